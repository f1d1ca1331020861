// Elementwise graph ops (add_requant, lut, lut_mul), the strided copy that materialises a layout view, and
// input quantization. All are HBM-bound grid-stride loops; LUTs are staged in LDS once per workgroup.
#include <algorithm>
#include <cmath>

#include "common.h"

namespace anvil {

constexpr int E_THREADS = 256;

static unsigned grid_for(long long n, int per_thread = 1) {
  long long b = (n + (long long)E_THREADS * per_thread - 1) / ((long long)E_THREADS * per_thread);
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return (unsigned)b;
}

// -------------------------------------------------------------------------------------------- add_requant
// out = clamp_out((a Ma + b Mb + 2^(s-1)) >> s), each product and the sum checked against int32
// (anvil/semantics.py:106-115).
template <typename TA, typename TB, typename TO>
__global__ __launch_bounds__(E_THREADS) void add_requant_kernel(const TA* __restrict__ a, const TB* __restrict__ b,
                                                                 int ma, int mb, int shift, long long rnd, long long n,
                                                                 TO* __restrict__ out, int lo, int hi,
                                                                 unsigned* flags) {
  unsigned bad = 0;
  for (long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x; i < n; i += (long long)gridDim.x * E_THREADS) {
    const long long pa = (long long)a[i] * ma, pb = (long long)b[i] * mb;
    const long long acc = pa + pb;
    bad |= (pa < I32_MIN) | (pa > I32_MAX) | (pb < I32_MIN) | (pb > I32_MAX) | (acc < I32_MIN) | (acc > I32_MAX);
    out[i] = (TO)requant_checked((int)acc, 1, shift, rnd, lo, hi, bad);
  }
  if (bad) raise_flag(flags, FLAG_OVERFLOW);
}

// ------------------------------------------------------------------------------------- 16-element chunks
// The vector kernels below take 16 elements a lane per step (chunk c = elements 16 c .. 16 c + 15): one 16-byte
// access per int8 operand, two per int16 operand, so every load and store is a full dwordx4 and a wave moves whole
// 1 KiB (or 2 KiB) spans. They need 16-byte aligned arrays; the n % 16 trailing elements go to the one-element
// kernels, whose arithmetic is the same.
template <typename T>
__device__ __forceinline__ void load16(const T* __restrict__ p, long long c, int v[16]) {
  if constexpr (sizeof(T) == 1) {
    const uint4 w = reinterpret_cast<const uint4*>(p)[c];
    const unsigned d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = (int)(int8_t)(d[e >> 2] >> (8 * (e & 3)));
  } else {
    const uint4 w0 = reinterpret_cast<const uint4*>(p)[2 * c], w1 = reinterpret_cast<const uint4*>(p)[2 * c + 1];
    const unsigned d[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = (int)(int16_t)(d[e >> 1] >> (16 * (e & 1)));
  }
}

// 16 results already inside T's range
template <typename T>
__device__ __forceinline__ void store16(T* __restrict__ p, long long c, const int v[16]) {
  if constexpr (sizeof(T) == 1) {
    reinterpret_cast<uint4*>(p)[c] = uint4{pack4(v[0], v[1], v[2], v[3]), pack4(v[4], v[5], v[6], v[7]),
                                           pack4(v[8], v[9], v[10], v[11]), pack4(v[12], v[13], v[14], v[15])};
  } else {
    unsigned d[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) d[q] = __builtin_amdgcn_perm((unsigned)v[2 * q + 1], (unsigned)v[2 * q], 0x05040100u);
    reinterpret_cast<uint4*>(p)[2 * c] = uint4{d[0], d[1], d[2], d[3]};
    reinterpret_cast<uint4*>(p)[2 * c + 1] = uint4{d[4], d[5], d[6], d[7]};
  }
}

// add_requant over 16-element chunks. CHECKED repeats add_requant_kernel's int32 checks; otherwise the graph's
// static proof keeps a Ma + b Mb + rnd inside int32 and it is computed in 32 bits, with 24-bit multiplies (MUL24)
// when |Ma|, |Mb| < 2^23 (|a|, |b| <= 2^15 as i8 / i16).
template <typename TA, typename TB, typename TO, bool CHECKED, bool MUL24>
__global__ __launch_bounds__(E_THREADS) void add_requant_vec(const TA* __restrict__ a, const TB* __restrict__ b,
                                                              int ma, int mb, int shift, int rnd, long long n16,
                                                              TO* __restrict__ out, unsigned* flags) {
  constexpr int lo = sizeof(TO) == 1 ? -128 : -32768, hi = sizeof(TO) == 1 ? 127 : 32767;
  unsigned bad = 0;
  for (long long c = (long long)blockIdx.x * E_THREADS + threadIdx.x; c < n16; c += (long long)gridDim.x * E_THREADS) {
    int va[16], vb[16], o[16];
    load16(a, c, va);
    load16(b, c, vb);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if constexpr (CHECKED) {
        const long long pa = (long long)va[e] * ma, pb = (long long)vb[e] * mb, acc = pa + pb;
        bad |= (pa < I32_MIN) | (pa > I32_MAX) | (pb < I32_MIN) | (pb > I32_MAX) | (acc < I32_MIN) | (acc > I32_MAX);
        o[e] = requant_checked((int)acc, 1, shift, rnd, lo, hi, bad);
      } else {
        const int x = MUL24 ? __mul24(va[e], ma) + __mul24(vb[e], mb) + rnd : va[e] * ma + vb[e] * mb + rnd;
        o[e] = min(max(x >> shift, lo), hi);
      }
    }
    store16(out, c, o);
  }
  if (CHECKED && bad) raise_flag(flags, FLAG_OVERFLOW);
}

// ------------------------------------------------------------------------------------------------ lut ops
__global__ __launch_bounds__(E_THREADS) void lut_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ table,
                                                         long long n, int8_t* __restrict__ out) {
  __shared__ int8_t t_s[256];
  t_s[threadIdx.x] = table[threadIdx.x];
  __syncthreads();
  for (long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x; i < n; i += (long long)gridDim.x * E_THREADS)
    out[i] = t_s[x[i] + 128];
}

__global__ __launch_bounds__(E_THREADS) void lut_mul_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ y,
                                                             const int8_t* __restrict__ table, int mult, int shift,
                                                             long long rnd, long long n, int8_t* __restrict__ out,
                                                             unsigned* flags) {
  __shared__ int8_t t_s[256];
  t_s[threadIdx.x] = table[threadIdx.x];
  __syncthreads();
  unsigned bad = 0;
  for (long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x; i < n; i += (long long)gridDim.x * E_THREADS)
    out[i] = (int8_t)requant_checked((int)t_s[x[i] + 128] * (int)y[i], mult, shift, rnd, -128, 127, bad);
  if (bad) raise_flag(flags, FLAG_OVERFLOW);
}

// lut and lut_mul over 16-element chunks. The table is staged rotated (the entry of v at index v & 255), so a
// lookup's index is the operand byte itself. lut_mul: |T[x] y| <= 2^14, so with |M| < 2^23 (MUL24) T[x] y M + rnd is
// one 24-bit multiply-add after the product; CHECKED keeps lut_mul_kernel's int32 checks.
__global__ __launch_bounds__(E_THREADS) void lut_vec(const int8_t* __restrict__ x, const int8_t* __restrict__ table,
                                                      long long n16, int8_t* __restrict__ out) {
  __shared__ int8_t t_s[256];
  t_s[threadIdx.x ^ 128] = table[threadIdx.x];
  __syncthreads();
  for (long long c = (long long)blockIdx.x * E_THREADS + threadIdx.x; c < n16; c += (long long)gridDim.x * E_THREADS) {
    const uint4 w = reinterpret_cast<const uint4*>(x)[c];
    const unsigned d[4] = {w.x, w.y, w.z, w.w};
    int o[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] = t_s[(d[e >> 2] >> (8 * (e & 3))) & 255];
    reinterpret_cast<uint4*>(out)[c] = uint4{pack4(o[0], o[1], o[2], o[3]), pack4(o[4], o[5], o[6], o[7]),
                                             pack4(o[8], o[9], o[10], o[11]), pack4(o[12], o[13], o[14], o[15])};
  }
}

template <bool CHECKED, bool MUL24>
__global__ __launch_bounds__(E_THREADS) void lut_mul_vec(const int8_t* __restrict__ x, const int8_t* __restrict__ y,
                                                          const int8_t* __restrict__ table, int mult, int shift,
                                                          int rnd, long long n16, int8_t* __restrict__ out,
                                                          unsigned* flags) {
  __shared__ int8_t t_s[256];
  t_s[threadIdx.x ^ 128] = table[threadIdx.x];
  __syncthreads();
  unsigned bad = 0;
  for (long long c = (long long)blockIdx.x * E_THREADS + threadIdx.x; c < n16; c += (long long)gridDim.x * E_THREADS) {
    const uint4 w = reinterpret_cast<const uint4*>(x)[c];
    const unsigned d[4] = {w.x, w.y, w.z, w.w};
    int vy[16], o[16];
    load16(y, c, vy);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int p = (int)t_s[(d[e >> 2] >> (8 * (e & 3))) & 255] * vy[e];
      if constexpr (CHECKED) {
        o[e] = requant_checked(p, mult, shift, rnd, -128, 127, bad);
      } else {
        const int v = MUL24 ? __mul24(p, mult) + rnd : p * mult + rnd;
        o[e] = min(max(v >> shift, -128), 127);
      }
    }
    store16(out, c, o);
  }
  if (CHECKED && bad) raise_flag(flags, FLAG_OVERFLOW);
}

// ------------------------------------------------------------------------------------------ strided copy
struct CopyArgs {
  const char* src;
  char* dst;
  int rank;
  long long dims[6];
  long long strides[6];
  long long n;
};

template <typename T>
__global__ __launch_bounds__(E_THREADS) void copy_strided_kernel(CopyArgs c) {
  const T* __restrict__ s = reinterpret_cast<const T*>(c.src);
  T* __restrict__ d = reinterpret_cast<T*>(c.dst);
  for (long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x; i < c.n; i += (long long)gridDim.x * E_THREADS) {
    long long rem = i, off = 0;
    for (int a = c.rank - 1; a >= 0; --a) {
      const long long q = rem / c.dims[a];
      off += (rem - q * c.dims[a]) * c.strides[a];
      rem = q;
    }
    d[i] = s[off];
  }
}

// A dense view (strides of a row-major array) with 16-byte-aligned ends is a plain byte copy: 16 bytes a lane,
// four independent loads in flight per lane per pass.
__global__ __launch_bounds__(E_THREADS) void copy_dense16_kernel(const uint4* __restrict__ s, uint4* __restrict__ d,
                                                                 long long n16) {
  const long long stride = (long long)gridDim.x * E_THREADS;
  long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 v0 = s[i], v1 = s[i + stride], v2 = s[i + 2 * stride], v3 = s[i + 3 * stride];
    d[i] = v0;
    d[i + stride] = v1;
    d[i + 2 * stride] = v2;
    d[i + 3 * stride] = v3;
  }
  for (; i < n16; i += stride) d[i] = s[i];
}

// --------------------------------------------------------------------------------------------- quantize
// A NaN or infinite x raises FLAG_NONFINITE (the reference refuses such an input before quantizing) and stores 0.
template <typename TI, typename TO>
__global__ __launch_bounds__(E_THREADS) void quantize_kernel(const TI* __restrict__ x, double scale, long long n,
                                                              TO* __restrict__ out, int lo, int hi, unsigned* flags) {
  bool bad = false;
  for (long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x; i < n; i += (long long)gridDim.x * E_THREADS) {
    const double xv = (double)x[i];
    const bool fin = isfinite(xv);
    bad |= !fin;
    double v = rint(xv / scale);
    v = v < lo ? lo : (v > hi ? hi : v);
    out[i] = fin ? (TO)v : (TO)0;
  }
  if (bad) raise_flag(flags, FLAG_NONFINITE);
}

// quantize over 16-element chunks: 64 (float) or 128 (double) input bytes and one or two 16-byte stores a lane; each
// element as in quantize_kernel (float64 division, round half to even, clamp; a non-finite element flags and stores 0)
template <typename TI, typename TO>
__global__ __launch_bounds__(E_THREADS) void quantize_vec(const TI* __restrict__ x, double scale, long long n16,
                                                           TO* __restrict__ out, int lo, int hi, unsigned* flags) {
  bool bad = false;
  for (long long c = (long long)blockIdx.x * E_THREADS + threadIdx.x; c < n16; c += (long long)gridDim.x * E_THREADS) {
    double xv[16];
    if constexpr (sizeof(TI) == 4) {
      const float4* p = reinterpret_cast<const float4*>(x) + 4 * c;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = p[q];
        xv[4 * q] = f.x, xv[4 * q + 1] = f.y, xv[4 * q + 2] = f.z, xv[4 * q + 3] = f.w;
      }
    } else {
      const double2* p = reinterpret_cast<const double2*>(x) + 8 * c;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const double2 f = p[q];
        xv[2 * q] = f.x, xv[2 * q + 1] = f.y;
      }
    }
    int o[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const bool fin = isfinite(xv[e]);
      bad |= !fin;
      double v = rint(xv[e] / scale);
      v = v < lo ? lo : (v > hi ? hi : v);
      o[e] = fin ? (int)v : 0;
    }
    store16(out, c, o);
  }
  if (bad) raise_flag(flags, FLAG_NONFINITE);
}

// the float prelude of a token model: out[r][c] = clamp_out(rint((wte[ids[r]][c] + wpe[r % T][c]) / scale)), the
// float32 tables read as float64, as the host computes x = wte[ids] + wpe[positions] in float64 and quantizes it
template <typename TO>
__global__ __launch_bounds__(E_THREADS) void embed_quantize_kernel(const int64_t* __restrict__ ids,
                                                                   const float* __restrict__ wte,
                                                                   const float* __restrict__ wpe, long long rows,
                                                                   int T, int C, int vocab, double scale,
                                                                   TO* __restrict__ out, int lo, int hi,
                                                                   unsigned* flags) {
  const long long n = rows * C;
  for (long long i = (long long)blockIdx.x * E_THREADS + threadIdx.x; i < n; i += (long long)gridDim.x * E_THREADS) {
    const long long r = i / C;
    const int c = (int)(i - r * C);
    const long long id = ids[r];
    if (id < 0 || id >= vocab) {
      raise_flag(flags, FLAG_RANGE);
      out[i] = 0;
      continue;
    }
    double v = rint(((double)wte[id * C + c] + (double)wpe[(r % T) * C + c]) / scale);
    v = v < lo ? lo : (v > hi ? hi : v);
    out[i] = (TO)v;
  }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// One-element kernel over elements [from, n) of the operands (the tail past the vector kernel's chunks, or every
// element when an operand is not 16-byte aligned).
template <typename TA, typename TB, typename TO>
static void launch_add_scalar(anvil_ctx* ctx, const TA* a, const TB* b, int ma, int mb, int s, long long from,
                              long long n, TO* out) {
  if (from >= n) return;
  const long long rnd = s ? (1ll << (s - 1)) : 0;
  const int lo = sizeof(TO) == 1 ? -128 : -32768, hi = sizeof(TO) == 1 ? 127 : 32767;
  ANVIL_LAUNCH((add_requant_kernel<TA, TB, TO>), dim3(grid_for(n - from)), dim3(E_THREADS), 0, ctx->stream,
               a + from, b + from, ma, mb, s, rnd, n - from, out + from, lo, hi, ctx->flags);
}

template <typename TA, typename TB, typename TO>
static void launch_add_typed(anvil_ctx* ctx, const TA* a, const TB* b, int ma, int mb, int s, long long n, TO* out,
                             bool unchecked) {
  const long long n16 = (al16(a) && al16(b) && al16(out)) ? n / 16 : 0;
  if (n16) {
    const int rnd = s ? (int)(1u << (s - 1)) : 0;
    const bool m24 = ma > -(1 << 23) && ma < (1 << 23) && mb > -(1 << 23) && mb < (1 << 23);
    const dim3 gr(grid_for(n16)), bl(E_THREADS);
    if (!unchecked)
      ANVIL_LAUNCH((add_requant_vec<TA, TB, TO, true, false>), gr, bl, 0, ctx->stream, a, b, ma, mb, s, rnd, n16, out,
                   ctx->flags);
    else if (m24)
      ANVIL_LAUNCH((add_requant_vec<TA, TB, TO, false, true>), gr, bl, 0, ctx->stream, a, b, ma, mb, s, rnd, n16, out,
                   ctx->flags);
    else
      ANVIL_LAUNCH((add_requant_vec<TA, TB, TO, false, false>), gr, bl, 0, ctx->stream, a, b, ma, mb, s, rnd, n16,
                   out, ctx->flags);
  }
  launch_add_scalar(ctx, a, b, ma, mb, s, n16 * 16, n, out);
}

// embed_quantize four columns a lane: one wave a row (a workgroup takes four rows, then strides by the grid), its
// lanes over the row's C / 4 float4 columns of the token's and the position's rows, so no lane divides by C; one
// 4-byte (i8) or 8-byte (i16) store. Each element as in embed_quantize_kernel, with the division replaced where
// that cannot change the result: q = fl(x fl(1 / scale)) is within 3 ulp of x / scale (inv a normal double), so
// rint(q) is the rint of the correctly rounded quotient unless q lies within 2^-50 |q| of a half-integer (the only
// points where rint changes value); such an element, and every element when inv is not normal, takes the quotient.
// q - floor(q) is exact, so the test is too; an infinite or NaN q fails it and takes the quotient.
template <typename TO>
__global__ __launch_bounds__(E_THREADS) void embed_quantize_vec4(const int64_t* __restrict__ ids,
                                                                 const float* __restrict__ wte,
                                                                 const float* __restrict__ wpe, long long rows,
                                                                 int T, int C, int vocab, double scale, double inv,
                                                                 int use_inv, TO* __restrict__ out, int lo, int hi,
                                                                 unsigned* flags) {
  const int c4 = C >> 2, lane = threadIdx.x & 63;
  const long long step = (long long)gridDim.x * (E_THREADS / 64);
  for (long long r = (long long)blockIdx.x * (E_THREADS / 64) + (threadIdx.x >> 6); r < rows; r += step) {
    const long long id = ids[r];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && lane == 0) raise_flag(flags, FLAG_RANGE);
    const float* te = wte + (ok ? id : 0) * C;
    const float* pe = wpe + (long long)(int)(r % T) * C;
    for (int j = lane; j < c4; j += 64) {
      int o[4] = {0, 0, 0, 0};
      if (ok) {
        const float4 w = reinterpret_cast<const float4*>(te)[j];
        const float4 p = reinterpret_cast<const float4*>(pe)[j];
        const double xs[4] = {(double)w.x + (double)p.x, (double)w.y + (double)p.y, (double)w.z + (double)p.z,
                              (double)w.w + (double)p.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const double q = xs[e] * inv;
          double v = rint(q);
          if (!(use_inv && fabs(q - floor(q) - 0.5) > 0x1p-50 * fabs(q))) v = rint(xs[e] / scale);
          v = v < lo ? lo : (v > hi ? hi : v);
          o[e] = (int)v;
        }
      }
      const long long i = r * c4 + j;
      if constexpr (sizeof(TO) == 1) {
        reinterpret_cast<unsigned*>(out)[i] = pack4(o[0], o[1], o[2], o[3]);
      } else {
        reinterpret_cast<uint2*>(out)[i] = uint2{__builtin_amdgcn_perm((unsigned)o[1], (unsigned)o[0], 0x05040100u),
                                                 __builtin_amdgcn_perm((unsigned)o[3], (unsigned)o[2], 0x05040100u)};
      }
    }
  }
}

template <typename TA, typename TB>
static void launch_add(anvil_ctx* ctx, const void* a, const void* b, int ma, int mb, int s, long long n, void* out,
                       int out_dtype, bool unchecked) {
  if (out_dtype == ANVIL_I8)
    launch_add_typed(ctx, (const TA*)a, (const TB*)b, ma, mb, s, n, (int8_t*)out, unchecked);
  else
    launch_add_typed(ctx, (const TA*)a, (const TB*)b, ma, mb, s, n, (int16_t*)out, unchecked);
}

}  // namespace anvil

using namespace anvil;

extern "C" {

int anvil_add_requant(anvil_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype, int32_t ma, int32_t mb,
                      int shift, int64_t n, void* out, int out_dtype) {
  return anvil_add_requant_ex(ctx, a, a_dtype, b, b_dtype, ma, mb, shift, n, out, out_dtype, 0);
}

int anvil_add_requant_ex(anvil_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype, int32_t ma,
                         int32_t mb, int shift, int64_t n, void* out, int out_dtype, int flags) {
  if (int r = check_ctx(ctx)) return r;
  if (flags & ~ANVIL_OP_UNCHECKED) return set_error(ANVIL_E_VALUE, "anvil_add_requant_ex: unknown flags %d", flags);
  const bool unchecked = (flags & ANVIL_OP_UNCHECKED) != 0;
  if (!a || !b || !out) return set_error(ANVIL_E_VALUE, "anvil_add_requant: null pointer");
  auto wide = [](int d) { return d == ANVIL_I8 || d == ANVIL_I16; };
  if (!wide(a_dtype) || !wide(b_dtype) || !wide(out_dtype))
    return set_error(ANVIL_E_VALUE, "add_requant operands and result must be i8 or i16");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (n < 0) return set_error(ANVIL_E_VALUE, "anvil_add_requant: negative size");
  if (n == 0) return ANVIL_OK;
  if (a_dtype == ANVIL_I8 && b_dtype == ANVIL_I8)
    launch_add<int8_t, int8_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype, unchecked);
  else if (a_dtype == ANVIL_I8)
    launch_add<int8_t, int16_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype, unchecked);
  else if (b_dtype == ANVIL_I8)
    launch_add<int16_t, int8_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype, unchecked);
  else
    launch_add<int16_t, int16_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype, unchecked);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_lut_i8(anvil_ctx* ctx, const int8_t* x, const int8_t* table, int64_t n, int8_t* out) {
  if (int r = check_ctx(ctx)) return r;
  if (!x || !table || !out) return set_error(ANVIL_E_VALUE, "anvil_lut_i8: null pointer");
  if (n < 0) return set_error(ANVIL_E_VALUE, "anvil_lut_i8: negative size");
  if (n == 0) return ANVIL_OK;
  const long long n16 = (al16(x) && al16(out)) ? n / 16 : 0;
  if (n16) ANVIL_LAUNCH(lut_vec, dim3(grid_for(n16)), dim3(E_THREADS), 0, ctx->stream, x, table, n16, out);
  if (n16 * 16 < n)
    ANVIL_LAUNCH(lut_kernel, dim3(grid_for(n - n16 * 16)), dim3(E_THREADS), 0, ctx->stream, x + n16 * 16, table,
                 (long long)(n - n16 * 16), out + n16 * 16);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_lut_mul(anvil_ctx* ctx, const int8_t* x, const int8_t* y, const int8_t* table, int32_t mult, int shift,
                  int64_t n, int8_t* out) {
  return anvil_lut_mul_ex(ctx, x, y, table, mult, shift, n, out, 0);
}

int anvil_lut_mul_ex(anvil_ctx* ctx, const int8_t* x, const int8_t* y, const int8_t* table, int32_t mult, int shift,
                     int64_t n, int8_t* out, int flags) {
  if (int r = check_ctx(ctx)) return r;
  if (flags & ~ANVIL_OP_UNCHECKED) return set_error(ANVIL_E_VALUE, "anvil_lut_mul_ex: unknown flags %d", flags);
  if (!x || !y || !table || !out) return set_error(ANVIL_E_VALUE, "anvil_lut_mul: null pointer");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (n < 0) return set_error(ANVIL_E_VALUE, "anvil_lut_mul: negative size");
  if (n == 0) return ANVIL_OK;
  const long long rnd = shift ? (1ll << (shift - 1)) : 0;
  const long long n16 = (al16(x) && al16(y) && al16(out)) ? n / 16 : 0;
  if (n16) {
    const dim3 gr(grid_for(n16)), bl(E_THREADS);
    if (!(flags & ANVIL_OP_UNCHECKED))
      ANVIL_LAUNCH((lut_mul_vec<true, false>), gr, bl, 0, ctx->stream, x, y, table, mult, shift, (int)rnd, n16, out,
                   ctx->flags);
    else if (mult > -(1 << 23) && mult < (1 << 23))
      ANVIL_LAUNCH((lut_mul_vec<false, true>), gr, bl, 0, ctx->stream, x, y, table, mult, shift, (int)rnd, n16, out,
                   ctx->flags);
    else
      ANVIL_LAUNCH((lut_mul_vec<false, false>), gr, bl, 0, ctx->stream, x, y, table, mult, shift, (int)rnd, n16,
                   out, ctx->flags);
  }
  const long long from = n16 * 16;
  if (from < n)
    ANVIL_LAUNCH(lut_mul_kernel, dim3(grid_for(n - from)), dim3(E_THREADS), 0, ctx->stream, x + from, y + from, table,
                 mult, shift, rnd, (long long)(n - from), out + from, ctx->flags);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_copy_strided(anvil_ctx* ctx, const void* src, void* dst, int elem_size, int rank, const int64_t* dims,
                       const int64_t* src_strides) {
  if (int r = check_ctx(ctx)) return r;
  if (!src || !dst || !dims || !src_strides) return set_error(ANVIL_E_VALUE, "anvil_copy_strided: null pointer");
  if (rank < 1 || rank > 6) return set_error(ANVIL_E_VALUE, "anvil_copy_strided: rank %d outside [1, 6]", rank);
  CopyArgs c;
  c.src = (const char*)src;
  c.dst = (char*)dst;
  c.rank = rank;
  c.n = 1;
  for (int i = 0; i < rank; ++i) {
    if (dims[i] < 1) return set_error(ANVIL_E_VALUE, "anvil_copy_strided: dim %d is %lld", i, (long long)dims[i]);
    c.dims[i] = dims[i];
    c.strides[i] = src_strides[i];
    c.n *= dims[i];
  }
  if (elem_size != 1 && elem_size != 2 && elem_size != 4)
    return set_error(ANVIL_E_VALUE, "anvil_copy_strided: element size %d", elem_size);
  bool dense = true;
  for (long long i = rank - 1, want = 1; i >= 0; want *= c.dims[i], --i) dense &= c.dims[i] == 1 || c.strides[i] == want;
  const long long bytes = c.n * elem_size;
  if (dense && bytes % 16 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0) {
    const long long n16 = bytes / 16;
    ANVIL_LAUNCH(copy_dense16_kernel, dim3(grid_for(n16, 4)), dim3(E_THREADS), 0, ctx->stream,
                 (const uint4*)src, (uint4*)dst, n16);
    ANVIL_LAUNCHED();
    return ANVIL_OK;
  }
  switch (elem_size) {
    case 1:
      ANVIL_LAUNCH(copy_strided_kernel<int8_t>, dim3(grid_for(c.n)), dim3(E_THREADS), 0, ctx->stream, c);
      break;
    case 2:
      ANVIL_LAUNCH(copy_strided_kernel<int16_t>, dim3(grid_for(c.n)), dim3(E_THREADS), 0, ctx->stream, c);
      break;
    case 4:
      ANVIL_LAUNCH(copy_strided_kernel<int32_t>, dim3(grid_for(c.n)), dim3(E_THREADS), 0, ctx->stream, c);
      break;
    default:
      return set_error(ANVIL_E_VALUE, "anvil_copy_strided: element size %d", elem_size);
  }
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_quantize(anvil_ctx* ctx, const void* x, int x_is_f64, double scale, int64_t n, void* out, int out_dtype) {
  if (int r = check_ctx(ctx)) return r;
  if (!x || !out) return set_error(ANVIL_E_VALUE, "anvil_quantize: null pointer");
  if (!(scale > 0)) return set_error(ANVIL_E_VALUE, "anvil_quantize: scale must be positive");
  if (out_dtype != ANVIL_I8 && out_dtype != ANVIL_I16) return set_error(ANVIL_E_VALUE, "quantize result i8 or i16");
  if (n <= 0) return n < 0 ? set_error(ANVIL_E_VALUE, "anvil_quantize: negative size") : ANVIL_OK;
  const int lo = dtype_lo(out_dtype), hi = dtype_hi(out_dtype);
  const long long n16 = (al16(x) && al16(out)) ? n / 16 : 0;
  if (n16) {
    const dim3 g16(grid_for(n16)), b16(E_THREADS);
    if (x_is_f64 && out_dtype == ANVIL_I8)
      ANVIL_LAUNCH((quantize_vec<double, int8_t>), g16, b16, 0, ctx->stream, (const double*)x, scale, n16,
                   (int8_t*)out, lo, hi, ctx->flags);
    else if (x_is_f64)
      ANVIL_LAUNCH((quantize_vec<double, int16_t>), g16, b16, 0, ctx->stream, (const double*)x, scale, n16,
                   (int16_t*)out, lo, hi, ctx->flags);
    else if (out_dtype == ANVIL_I8)
      ANVIL_LAUNCH((quantize_vec<float, int8_t>), g16, b16, 0, ctx->stream, (const float*)x, scale, n16,
                   (int8_t*)out, lo, hi, ctx->flags);
    else
      ANVIL_LAUNCH((quantize_vec<float, int16_t>), g16, b16, 0, ctx->stream, (const float*)x, scale, n16,
                   (int16_t*)out, lo, hi, ctx->flags);
  }
  const long long from = n16 * 16;
  if (from == n) {
    ANVIL_LAUNCHED();
    return ANVIL_OK;
  }
  n -= from;
  x = (const char*)x + from * (x_is_f64 ? 8 : 4);
  out = (char*)out + from * (out_dtype == ANVIL_I8 ? 1 : 2);
  dim3 gr(grid_for(n)), bl(E_THREADS);
  if (x_is_f64 && out_dtype == ANVIL_I8)
    ANVIL_LAUNCH((quantize_kernel<double, int8_t>), gr, bl, 0, ctx->stream, (const double*)x, scale, (long long)n,
                       (int8_t*)out, lo, hi, ctx->flags);
  else if (x_is_f64)
    ANVIL_LAUNCH((quantize_kernel<double, int16_t>), gr, bl, 0, ctx->stream, (const double*)x, scale,
                       (long long)n, (int16_t*)out, lo, hi, ctx->flags);
  else if (out_dtype == ANVIL_I8)
    ANVIL_LAUNCH((quantize_kernel<float, int8_t>), gr, bl, 0, ctx->stream, (const float*)x, scale, (long long)n,
                       (int8_t*)out, lo, hi, ctx->flags);
  else
    ANVIL_LAUNCH((quantize_kernel<float, int16_t>), gr, bl, 0, ctx->stream, (const float*)x, scale,
                       (long long)n, (int16_t*)out, lo, hi, ctx->flags);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_embed_quantize(anvil_ctx* ctx, const int64_t* ids, int64_t rows, int T, int C, const float* wte,
                         int vocab, const float* wpe, double scale, void* out, int out_dtype) {
  if (!ids || !wte || !wpe || !out) return set_error(ANVIL_E_VALUE, "anvil_embed_quantize: null pointer");
  if (rows < 0 || T < 1 || C < 1 || vocab < 1 || rows % T)
    return set_error(ANVIL_E_VALUE, "anvil_embed_quantize: rows %lld must be a multiple of T %d (C %d, vocab %d)",
                     (long long)rows, T, C, vocab);
  if (!(scale > 0) || scale == HUGE_VAL) return set_error(ANVIL_E_VALUE, "anvil_embed_quantize: scale must be > 0");
  if (out_dtype != ANVIL_I8 && out_dtype != ANVIL_I16)
    return set_error(ANVIL_E_VALUE, "anvil_embed_quantize: result dtype must be i8 or i16");
  if (rows * C / C != rows) return set_error(ANVIL_E_VALUE, "anvil_embed_quantize: size overflow");
  if (int r = check_ctx(ctx)) return r;
  if (rows == 0) return ANVIL_OK;
  const long long n = rows * C;
  const int lo = dtype_lo(out_dtype), hi = dtype_hi(out_dtype);
  if (C % 4 == 0 && al16(wte) && al16(wpe) && ((uintptr_t)out & (out_dtype == ANVIL_I8 ? 3 : 7)) == 0) {
    const dim3 gr((unsigned)std::min<long long>((rows + 3) / 4, 65536)), bl(E_THREADS);   // four rows a workgroup
    const double inv = 1.0 / scale;
    const int use_inv = std::isnormal(inv) ? 1 : 0;
    if (out_dtype == ANVIL_I8)
      ANVIL_LAUNCH(embed_quantize_vec4<int8_t>, gr, bl, 0, ctx->stream, ids, wte, wpe, (long long)rows, T, C, vocab,
                   scale, inv, use_inv, (int8_t*)out, lo, hi, ctx->flags);
    else
      ANVIL_LAUNCH(embed_quantize_vec4<int16_t>, gr, bl, 0, ctx->stream, ids, wte, wpe, (long long)rows, T, C, vocab,
                   scale, inv, use_inv, (int16_t*)out, lo, hi, ctx->flags);
    ANVIL_LAUNCHED();
    return ANVIL_OK;
  }
  if (out_dtype == ANVIL_I8)
    ANVIL_LAUNCH(embed_quantize_kernel<int8_t>, dim3(grid_for(n)), dim3(E_THREADS), 0, ctx->stream, ids, wte, wpe,
                       (long long)rows, T, C, vocab, scale, (int8_t*)out, lo, hi, ctx->flags);
  else
    ANVIL_LAUNCH(embed_quantize_kernel<int16_t>, dim3(grid_for(n)), dim3(E_THREADS), 0, ctx->stream, ids, wte,
                       wpe, (long long)rows, T, C, vocab, scale, (int16_t*)out, lo, hi, ctx->flags);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

}  // extern "C"
