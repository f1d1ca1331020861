// Elementwise graph ops (add_requant, lut, lut_mul), the strided copy that materialises a layout view, and
// input quantization. All are HBM-bound grid-stride loops; LUTs are staged in LDS once per workgroup.
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

template <typename TA, typename TB>
static void launch_add(anvil_ctx* ctx, const void* a, const void* b, int ma, int mb, int s, long long n, void* out,
                       int out_dtype) {
  const long long rnd = s ? (1ll << (s - 1)) : 0;
  if (out_dtype == ANVIL_I8)
    ANVIL_LAUNCH((add_requant_kernel<TA, TB, int8_t>), dim3(grid_for(n)), dim3(E_THREADS), 0, ctx->stream,
                       (const TA*)a, (const TB*)b, ma, mb, s, rnd, n, (int8_t*)out, -128, 127, ctx->flags);
  else
    ANVIL_LAUNCH((add_requant_kernel<TA, TB, int16_t>), dim3(grid_for(n)), dim3(E_THREADS), 0, ctx->stream,
                       (const TA*)a, (const TB*)b, ma, mb, s, rnd, n, (int16_t*)out, -32768, 32767, ctx->flags);
}

}  // namespace anvil

using namespace anvil;

extern "C" {

int anvil_add_requant(anvil_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype, int32_t ma, int32_t mb,
                      int shift, int64_t n, void* out, int out_dtype) {
  if (int r = check_ctx(ctx)) return r;
  if (!a || !b || !out) return set_error(ANVIL_E_VALUE, "anvil_add_requant: null pointer");
  auto wide = [](int d) { return d == ANVIL_I8 || d == ANVIL_I16; };
  if (!wide(a_dtype) || !wide(b_dtype) || !wide(out_dtype))
    return set_error(ANVIL_E_VALUE, "add_requant operands and result must be i8 or i16");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (n < 0) return set_error(ANVIL_E_VALUE, "anvil_add_requant: negative size");
  if (n == 0) return ANVIL_OK;
  if (a_dtype == ANVIL_I8 && b_dtype == ANVIL_I8)
    launch_add<int8_t, int8_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype);
  else if (a_dtype == ANVIL_I8)
    launch_add<int8_t, int16_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype);
  else if (b_dtype == ANVIL_I8)
    launch_add<int16_t, int8_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype);
  else
    launch_add<int16_t, int16_t>(ctx, a, b, ma, mb, shift, n, out, out_dtype);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_lut_i8(anvil_ctx* ctx, const int8_t* x, const int8_t* table, int64_t n, int8_t* out) {
  if (int r = check_ctx(ctx)) return r;
  if (!x || !table || !out) return set_error(ANVIL_E_VALUE, "anvil_lut_i8: null pointer");
  if (n < 0) return set_error(ANVIL_E_VALUE, "anvil_lut_i8: negative size");
  if (n == 0) return ANVIL_OK;
  ANVIL_LAUNCH(lut_kernel, dim3(grid_for(n)), dim3(E_THREADS), 0, ctx->stream, x, table, (long long)n, out);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

int anvil_lut_mul(anvil_ctx* ctx, const int8_t* x, const int8_t* y, const int8_t* table, int32_t mult, int shift,
                  int64_t n, int8_t* out) {
  if (int r = check_ctx(ctx)) return r;
  if (!x || !y || !table || !out) return set_error(ANVIL_E_VALUE, "anvil_lut_mul: null pointer");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (n < 0) return set_error(ANVIL_E_VALUE, "anvil_lut_mul: negative size");
  if (n == 0) return ANVIL_OK;
  const long long rnd = shift ? (1ll << (shift - 1)) : 0;
  ANVIL_LAUNCH(lut_mul_kernel, dim3(grid_for(n)), dim3(E_THREADS), 0, ctx->stream, x, y, table, mult, shift,
                     rnd, (long long)n, out, ctx->flags);
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
