// Row reductions of the graph: rmsnorm_int and softmax_lut. One wavefront (64 lanes) per row; the row
// statistics (sum of squares, max, exp sum) are reduced across the wave with DPP-backed shuffles, so every lane
// ends with the same exact integer and the per-element pass needs no LDS round trip.
#include "common.h"

namespace anvil {

constexpr int R_THREADS = 256, R_WAVES = R_THREADS / 64;

__device__ __forceinline__ long long wave_sum(long long v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

// Python floor division (the reference's `//`) on int64.
__device__ __forceinline__ long long floordiv(long long n, long long d) {
  long long q = n / d;
  if ((n % d != 0) && ((n < 0) != (d < 0))) --q;
  return q;
}

// ---------------------------------------------------------------------------------------------- rmsnorm_int
// Per row (anvil/semantics.py:164-182): ss = e + sum((x^2 + 2^(c-1)) >> c); (i, k) = rsqrt_index(ss, n);
// out = requant(x * w * lut[i], M, s + k).
template <typename T>
__global__ __launch_bounds__(R_THREADS) void rmsnorm_kernel(const T* __restrict__ x, const int8_t* __restrict__ w,
                                                             const int* __restrict__ lut, int lut_len, int mult,
                                                             int shift, int c, int e, long long rows, int cols,
                                                             int8_t* __restrict__ out, unsigned* flags) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * R_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  const long long rc = round_term(c);
  long long ss = 0;
  for (int j = lane; j < cols; j += 64) {
    const long long v = xr[j];
    long long sq = v * v;
    if (c) sq = (sq + rc) >> c;
    ss += sq;
  }
  ss = wave_sum(ss) + e;
  unsigned bad = ss > I32_MAX;
  int k = 0;
  long long idx = ss;
  while (idx >= lut_len) {
    idx >>= 2;
    ++k;
  }
  const int sh = shift + k;
  if (sh > 31) {
    if (lane == 0) raise_flag(flags, FLAG_SHIFT);
    return;
  }
  const long long r = lut[idx];
  const long long rnd = round_term(sh);
  int8_t* o = out + row * cols;
  for (int j = lane; j < cols; j += 64) {
    const long long xwr = (long long)xr[j] * w[j] * r;
    bad |= (xwr < I32_MIN) | (xwr > I32_MAX);
    o[j] = (int8_t)requant_checked((int)xwr, mult, sh, rnd, -128, 127, bad);
  }
  if (bad) raise_flag(flags, FLAG_OVERFLOW);
}

// ---------------------------------------------------------------------------------------------- softmax_lut
// Per row i of (..., t1, t2) (anvil/lower/graph_to_tensor.py:352-398): kept columns j <= i when causal;
// m = max(-128, max kept x); e_j = lut[x_j - m + 255]; S = sum e; p_j = (e_j one + S // 2) // S, masked 0.
template <typename TO>
__global__ __launch_bounds__(R_THREADS) void softmax_kernel(const int8_t* __restrict__ x, const int* __restrict__ lut,
                                                             int one, int causal, long long rows, int t1, int t2,
                                                             TO* __restrict__ out, unsigned* flags) {
  __shared__ int lut_s[256];
  lut_s[threadIdx.x] = lut[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * R_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int i = (int)(row % t1);
  const int kept = causal ? min(i + 1, t2) : t2;
  const int8_t* xr = x + row * t2;
  int m = -128;
  for (int j = lane; j < kept; j += 64) m = max(m, (int)xr[j]);
  m = wave_max(m);
  long long S = 0;
  for (int j = lane; j < kept; j += 64) S += lut_s[xr[j] - m + 255];
  S = wave_sum(S);
  unsigned bad = (S < I32_MIN) | (S > I32_MAX);
  if (S == 0) {
    if (lane == 0) raise_flag(flags, FLAG_ZERODIV);
    return;
  }
  const long long half = floordiv(S, 2);
  TO* o = out + row * t2;
  if (S > 0 && S <= I32_MAX) {
    const unsigned us = (unsigned)S;
    for (int j = lane; j < t2; j += 64) {
      long long p = 0;
      if (j < kept) {
        const long long n = (long long)lut_s[xr[j] - m + 255] * one + half;
        bad |= (n < I32_MIN) | (n > I32_MAX);
        p = n >= 0 ? (long long)((unsigned)n / us) : floordiv(n, S);
      }
      o[j] = (TO)p;
    }
  } else {
    for (int j = lane; j < t2; j += 64) {
      long long p = 0;
      if (j < kept) {
        const long long n = (long long)lut_s[xr[j] - m + 255] * one + half;
        bad |= (n < I32_MIN) | (n > I32_MAX);
        p = floordiv(n, S);
      }
      o[j] = (TO)p;
    }
  }
  if (bad) raise_flag(flags, FLAG_OVERFLOW);
}

}  // namespace anvil

using namespace anvil;

extern "C" int anvil_rmsnorm_int(anvil_ctx* ctx, const void* x, int x_dtype, const int8_t* w, const int32_t* lut,
                                 int lut_len, int32_t mult, int shift, int ss_shift, int32_t ss_init, int64_t rows,
                                 int cols, int8_t* out) {
  if (int r = check_ctx(ctx)) return r;
  if (!x || !w || !lut || !out) return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: null pointer");
  if (rows < 0 || cols < 1 || lut_len < 1) return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: bad size");
  if (x_dtype != ANVIL_I8 && x_dtype != ANVIL_I16) return set_error(ANVIL_E_VALUE, "rmsnorm x must be i8 or i16");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (ss_shift < 0 || ss_shift > 30) return set_error(ANVIL_E_VALUE, "ss_shift %d outside [0, 30]", ss_shift);
  if (ss_init < 0) return set_error(ANVIL_E_VALUE, "ss_init %d negative", ss_init);
  if (rows == 0) return ANVIL_OK;
  const long long blocks = (rows + R_WAVES - 1) / R_WAVES;
  if (blocks > (1ll << 31) - 1) return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: too many rows");
  if (x_dtype == ANVIL_I8)
    hipLaunchKernelGGL(rmsnorm_kernel<int8_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream,
                       (const int8_t*)x, w, lut, lut_len, mult, shift, ss_shift, ss_init, (long long)rows, cols, out,
                       ctx->flags);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<int16_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream,
                       (const int16_t*)x, w, lut, lut_len, mult, shift, ss_shift, ss_init, (long long)rows, cols,
                       out, ctx->flags);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

extern "C" int anvil_softmax_lut(anvil_ctx* ctx, const int8_t* x, const int32_t* lut, int32_t one, int causal,
                                 int64_t batch, int t1, int t2, void* out, int out_dtype) {
  if (int r = check_ctx(ctx)) return r;
  if (!x || !lut || !out) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: null pointer");
  if (batch < 0 || t1 < 1 || t2 < 1) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: bad size");
  if (out_dtype != ANVIL_I8 && out_dtype != ANVIL_I32)
    return set_error(ANVIL_E_VALUE, "softmax result must be i8 or i32");
  if (one < 1 || (out_dtype == ANVIL_I8 && one > 127))
    return set_error(ANVIL_E_VALUE, "one=%d does not fit the result dtype", one);
  const long long rows = batch * t1;
  if (rows == 0) return ANVIL_OK;
  const long long blocks = (rows + R_WAVES - 1) / R_WAVES;
  if (blocks > (1ll << 31) - 1) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: too many rows");
  if (out_dtype == ANVIL_I8)
    hipLaunchKernelGGL(softmax_kernel<int8_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream, x, lut, one,
                       causal, rows, t1, t2, (int8_t*)out, ctx->flags);
  else
    hipLaunchKernelGGL(softmax_kernel<int32_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream, x, lut, one,
                       causal, rows, t1, t2, (int32_t*)out, ctx->flags);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}
