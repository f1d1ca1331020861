// int8 x int8 -> int32 GEMM on CDNA4 MFMA with the fused requant [+ LUT] epilogue of qmatmul / qlinear.
//
// C[b][m][n] = epilogue(sum_k A[b][m][k] * Bt[b][n][k]): both operands K-contiguous, so every lane of an MFMA
// operand reads 16 consecutive K bytes straight from an LDS row. Workgroup tile BM x BN, BK bytes of K per
// stage, two LDS stages (the next stage's global loads are in flight while the current one feeds the MFMAs).
// 4 waves in a 2 x 2 grid; each wave owns (BM/2) x (BN/2) outputs as 32 x 32 MFMA tiles
// (v_mfma_i32_32x32x32_i8: A 32 x 32 bytes, B 32 x 32 bytes, 16 int32 accumulators per lane).
//
// MFMA operand layout: lane l supplies row (l % 32) of A / column (l % 32) of B and 16 K bytes at offset
// 16 * (l / 32) of the 32-byte K slice; A and B use the same K mapping, so the dot product does not depend on
// the order in which the hardware pairs the bytes. Accumulator r of lane l holds
// C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
#include "common.h"

namespace anvil {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const int8_t* A;
  const int8_t* B;
  void* C;
  int M, N, K;
  int batch1;        // blockIdx.y = b0 * batch1 + b1
  int tiles_n;
  long long sa0, sa1, lda, sb0, sb1, ldb, sc0, sc1, ldc;
  int mult, shift;
  long long rnd;
  const int8_t* lut;
  int out_dtype;
  unsigned* flags;
};

constexpr int G_BM = 128, G_BN = 128, G_BK = 64, G_LDK = G_BK + 16, G_THREADS = 256;

// One 16-byte K chunk of one operand row, zero outside [0, rows) x [0, K).
template <bool VEC>
__device__ __forceinline__ v4i load_chunk(const int8_t* __restrict__ base, long long ld, int row, int rows, int k,
                                          int K) {
  v4i v = {0, 0, 0, 0};
  if (row >= rows) return v;
  const int8_t* p = base + (long long)row * ld + k;
  if (VEC) {
    if (k < K) v = *reinterpret_cast<const v4i*>(p);
  } else {
    unsigned w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (k + i < K) w[i >> 2] |= (unsigned)(uint8_t)p[i] << (8 * (i & 3));
    v = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
  return v;
}

template <bool VEC>
__global__ __launch_bounds__(G_THREADS) void gemm_i8_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) int8_t As[2][G_BM * G_LDK];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][G_BN * G_LDK];
  __shared__ int8_t lut_s[256];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tile = blockIdx.x;
  const int m0 = (tile / g.tiles_n) * G_BM, n0 = (tile % g.tiles_n) * G_BN;
  const int b0 = blockIdx.y / g.batch1, b1 = blockIdx.y % g.batch1;
  const int8_t* __restrict__ A = g.A + b0 * g.sa0 + b1 * g.sa1 + (long long)m0 * g.lda;
  const int8_t* __restrict__ B = g.B + b0 * g.sb0 + b1 * g.sb1 + (long long)n0 * g.ldb;
  const int rows_a = g.M - m0, rows_b = g.N - n0;

  if (g.lut) lut_s[t] = g.lut[t];

  // loader mapping: 4 threads per 64-byte row, 64 rows per pass, 2 passes per operand tile
  const int lc = (t & 3) * 16, lr = t >> 2;
  v4i ra[2], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      ra[p] = load_chunk<VEC>(A, g.lda, lr + 64 * p, rows_a, k0 + lc, g.K);
      rb[p] = load_chunk<VEC>(B, g.ldb, lr + 64 * p, rows_b, k0 + lc, g.K);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      *reinterpret_cast<v4i*>(&As[buf][(lr + 64 * p) * G_LDK + lc]) = ra[p];
      *reinterpret_cast<v4i*>(&Bs[buf][(lr + 64 * p) * G_LDK + lc]) = rb[p];
    }
  };

  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int nk = (g.K + G_BK - 1) / G_BK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int arow = wm * 64 + (lane & 31), brow = wn * 64 + (lane & 31), kof = (lane >> 5) * 16;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * G_BK);
#pragma unroll
    for (int ks = 0; ks < G_BK / 32; ++ks) {
      v4i a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const v4i*>(&As[cur][(arow + 32 * i) * G_LDK + ks * 32 + kof]);
        b[i] = *reinterpret_cast<const v4i*>(&Bs[cur][(brow + 32 * i) * G_LDK + ks * 32 + kof]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // epilogue: checked requant, clamp to the result dtype, optional LUT; one writer per output element
  const int lo = g.out_dtype == ANVIL_I8 ? -128 : -32768, hi = g.out_dtype == ANVIL_I8 ? 127 : 32767;
  unsigned bad = 0;
  char* Cb = reinterpret_cast<char*>(g.C);
  const long long cbase = b0 * g.sc0 + b1 * g.sc1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = n0 + wn * 64 + j * 32 + (lane & 31);
        if (row < g.M && col < g.N) {
          int v = requant_checked(acc[i][j][r], g.mult, g.shift, g.rnd, lo, hi, bad);
          const long long off = cbase + (long long)row * g.ldc + col;
          if (g.out_dtype == ANVIL_I8) {
            if (g.lut) v = lut_s[v + 128];
            reinterpret_cast<int8_t*>(Cb)[off] = (int8_t)v;
          } else {
            reinterpret_cast<int16_t*>(Cb)[off] = (int16_t)v;
          }
        }
      }
  if (bad) raise_flag(g.flags, FLAG_OVERFLOW);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace anvil

using namespace anvil;

extern "C" int anvil_gemm_i8(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1,
                             int M, int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut,
                             int out_dtype) {
  if (int r = check_ctx(ctx)) return r;
  if (!A || !Bt || !C || !strides) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: null pointer");
  if (batch0 < 1 || batch1 < 1 || M < 1 || N < 1 || K < 1)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: non-positive size (batch %d x %d, M %d, N %d, K %d)", batch0,
                     batch1, M, N, K);
  if ((long long)batch0 * batch1 > 65535) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: batch above 65535");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (out_dtype != ANVIL_I8 && out_dtype != ANVIL_I16)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: result dtype must be i8 or i16");
  if (lut && out_dtype != ANVIL_I8) return set_error(ANVIL_E_VALUE, "a LUT epilogue needs an i8 result");
  GemmArgs g;
  g.A = A;
  g.B = Bt;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.batch1 = batch1;
  g.sa0 = strides[0];
  g.sa1 = strides[1];
  g.lda = strides[2];
  g.sb0 = strides[3];
  g.sb1 = strides[4];
  g.ldb = strides[5];
  g.sc0 = strides[6];
  g.sc1 = strides[7];
  g.ldc = strides[8];
  g.mult = mult;
  g.shift = shift;
  g.rnd = shift ? (1ll << (shift - 1)) : 0;
  g.lut = lut;
  g.out_dtype = out_dtype;
  g.flags = ctx->flags;
  const int tiles_m = (M + G_BM - 1) / G_BM;
  g.tiles_n = (N + G_BN - 1) / G_BN;
  if ((long long)tiles_m * g.tiles_n > (1ll << 31) - 1) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: too many tiles");
  auto ok16 = [](long long v) { return (v & 15) == 0; };
  const bool vec = (K & 15) == 0 && aligned16(A) && aligned16(Bt) && ok16(g.lda) && ok16(g.ldb) &&
                   (batch0 == 1 || (ok16(g.sa0) && ok16(g.sb0))) && (batch1 == 1 || (ok16(g.sa1) && ok16(g.sb1)));
  dim3 grid(tiles_m * g.tiles_n, batch0 * batch1);
  if (vec)
    hipLaunchKernelGGL(gemm_i8_kernel<true>, grid, dim3(G_THREADS), 0, ctx->stream, g);
  else
    hipLaunchKernelGGL(gemm_i8_kernel<false>, grid, dim3(G_THREADS), 0, ctx->stream, g);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}
