// int8 x int8 -> int32 GEMM on CDNA4 MFMA with the fused requant [+ LUT] epilogue of qmatmul / qlinear.
//
// C[b][m][n] = epilogue(sum_k A[b][m][k] * Bt[b][n][k]); both operands are K-contiguous, so every MFMA operand
// lane reads 16 consecutive K bytes from one LDS row.
//
// Workgroup: 256 threads = 4 waves in a 2 x 2 grid over a BM x BN output tile; BK bytes of K per pipeline stage,
// two LDS stages (the next stage's global loads are in flight while the current stage feeds the MFMAs). Each wave
// owns (BM/2) x (BN/2) outputs as 32 x 32 tiles of v_mfma_i32_32x32x32_i8.
//
// The MFMA computes D = Bt_tile . A_tile^T (operand roles swapped), so accumulator r of lane l holds
// C[m = 32 tm + l % 32][n = 32 tn + 8 (r / 4) + 4 (l / 32) + r % 4]: four consecutive output columns per lane, which
// pack into one dword (i8) or two (i16) for the LDS-staged epilogue. Both operands use the same K mapping
// (lane l supplies 16 K bytes at offset 16 (l / 32) of each 32-byte K slice), so the hardware's pairing order of the
// bytes cannot change the dot product.
//
// LDS rows are BK bytes with an XOR swizzle of their 16-byte chunks (swz below), so the lanes served together by a
// ds_read_b128 (consecutive rows, one logical chunk) hit distinct banks.
//
// Epilogue: requant (64-bit and checked against int32 unless the graph's static proof guarantees every value
// fits, then 32-bit), clamp, optional LUT, staged through LDS as a row-major tile, then written with 16-byte stores.
//
// Tile order: workgroup ids are spread round-robin over the 8 XCDs, so consecutive logical tiles are placed on one
// XCD, and logical tiles run in column groups of GROUP_M row tiles so concurrently running tiles share A and B rows
// in that XCD's L2.
//
// causal = 1: tiles strictly above the diagonal (every n > every m) are skipped (their values are never read);
// causal = 2: the K loop stops at m0 + BM (A[m][k] = 0 for k > m, e.g. a causal softmax output).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace anvil {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const int8_t* A;
  const int8_t* B;
  void* C;
  int M, N, K;
  int batch1;
  int tiles_m, tiles_n;
  long long sa0, sa1, lda, sb0, sb1, ldb, sc0, sc1, ldc;
  // bytes from one 64-byte K block of an operand row to the next: 64 for row-major operands; for K-blocked ones
  // (fast kernels only) the block stride, with lda / ldb then 64 (row r's block j at r 64 + j kba)
  long long kba, kbb;
  long long kbc;        // the same for the result's 64-column blocks (64: row-major; fast kernels only otherwise)
  int mult, shift, rnd;
  const int8_t* lut;
  unsigned* flags;
  int causal;
  int vec_store;
  // fused residual add (fast kernel only): D = clamp_i8((R ma + y mb + rnd2) >> shift2), y written when store_y
  const int8_t* R;
  int8_t* D;
  long long sr0, sr1, ldr, sd0, sd1, ldd;
  int ma, mb, shift2, rnd2;
  int res, store_y, vec_res;
  int nbatch;                     // batch0 * batch1 (persistent kernel)
  // split-K (fast kernel, batch 1): workgroup (tile, z) stores the int32 sums of K bytes [z kchunk, (z + 1) kchunk)
  // as partial tile (tile, z) of ws; splitk_reduce adds the partial tiles up
  int* ws;
  int kchunk, splits;
  // fused rmsnorm of D (gemm_i8_fast with NORM, one tile spanning D's rows): H = rmsnorm_int(D, nw, nlut, nmult,
  // nshift), H row-major (row stride ldh) or K-blocked (block stride kbh); nbits = the bit length of nlut_len
  const int8_t* nw;
  const int* nlut;
  int8_t* H;
  long long ldh, kbh;
  int nlut_len, nbits, nmult, nshift;
};

constexpr int G_THREADS = 256;
constexpr int GROUP_M = 4;

// Element offset of result (m, n) from the batch entry's base: row-major (kbc = 64) or K-blocked (ldc = 64, column
// block n / 64 at kbc). A 16-byte store chunk never crosses a 64-column block.
__device__ __forceinline__ long long cpos(const GemmArgs& g, int m, int n) {
  return (long long)m * g.ldc + (long long)(n >> 6) * g.kbc + (n & 63);
}

// Bytes of a tile's operand rows that its buffer descriptor covers: rows whole rows of a row-major operand (kb = 64),
// or, K-blocked, those rows in every K block; anything past reads as zero.
__device__ __forceinline__ int operand_bytes(int rows, long long ld, long long kb, int K) {
  // row-major: up to the last row's K-th byte, not its row stride: an operand that is a column slice of a wider
  // array (one head of q, say) must not reach past that array's last row, where its allocation may end
  return kb == 64 ? (int)((rows - 1) * ld + K) : (int)(rows * 64 + ((K + 63) / 64 - 1) * kb);
}

// Physical 16-byte chunk of logical chunk `chunk` in LDS row `row`. gfx950's LDS serves a ds_read_b128 from 64
// banks (256 bytes a cycle) to 16 lanes at a time, taken as four blocks of four consecutive lanes whose block
// indices k differ in the pattern {0, 3, 5, 6} (+ 8 m, and the complementary {1, 2, 4, 7}); measured on MI355X with
// a read-pattern probe. A fragment read puts rows 4 k + j (j = 0..3) of one logical chunk in block k, so the
// swizzle must differ for k = 0, 3, 5, 6 at each j: chunk ^ ((row ^ row >> 2) & 3) = chunk ^ ((j ^ k) & 3) does, and
// reads at 195 B/clk/CU against 108 for the 2-way-conflicting ((row >> 1) ^ (row >> 3)) & 3.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  static_assert(BK == 64 || BK == 128, "swizzle defined for 64- and 128-byte rows");
  if (BK == 64) return chunk ^ ((row ^ (row >> 2)) & 3);
  return chunk ^ ((row ^ (row >> 3)) & 7);
}

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

template <bool CHECKED>
__device__ __forceinline__ int rq(int acc, const GemmArgs& g, int lo, int hi, unsigned& bad) {
  if (CHECKED) return requant_checked(acc, g.mult, g.shift, (long long)g.rnd, lo, hi, bad);
  const int v = (acc * g.mult + g.rnd) >> g.shift;     // the static proof keeps acc * M + rnd inside int32
  return min(max(v, lo), hi);
}

template <int BM, int BN, int BK, int WGM, int PF, int OSZ, bool CHECKED, bool VEC>
__global__ __launch_bounds__(G_THREADS) void gemm_i8_kernel(GemmArgs g) {
  constexpr int WGN = 4 / WGM;                           // waves along M x along N
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static_assert(WGM * WGN == 4 && TM >= 1 && TN >= 1, "wave grid");
  constexpr int CPR = BK / 16;
  constexpr int A_PASS = BM * CPR / G_THREADS, B_PASS = BN * CPR / G_THREADS;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int SROW = BN * OSZ + 16;                    // epilogue staging row stride (bytes)
  constexpr int LDS_MAIN = 2 * STAGE, LDS_EPI = BM * SROW;
  constexpr int LDS_BYTES = LDS_MAIN > LDS_EPI ? LDS_MAIN : LDS_EPI;
  static_assert(A_PASS >= 1 && B_PASS >= 1 && (BM * CPR) % G_THREADS == 0 && (BN * CPR) % G_THREADS == 0, "tile");
  __shared__ __attribute__((aligned(16))) int8_t smem[LDS_BYTES];
  __shared__ int8_t lut_s[256];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  // XCD-aware, grouped tile order
  const int ntiles = g.tiles_m * g.tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int in_group = GROUP_M * g.tiles_n;
  const int first_m = (pid / in_group) * GROUP_M;
  const int gsize = min(g.tiles_m - first_m, GROUP_M);
  const int tile_m = first_m + (pid % in_group) % gsize;
  const int tile_n = (pid % in_group) / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  if (g.causal == 1 && n0 > m0 + BM - 1) return;

  const int b0 = blockIdx.y / g.batch1, b1 = blockIdx.y % g.batch1;
  const int8_t* __restrict__ A = g.A + b0 * g.sa0 + b1 * g.sa1 + (long long)m0 * g.lda;
  const int8_t* __restrict__ B = g.B + b0 * g.sb0 + b1 * g.sb1 + (long long)n0 * g.ldb;
  const int rows_a = g.M - m0, rows_b = g.N - n0;
  const int K = g.causal == 2 ? min(g.K, m0 + BM) : g.K;

  if (g.lut) lut_s[t ^ 128] = g.lut[t];               // rotated: the entry of v at index v & 255

  const int lc = t % CPR, lr = t / CPR;
  constexpr int RSTEP = G_THREADS / CPR;
  // PF register sets of staged global loads: the loads of stage s are issued PF iterations before stage s is
  // written to LDS, so PF iterations of MFMA work cover their latency.
  v4i ra[PF][A_PASS], rb[PF][B_PASS];
  auto gload = [&](int set, int k0) {
#pragma unroll
    for (int p = 0; p < A_PASS; ++p) ra[set][p] = load_chunk<VEC>(A, g.lda, lr + RSTEP * p, rows_a, k0 + lc * 16, K);
#pragma unroll
    for (int p = 0; p < B_PASS; ++p) rb[set][p] = load_chunk<VEC>(B, g.ldb, lr + RSTEP * p, rows_b, k0 + lc * 16, K);
  };
  auto lstore = [&](int set, int buf) {
    int8_t* As = smem + buf * STAGE;
    int8_t* Bs = As + BM * BK;
#pragma unroll
    for (int p = 0; p < A_PASS; ++p) {
      const int r = lr + RSTEP * p;
      *reinterpret_cast<v4i*>(As + r * BK + swz<BK>(r, lc) * 16) = ra[set][p];
    }
#pragma unroll
    for (int p = 0; p < B_PASS; ++p) {
      const int r = lr + RSTEP * p;
      *reinterpret_cast<v4i*>(Bs + r * BK + swz<BK>(r, lc) * 16) = rb[set][p];
    }
  };

  v16i acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int half = lane >> 5, l32 = lane & 31;
  auto compute = [&](int buf) {
    const int8_t* As = smem + buf * STAGE;
    const int8_t* Bs = As + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      v4i af[TM], bf[TN];
      const int ch = ks * 2 + half;
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int r = wm * WM + j * 32 + l32;
        af[j] = *reinterpret_cast<const v4i*>(As + r * BK + swz<BK>(r, ch) * 16);
      }
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int r = wn * WN + i * 32 + l32;
        bf[i] = *reinterpret_cast<const v4i*>(Bs + r * BK + swz<BK>(r, ch) * 16);
      }
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[i], af[j], acc[i][j], 0, 0, 0);
    }
  };

  const int nk = (K + BK - 1) / BK;
#pragma unroll
  for (int s = 0; s < PF; ++s)
    if (s < nk) gload(s, s * BK);
  lstore(0, 0);
  __syncthreads();
  for (int kt0 = 0; kt0 < nk; kt0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int kt = kt0 + u;
      if (kt < nk) {
        if (kt + PF < nk) gload(u, (kt + PF) * BK);          // stage kt + PF has the parity of stage kt
        compute(kt & 1);
        if (kt + 1 < nk) lstore((u + 1) % PF, (kt + 1) & 1);
        __syncthreads();
      }
    }
  }

  // epilogue: requant (+ LUT) into an LDS row-major staging tile, then 16-byte global stores
  const int lo = OSZ == 1 ? -128 : -32768, hi = OSZ == 1 ? 127 : 32767;
  unsigned bad = 0;
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m_l = wm * WM + j * 32 + l32;
        const int n_l = wn * WN + i * 32 + 8 * q + 4 * half;
        int v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = rq<CHECKED>(acc[i][j][4 * q + e], g, lo, hi, bad);
          if (OSZ == 1 && g.lut) v[e] = lut_s[(uint8_t)v[e]];
        }
        int8_t* dst = smem + m_l * SROW + n_l * OSZ;
        if (OSZ == 1) {
          *reinterpret_cast<unsigned*>(dst) =
              (unsigned)(v[0] & 255) | ((unsigned)(v[1] & 255) << 8) | ((unsigned)(v[2] & 255) << 16) | ((unsigned)v[3] << 24);
        } else {
          *reinterpret_cast<unsigned*>(dst) = (unsigned)(v[0] & 0xffff) | ((unsigned)v[1] << 16);
          *reinterpret_cast<unsigned*>(dst + 4) = (unsigned)(v[2] & 0xffff) | ((unsigned)v[3] << 16);
        }
      }
  if (CHECKED && bad) raise_flag(g.flags, FLAG_OVERFLOW);
  __syncthreads();

  constexpr int CH_ROW = BN * OSZ / 16;                  // 16-byte chunks per staged row
  constexpr int ROWS_PER_PASS = G_THREADS / CH_ROW;
  const int cc = t % CH_ROW, rr0 = t / CH_ROW;
  char* Cb = reinterpret_cast<char*>(g.C) + (b0 * g.sc0 + b1 * g.sc1) * OSZ;
  const int cols_valid = min(BN, g.N - n0);
  const int cfirst = cc * 16 / OSZ;                      // first column of this chunk within the tile
#pragma unroll 4
  for (int rr = rr0; rr < BM; rr += ROWS_PER_PASS) {
    const int m = m0 + rr;
    if (m >= g.M) break;
    const int8_t* src = smem + rr * SROW + cc * 16;
    char* dst = Cb + cpos(g, m, n0 + cfirst) * OSZ;
    if (g.vec_store && cfirst + 16 / OSZ <= cols_valid) {
      *reinterpret_cast<v4i*>(dst) = *reinterpret_cast<const v4i*>(src);
    } else {
      for (int e = 0; e < 16 / OSZ; ++e)
        if (cfirst + e < cols_valid) {
          if (OSZ == 1)
            dst[e] = src[e];
          else
            reinterpret_cast<int16_t*>(dst)[e] = reinterpret_cast<const int16_t*>(src)[e];
        }
    }
  }
}

// ---------------------------------------------------------------------------------------------- fast path
// The production kernel for proven graphs with 16-byte aligned, K-contiguous operands (every block GEMM).
//
// Operand tiles go global -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging): each wave instruction fills one
// contiguous KiB of LDS, lane l its 16 bytes, and the lane's global address is chosen so the KiB holds 16 swizzled
// rows. The buffer resource's record count ends at the tile's last valid row and an out-of-range K chunk gets an
// out-of-range offset, so the hardware writes zeros there: no branches around loads. Three LDS stages live in three
// distinct arrays (so the compiler tracks each one's outstanding loads separately); iteration kt waits for its own
// stage-kt loads (s_waitcnt vmcnt(G), G = one stage's loads still in flight), meets the other waves at s_barrier,
// issues stage kt + 2 into the array stage kt - 1 used, then runs stage kt's MFMAs. The epilogue reuses the three
// arrays as its staging tile. MUL24: every |acc| and |M| is below 2^23 (host-proven), so acc * M + rnd is one
// 24-bit multiply-add.


// 16 bytes per lane from buffer offset voff into LDS at lds + 16 * lane (lds must be wave-uniform)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, int8_t* lds, unsigned voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

__device__ __forceinline__ void wait_vmcnt(int n) {
  // s_waitcnt with vmcnt = n (0..15), expcnt and lgkmcnt left at their "no wait" maxima
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
}

// all waves' LDS writes for a stage have landed once each has waited for its own loads and the barrier is passed;
// the acquire fence keeps the following LDS reads below the barrier without waiting on later loads
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// s_waitcnt vmcnt(N) lgkmcnt(0): this wave's loads beyond the newest N have landed and its LDS accesses are done
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
}

// workgroups per CU the register budget is sized for: 3 for 128 x 128, 2 for 256 x 128 / 128 x 256 (AGPR + VGPR <= 256
// a lane, two waves a SIMD), 1 for 256 x 256
template <int BM, int BN>
constexpr int fast_occupancy() { return BM * BN <= 128 * 128 ? 3 : (BM * BN <= 256 * 128 ? 2 : 1); }

// (x >> sh) & 255 by one SDWA shift (byte 0 written, the rest zeroed): the LUT index of a clamped int8 result
__device__ __forceinline__ unsigned sra_byte(int x, int sh) {
  unsigned d;
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
      : "=v"(d) : "s"(sh), "v"(x));
  return d;
}

// requant (+ LUT) of one lane's 16 accumulators into 16 results. With the rotated LUT (LUT 1: int8 results, the
// table staged so that the entry of v sits at index v & 255) the clamp runs before the shift, with bounds
// [-128, 127] << shift saturated to int32, and one SDWA shift gives the lookup index. The widened table (LUT 2, entry
// u = lut[clamp(u - 2^(31 - shift), -128, 127) + 128]) is indexed by (x + 2^31) >> shift, unsigned.
template <int OSZ, bool MUL24, int LUT>
__device__ __forceinline__ void requant16(const v16i& a, int mult, int rnd, int shift, const int8_t* lut_s, int v[16]) {
  if constexpr (LUT == 2) {
    static_assert(OSZ == 1, "a LUT epilogue has int8 results");
    const unsigned rndw = (unsigned)rnd ^ 0x80000000u;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const unsigned u = (unsigned)(MUL24 ? __mul24(a[e], mult) : a[e] * mult) + rndw;
      v[e] = lut_s[u >> shift];
    }
  } else if constexpr (LUT == 1) {
    static_assert(OSZ == 1, "a LUT epilogue has int8 results");
    const int clo = (int)max(-128ll << shift, (long long)INT32_MIN);
    const int chi = (int)min((128ll << shift) - 1, (long long)INT32_MAX);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int x = MUL24 ? (__mul24(a[e], mult) + rnd) : (a[e] * mult + rnd);
      v[e] = lut_s[sra_byte(med3i(x, clo, chi), shift)];
    }
  } else {
    const int lo = OSZ == 1 ? -128 : -32768, hi = OSZ == 1 ? 127 : 32767;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int x = MUL24 ? (__mul24(a[e], mult) + rnd) : (a[e] * mult + rnd);
      v[e] = min(max(x >> shift, lo), hi);
    }
  }
}


// Epilogue from registers: tile (i, j) of this lane is row mrow + 32 j, columns ncol + 32 i .. + 15. Interior tiles
// issue every residual load first, then requantize and store 16 bytes a lane; edge tiles store element by element.
template <int BM, int BN, int WM, int WN, int TM, int TN, int OSZ, bool MUL24>
__device__ __forceinline__ void direct_epilogue(const GemmArgs& g, const v16i (&acc)[TN][TM], const int8_t* lut_s,
                                                bool wide, int mrow, int ncol, int m0, int n0, int b0, int b1) {
  char* Cb = reinterpret_cast<char*>(g.C) + (b0 * g.sc0 + b1 * g.sc1) * OSZ;
  const bool res = OSZ == 1 && g.res;
  const int8_t* Rb = g.R + b0 * g.sr0 + b1 * g.sr1;
  int8_t* Db = g.D + b0 * g.sd0 + b1 * g.sd1;
  const bool interior = m0 + BM <= g.M && n0 + BN <= g.N &&
                        (res ? (g.vec_res != 0 && (!g.store_y || g.vec_store != 0)) : g.vec_store != 0);
  const int mult = g.mult, rnd = g.rnd, shift = g.shift;
  auto run = [&](auto lut_c, auto full_c) {
    constexpr int LUT = decltype(lut_c)::value;
    constexpr bool FULL = decltype(full_c)::value;
    v4i rv[TM][TN];
    if (FULL && res) {
#pragma unroll
      for (int j = 0; j < TM; ++j)
#pragma unroll
        for (int i = 0; i < TN; ++i)
          rv[j][i] = *reinterpret_cast<const v4i*>(Rb + (long long)(mrow + 32 * j) * g.ldr + ncol + 32 * i);
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int m = mrow + 32 * j;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int n = ncol + 32 * i;
        int v[16];
        requant16<OSZ, MUL24, LUT>(acc[i][j], mult, rnd, shift, lut_s, v);
        if (FULL) {
          if (res) {
            const int ma = g.ma, mb = g.mb, rnd2 = g.rnd2, sh2 = g.shift2;
            v4i ov;
            if (PackedAdd::applies(ma, mb)) {
              // multipliers below 2^24: y packed, then full-rate byte multiplies (PackedAdd)
              const PackedAdd add(ma, mb, rnd2, sh2);
#pragma unroll
              for (int q = 0; q < 4; ++q)
                ov[q] = (int)add((unsigned)rv[j][i][q], pack4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]));
            } else {
              // clamp before the shift, then one SDWA shift into each byte lane
              const int clo2 = (int)max(-128ll << sh2, (long long)INT32_MIN);
              const int chi2 = (int)min((128ll << sh2) - 1, (long long)INT32_MAX);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                int o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const int r = (int)(int8_t)((unsigned)rv[j][i][q] >> (8 * e));
                  o[e] = med3i(r * ma + v[4 * q + e] * mb + rnd2, clo2, chi2);   // proven inside int32
                }
                ov[q] = (int)sra_pack4(o[0], o[1], o[2], o[3], sh2);
              }
            }
            *reinterpret_cast<v4i*>(Db + (long long)m * g.ldd + n) = ov;
            if (!g.store_y) continue;
          }
          if (OSZ == 1) {
            v4i w;
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = (int)pack4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
            *reinterpret_cast<v4i*>(Cb + cpos(g, m, n)) = w;
          } else {
            v4i w0, w1;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              w0[q] = (int)__builtin_amdgcn_perm((unsigned)v[2 * q + 1], (unsigned)v[2 * q], 0x05040100u);
              w1[q] = (int)__builtin_amdgcn_perm((unsigned)v[2 * q + 9], (unsigned)v[2 * q + 8], 0x05040100u);
            }
            char* d = Cb + cpos(g, m, n) * 2;
            *reinterpret_cast<v4i*>(d) = w0;
            *reinterpret_cast<v4i*>(d + 16) = w1;
          }
        } else if (m < g.M) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            if (n + e >= g.N) break;
            if (res) {
              const int r = Rb[(long long)m * g.ldr + n + e];
              Db[(long long)m * g.ldd + n + e] =
                  (int8_t)min(max((r * g.ma + v[e] * g.mb + g.rnd2) >> g.shift2, -128), 127);
              if (!g.store_y) continue;
            }
            if (OSZ == 1)
              Cb[cpos(g, m, n) + e] = (int8_t)v[e];
            else
              reinterpret_cast<int16_t*>(Cb)[cpos(g, m, n) + e] = (int16_t)v[e];
          }
        }
      }
    }
  };
  const bool lut = OSZ == 1 && g.lut;
  auto pick = [&](auto full_c) {
    if constexpr (OSZ == 1) {
      if (lut && wide) return run(std::integral_constant<int, 2>{}, full_c);
      if (lut) return run(std::integral_constant<int, 1>{}, full_c);
    }
    run(std::integral_constant<int, 0>{}, full_c);
  };
  if (interior) pick(std::true_type{}); else pick(std::false_type{});
}

// Bytes of the persistent kernel's lookup table: the largest power of two up to 32 KiB that fits beside `stages`
// bytes of pipeline stages in the 160 KiB of LDS.
constexpr int table_bytes(int stages) {
  int b = 32768;
  while (b > 256 && stages + b > 160 * 1024) b >>= 1;
  return b;
}

// The register epilogue of an interior tile with int8 results and no fused add, one group at a time: requant (+ LUT)
// and one 16-byte store a group at p + the group's offset. A LUT widened to the whole range of x >> shift (WIDE,
// the table's entry u holding lut[clamp(u - 2^(31 - shift), -128, 127)]) takes its index as (x + 2^31) >> shift,
// unsigned: the 2^31 rides in the rounding constant, and no clamp is needed, as the proof keeps x inside int32.
// Without a LUT the clamp runs before the shift and one SDWA shift writes each byte of the packed dword.
template <int TM, int TN, bool MUL24, int MODE>   // MODE 0: no LUT, 1: the rotated 256-entry LUT, 2: WIDE
__device__ __forceinline__ void plain_epilogue(const GemmArgs& g, const v16i (&acc)[TN][TM], const uint8_t* tab,
                                               int8_t* p) {
  const int mult = g.mult, shift = g.shift;
  const int clo = (int)max(-128ll << shift, (long long)INT32_MIN);
  const int chi = (int)min((128ll << shift) - 1, (long long)INT32_MAX);
  const unsigned rndw = (unsigned)g.rnd ^ 0x80000000u;
#pragma unroll
  for (int j = 0; j < TM; ++j)
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const v16i& a = acc[i][j];
      v4i w;
      if constexpr (MODE == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int x[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            x[e] = med3i(MUL24 ? __mul24(a[4 * q + e], mult) + g.rnd : a[4 * q + e] * mult + g.rnd, clo, chi);
          w[q] = (int)sra_pack4(x[0], x[1], x[2], x[3], shift);
        }
      } else {
        int v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if constexpr (MODE == 2) {
            const unsigned u = (unsigned)(MUL24 ? __mul24(a[e], mult) : a[e] * mult) + rndw;
            v[e] = tab[u >> shift];
          } else {
            const int x = MUL24 ? (__mul24(a[e], mult) + g.rnd) : (a[e] * mult + g.rnd);
            v[e] = tab[sra_byte(med3i(x, clo, chi), shift)];
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = (int)pack4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
      }
      // group (i, j): row + 32 j, column + 32 i; a wave's columns start at a multiple of 64 (+ 16 for the upper
      // half-wave), so column + 32 i lies in 64-column block i / 2 at offset 32 (i % 2)
      *reinterpret_cast<v4i*>(p + 32 * j * g.ldc + (i >> 1) * g.kbc + 32 * (i & 1)) = w;
    }
}

// One output tile of the fast kernel: logical tile pid of batch entry bz (the XCD remap below assumes pid and the
// workgroup id agree modulo 8).
template <int BM, int BN, int WM, int WN, int TM, int TN, int OSZ, bool MUL24>
__device__ void splitk_finish(const GemmArgs& g, const v16i (&acc)[TN][TM], const int8_t* lut_s, int tile, int m0,
                              int n0, int mrow, int ncol);

// KFULL: K (of the product, or of each split-K chunk) is a whole number of 64-byte blocks, so no chunk of a stage
// below K needs the per-lane K bound: a load's offset is its lane's fixed offset plus the stage's block offset (one
// add). A stage at or past K is issued only to keep each stage's load count fixed and is never read: its offsets
// reach the next rows' bytes inside the buffer resource, or zeros past it. With three stages KFULL also means
// whole rotations (K a multiple of 192), which the launches check.
template <int BM, int BN, int WGM, int NS, int OSZ, bool MUL24, bool SPLIT = false, bool KFULL = false, bool RES = true,
          bool NORM = false>
__device__ __forceinline__ void fast_tile(const GemmArgs& g, int pid, const int bz) {
  constexpr int BK = 64, CPR = BK / 16;
  constexpr int WGN = 4 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static_assert(WGM * WGN == 4 && TM >= 1 && TN >= 1, "wave grid");
  static_assert(NS == 3 || NS == 4, "three or four LDS stages");
  constexpr int IA = BM * CPR / 64, IB = BN * CPR / 64;  // wave instructions (KiB) per operand per stage
  static_assert(IA % 4 == 0 && IB % 4 == 0, "each wave issues an equal share of a stage");
  constexpr int JA = IA / 4, JB = IB / 4, G = JA + JB;   // per-wave loads per stage
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int SROW = BN * OSZ + 16;
  constexpr int ROWS_PER_ARR_MIN = (BM + NS - 1) / NS;
  constexpr int ARR = STAGE > ROWS_PER_ARR_MIN * SROW ? STAGE : ROWS_PER_ARR_MIN * SROW;
  constexpr int RPA = ARR / SROW;                        // staging rows per array
  __shared__ __attribute__((aligned(1024))) int8_t L0[ARR];
  __shared__ __attribute__((aligned(1024))) int8_t L1[ARR];
  __shared__ __attribute__((aligned(1024))) int8_t L2[ARR];
  __shared__ __attribute__((aligned(1024))) int8_t L3[NS == 4 ? ARR : 16];
  __shared__ int8_t lut_s[256];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  const int ntiles = g.tiles_m * g.tiles_n;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int in_group = GROUP_M * g.tiles_n;
  const int first_m = (pid / in_group) * GROUP_M;
  const int gsize = min(g.tiles_m - first_m, GROUP_M);
  const int tile_m = first_m + (pid % in_group) % gsize;
  const int tile_n = (pid % in_group) / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  if (g.causal == 1 && n0 > m0 + BM - 1) return;

  // split-K: bz is the K chunk (the batch is 1), and the chunk's first byte becomes the operands' K origin
  const int b0 = SPLIT ? 0 : bz / g.batch1, b1 = SPLIT ? 0 : bz % g.batch1;
  const int kbeg = SPLIT ? bz * g.kchunk : 0;
  const int8_t* Ab = g.A + b0 * g.sa0 + b1 * g.sa1 + (long long)m0 * g.lda + (kbeg >> 6) * g.kba;
  const int8_t* Bb = g.B + b0 * g.sb0 + b1 * g.sb1 + (long long)n0 * g.ldb + (kbeg >> 6) * g.kbb;
  const int rows_a = min(g.M - m0, BM), rows_b = min(g.N - n0, BN);
  const int K = SPLIT ? min(g.K - kbeg, g.kchunk) : (g.causal == 2 ? min(g.K, m0 + BM) : g.K);
  const __amdgpu_buffer_rsrc_t ra = uniform_rsrc(Ab, operand_bytes(rows_a, g.lda, g.kba, K));
  const __amdgpu_buffer_rsrc_t rb = uniform_rsrc(Bb, operand_bytes(rows_b, g.ldb, g.kbb, K));

  if (g.lut) lut_s[t ^ 128] = g.lut[t];               // rotated: the entry of v at index v & 255

  // per-lane global byte offsets (without k0) of the chunks this wave loads, and their K offsets
  unsigned offa[JA], offb[JB];
  int ka[JA], kb[JB];
#pragma unroll
  for (int j = 0; j < JA; ++j) {
    const int P = (wave + 4 * j) * 64 + lane, row = P / CPR, c = swz<BK>(row, P % CPR);
    offa[j] = (unsigned)(row * g.lda + (c >> 2) * g.kba + (c & 3) * 16);
    ka[j] = c * 16;
  }
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const int P = (wave + 4 * j) * 64 + lane, row = P / CPR, c = swz<BK>(row, P % CPR);
    offb[j] = (unsigned)(row * g.ldb + (c >> 2) * g.kbb + (c & 3) * 16);
    kb[j] = c * 16;
  }
  // a stage at or past K loads zeros (every offset out of range): issuing is unconditional, so the compiler's
  // per-array tracking of outstanding LDS writes stays exact (a branch around the loads would make it wait for all)
  auto issue = [&](int8_t* arr, int k0) {
    const unsigned oa = (unsigned)((k0 >> 6) * g.kba), ob = (unsigned)((k0 >> 6) * g.kbb);
#pragma unroll
    for (int j = 0; j < JA; ++j)
      dma16(ra, arr + (wave + 4 * j) * 1024, KFULL ? offa[j] + oa : (k0 + ka[j] < K ? offa[j] + oa : OOB));
#pragma unroll
    for (int j = 0; j < JB; ++j)
      dma16(rb, arr + BM * BK + (wave + 4 * j) * 1024, KFULL ? offb[j] + ob : (k0 + kb[j] < K ? offb[j] + ob : OOB));
  };

  v16i acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // MFMA fragments are double-buffered in registers: the next k-step's fragments are read from LDS while the
  // current k-step's MFMAs run, so LDS latency never sits between two MFMA groups
  const int half = lane >> 5, l32 = lane & 31;
  v4i af[2][TM], bf[2][TN];
  auto load_frags = [&](int set, const int8_t* arr, int ks) {
    const int ch = ks * 2 + half;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int r = wm * WM + j * 32 + l32;
      af[set][j] = *reinterpret_cast<const v4i*>(arr + r * BK + (swz<BK>(r, ch) << 4));
    }
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int r = wn * WN + i * 32 + l32;
      bf[set][i] = *reinterpret_cast<const v4i*>(arr + BM * BK + r * BK + (swz<BK>(r, ch) << 4));
    }
  };
  auto mm = [&](int set) {
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[set][i], af[set][j], acc[i][j], 0, 0, 0);
  };
  // One pipeline step over stage kt (in `cur`, complete and visible on entry, its first fragments in set 0):
  // stage kt + NS - 1 goes into `nxt` (the array of stage kt - 1, which every wave finished reading before the
  // previous step's barrier); then the k-steps of stage kt run, and before the last one this wave waits for its
  // share of stage kt + 1 (the loads still allowed in flight are stages kt + 2 .. kt + NS - 1) and for its own LDS
  // reads of stage kt, meets the other waves at the barrier, and prefetches stage kt + 1's first fragments from
  // `next` during the last k-step's MFMAs. Past the last stage those reads are harmless and unused.
  constexpr int KS = BK / 32;
  static_assert(KS % 2 == 0, "fragment sets alternate within a stage");
  const int nk = (K + BK - 1) / BK;
  auto step = [&](int kt, const int8_t* cur, int8_t* nxt, const int8_t* next) {
    issue(nxt, (kt + NS - 1) * BK);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS - 1; ++ks) {
      load_frags((ks + 1) & 1, cur, ks + 1);
      __builtin_amdgcn_sched_barrier(0);            // keep the prefetch ahead of the MFMAs it overlaps
      mm(ks & 1);
      __builtin_amdgcn_sched_barrier(0);            // and the waits below after them
    }
    wait_vm_lgkm0<(NS - 2) * G>();
    stage_barrier();
    load_frags(0, next, 0);
    __builtin_amdgcn_sched_barrier(0);
    mm((KS - 1) & 1);
  };

  issue(L0, 0);
  issue(L1, BK);
  if (NS == 4) issue(L2, 2 * BK);
  wait_vm_lgkm0<(NS - 2) * G>();
  stage_barrier();
  load_frags(0, L0, 0);
  int kt = 0;
  if (NS == 3 && KFULL) {
    // KFULL launches have nk % 3 == 0: whole rotations and no tail steps, so the accumulators reach the epilogue from
    // one place (tail steps leave several, and the compiler then copies every accumulator where they join)
    for (; kt < nk; kt += 3) {
      step(kt, L0, L2, L1);
      step(kt + 1, L1, L0, L2);
      step(kt + 2, L2, L1, L0);
    }
  } else if (NS == 3) {
    for (; kt + 3 <= nk; kt += 3) {
      step(kt, L0, L2, L1);
      step(kt + 1, L1, L0, L2);
      step(kt + 2, L2, L1, L0);
    }
    if (kt < nk) step(kt, L0, L2, L1);
    if (kt + 1 < nk) step(kt + 1, L1, L0, L2);
  } else {
    for (; kt + 4 <= nk; kt += 4) {
      step(kt, L0, L3, L1);
      step(kt + 1, L1, L0, L2);
      step(kt + 2, L2, L1, L3);
      step(kt + 3, L3, L2, L0);
    }
    if (kt < nk) step(kt, L0, L3, L1);
    if (kt + 1 < nk) step(kt + 1, L1, L0, L2);
    if (kt + 2 < nk) step(kt + 2, L2, L1, L3);
  }
  if constexpr (SPLIT) {
    splitk_finish<BM, BN, WM, WN, TM, TN, OSZ, MUL24>(g, acc, lut_s, tile_m * g.tiles_n + tile_n, m0, n0,
                                                      wm * WM + l32, wn * WN + 4 * half);
    return;
  }

  // the staged tile leaves in 16-byte chunks, chunk idx = t + pass * G_THREADS of the tile: row idx / CH_ROW,
  // column chunk idx % CH_ROW (a thread keeps one column chunk when CH_ROW divides the thread count)
  constexpr int CH_ROW = BN * OSZ / 16;
  static_assert((BM * CH_ROW) % G_THREADS == 0, "whole store passes");
  constexpr int PASSES = BM * CH_ROW / G_THREADS;
  auto rr_of = [&](int pass) { return (t + pass * G_THREADS) / CH_ROW; };
  auto cf_of = [&](int pass) { return (t + pass * G_THREADS) % CH_ROW * 16 / OSZ; };   // first column
  const int cols_valid = min(BN, g.N - n0);
  const bool res = RES && g.res != 0;   // RES false: no fused add, its code compiled out
  // interior tile: every chunk is read from LDS (and the residual from memory) before the first store, so the
  // reads' latencies overlap instead of serialising pass by pass
  const bool full = m0 + BM <= g.M && cols_valid == BN && (res ? g.vec_res != 0 : g.vec_store != 0) &&
                    (!res || !g.store_y || g.vec_store) && (!res || (long long)BM * g.ldr * OSZ < (1ll << 31));
  // An interior tile's residual chunks (R has the result's dtype) are loaded now, so their latency overlaps the
  // staging below. With an i8 result the loads are issued whatever the tile (out of range, so loading nothing,
  // without a residual): they are then the newest NR loads, and waiting for all but those retires the pipeline's
  // last (zero-filling) stage loads before the staging overwrites their arrays. An i16 result (twice the chunks,
  // whose registers the staging needs) loads its residual chunks in the store phase, and the wait is for all.
  constexpr int NR = OSZ == 1 && RES ? PASSES : 0;
  const bool res_full = res && full;
  const int8_t* Rb = g.R + (b0 * g.sr0 + b1 * g.sr1 + (long long)m0 * g.ldr + n0) * OSZ;
  const __amdgpu_buffer_rsrc_t rres = uniform_rsrc(res_full ? Rb : g.A, res_full ? (int)(BM * g.ldr * OSZ) : 0);
  v4i rv[NR > 0 ? NR : 1];
#pragma unroll
  for (int pass = 0; pass < NR; ++pass)
    rv[pass] = __builtin_bit_cast(
        v4i, __builtin_amdgcn_raw_buffer_load_b128(
                 rres, res_full ? (unsigned)((rr_of(pass) * g.ldr + cf_of(pass)) * OSZ) : OOB, 0, 0));

  // epilogue: requant (+ LUT) into the staging tile spread over the stage arrays (RPA rows each), then 16-byte
  // stores
  wait_vm_lgkm0<NR>();
  stage_barrier();
  const int lo = OSZ == 1 ? -128 : -32768, hi = OSZ == 1 ? 127 : 32767;
  auto srow = [&](int r) -> int8_t* {
    if (r < RPA) return L0 + r * SROW;
    if (r < 2 * RPA) return L1 + (r - RPA) * SROW;
    if (NS == 3 || r < 3 * RPA) return L2 + (r - 2 * RPA) * SROW;
    return L3 + (r - 3 * RPA) * SROW;
  };
  // the LUT choice is made once, outside the loops: a per-element branch would split the requant into basic blocks
  // that each wait for their LDS reads
  int8_t* rowp[TM];
#pragma unroll
  for (int j = 0; j < TM; ++j) rowp[j] = srow(wm * WM + j * 32 + l32);
  const int mult = g.mult, rnd = g.rnd, shift = g.shift;
  // i8 without a LUT: the clamp runs before the shift (bounds [-128, 127] << shift, saturated to int32) and one SDWA
  // shift writes each byte of the packed dword
  const int clo = (int)max(-128ll << shift, (long long)INT32_MIN), chi = (int)min((128ll << shift) - 1, (long long)INT32_MAX);
  auto stage = [&](auto lut_c) {
    constexpr bool LUT = decltype(lut_c)::value;
#pragma unroll
    for (int j = 0; j < TM; ++j)
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n_l = wn * WN + i * 32 + 8 * q + 4 * half;
          if constexpr (OSZ == 1 && !LUT) {
            int x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int a = acc[i][j][4 * q + e];
              x[e] = med3i(MUL24 ? (__mul24(a, mult) + rnd) : (a * mult + rnd), clo, chi);
            }
            *reinterpret_cast<unsigned*>(rowp[j] + n_l) = sra_pack4(x[0], x[1], x[2], x[3], shift);
            continue;
          }
          int v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int a = acc[i][j][4 * q + e];
            const int x = MUL24 ? (__mul24(a, mult) + rnd) : (a * mult + rnd);
            v[e] = min(max(x >> shift, lo), hi);
            if (LUT) v[e] = lut_s[(uint8_t)v[e]];
          }
          if (OSZ == 1) {
            const unsigned t01 = __builtin_amdgcn_perm((unsigned)v[1], (unsigned)v[0], 0x0c0c0400u);
            const unsigned t23 = __builtin_amdgcn_perm((unsigned)v[3], (unsigned)v[2], 0x0c0c0400u);
            *reinterpret_cast<unsigned*>(rowp[j] + n_l) = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
          } else {
            *reinterpret_cast<unsigned*>(rowp[j] + 2 * n_l) = __builtin_amdgcn_perm((unsigned)v[1], (unsigned)v[0], 0x05040100u);
            *reinterpret_cast<unsigned*>(rowp[j] + 2 * n_l + 4) =
                __builtin_amdgcn_perm((unsigned)v[3], (unsigned)v[2], 0x05040100u);
          }
        }
  };
  if (OSZ == 1 && g.lut)
    stage(std::true_type{});
  else
    stage(std::false_type{});
  wait_vm_lgkm0<63>();                                   // the staging writes, not the residual loads
  stage_barrier();

  char* Cb = reinterpret_cast<char*>(g.C) + (b0 * g.sc0 + b1 * g.sc1) * OSZ;
  if (full) {
    v4i ch[PASSES];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass)
      ch[pass] = *reinterpret_cast<const v4i*>(srow(rr_of(pass)) + cf_of(pass) * OSZ);
    if (res) {
      int8_t* Db = g.D + (b0 * g.sd0 + b1 * g.sd1 + (long long)m0 * g.ldd + n0) * OSZ;
      const int ma = g.ma, mb = g.mb, rnd2 = g.rnd2, sh2 = g.shift2;
      // clamp before the shift (bounds [lo, hi] << sh2, saturated to int32), then the shift: for i8 one SDWA shift
      // into each byte lane
      constexpr long long LO = OSZ == 1 ? -128 : -32768, HI = OSZ == 1 ? 127 : 32767;
      const int clo2 = (int)max(LO << sh2, (long long)INT32_MIN);
      const int chi2 = (int)min(((HI + 1) << sh2) - 1, (long long)INT32_MAX);
      if (OSZ == 1 && PackedAdd::applies(ma, mb)) {
        // multipliers below 2^24: full-rate byte multiplies (PackedAdd) instead of 32-bit ones
        const PackedAdd add(ma, mb, rnd2, sh2);
        // NORM: H = rmsnorm_int(D) row by row (anvil/semantics.py:164-182 with ss_shift = ss_init = 0): the tile
        // spans D's rows, CH_ROW consecutive lanes hold one row's chunks, and a lane's columns are the same in every
        // pass (CH_ROW divides the thread count), so its 16 weights load once
        static_assert(!NORM || (OSZ == 1 && RES && G_THREADS % CH_ROW == 0), "a fused rmsnorm of int8 D rows");
        v4i nwv = {0, 0, 0, 0};
        if constexpr (NORM) nwv = *reinterpret_cast<const v4i*>(g.nw + cf_of(0));
        auto norm_chunk = [&](const v4i& d, int rr, int cf) {
          int ss = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) ss = __builtin_amdgcn_sdot4(d[q], d[q], ss, false);
          ss = lane_group_sum<CH_ROW>(ss);
          const int k = rsqrt_shift(ss, g.nlut_len, g.nbits);       // (idx, k) = rsqrt_index(ss, n)
          const int rm = g.nlut[ss >> (2 * k)] * g.nmult;            // proven below 2^23 in magnitude
          const int sh = g.nshift + k;
          const int rnd = sh ? 1 << (sh - 1) : 0;
          const int lo = sh >= 24 ? INT32_MIN : -128 * (1 << sh), hi = sh >= 24 ? INT32_MAX : 128 * (1 << sh) - 1;
          v4i h;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const unsigned xd = (unsigned)d[q], wd = (unsigned)nwv[q];
            // proven: x w r M + rnd inside int32, |x w| and |r M| below 2^23
            const int y0 = med3i(mad_i24v(mul_sbytes<0>(xd, wd), rm, rnd), lo, hi);
            const int y1 = med3i(mad_i24v(mul_sbytes<1>(xd, wd), rm, rnd), lo, hi);
            const int y2 = med3i(mad_i24v(mul_sbytes<2>(xd, wd), rm, rnd), lo, hi);
            const int y3 = med3i(mad_i24v(mul_sbytes<3>(xd, wd), rm, rnd), lo, hi);
            h[q] = (int)sra_pack4v(y0, y1, y2, y3, sh);
          }
          const long long m = m0 + rr;
          *reinterpret_cast<v4i*>(g.H + (g.kbh ? m * 64 + (cf >> 6) * g.kbh + (cf & 63) : m * g.ldh + cf)) = h;
        };
#pragma unroll
        for (int pass = 0; pass < PASSES; ++pass) {
          v4i ov;
#pragma unroll
          for (int q = 0; q < 4; ++q) ov[q] = (int)add((unsigned)rv[pass][q], (unsigned)ch[pass][q]);
          *reinterpret_cast<v4i*>(Db + ((long long)rr_of(pass) * g.ldd + cf_of(pass)) * OSZ) = ov;
          if constexpr (NORM) norm_chunk(ov, rr_of(pass), cf_of(pass));
        }
        if (!g.store_y) return;
#pragma unroll
        for (int pass = 0; pass < PASSES; ++pass)
          *reinterpret_cast<v4i*>(Cb + cpos(g, m0 + rr_of(pass), n0 + cf_of(pass)) * OSZ) = ch[pass];
        return;
      }
#pragma unroll
      for (int pass = 0; pass < PASSES; ++pass) {
        v4i ov, r16 = {0, 0, 0, 0};
        if constexpr (OSZ == 2)
          r16 = *reinterpret_cast<const v4i*>(Rb + ((long long)rr_of(pass) * g.ldr + cf_of(pass)) * 2);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (OSZ == 1) {
            int o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int y = (int)(int8_t)((unsigned)ch[pass][q] >> (8 * e));
              const int r = (int)(int8_t)((unsigned)rv[pass][q] >> (8 * e));
              o[e] = med3i(r * ma + y * mb + rnd2, clo2, chi2);              // proven inside int32
            }
            ov[q] = (int)sra_pack4(o[0], o[1], o[2], o[3], sh2);
          } else {
            int o[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const int y = (int)(int16_t)((unsigned)ch[pass][q] >> (16 * e));
              const int r = (int)(int16_t)((unsigned)r16[q] >> (16 * e));
              o[e] = med3i(r * ma + y * mb + rnd2, clo2, chi2) >> sh2;       // proven inside int32
            }
            ov[q] = (int)__builtin_amdgcn_perm((unsigned)o[1], (unsigned)o[0], 0x05040100u);
          }
        }
        *reinterpret_cast<v4i*>(Db + ((long long)rr_of(pass) * g.ldd + cf_of(pass)) * OSZ) = ov;
      }
      if (!g.store_y) return;
    }
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass)
      *reinterpret_cast<v4i*>(Cb + cpos(g, m0 + rr_of(pass), n0 + cf_of(pass)) * OSZ) = ch[pass];
    return;
  }
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    const int rr = rr_of(pass), cfirst = cf_of(pass);
    const int m = m0 + rr;
    if (m >= g.M) break;                                 // rows grow with the pass
    const int8_t* src = srow(rr) + cfirst * OSZ;
    if (OSZ == 2 && res) {
      // the fused add_requant on i16 values, element by element over the chunk's 8 columns
      const int16_t* rp = reinterpret_cast<const int16_t*>(g.R) + b0 * g.sr0 + b1 * g.sr1 + (long long)m * g.ldr + n0 +
                          cfirst;
      int16_t* dp = reinterpret_cast<int16_t*>(g.D) + b0 * g.sd0 + b1 * g.sd1 + (long long)m * g.ldd + n0 + cfirst;
      for (int e = 0; e < 8; ++e)
        if (cfirst + e < cols_valid) {
          const int y = reinterpret_cast<const int16_t*>(src)[e];
          dp[e] = (int16_t)min(max(((int)rp[e] * g.ma + y * g.mb + g.rnd2) >> g.shift2, -32768), 32767);
        }
      if (!g.store_y) continue;
    }
    if (OSZ == 1 && res) {
      // the fused add_requant: 16 results from the staged y chunk and the residual chunk at the same position
      const int8_t* rp = g.R + b0 * g.sr0 + b1 * g.sr1 + (long long)m * g.ldr + n0 + cfirst;
      int8_t* dp = g.D + b0 * g.sd0 + b1 * g.sd1 + (long long)m * g.ldd + n0 + cfirst;
      if (g.vec_res && cfirst + 16 <= cols_valid) {
        const v4i yv = *reinterpret_cast<const v4i*>(src);
        const v4i rv = *reinterpret_cast<const v4i*>(rp);
        v4i ov;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int y = (int)(int8_t)((unsigned)yv[q] >> (8 * e)), r = (int)(int8_t)((unsigned)rv[q] >> (8 * e));
            o[e] = min(max((r * g.ma + y * g.mb + g.rnd2) >> g.shift2, -128), 127);   // proven inside int32
          }
          ov[q] = (int)((unsigned)(o[0] & 255) | ((unsigned)(o[1] & 255) << 8) | ((unsigned)(o[2] & 255) << 16) |
                        ((unsigned)o[3] << 24));
        }
        *reinterpret_cast<v4i*>(dp) = ov;
      } else {
        for (int e = 0; e < 16; ++e)
          if (cfirst + e < cols_valid)
            dp[e] = (int8_t)min(max(((int)rp[e] * g.ma + (int)src[e] * g.mb + g.rnd2) >> g.shift2, -128), 127);
      }
      if (!g.store_y) continue;
    }
    char* dst = Cb + cpos(g, m, n0 + cfirst) * OSZ;
    if (g.vec_store && cfirst + 16 / OSZ <= cols_valid) {
      *reinterpret_cast<v4i*>(dst) = *reinterpret_cast<const v4i*>(src);
    } else {
      for (int e = 0; e < 16 / OSZ; ++e)
        if (cfirst + e < cols_valid) {
          if (OSZ == 1)
            dst[e] = src[e];
          else
            reinterpret_cast<int16_t*>(dst)[e] = reinterpret_cast<const int16_t*>(src)[e];
        }
    }
  }
}

// Split-K end of a tile: this K chunk's int32 accumulators become partial tile (tile, chunk) of ws, BM x BN
// row-major, with plain 16-byte stores; splitk_reduce sums a tile's chunks in the next launch (the kernel boundary
// is the only synchronisation). Accumulator r of lane l in tile (i, j) is tile row mrow + 32 j, column
// ncol + 32 i + 8 (r / 4) + r % 4 (mrow, ncol relative to the tile).
template <int BM, int BN, int WM, int WN, int TM, int TN, int OSZ, bool MUL24>
__device__ void splitk_finish(const GemmArgs& g, const v16i (&acc)[TN][TM], const int8_t* lut_s, int tile, int m0,
                              int n0, int mrow, int ncol) {
  int* part = g.ws + ((long long)tile * g.splits + blockIdx.y) * (BM * BN);
#pragma unroll
  for (int j = 0; j < TM; ++j)
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<v4i*>(part + (mrow + 32 * j) * BN + ncol + 32 * i + 8 * q) =
            v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
  wait_vmcnt(0);                                         // trailing zero-fill stage loads land before exit
}

// The second launch of a split-K product: workgroup (tile, band) sums the g.splits partial tiles of 16 rows of one
// 128 x 128 output tile, four consecutive sums a thread, and requantizes (+ LUT) them into C.
template <int OSZ, bool MUL24>
__global__ __launch_bounds__(G_THREADS) void splitk_reduce(GemmArgs g) {
  constexpr int T = 128, BAND = 16;
  __shared__ int8_t lut_s[256];
  const int tile = blockIdx.x / (T / BAND), band = blockIdx.x % (T / BAND);
  const int tm = tile / g.tiles_n, tn = tile % g.tiles_n;
  const bool lut = OSZ == 1 && g.lut;
  if (lut) lut_s[threadIdx.x ^ 128] = g.lut[threadIdx.x];   // rotated: the entry of v at index v & 255
  __syncthreads();
  const int rr = band * BAND + threadIdx.x / 32 * 2, c4 = threadIdx.x % 32 * 4;
  const int lo = OSZ == 1 ? -128 : -32768, hi = OSZ == 1 ? 127 : 32767;
  const int* tp = g.ws + (long long)tile * g.splits * (T * T);
  char* Cb = reinterpret_cast<char*>(g.C);
  const int n = tn * T + c4;
  if (n >= g.N) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {                          // two rows a thread
    const int m = tm * T + rr + h;
    if (m >= g.M) break;
    v4i a = *reinterpret_cast<const v4i*>(tp + (rr + h) * T + c4);
    for (int z = 1; z < g.splits; ++z) a += *reinterpret_cast<const v4i*>(tp + (long long)z * (T * T) + (rr + h) * T + c4);
    int v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int x = MUL24 ? (__mul24(a[e], g.mult) + g.rnd) : (a[e] * g.mult + g.rnd);
      v[e] = min(max(x >> g.shift, lo), hi);
      if (lut) v[e] = lut_s[(uint8_t)v[e]];
    }
    char* c = Cb + cpos(g, m, n) * OSZ;
    if (OSZ == 1 && g.vec_store && n + 3 < g.N) {
      *reinterpret_cast<unsigned*>(c) = pack4(v[0], v[1], v[2], v[3]);
    } else {
      for (int e = 0; e < 4 && n + e < g.N; ++e) {
        if (OSZ == 1)
          c[e] = (char)v[e];
        else
          reinterpret_cast<int16_t*>(c)[e] = (int16_t)v[e];
      }
    }
  }
}

template <int BM, int BN, int WGM, int NS, int OSZ, bool MUL24, bool KFULL>
__global__ __launch_bounds__(G_THREADS, (fast_occupancy<BM, BN>())) void gemm_i8_splitk(GemmArgs g) {
  fast_tile<BM, BN, WGM, NS, OSZ, MUL24, true, KFULL, false>(g, blockIdx.x, blockIdx.y);
}

// RES: the product may carry a fused residual add (a kernel without one has none of its code); NORM: and a fused
// rmsnorm of its sum
template <int BM, int BN, int WGM, int NS, int OSZ, bool MUL24, bool KFULL = false, bool RES = true, bool NORM = false>
__global__ __launch_bounds__(G_THREADS, (fast_occupancy<BM, BN>())) void gemm_i8_fast(GemmArgs g) {
  fast_tile<BM, BN, WGM, NS, OSZ, MUL24, false, KFULL, RES, NORM>(g, blockIdx.x, blockIdx.y);
}

// Up to GEMM_GROUP_MAX independent products in one launch (q, k and v of one input, say): member i owns the
// workgroups [first[i], first[i + 1]) (first[i] a multiple of 8, so each member's tiles keep their XCD placement),
// batch entry by batch entry like the single kernel's grid. One grid leaves one tail where separate launches leave
// one per product, and the launch gaps between them go.
constexpr int GEMM_GROUP_MAX = 4;
struct GemmGroupArgs {
  GemmArgs g[GEMM_GROUP_MAX];
  int first[GEMM_GROUP_MAX + 1];
  int n;
};

template <int BM, int BN, int WGM, int NS, int OSZ, bool MUL24, bool KFULL>
__global__ __launch_bounds__(G_THREADS, (fast_occupancy<BM, BN>())) void gemm_i8_fast_group(GemmGroupArgs a) {
  const int w = blockIdx.x;
  int i = 0;
#pragma unroll
  for (int j = 1; j < GEMM_GROUP_MAX; ++j) i += (j < a.n && w >= a.first[j]) ? 1 : 0;
  const GemmArgs& g = a.g[i];
  const int ntiles = g.tiles_m * g.tiles_n, local = w - a.first[i];
  const int bz = local / ntiles;
  if (bz >= g.nbatch) return;                            // padding up to the next member's multiple of 8
  fast_tile<BM, BN, WGM, NS, OSZ, MUL24, false, KFULL, false>(g, local - bz * ntiles, bz);   // no member has an add
}

// Persistent kernel with a register epilogue. Bt rows are loaded into LDS permuted within each 32-row group (LDS row c
// holds Bt row bperm(c)), so accumulator r of lane l is output column 16 (l / 32) + r of its 32 x 32 tile: each lane
// owns 16 consecutive columns of one row and writes them with one 16-byte store (two for i16), with no LDS staging.
// gridDim.x workgroups (a multiple of 8) walk every tile of every batch entry. XCD x (workgroups x, x + 8, ...) owns the contiguous logical tile range
// [x * chunk, (x + 1) * chunk) and its workgroups take consecutive tiles of it, so the tiles in flight on one XCD share
// A row bands and B column panels in that XCD's L2. The LDS pipeline runs on across tiles: the last two stages of a
// tile issue the next tile's first two stages, and the epilogue (registers only) runs while they load. A tile's K
// loop must be a whole number of array rotations (nk % NS == 0), so every tile starts in L0.
template <int BM, int BN, int BK, int NS>
constexpr int persist_occupancy() { return NS * (BM + BN) * BK + 256 <= 80 * 1024 ? 2 : 1; }

// NW waves in a (NW / WGN) x WGN grid over the BM x BN tile
template <int BM, int BN, int BK, int NS, int NW, int WGN, int OSZ, bool MUL24, bool KFULL>
__global__ __launch_bounds__(NW * 64, (persist_occupancy<BM, BN, BK, NS>())) void gemm_i8_persist(GemmArgs g) {
  constexpr int CPR = BK / 16, KS = BK / 32, WGM = NW / WGN;
  static_assert(NS >= 2 && NS <= 6, "two to six LDS stages");
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static_assert(WGM * WGN == NW && TM >= 1 && TN >= 1, "wave grid");
  static_assert(KS % 2 == 0, "fragment sets alternate within a stage");
  constexpr int IA = BM * CPR / 64, IB = BN * CPR / 64;
  static_assert(IA % NW == 0 && IB % NW == 0, "each wave issues an equal share of a stage");
  constexpr int JA = IA / NW, JB = IB / NW, G = JA + JB;
  constexpr int STAGE = (BM + BN) * BK;
  // the LUT first, at LDS address 0 (an alignment above the stages' puts it first), so that a lookup's address is
  // its index: the 256-entry table rotated, or widened to TAB entries (plain_epilogue)
  constexpr int TAB = table_bytes(NS * STAGE);
  __shared__ __attribute__((aligned(2048))) int8_t lut_s[TAB];
  __shared__ __attribute__((aligned(1024))) int8_t L0[STAGE];
  __shared__ __attribute__((aligned(1024))) int8_t L1[STAGE];
  __shared__ __attribute__((aligned(1024))) int8_t L2[NS > 2 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) int8_t L3[NS > 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) int8_t L4[NS > 4 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) int8_t L5[NS > 5 ? STAGE : 16];
  // the array of pipeline stage u (mod NS), chosen at compile time so that every LDS access has a known array
  auto arr = [&](auto u) -> int8_t* {
    constexpr int U = decltype(u)::value % NS;
    if constexpr (U == 0) return L0;
    else if constexpr (U == 1) return L1;
    else if constexpr (U == 2) return L2;
    else if constexpr (U == 3) return L3;
    else if constexpr (U == 4) return L4;
    else return L5;
  };

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int half = lane >> 5, l32 = lane & 31;

  const int per_batch = g.tiles_m * g.tiles_n, total = per_batch * g.nbatch;
  const int per_xcd = gridDim.x >> 3, xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int chunk = (total + 7) >> 3, lo_t = xcd * chunk, hi_t = min(total, lo_t + chunk);
  const int in_group = GROUP_M * g.tiles_n;
  struct Tile {
    int m0, n0, b0, b1;
    bool valid;
  };
  auto tile_of = [&](int it) {
    Tile T;
    const int L = lo_t + it * per_xcd + slot;
    T.valid = L < hi_t;
    const int b = T.valid ? L / per_batch : 0, pid = T.valid ? L % per_batch : 0;
    const int first_m = (pid / in_group) * GROUP_M;
    const int gsize = min(g.tiles_m - first_m, GROUP_M);
    T.m0 = (first_m + (pid % in_group) % gsize) * BM;
    T.n0 = ((pid % in_group) / gsize) * BN;
    T.b0 = b / g.batch1;
    T.b1 = b % g.batch1;
    return T;
  };
  // an invalid tile gets empty descriptors: its loads read zeros and are never used
  auto rsrc_a = [&](const Tile& T) {
    return uniform_rsrc(g.A + T.b0 * g.sa0 + T.b1 * g.sa1 + (long long)T.m0 * g.lda,
                        T.valid ? operand_bytes(min(g.M - T.m0, BM), g.lda, g.kba, g.K) : 0);
  };
  auto rsrc_b = [&](const Tile& T) {
    return uniform_rsrc(g.B + T.b0 * g.sb0 + T.b1 * g.sb1 + (long long)T.n0 * g.ldb,
                        T.valid ? operand_bytes(min(g.N - T.n0, BN), g.ldb, g.kbb, g.K) : 0);
  };

  Tile cur = tile_of(0);
  if (!cur.valid) return;
  // a table of 2^(32 - shift) entries fits: widened, entry u = lut[clamp(u - 2^(31 - shift), -128, 127) + 128]
  const bool wide = OSZ == 1 && g.lut && g.shift >= 1 && g.shift <= 31 && (1ll << (32 - g.shift)) <= TAB;
  if (wide) {
    const int n = 1 << (32 - g.shift), mid = 1 << (31 - g.shift);
    for (int u = t; u < n; u += NW * 64) lut_s[u] = g.lut[min(max(u - mid, -128), 127) + 128];
  } else if (g.lut && t < 256) {
    lut_s[t ^ 128] = g.lut[t];   // rotated: the entry of v at index v & 255
  }

  unsigned offa[JA], offb[JB];
  int ka[JA], kb[JB];
#pragma unroll
  for (int j = 0; j < JA; ++j) {
    const int P = (wave + NW * j) * 64 + lane, row = P / CPR, c = swz<BK>(row, P % CPR);
    offa[j] = (unsigned)(row * g.lda + (c >> 2) * g.kba + (c & 3) * 16);
    ka[j] = c * 16;
  }
#pragma unroll
  for (int j = 0; j < JB; ++j) {
    const int P = (wave + NW * j) * 64 + lane, row = P / CPR, c = swz<BK>(row, P % CPR);
    offb[j] = (unsigned)(((row & ~31) | bperm(row & 31)) * g.ldb + (c >> 2) * g.kbb + (c & 3) * 16);
    kb[j] = c * 16;
  }
  const int K = g.K;
  auto issue = [&](int8_t* arr, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, int k0) {
    // KFULL (K a whole number of BK-byte stages): no per-lane K bound, as in fast_tile; past the last tile the
    // descriptors are empty and every load reads zeros
    const unsigned oa = (unsigned)((k0 >> 6) * g.kba), ob = (unsigned)((k0 >> 6) * g.kbb);
#pragma unroll
    for (int j = 0; j < JA; ++j)
      dma16(ra, arr + (wave + NW * j) * 1024, KFULL ? offa[j] + oa : (k0 + ka[j] < K ? offa[j] + oa : OOB));
#pragma unroll
    for (int j = 0; j < JB; ++j)
      dma16(rb, arr + BM * BK + (wave + NW * j) * 1024, KFULL ? offb[j] + ob : (k0 + kb[j] < K ? offb[j] + ob : OOB));
  };

  v16i acc[TN][TM];
  v4i af[2][TM], bf[2][TN];
  auto load_frags = [&](int set, const int8_t* arr, int ks) {
    const int ch = ks * 2 + half;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int r = wm * WM + j * 32 + l32;
      af[set][j] = *reinterpret_cast<const v4i*>(arr + r * BK + (swz<BK>(r, ch) << 4));
    }
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int r = wn * WN + i * 32 + l32;
      bf[set][i] = *reinterpret_cast<const v4i*>(arr + BM * BK + r * BK + (swz<BK>(r, ch) << 4));
    }
  };
  // the MFMAs of a k-step at raised wave priority: with two waves a SIMD and no second workgroup on the CU, the
  // wave issuing them goes first while the other reads fragments (fc 88.9 -> 87.9 us; in the 256 x 128 kernel,
  // two workgroups a CU, the same slowed every product)
  auto mm = [&](int set) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[set][i], af[set][j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  };
  const int nk = (K + BK - 1) / BK;
  __amdgpu_buffer_rsrc_t ra = rsrc_a(cur), rb = rsrc_b(cur);
  // one pipeline step, as in gemm_i8_fast; stage kt + 2 belongs to the next tile once it passes this tile's K
  auto step = [&](int kt, const int8_t* curA, int8_t* nxt, const int8_t* next, __amdgpu_buffer_rsrc_t ran,
                  __amdgpu_buffer_rsrc_t rbn) {
    const bool over = kt + NS - 1 >= nk;
    issue(nxt, over ? ran : ra, over ? rbn : rb, (over ? kt + NS - 1 - nk : kt + NS - 1) * BK);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS - 1; ++ks) {
      load_frags((ks + 1) & 1, curA, ks + 1);
      __builtin_amdgcn_sched_barrier(0);
      mm(ks & 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm_lgkm0<(NS - 2) * G>();
    stage_barrier();
    load_frags(0, next, 0);
    __builtin_amdgcn_sched_barrier(0);
    mm((KS - 1) & 1);
  };

  static_for<NS - 1>([&](auto u) { issue(arr(u), ra, rb, decltype(u)::value * BK); });
  wait_vm_lgkm0<(NS - 2) * G>();
  stage_barrier();
  load_frags(0, L0, 0);
  for (int it = 0;; ++it) {
    const Tile nt = tile_of(it + 1);
    const __amdgpu_buffer_rsrc_t ran = rsrc_a(nt), rbn = rsrc_b(nt);
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int kt = 0; kt < nk; kt += NS) {
      static_for<NS>([&](auto u) {
        constexpr int U = decltype(u)::value;
        step(kt + U, arr(u), arr(std::integral_constant<int, U + NS - 1>{}), arr(std::integral_constant<int, U + 1>{}),
             ran, rbn);
      });
    }
    const int mrow = cur.m0 + wm * WM + l32, ncol = cur.n0 + wn * WN + 16 * half;
    if (OSZ == 1 && !g.res && g.vec_store != 0 && cur.m0 + BM <= g.M && cur.n0 + BN <= g.N) {
      if constexpr (OSZ == 1) {
        int8_t* p = reinterpret_cast<int8_t*>(g.C) + cur.b0 * g.sc0 + cur.b1 * g.sc1 + cpos(g, mrow, ncol);
        const uint8_t* tab = reinterpret_cast<const uint8_t*>(lut_s);
        if (wide) plain_epilogue<TM, TN, MUL24, 2>(g, acc, tab, p);
        else if (g.lut) plain_epilogue<TM, TN, MUL24, 1>(g, acc, tab, p);
        else plain_epilogue<TM, TN, MUL24, 0>(g, acc, tab, p);
      }
    } else {
      direct_epilogue<BM, BN, WM, WN, TM, TN, OSZ, MUL24>(g, acc, lut_s, wide, mrow, ncol, cur.m0, cur.n0, cur.b0,
                                                          cur.b1);
    }
    if (!nt.valid) break;
    cur = nt;
    ra = ran;
    rb = rbn;
  }
  wait_vmcnt(0);   // the trailing zero loads land in LDS before the workgroup's LDS is released
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int BM, int BN, int BK, int NS, bool MUL24, int NW = 4, int WGN = 2>
static void launch_persist(GemmArgs& g, int osz, int batch, int num_cu, hipStream_t s) {
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BN - 1) / BN;
  g.nbatch = batch;
  const long long total = (long long)g.tiles_m * g.tiles_n * batch;
  const int slots = 8 * ((num_cu * persist_occupancy<BM, BN, BK, NS>()) / 8);
  const int nwg = (int)std::min<long long>(slots, 8 * ((total + 7) / 8));
  const bool kfull = g.K % BK == 0;
  if (osz == 1 && kfull)
    ANVIL_LAUNCH((gemm_i8_persist<BM, BN, BK, NS, NW, WGN, 1, MUL24, true>), dim3(nwg), dim3(NW * 64), 0, s, g);
  else if (osz == 1)
    ANVIL_LAUNCH((gemm_i8_persist<BM, BN, BK, NS, NW, WGN, 1, MUL24, false>), dim3(nwg), dim3(NW * 64), 0, s, g);
  else if (kfull)
    ANVIL_LAUNCH((gemm_i8_persist<BM, BN, BK, NS, NW, WGN, 2, MUL24, true>), dim3(nwg), dim3(NW * 64), 0, s, g);
  else
    ANVIL_LAUNCH((gemm_i8_persist<BM, BN, BK, NS, NW, WGN, 2, MUL24, false>), dim3(nwg), dim3(NW * 64), 0, s, g);
}

// KF: the shapes the planner takes (256 x 128 and 128 x 128, three stages) have a KFULL form, used when K is a whole
// number of stage rotations (K % 192 == 0) and not truncated per tile (causal mode 2); the benchmarking-override
// shapes keep the per-lane K bound
template <int BM, int BN, int WGM, int NS, bool MUL24, bool KF = false>
static void launch_fast(GemmArgs& g, int osz, int batch, hipStream_t s) {
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BN - 1) / BN;
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  const bool kfull = KF && g.K % (64 * NS) == 0 && g.causal != 2;
  auto go = [&](auto res_c) {
    constexpr bool R = decltype(res_c)::value;
    if (osz == 1 && kfull)
      ANVIL_LAUNCH((gemm_i8_fast<BM, BN, WGM, NS, 1, MUL24, KF, R>), grid, dim3(G_THREADS), 0, s, g);
    else if (osz == 1)
      ANVIL_LAUNCH((gemm_i8_fast<BM, BN, WGM, NS, 1, MUL24, false, R>), grid, dim3(G_THREADS), 0, s, g);
    else if (kfull)
      ANVIL_LAUNCH((gemm_i8_fast<BM, BN, WGM, NS, 2, MUL24, KF, R>), grid, dim3(G_THREADS), 0, s, g);
    else
      ANVIL_LAUNCH((gemm_i8_fast<BM, BN, WGM, NS, 2, MUL24, false, R>), grid, dim3(G_THREADS), 0, s, g);
  };
  if (g.res) go(std::true_type{}); else go(std::false_type{});
}

// The fused add + rmsnorm product (anvil_gemm_i8_add_norm): BM x BN tiles, BN = N, so each tile spans its rows
template <int BM, int BN>
static void launch_fast_norm(GemmArgs& g, bool mul24, hipStream_t s) {
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = 1;
  const dim3 grid(g.tiles_m, 1);
  if (mul24)
    ANVIL_LAUNCH((gemm_i8_fast<BM, BN, 2, 3, 1, true, false, true, true>), grid, dim3(G_THREADS), 0, s, g);
  else
    ANVIL_LAUNCH((gemm_i8_fast<BM, BN, 2, 3, 1, false, false, true, true>), grid, dim3(G_THREADS), 0, s, g);
}

template <int BM, int BN, int WGM, int NS, bool MUL24>
static bool launch_fast_group(GemmArgs* gs, const int* batch, int n, int osz, hipStream_t s) {
  GemmGroupArgs a{};
  long long w = 0;
  for (int i = 0; i < n; ++i) {
    gs[i].tiles_m = (gs[i].M + BM - 1) / BM;
    gs[i].tiles_n = (gs[i].N + BN - 1) / BN;
    gs[i].nbatch = batch[i];
    a.g[i] = gs[i];
    a.first[i] = (int)w;
    w += ((long long)gs[i].tiles_m * gs[i].tiles_n * batch[i] + 7) / 8 * 8;
    if (w > (1ll << 31) - 1) return false;
  }
  a.first[n] = (int)w;
  a.n = n;
  bool kfull = true;
  for (int i = 0; i < n; ++i) kfull = kfull && gs[i].K % (64 * NS) == 0 && gs[i].causal != 2;
  if (osz == 1 && kfull)
    ANVIL_LAUNCH((gemm_i8_fast_group<BM, BN, WGM, NS, 1, MUL24, true>), dim3((unsigned)w), dim3(G_THREADS), 0, s, a);
  else if (osz == 1)
    ANVIL_LAUNCH((gemm_i8_fast_group<BM, BN, WGM, NS, 1, MUL24, false>), dim3((unsigned)w), dim3(G_THREADS), 0, s, a);
  else if (kfull)
    ANVIL_LAUNCH((gemm_i8_fast_group<BM, BN, WGM, NS, 2, MUL24, true>), dim3((unsigned)w), dim3(G_THREADS), 0, s, a);
  else
    ANVIL_LAUNCH((gemm_i8_fast_group<BM, BN, WGM, NS, 2, MUL24, false>), dim3((unsigned)w), dim3(G_THREADS), 0, s, a);
  return true;
}

// Few-tile products with a long K (a handful of rows against a wide weight, as in decoding): one workgroup of four
// groups of four waves per 64 x 64 output tile. Group grp sums the K chunks [grp S, (grp + 1) S) of the tile (S = a
// quarter of them, chunks of 128 bytes = four MFMA steps), its four waves on 32 x 32 sub-tiles in a 2 x 2 grid; the
// groups' partial sums meet in LDS and group 0 requantises. A group's chunk comes into LDS by direct-to-LDS loads
// (64 rows x 128 bytes of each operand, 16-byte pieces XOR-swizzled by row so fragment reads spread over the
// banks), two buffers a group, the next chunk loading while the current one feeds the MFMAs. Every group walks the
// same number of chunks (pieces past its K range or past K load zeros), so the workgroup barriers line up. B rows
// enter the MFMA in bperm order: accumulator r of lane l then holds column 16 (l / 32) + r of the lane's row l % 32,
// 16 consecutive outputs, one 16-byte store (i8).
constexpr int SMALL_SK = 4, SMALL_CK = 128;               // K groups a tile; K bytes a chunk

template <int OSZ, bool MUL24>
__global__ __launch_bounds__(SMALL_SK * 256) void gemm_i8_small(GemmArgs g) {
  constexpr int TILE = 64 * SMALL_CK;                     // one operand's chunk: 64 rows of 128 bytes
  // Each group's two buffers ([A | B] chunk) are arrays of their own, reached through a switch on the group, so the
  // compiler sees which array every load fills and every read reads, and keeps the newer chunk's loads in flight
  // across the older chunk's reads (with one array, or a group index into one, every read waited for every load).
  __shared__ __attribute__((aligned(1024))) int8_t s00[2 * TILE], s01[2 * TILE], s10[2 * TILE], s11[2 * TILE];
  __shared__ __attribute__((aligned(1024))) int8_t s20[2 * TILE], s21[2 * TILE], s30[2 * TILE], s31[2 * TILE];
  static_assert(SMALL_SK == 4, "four groups");
  __shared__ int8_t lut_s[256];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int grp = wave >> 2, wq = wave & 3, wm = wq >> 1, wn = wq & 1;
  const int l32 = lane & 31, half = lane >> 5;
  const int tm = blockIdx.x / g.tiles_n, tn = blockIdx.x % g.tiles_n;
  const int am0 = tm * 64, bn0 = tn * 64;
  const int rows_a = min(g.M - am0, 64), rows_b = min(g.N - bn0, 64);
  const __amdgpu_buffer_rsrc_t ra =
      uniform_rsrc(g.A + (long long)am0 * g.lda, operand_bytes(rows_a, g.lda, g.kba, g.K));
  const __amdgpu_buffer_rsrc_t rb =
      uniform_rsrc(g.B + (long long)bn0 * g.ldb, operand_bytes(rows_b, g.ldb, g.kbb, g.K));
  if (g.lut && t < 256) lut_s[t ^ 128] = g.lut[t];        // rotated: the entry of v at index v & 255
  const int nck = (g.K + SMALL_CK - 1) / SMALL_CK;        // chunks of the product
  const int S = (nck + SMALL_SK - 1) / SMALL_SK;          // chunks a group (the last group's may run past K)
  const int kend = min(g.K, (grp + 1) * S * SMALL_CK);    // this group's K bytes end here
  // this wave's two load instructions of each operand: rows 8 i + lane / 8 (i = wq, wq + 4), global piece
  // (lane % 8) ^ swizzle, landing in LDS piece lane % 8 of that row
  int pk[2];                                              // the piece's K offset in a chunk
  unsigned rowa[2], rowb[2];                              // the row's byte offset, or OOB past the tile's rows
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 8 * (wq + 4 * j) + (lane >> 3);
    pk[j] = 16 * swz<128>(r, lane & 7);
    rowa[j] = r < rows_a ? (unsigned)(r * g.lda) : OOB;
    rowb[j] = r < rows_b ? (unsigned)(r * g.ldb) : OOB;
  }
  // a chunk's pieces start at multiples of 16 below a 64-byte block's end, so block k >> 6 holds all 16 bytes
  auto issue = [&](int c, int8_t* base) __attribute__((always_inline)) {   // chunk c of this group into base
    const int k0 = (grp * S + c) * SMALL_CK;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int k = k0 + pk[j];
      const bool kin = k < kend;
      const unsigned ka = (unsigned)((k >> 6) * g.kba + (k & 63)), kb = (unsigned)((k >> 6) * g.kbb + (k & 63));
      dma16(ra, base + (wq + 4 * j) * 1024, kin && rowa[j] != OOB ? rowa[j] + ka : OOB);
      dma16(rb, base + TILE + (wq + 4 * j) * 1024, kin && rowb[j] != OOB ? rowb[j] + kb : OOB);
    }
  };
  const int ar = wm * 32 + l32, br = wn * 32 + bperm(l32);
  v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  auto compute = [&](const int8_t* base) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {                         // MFMA step j: logical pieces 2 j and 2 j + 1
      const int q = 2 * j + half;
      const v4i af = *reinterpret_cast<const v4i*>(base + ar * SMALL_CK + 16 * swz<128>(ar, q));
      const v4i bf = *reinterpret_cast<const v4i*>(base + TILE + br * SMALL_CK + 16 * swz<128>(br, q));
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af, acc, 0, 0, 0);
    }
  };
  // chunk c lives in buffer c % 2; chunk c + 1 loads while chunk c is read (past the group's chunks every piece is
  // out of range: zeros). The waits leave the newer chunk's four loads of this wave in flight; the barriers (no
  // release fence, which would wait for those loads too) make every wave's pieces visible, then free the buffer for
  // the chunk after next.
  auto walk = [&](int8_t* b0, int8_t* b1) __attribute__((always_inline)) {   // inlined: b0, b1 known arrays
    issue(0, b0);
    for (int c = 0; c < S; c += 2) {
      issue(c + 1, b1);
      wait_vmcnt(4);
      stage_barrier();
      compute(b0);
      __builtin_amdgcn_s_waitcnt(0xC07F);                 // lgkmcnt(0): this wave's reads of b0 are done
      stage_barrier();
      if (c + 1 >= S) break;
      issue(c + 2, b0);
      wait_vmcnt(4);
      stage_barrier();
      compute(b1);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      stage_barrier();
    }
    wait_vmcnt(0);                                        // the last (all-zero) chunk's loads land before LDS reuse
    __syncthreads();
    if (grp > 0) {                                        // the partial sums, into the group's first buffer (16 KiB)
      int* pp = reinterpret_cast<int*>(b0) + (wq * 64 + lane) * 16;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<v4i*>(pp + 4 * q) = v4i{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
    }
    __syncthreads();
  };
  switch (grp) {
    case 0: walk(s00, s01); break;
    case 1: walk(s10, s11); break;
    case 2: walk(s20, s21); break;
    default: walk(s30, s31); break;
  }
  if (grp > 0) return;
  for (const int8_t* b : {s10, s20, s30}) {
    const int* pp = reinterpret_cast<const int*>(b) + (wq * 64 + lane) * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const v4i x = *reinterpret_cast<const v4i*>(pp + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[4 * q + e] += x[e];
    }
  }
  const int m = am0 + ar, n = bn0 + wn * 32 + 16 * half;
  if (m >= g.M || n >= g.N) return;
  const int lo = OSZ == 1 ? -128 : -32768, hi = OSZ == 1 ? 127 : 32767;
  int v[16];
  auto requant = [&](auto lut) {                          // the LUT choice outside the element loop
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int x = MUL24 ? (__mul24(acc[r], g.mult) + g.rnd) : (acc[r] * g.mult + g.rnd);
      v[r] = min(max(x >> g.shift, lo), hi);
      if constexpr (decltype(lut)::value) v[r] = lut_s[(uint8_t)v[r]];
    }
  };
  if (OSZ == 1 && g.lut)
    requant(std::true_type{});
  else
    requant(std::false_type{});
  char* c = reinterpret_cast<char*>(g.C) + cpos(g, m, n) * OSZ;
  if (g.vec_store && n + 16 <= g.N) {
    if (OSZ == 1) {
      *reinterpret_cast<v4i*>(c) = v4i{(int)pack4(v[0], v[1], v[2], v[3]), (int)pack4(v[4], v[5], v[6], v[7]),
                                       (int)pack4(v[8], v[9], v[10], v[11]), (int)pack4(v[12], v[13], v[14], v[15])};
    } else {
      v4i w0, w1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        w0[q] = (int)__builtin_amdgcn_perm((unsigned)v[2 * q + 1], (unsigned)v[2 * q], 0x05040100u);
        w1[q] = (int)__builtin_amdgcn_perm((unsigned)v[2 * q + 9], (unsigned)v[2 * q + 8], 0x05040100u);
      }
      *reinterpret_cast<v4i*>(c) = w0;
      *reinterpret_cast<v4i*>(c + 16) = w1;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (n + e >= g.N) break;
      if (OSZ == 1)
        reinterpret_cast<int8_t*>(g.C)[cpos(g, m, n + e)] = (int8_t)v[e];
      else
        reinterpret_cast<int16_t*>(g.C)[cpos(g, m, n + e)] = (int16_t)v[e];
    }
  }
}

template <bool MUL24>
static void launch_small(GemmArgs& g, int osz, hipStream_t s) {
  g.tiles_m = (g.M + 63) / 64;
  g.tiles_n = (g.N + 63) / 64;
  const dim3 grid(g.tiles_m * g.tiles_n);
  if (osz == 1)
    ANVIL_LAUNCH((gemm_i8_small<1, MUL24>), grid, dim3(SMALL_SK * 256), 0, s, g);
  else
    ANVIL_LAUNCH((gemm_i8_small<2, MUL24>), grid, dim3(SMALL_SK * 256), 0, s, g);
}

// Narrow products over many rows: K and N each 32 or 64 (the reference's frozen models, C = 32: q, k, v, y with
// its residual add, gate, up, down), where a 128-row tile leaves most of every MFMA and of its operand loads unused.
// One wave takes a block of 32 rows at a time (walking blocks grid-stride, the next block's rows loading during
// this one's epilogue): its A rows load as MFMA fragments (lane l: row l % 32, 16 K bytes at 16 (l / 32) + 32 k,
// 1 KiB contiguous for a dense 32-byte row), the weights' fragments stay in registers for the whole walk, and up to
// four products that share A (q, k and v of one input) run in the same pass. B rows enter the MFMA in bperm order,
// so a lane's 16 accumulators are 16 consecutive columns of its row: one 16-byte store (i8), or two (i16).
// RES: the fused add_requant of anvil_gemm_i8_add (one member): D = clamp((R ma + y mb + rnd2) >> shift2) in the
// result's dtype, y stored when store_y.
struct SkinnyArgs {
  GemmArgs g[GEMM_GROUP_MAX];
  int n;                  // members, sharing A, M and K
  int nblocks;            // blocks of 32 rows
};

template <int NT, int KS, int OSZ, bool MUL24, bool RES>
__global__ __launch_bounds__(G_THREADS) void gemm_i8_skinny(SkinnyArgs sa) {
  __shared__ int8_t lut_s[GEMM_GROUP_MAX][256];
  const int t = threadIdx.x, lane = t & 63;
  const int l32 = lane & 31, half = lane >> 5;
  const GemmArgs& g0 = sa.g[0];
#pragma unroll
  for (int j = 0; j < GEMM_GROUP_MAX; ++j)
    if (j < sa.n && sa.g[j].lut) lut_s[j][t ^ 128] = sa.g[j].lut[t];   // rotated: entry of v at index v & 255
  __syncthreads();
  // the members' weight fragments: B row 32 nt + bperm(l32), K bytes 32 ks + 16 half
  v4i bf[GEMM_GROUP_MAX][NT][KS];
#pragma unroll
  for (int j = 0; j < GEMM_GROUP_MAX; ++j)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const GemmArgs& g = sa.g[j < sa.n ? j : 0];
        const int r = 32 * nt + bperm(l32), k = 32 * ks + 16 * half;
        bf[j][nt][ks] = j < sa.n && r < g.N && k < g.K
                            ? *reinterpret_cast<const v4i*>(g.B + (long long)r * g.ldb + (k >> 6) * g.kbb + (k & 63))
                            : v4i{0, 0, 0, 0};
      }
  const __amdgpu_buffer_rsrc_t ra = uniform_rsrc(g0.A, operand_bytes(g0.M, g0.lda, g0.kba, g0.K));
  auto aoff = [&](int blk, int ks) -> unsigned {        // this lane's A fragment of block blk, or out of range
    const int m = 32 * blk + l32, k = 32 * ks + 16 * half;
    return blk < sa.nblocks && m < g0.M && k < g0.K ? (unsigned)(m * g0.lda + (k >> 6) * g0.kba + (k & 63)) : OOB;
  };
  const int wave = blockIdx.x * (G_THREADS / 64) + (t >> 6), nwaves = gridDim.x * (G_THREADS / 64);
  v4i af[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    af[ks] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, aoff(wave, ks), 0, 0));
  constexpr int LO = OSZ == 1 ? -128 : -32768, HI = OSZ == 1 ? 127 : 32767;
  for (int blk = wave; blk < sa.nblocks; blk += nwaves) {
    v4i an[KS];                                          // the next block's rows load during this block's work
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      an[ks] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, aoff(blk + nwaves, ks), 0, 0));
    const int m = 32 * blk + l32;
#pragma unroll
    for (int j = 0; j < GEMM_GROUP_MAX; ++j) {
      if (j >= sa.n) break;
      const GemmArgs& g = sa.g[j];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j][nt][ks], af[ks], acc, 0, 0, 0);
        const int n = 32 * nt + 16 * half;
        if (m >= g0.M || n >= g.N) continue;
        int v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int x = MUL24 ? (__mul24(acc[r], g.mult) + g.rnd) : (acc[r] * g.mult + g.rnd);
          v[r] = min(max(x >> g.shift, LO), HI);
        }
        if (OSZ == 1 && g.lut) {
#pragma unroll
          for (int r = 0; r < 16; ++r) v[r] = lut_s[j][(uint8_t)v[r]];
        }
        const bool whole = n + 16 <= g.N;
        if constexpr (RES) {                             // D = clamp((R ma + y mb + rnd2) >> shift2), proven in int32
          int o[16];
          if constexpr (OSZ == 1) {
            const int8_t* rp = g.R + (long long)m * g.ldr + n;
            v4i rv = {0, 0, 0, 0};
            if (whole && g.vec_res) rv = *reinterpret_cast<const v4i*>(rp);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int r = whole && g.vec_res ? (int)(int8_t)((unsigned)rv[e >> 2] >> (8 * (e & 3)))
                                               : (n + e < g.N ? (int)rp[e] : 0);
              o[e] = min(max((r * g.ma + v[e] * g.mb + g.rnd2) >> g.shift2, LO), HI);
            }
          } else {
            const int16_t* rp = reinterpret_cast<const int16_t*>(g.R) + (long long)m * g.ldr + n;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int r = n + e < g.N ? (int)rp[e] : 0;
              o[e] = min(max((r * g.ma + v[e] * g.mb + g.rnd2) >> g.shift2, LO), HI);
            }
          }
          char* dp = reinterpret_cast<char*>(g.D) + ((long long)m * g.ldd + n) * OSZ;
          if (whole && g.vec_res) {
            if (OSZ == 1) {
              *reinterpret_cast<v4i*>(dp) = v4i{(int)pack4(o[0], o[1], o[2], o[3]), (int)pack4(o[4], o[5], o[6], o[7]),
                                                (int)pack4(o[8], o[9], o[10], o[11]),
                                                (int)pack4(o[12], o[13], o[14], o[15])};
            } else {
              v4i w0, w1;
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                w0[q] = (int)__builtin_amdgcn_perm((unsigned)o[2 * q + 1], (unsigned)o[2 * q], 0x05040100u);
                w1[q] = (int)__builtin_amdgcn_perm((unsigned)o[2 * q + 9], (unsigned)o[2 * q + 8], 0x05040100u);
              }
              *reinterpret_cast<v4i*>(dp) = w0;
              *reinterpret_cast<v4i*>(dp + 16) = w1;
            }
          } else {
            for (int e = 0; e < 16 && n + e < g.N; ++e) {
              if (OSZ == 1)
                reinterpret_cast<int8_t*>(dp)[e] = (int8_t)o[e];
              else
                reinterpret_cast<int16_t*>(dp)[e] = (int16_t)o[e];
            }
          }
          if (!g.store_y) continue;
        }
        char* c = reinterpret_cast<char*>(g.C) + cpos(g, m, n) * OSZ;
        if (whole && g.vec_store) {
          if (OSZ == 1) {
            *reinterpret_cast<v4i*>(c) = v4i{(int)pack4(v[0], v[1], v[2], v[3]), (int)pack4(v[4], v[5], v[6], v[7]),
                                             (int)pack4(v[8], v[9], v[10], v[11]),
                                             (int)pack4(v[12], v[13], v[14], v[15])};
          } else {
            v4i w0, w1;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              w0[q] = (int)__builtin_amdgcn_perm((unsigned)v[2 * q + 1], (unsigned)v[2 * q], 0x05040100u);
              w1[q] = (int)__builtin_amdgcn_perm((unsigned)v[2 * q + 9], (unsigned)v[2 * q + 8], 0x05040100u);
            }
            *reinterpret_cast<v4i*>(c) = w0;
            *reinterpret_cast<v4i*>(c + 16) = w1;
          }
        } else {
          for (int e = 0; e < 16 && n + e < g.N; ++e) {
            if (OSZ == 1)
              reinterpret_cast<int8_t*>(g.C)[cpos(g, m, n + e)] = (int8_t)v[e];
            else
              reinterpret_cast<int16_t*>(g.C)[cpos(g, m, n + e)] = (int16_t)v[e];
          }
        }
      }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) af[ks] = an[ks];
  }
}

// Whether a fast-path product (one member of a group, or the product of a fused add) takes gemm_i8_skinny: batch 1, no
// causal mode or split, K and N each 32 or 64, at least 4096 rows.
static bool skinny_ok(const GemmArgs& g, int batch) {
  return batch == 1 && g.causal == 0 && (g.K == 32 || g.K == 64) && (g.N == 32 || g.N == 64) && g.M >= 4096 &&
         (long long)g.M * g.lda < (1ll << 31);
}

template <bool MUL24>
static void launch_skinny(const GemmArgs* gs, int n, int osz, int num_cu, hipStream_t s) {
  SkinnyArgs sa;
  for (int i = 0; i < n; ++i) sa.g[i] = gs[i];
  for (int i = n; i < GEMM_GROUP_MAX; ++i) sa.g[i] = gs[0];
  sa.n = n;
  sa.nblocks = (gs[0].M + 31) / 32;
  const int nt = (gs[0].N + 31) / 32, ks = (gs[0].K + 31) / 32;
  const bool res = gs[0].res != 0;
  const dim3 grid((unsigned)std::min<long long>((sa.nblocks + 3) / 4, 8ll * num_cu));
  auto go = [&](auto kernel) { ANVIL_LAUNCH(kernel, grid, dim3(G_THREADS), 0, s, sa); };
#define ANVIL_SKINNY(NT, KS, OSZ, RES) \
  if (nt == NT && ks == KS && osz == OSZ && res == RES) return go(gemm_i8_skinny<NT, KS, OSZ, MUL24, RES>);
  ANVIL_SKINNY(1, 1, 1, false) ANVIL_SKINNY(1, 2, 1, false) ANVIL_SKINNY(2, 1, 1, false) ANVIL_SKINNY(2, 2, 1, false)
  ANVIL_SKINNY(1, 1, 2, false) ANVIL_SKINNY(1, 2, 2, false) ANVIL_SKINNY(2, 1, 2, false) ANVIL_SKINNY(2, 2, 2, false)
  ANVIL_SKINNY(1, 1, 1, true) ANVIL_SKINNY(1, 2, 1, true) ANVIL_SKINNY(2, 1, 1, true) ANVIL_SKINNY(2, 2, 1, true)
  ANVIL_SKINNY(1, 1, 2, true) ANVIL_SKINNY(1, 2, 2, true) ANVIL_SKINNY(2, 1, 2, true) ANVIL_SKINNY(2, 2, 2, true)
#undef ANVIL_SKINNY
}

// Whether a fast-path product takes gemm_i8_small: one product (batch 1, no causal mode, no fused add) whose 128 x 128
// tiles fill at most a quarter of the CUs, with K >= 512.
static bool small_plan(const GemmArgs& g, int batch, int num_cu) {
  if (batch != 1 || g.causal != 0 || g.res || g.K < 512) return false;
  const long long tiles = (long long)((g.M + 127) / 128) * ((g.N + 127) / 128);
  return tiles * 4 <= num_cu;
}

constexpr int SPLITK_MAX = 4;                             // K chunks of one product (partial tiles kept per tile)

// Split-K on 128 x 128 tiles (three LDS stages, three workgroups per CU): grid (tiles, splits) storing partial
// tiles, then the reduction, eight workgroups per tile.
template <bool MUL24>
static void launch_splitk(GemmArgs& g, int osz, hipStream_t s) {
  g.tiles_m = (g.M + 127) / 128;
  g.tiles_n = (g.N + 127) / 128;
  dim3 grid(g.tiles_m * g.tiles_n, g.splits);
  const dim3 rgrid(g.tiles_m * g.tiles_n * 8);
  const bool kfull = g.K % 192 == 0 && g.kchunk % 192 == 0;   // every chunk whole rotations of three stages
  if (osz == 1) {
    if (kfull)
      ANVIL_LAUNCH((gemm_i8_splitk<128, 128, 2, 3, 1, MUL24, true>), grid, dim3(G_THREADS), 0, s, g);
    else
      ANVIL_LAUNCH((gemm_i8_splitk<128, 128, 2, 3, 1, MUL24, false>), grid, dim3(G_THREADS), 0, s, g);
    ANVIL_LAUNCH((splitk_reduce<1, MUL24>), rgrid, dim3(G_THREADS), 0, s, g);
  } else {
    if (kfull)
      ANVIL_LAUNCH((gemm_i8_splitk<128, 128, 2, 3, 2, MUL24, true>), grid, dim3(G_THREADS), 0, s, g);
    else
      ANVIL_LAUNCH((gemm_i8_splitk<128, 128, 2, 3, 2, MUL24, false>), grid, dim3(G_THREADS), 0, s, g);
    ANVIL_LAUNCH((splitk_reduce<2, MUL24>), rgrid, dim3(G_THREADS), 0, s, g);
  }
}

// Whether a fast-path product splits K, and into how many chunks: a single product (batch 1, no causal mode or fused
// add) with K >= 2048 whose 128 x 128 output tiles fill at most a quarter of the CUs splits into two to SPLITK_MAX
// chunks of whole 64-byte K blocks; `force` (ANVIL_GEMM_SPLITK) splits any such product. Measured on MI355X (two
// launches, partial tiles through the workspace): 256 x 3072 x 3072 (48 tiles) 22.1 -> 17.8 us; at K = 768
// (256 x 768 x 768, 12 tiles) the second launch costs more than the split saves, 11.4 -> 13.3 us.
static bool splitk_plan(const GemmArgs& g, int batch, int num_cu, bool force, int& splits, int& kchunk) {
  if (batch != 1 || g.causal != 0 || g.res) return false;
  const long long tiles = (long long)((g.M + 127) / 128) * ((g.N + 127) / 128);
  if (!force && (tiles * 4 > num_cu || g.K < 2048)) return false;
  long long want = std::max<long long>(2, (2ll * num_cu + tiles - 1) / tiles);
  want = std::min<long long>(std::min<long long>(want, SPLITK_MAX), std::max(1, g.K / 128));
  kchunk = (int)(((g.K + want - 1) / want + 63) / 64 * 64);
  splits = (g.K + kchunk - 1) / kchunk;
  return force || splits >= 2;
}

// The fast-path configuration of a product, named by the context's benchmarking override values: 39 and 40 the
// persistent 256 x 256 (K blocks of 64) and 256 x 128 (K blocks of 128) kernels, 11 - 20 the one-tile-per-workgroup
// shapes of the switch in launch_fast_choice. An override the product cannot take falls through to the rules.
static int fast_choice(const GemmArgs& g, int batch, int cfg, int num_cu) {
  // the persistent 256 x 256 kernel: one workgroup of 8 waves per CU, four 32 KiB LDS stages, wave tiles 64 x 128
  const bool persist_ok = g.causal == 0 && ((g.K + 63) / 64) % 4 == 0;
  const bool persist128_ok = g.causal == 0 && ((g.K + 127) / 128) % 3 == 0;
  const bool persist128x2_ok = g.causal == 0 && ((g.K + 127) / 128) % 2 == 0;
  if ((cfg == 39 && persist_ok) || (cfg == 40 && persist128_ok) || ((cfg == 41 || cfg == 42) && persist128x2_ok) ||
      (cfg >= 11 && cfg <= 20))
    return cfg;
  // measured on MI355X (block GEMM shapes, K 768 and 3072): wide products with at least six 256 x 256 tiles per CU
  // take the persistent kernel (it halves the L2 traffic per MFMA of the 256 x 128 tile); 256 x 128 tiles with three
  // LDS stages (72 KiB) run two workgroups per CU, which hide each other's pipeline fill and epilogue; small problems
  // keep the 128 x 128 tile (more workgroups)
  const long long tiles256 = (long long)((g.M + 255) / 256) * ((g.N + 255) / 256) * batch;
  // Wide and long (N, K >= 2048): 256 x 256 tiles with 128-byte K blocks in two LDS stages (128 KiB). Its loads fetch
  // whole 128-byte lines of each row, and a stage (four k-steps) covers the next one's latency once K is long.
  // Measured: 16384 x 3072 x 3072 147 us against 188 us on 64-byte K blocks; at K = 768 (fc) it loses, 100 vs 97 us.
  if (persist128x2_ok && g.N >= 2048 && g.K >= 2048 && tiles256 >= (long long)num_cu) return 41;
  if (persist_ok && g.N >= 2048 && tiles256 >= 6ll * num_cu) return 39;
  // Long K, N below 2048 (the block's proj, K 3072, N 768): the persistent kernel on 256 x 128 tiles with 128-byte
  // K blocks. Its loads fetch 128 contiguous bytes of each row (the 64-byte rows of a K block of 64 reach about half
  // the L2 bandwidth), and the tiles (768 at proj) divide evenly over one workgroup per CU. Measured: proj 87.5 ->
  // 82.5 us alone, about 5 us a step with its fused residual add. Short K (q, y) gains nothing and fc loses on it.
  // Otherwise, N a multiple of 192 without a fused add: 256 x 192 tiles, one workgroup per CU with whole tiles
  // (with the fused add its heavier epilogue has no second workgroup beside it and loses to 256 x 128).
  // Both rules serve a row-major A, whose 64-byte row pieces are the slow pattern: with A K-blocked (64-byte blocks
  // of consecutive rows contiguous) the 256 x 128 tile with K blocks of 64 is faster (proj 72 against 80 us).
  const bool a_rows = g.kba == 64;
  const long long tiles128 = (long long)((g.M + 255) / 256) * ((g.N + 127) / 128) * batch;
  if (a_rows && g.K >= 2048 && g.N < 2048 && persist128_ok && tiles128 >= 2ll * num_cu) return 40;
  const long long tiles192 = (long long)((g.M + 255) / 256) * (g.N / 192) * batch;
  if (a_rows && g.K >= 2048 && g.N % 192 == 0 && g.N < 2048 && !g.res && tiles192 >= 2ll * num_cu) return 19;
  if ((long long)g.M * g.N * batch >= 256ll * 128 * 512 && g.M >= 256 && g.N >= 128) return 16;
  return 13;
}

template <bool MUL24>
static void launch_fast_choice(GemmArgs& g, int osz, int batch, hipStream_t s, int choice, int num_cu) {
  switch (choice) {
    case 39: return launch_persist<256, 256, 64, 4, MUL24, 8, 2>(g, osz, batch, num_cu, s);
    case 40: return launch_persist<256, 128, 128, 3, MUL24, 8, 2>(g, osz, batch, num_cu, s);
    case 41: return launch_persist<256, 256, 128, 2, MUL24, 8, 2>(g, osz, batch, num_cu, s);
    case 42: return launch_persist<256, 128, 128, 2, MUL24, 8, 2>(g, osz, batch, num_cu, s);
    case 11: return launch_fast<256, 256, 2, 3, MUL24>(g, osz, batch, s);
    case 12: return launch_fast<256, 256, 2, 4, MUL24>(g, osz, batch, s);
    case 14: return launch_fast<128, 128, 2, 4, MUL24>(g, osz, batch, s);
    case 15: return launch_fast<256, 128, 2, 4, MUL24>(g, osz, batch, s);
    case 16: return launch_fast<256, 128, 2, 3, MUL24, true>(g, osz, batch, s);
    case 17: return launch_fast<128, 256, 2, 3, MUL24>(g, osz, batch, s);
    case 18: return launch_fast<128, 192, 2, 3, MUL24>(g, osz, batch, s);
    case 19: return launch_fast<256, 192, 2, 3, MUL24>(g, osz, batch, s);
    case 20: return launch_fast<256, 192, 2, 4, MUL24>(g, osz, batch, s);
    default: return launch_fast<128, 128, 2, 3, MUL24, true>(g, osz, batch, s);
  }
}

template <int BM, int BN, int BK, int WGM, int PF, bool CHECKED>
static void launch_cfg(GemmArgs& g, int osz, bool vec, int batch, hipStream_t s) {
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BN - 1) / BN;
  dim3 grid(g.tiles_m * g.tiles_n, batch);
  if (osz == 1) {
    if (vec)
      ANVIL_LAUNCH((gemm_i8_kernel<BM, BN, BK, WGM, PF, 1, CHECKED, true>), grid, dim3(G_THREADS), 0, s, g);
    else
      ANVIL_LAUNCH((gemm_i8_kernel<BM, BN, BK, WGM, PF, 1, CHECKED, false>), grid, dim3(G_THREADS), 0, s, g);
  } else {
    if (vec)
      ANVIL_LAUNCH((gemm_i8_kernel<BM, BN, BK, WGM, PF, 2, CHECKED, true>), grid, dim3(G_THREADS), 0, s, g);
    else
      ANVIL_LAUNCH((gemm_i8_kernel<BM, BN, BK, WGM, PF, 2, CHECKED, false>), grid, dim3(G_THREADS), 0, s, g);
  }
}

// Tile shape by problem: 128 x 128 for checked runs (its epilogue keeps the 64-bit checks in registers) and small
// problems, 256 x 64 with the four waves stacked along M when N <= 64 (attention's P.V), 256 x 256 otherwise.
// cfg (the context's ANVIL_GEMM_CFG, a benchmarking override) pins one shape for every unchecked GEMM.
static void launch_gemm(GemmArgs& g, bool checked, int osz, bool vec, int batch, hipStream_t s, int cfg) {
  if (checked) return launch_cfg<128, 128, 64, 2, 1, true>(g, osz, vec, batch, s);
  switch (cfg) {
    case 1: return launch_cfg<256, 256, 64, 2, 1, false>(g, osz, vec, batch, s);
    case 2: return launch_cfg<256, 256, 64, 2, 2, false>(g, osz, vec, batch, s);
    case 3: return launch_cfg<256, 128, 64, 2, 2, false>(g, osz, vec, batch, s);
    case 4: return launch_cfg<128, 128, 64, 2, 2, false>(g, osz, vec, batch, s);
    case 5: return launch_cfg<256, 256, 128, 2, 1, false>(g, osz, vec, batch, s);
    case 6: return launch_cfg<128, 256, 64, 2, 2, false>(g, osz, vec, batch, s);
    default: break;
  }
  if (g.N <= 64)
    launch_cfg<256, 64, 64, 4, 2, false>(g, osz, vec, batch, s);
  else if (g.M <= 128 || g.N <= 128)
    launch_cfg<128, 128, 64, 2, 2, false>(g, osz, vec, batch, s);
  else
    launch_cfg<256, 256, 64, 2, 2, false>(g, osz, vec, batch, s);
}

// Static split-K scratch of anvil_gemm_i8_noalloc: SCRATCH_SUMS int32 partial sums. Each device holds its own copy
// until the process ends; the library only ever uses it through the per-device address hipGetSymbolAddress returns
// (the array's name is a host-side stand-in in host code). A split-K run writes every partial sum before it reads it,
// so nothing needs clearing between calls. Calls on one stream run in order; calls from two streams could overlap on
// the device and race, so a device's scratch belongs to the first context that splits into it, until that context
// is destroyed (its stream drained first), and any other context's split is refused.
constexpr long long SCRATCH_SUMS = 1ll << 22;     // 16 MiB: 64 tiles of 128 x 128 in four K chunks
constexpr int SCRATCH_DEVICES = 64;
static __device__ __align__(256) int scratch[SCRATCH_SUMS];
static int* g_scratch[SCRATCH_DEVICES];
static anvil_ctx* g_scratch_owner[SCRATCH_DEVICES];
static std::mutex g_scratch_mu;

// The device's scratch for ctx: claimed on first use, refused while another context holds it.
static int claim_scratch(anvil_ctx* ctx, int** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[ctx->device]) return set_error(ANVIL_E_RUNTIME, "anvil_gemm_i8_noalloc: scratch not set up");
  if (g_scratch_owner[ctx->device] && g_scratch_owner[ctx->device] != ctx)
    return set_error(ANVIL_E_RUNTIME,
                     "anvil_gemm_i8_noalloc: device %d's static split-K scratch belongs to another context until it "
                     "is destroyed (split-K calls from two contexts could overlap on the device)", ctx->device);
  g_scratch_owner[ctx->device] = ctx;
  *out = g_scratch[ctx->device];
  return ANVIL_OK;
}

void gemm_scratch_release(anvil_ctx* ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (ctx->device >= 0 && ctx->device < SCRATCH_DEVICES && g_scratch_owner[ctx->device] == ctx)
    g_scratch_owner[ctx->device] = nullptr;
}

int gemm_scratch_setup(int device) {
  if (device < 0 || device >= SCRATCH_DEVICES)
    return set_error(ANVIL_E_VALUE, "device %d beyond the %d the static GEMM scratch serves", device, SCRATCH_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device]) return ANVIL_OK;
  void* ptr = nullptr;
  ANVIL_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  g_scratch[device] = static_cast<int*>(ptr);
  return ANVIL_OK;
}

}  // namespace anvil

using namespace anvil;

struct AddEpilogue {
  const int8_t* R;     // R and D have the product's result dtype (i8 or i16)
  int8_t* D;
  const int64_t* rstrides;
  int ma, mb, shift2;
};

// A validated product and the kernel family it takes.
struct Prepared {
  GemmArgs g;
  int osz, batch;
  bool checked, vec, fast, mul24, force_split;
};

// Argument checks that need no context (a group checks every member before any launch).
static int gemm_validate(const int8_t* A, const int8_t* Bt, const void* C, int batch0, int batch1, int M, int N, int K,
                         const int64_t* strides, int32_t mult, int shift, const int8_t* lut, int out_dtype, int flags,
                         const AddEpilogue* add) {
  if (!A || !Bt || (!C && !add) || !strides) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: null pointer");
  if (batch0 < 1 || batch1 < 1 || M < 1 || N < 1 || K < 1)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: non-positive size (batch %d x %d, M %d, N %d, K %d)", batch0,
                     batch1, M, N, K);
  if ((long long)batch0 * batch1 > 65535) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: batch above 65535");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (out_dtype != ANVIL_I8 && out_dtype != ANVIL_I16)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: result dtype must be i8 or i16");
  if (lut && out_dtype != ANVIL_I8) return set_error(ANVIL_E_VALUE, "a LUT epilogue needs an i8 result");
  if (flags & ~(ANVIL_GEMM_UNCHECKED | ANVIL_GEMM_CAUSAL_SKIP | ANVIL_GEMM_CAUSAL_K | ANVIL_GEMM_MUL24 |
                ANVIL_GEMM_SPLITK | ANVIL_GEMM_A_KBLOCK | ANVIL_GEMM_B_KBLOCK | ANVIL_GEMM_C_KBLOCK))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: unknown flags %d", flags);
  for (int o = 0; o < 3; ++o) {                          // K-blocked operands and result: block stride and reach
    const int flag = o == 0 ? ANVIL_GEMM_A_KBLOCK : (o == 1 ? ANVIL_GEMM_B_KBLOCK : ANVIL_GEMM_C_KBLOCK);
    if (!(flags & flag)) continue;
    const long long kb = strides[2 + 3 * o];
    const int blocks = ((o == 2 ? N : K) + 63) / 64;
    if (!(flags & ANVIL_GEMM_UNCHECKED))
      return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: K-blocked operands need ANVIL_GEMM_UNCHECKED");
    if (kb < 64 || kb % 16 || (long long)blocks * kb + 256ll * 64 >= (1ll << 31))
      return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: K-block stride %lld of %s out of range", kb,
                       o == 0 ? "A" : (o == 1 ? "Bt" : "C"));
  }
  if ((flags & ANVIL_GEMM_SPLITK) && (!(flags & ANVIL_GEMM_UNCHECKED) ||
                                      (flags & (ANVIL_GEMM_CAUSAL_SKIP | ANVIL_GEMM_CAUSAL_K)) || add ||
                                      (long long)batch0 * batch1 != 1))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: SPLITK needs UNCHECKED, batch 1, no causal mode and no fused add");
  if ((flags & ANVIL_GEMM_MUL24) && (mult >= (1 << 23) || mult < -(1 << 23)))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: MUL24 needs |mult| < 2^23 (got %d)", mult);
  if ((flags & ANVIL_GEMM_CAUSAL_SKIP) && (flags & ANVIL_GEMM_CAUSAL_K))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: the two causal modes exclude each other");
  if (add) {
    if (!add->R || !add->D || !add->rstrides) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add: null pointer");
    if (!(flags & ANVIL_GEMM_UNCHECKED) || (flags & (ANVIL_GEMM_CAUSAL_SKIP | ANVIL_GEMM_CAUSAL_K)))
      return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add: needs ANVIL_GEMM_UNCHECKED and no causal mode");
    if (add->shift2 < 0 || add->shift2 > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", add->shift2);
  }
  return ANVIL_OK;
}

static int gemm_prepare(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1, int M,
                        int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut,
                        int out_dtype, int flags, const AddEpilogue* add, Prepared& p) {
  if (int r = gemm_validate(A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags, add))
    return r;
  if (int r = check_ctx(ctx)) return r;
  GemmArgs g{};
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
  g.kba = 64;
  if (flags & ANVIL_GEMM_A_KBLOCK) g.kba = g.lda, g.lda = 64;
  g.sb0 = strides[3];
  g.sb1 = strides[4];
  g.ldb = strides[5];
  g.kbb = 64;
  if (flags & ANVIL_GEMM_B_KBLOCK) g.kbb = g.ldb, g.ldb = 64;
  g.sc0 = strides[6];
  g.sc1 = strides[7];
  g.ldc = strides[8];
  g.kbc = 64;
  if (flags & ANVIL_GEMM_C_KBLOCK) g.kbc = g.ldc, g.ldc = 64;
  g.mult = mult;
  g.shift = shift;
  g.rnd = shift ? (int)(1u << (shift - 1)) : 0;
  g.lut = lut;
  g.flags = ctx->flags;
  g.causal = (flags & ANVIL_GEMM_CAUSAL_SKIP) ? 1 : ((flags & ANVIL_GEMM_CAUSAL_K) ? 2 : 0);
  const bool checked = !(flags & ANVIL_GEMM_UNCHECKED);
  auto ok16 = [](long long v) { return (v & 15) == 0; };
  const bool vec = (K & 15) == 0 && aligned16(A) && aligned16(Bt) && ok16(g.lda) && ok16(g.ldb) &&
                   (batch0 == 1 || (ok16(g.sa0) && ok16(g.sb0))) && (batch1 == 1 || (ok16(g.sa1) && ok16(g.sb1)));
  const int osz = out_dtype == ANVIL_I8 ? 1 : 2;
  g.vec_store = C && aligned16(C) && ok16(g.ldc * osz) && (batch0 == 1 || ok16(g.sc0 * osz)) &&
                (batch1 == 1 || ok16(g.sc1 * osz));
  if ((long long)((M + 127) / 128) * ((N + 63) / 64) > (1ll << 31) - 1)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: too many tiles");
  const bool force_generic = !add && ctx->gemm_cfg >= 1 && ctx->gemm_cfg <= 6;   // benchmarking override
  const bool fast = !checked && vec && !force_generic && 256ll * g.lda < (1ll << 31) && 256ll * g.ldb < (1ll << 31);
  if (add) {
    if (!fast)
      return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add: operands must be 16-byte aligned with K a multiple of 16");
    const int64_t* rs = add->rstrides;
    g.R = add->R;
    g.D = add->D;
    g.sr0 = rs[0], g.sr1 = rs[1], g.ldr = rs[2], g.sd0 = rs[3], g.sd1 = rs[4], g.ldd = rs[5];
    g.ma = add->ma, g.mb = add->mb, g.shift2 = add->shift2;
    g.rnd2 = add->shift2 ? (int)(1u << (add->shift2 - 1)) : 0;
    g.res = 1;
    g.store_y = C != nullptr;
    g.vec_res = aligned16(g.R) && aligned16(g.D) && ok16(g.ldr * osz) && ok16(g.ldd * osz) &&
                (batch0 == 1 || (ok16(g.sr0 * osz) && ok16(g.sd0 * osz))) &&
                (batch1 == 1 || (ok16(g.sr1 * osz) && ok16(g.sd1 * osz)));
  }
  p.g = g;
  p.osz = osz;
  p.batch = batch0 * batch1;
  p.checked = checked;
  p.vec = vec;
  p.fast = fast;
  p.mul24 = (flags & ANVIL_GEMM_MUL24) != 0;
  p.force_split = (flags & ANVIL_GEMM_SPLITK) != 0;
  if ((flags & (ANVIL_GEMM_A_KBLOCK | ANVIL_GEMM_B_KBLOCK | ANVIL_GEMM_C_KBLOCK)) && !fast)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: K-blocked operands need 16-byte aligned operands with K a multiple "
                                    "of 16 (and no benchmarking override)");
  if (p.force_split && !fast)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8: SPLITK needs 16-byte aligned operands with K a multiple of 16");
  return ANVIL_OK;
}

// The context's split-K workspace, grown to hold `sums` partial sums (written before they are read: no clearing).
// The buffer it outgrows is retired, not freed: a graph captured earlier may still replay launches that use it.
static int ensure_workspace(anvil_ctx* ctx, long long sums) {
  if (ctx->ws_elems >= sums) return ANVIL_OK;
  if (ctx->ws) ctx->ws_retired.push_back(ctx->ws);
  ctx->ws = nullptr;
  ctx->ws_elems = 0;
  ANVIL_HIP(hipMalloc(&ctx->ws, sizeof(int) * sums));
  ctx->ws_elems = sums;
  return ANVIL_OK;
}

// Launch a prepared product. A split-K product keeps its partial tiles in the context's workspace (allocated on
// first use), or with `noalloc` in the static scratch, within whose size it must then fit.
static int gemm_launch(anvil_ctx* ctx, Prepared& p, bool noalloc = false) {
  if (!p.fast) {
    launch_gemm(p.g, p.checked, p.osz, p.vec, p.batch, ctx->stream, ctx->gemm_cfg);
    return ANVIL_OK;
  }
  int splits = 0, kchunk = 0;
  if (!p.force_split && !ctx->gemm_cfg && skinny_ok(p.g, p.batch)) {
    if (p.mul24)
      launch_skinny<true>(&p.g, 1, p.osz, ctx->num_cu, ctx->stream);
    else
      launch_skinny<false>(&p.g, 1, p.osz, ctx->num_cu, ctx->stream);
    return ANVIL_OK;
  }
  if (!p.force_split && !ctx->gemm_cfg && small_plan(p.g, p.batch, ctx->num_cu)) {
    if (p.mul24)
      launch_small<true>(p.g, p.osz, ctx->stream);
    else
      launch_small<false>(p.g, p.osz, ctx->stream);
    return ANVIL_OK;
  }
  if (splitk_plan(p.g, p.batch, ctx->num_cu, p.force_split, splits, kchunk)) {
    const long long tiles = (long long)((p.g.M + 127) / 128) * ((p.g.N + 127) / 128);
    const long long sums = tiles * splits * 128 * 128;   // one int32 partial tile per (tile, chunk)
    if (noalloc) {
      if (sums > SCRATCH_SUMS)
        return set_error(ANVIL_E_VALUE,
                         "anvil_gemm_i8_noalloc: a split-K product of %lld partial sums (%lld tiles of 128 x 128 in "
                         "%d K chunks) exceeds the static scratch (%lld sums)", sums, tiles, splits, SCRATCH_SUMS);
      if (int r = claim_scratch(ctx, &p.g.ws)) return r;
    } else {
      if (int r = ensure_workspace(ctx, sums)) return r;
      p.g.ws = ctx->ws;
    }
    p.g.splits = splits;
    p.g.kchunk = kchunk;
    if (p.mul24)
      launch_splitk<true>(p.g, p.osz, ctx->stream);
    else
      launch_splitk<false>(p.g, p.osz, ctx->stream);
    return ANVIL_OK;
  }
  int choice = fast_choice(p.g, p.batch, ctx->gemm_cfg, ctx->num_cu);
  if (p.g.res && p.osz == 2 && choice >= 39)   // the persistent kernels' register epilogue adds int8 results only
    choice = (long long)p.g.M * p.g.N * p.batch >= 256ll * 128 * 512 && p.g.M >= 256 && p.g.N >= 128 ? 16 : 13;
  if (p.mul24)
    launch_fast_choice<true>(p.g, p.osz, p.batch, ctx->stream, choice, ctx->num_cu);
  else
    launch_fast_choice<false>(p.g, p.osz, p.batch, ctx->stream, choice, ctx->num_cu);
  return ANVIL_OK;
}

static int gemm_entry(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1, int M,
                      int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut, int out_dtype,
                      int flags, const AddEpilogue* add, bool noalloc = false) {
  Prepared p;
  if (int r = gemm_prepare(ctx, A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags, add, p))
    return r;
  if (int r = gemm_launch(ctx, p, noalloc)) return r;
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

// Independent products in one launch when every one of them takes the same one-tile-per-workgroup kernel (256 x 128
// or 128 x 128) with the same result type and requant multiply, else one launch each (in order).
extern "C" int anvil_gemm_i8_group(anvil_ctx* ctx, const anvil_gemm_desc* d, int count) {
  if (!d) return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_group: null pointer");
  if (count < 1 || count > GEMM_GROUP_MAX)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_group: count %d outside [1, %d]", count, GEMM_GROUP_MAX);
  for (int i = 0; i < count; ++i)
    if (int r = gemm_validate(d[i].A, d[i].Bt, d[i].C, d[i].batch0, d[i].batch1, d[i].M, d[i].N, d[i].K, d[i].strides,
                              d[i].mult, d[i].shift, d[i].lut, d[i].out_dtype, d[i].flags, nullptr))
      return r;
  Prepared p[GEMM_GROUP_MAX];
  for (int i = 0; i < count; ++i)
    if (int r = gemm_prepare(ctx, d[i].A, d[i].Bt, d[i].C, d[i].batch0, d[i].batch1, d[i].M, d[i].N, d[i].K,
                             d[i].strides, d[i].mult, d[i].shift, d[i].lut, d[i].out_dtype, d[i].flags, nullptr, p[i]))
      return r;
  // narrow products sharing their left operand (the frozen models' q, k and v; gate and up): one gemm_i8_skinny pass
  bool skinny = count > 1 && !ctx->gemm_cfg;
  for (int i = 0; i < count && skinny; ++i)
    skinny = p[i].fast && !p[i].force_split && skinny_ok(p[i].g, p[i].batch) && p[i].osz == p[0].osz &&
             p[i].mul24 == p[0].mul24 && p[i].g.A == p[0].g.A && p[i].g.lda == p[0].g.lda &&
             p[i].g.kba == p[0].g.kba && p[i].g.M == p[0].g.M && p[i].g.K == p[0].g.K && p[i].g.N == p[0].g.N;
  if (skinny) {
    GemmArgs gs[GEMM_GROUP_MAX];
    for (int i = 0; i < count; ++i) gs[i] = p[i].g;
    if (p[0].mul24)
      launch_skinny<true>(gs, count, p[0].osz, ctx->num_cu, ctx->stream);
    else
      launch_skinny<false>(gs, count, p[0].osz, ctx->num_cu, ctx->stream);
    ANVIL_LAUNCHED();
    return ANVIL_OK;
  }
  // one launch when every member takes the same one-tile-per-workgroup kernel: 256 x 128 tiles, or 128 x 128 tiles
  // for smaller products (config 3's q, k and v, 256 tiles each), none of them splitting K
  int shape = 0;
  bool one = count > 1;
  for (int i = 0; i < count && one; ++i) {
    const int c = fast_choice(p[i].g, p[i].batch, ctx->gemm_cfg, ctx->num_cu);
    int splits = 0, kchunk = 0;
    one = p[i].fast && p[i].osz == p[0].osz && p[i].mul24 == p[0].mul24 && (c == 16 || c == 13) &&
          (i == 0 || c == shape) && !splitk_plan(p[i].g, p[i].batch, ctx->num_cu, p[i].force_split, splits, kchunk);
    shape = c;
  }
  if (one) {
    GemmArgs gs[GEMM_GROUP_MAX];
    int batch[GEMM_GROUP_MAX];
    for (int i = 0; i < count; ++i) gs[i] = p[i].g, batch[i] = p[i].batch;
    if (shape == 16)
      one = p[0].mul24 ? launch_fast_group<256, 128, 2, 3, true>(gs, batch, count, p[0].osz, ctx->stream)
                       : launch_fast_group<256, 128, 2, 3, false>(gs, batch, count, p[0].osz, ctx->stream);
    else
      one = p[0].mul24 ? launch_fast_group<128, 128, 2, 3, true>(gs, batch, count, p[0].osz, ctx->stream)
                       : launch_fast_group<128, 128, 2, 3, false>(gs, batch, count, p[0].osz, ctx->stream);
  }
  if (!one)
    for (int i = 0; i < count; ++i)
      if (int r = gemm_launch(ctx, p[i])) return r;
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

extern "C" int anvil_gemm_i8_ex(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1,
                                int M, int N, int K, const int64_t* strides, int32_t mult, int shift,
                                const int8_t* lut, int out_dtype, int flags) {
  return gemm_entry(ctx, A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags, nullptr);
}

extern "C" int anvil_gemm_i8_noalloc(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0,
                                     int batch1, int M, int N, int K, const int64_t* strides, int32_t mult, int shift,
                                     const int8_t* lut, int out_dtype, int flags) {
  return gemm_entry(ctx, A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags, nullptr, true);
}

extern "C" int anvil_workspace_sums(anvil_ctx* ctx, long long* sums) {
  if (int r = check_ctx(ctx)) return r;
  if (!sums) return set_error(ANVIL_E_VALUE, "anvil_workspace_sums: null pointer");
  *sums = ctx->ws_elems;
  return ANVIL_OK;
}

extern "C" int anvil_gemm_i8_add(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, int8_t* C, int batch0,
                                 int batch1, int M, int N, int K, const int64_t* strides, int32_t mult, int shift,
                                 const int8_t* lut, const int8_t* R, int32_t ma, int32_t mb, int shift2, int8_t* D,
                                 const int64_t* rstrides, int flags) {
  const AddEpilogue add{R, D, rstrides, ma, mb, shift2};
  return gemm_entry(ctx, A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, ANVIL_I8, flags, &add);
}

extern "C" int anvil_gemm_i8_add_ex(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0,
                                    int batch1, int M, int N, int K, const int64_t* strides, int32_t mult, int shift,
                                    const int8_t* lut, int out_dtype, const void* R, int32_t ma, int32_t mb,
                                    int shift2, void* D, const int64_t* rstrides, int flags) {
  const AddEpilogue add{static_cast<const int8_t*>(R), static_cast<int8_t*>(D), rstrides, ma, mb, shift2};
  return gemm_entry(ctx, A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, flags, &add);
}

extern "C" int anvil_gemm_i8_add_norm(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, int8_t* C, int M, int N, int K,
                                      const int64_t* strides, int32_t mult, int shift, const int8_t* lut,
                                      const int8_t* R, int32_t ma, int32_t mb, int shift2, int8_t* D,
                                      const int64_t* rstrides, const anvil_norm_epilogue* norm, int flags) {
  if (!norm || !norm->w || !norm->lut || !norm->out)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: null rmsnorm weights, table or result");
  if (!(flags & ANVIL_GEMM_UNCHECKED) || !(flags & ANVIL_GEMM_NORM_S24) || (flags & (ANVIL_GEMM_SPLITK | ANVIL_GEMM_CAUSAL_SKIP | ANVIL_GEMM_CAUSAL_K)))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: flags must hold ANVIL_GEMM_UNCHECKED and "
                                    "ANVIL_GEMM_NORM_S24, without a causal mode or split-K");
  if ((N != 128 && N != 256) || M % 128 != 0)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: needs N of 128 or 256 (one tile a row band) and M a "
                                    "multiple of 128 (M %d, N %d)", M, N);
  if (!PackedAdd::applies(ma, mb))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: add multipliers must be below 2^24 in magnitude");
  if (norm->lut_len < 1 || norm->shift < 0 || norm->shift > 31)
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: rsqrt table of %d entries, shift %d", norm->lut_len,
                     norm->shift);
  const bool kb = norm->kb != 0;
  if (!aligned16(norm->out) || !aligned16(norm->w) || (kb ? norm->ld != 64 || norm->kb % 16 || (long long)M * 64 > norm->kb
                                                          : norm->ld < N || norm->ld % 16))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: the result H and the weights must be 16-byte aligned, "
                                    "H row-major with a row stride >= N and a multiple of 16, or K-blocked");
  const AddEpilogue add{R, D, rstrides, ma, mb, shift2};
  Prepared p;
  if (int r = gemm_prepare(ctx, A, Bt, C, 1, 1, M, N, K, strides, mult, shift, lut, ANVIL_I8, flags & ~ANVIL_GEMM_NORM_S24,
                           &add, p))
    return r;
  if (!p.fast || p.osz != 1 || !p.g.vec_res || (C && !p.g.vec_store) || 128ll * p.g.ldr >= (1ll << 31))
    return set_error(ANVIL_E_VALUE, "anvil_gemm_i8_add_norm: needs the fast path with 16-byte aligned operands, "
                                    "results and row strides");
  p.g.nw = norm->w;
  p.g.nlut = norm->lut;
  p.g.nlut_len = norm->lut_len;
  p.g.nbits = 32 - __builtin_clz((unsigned)norm->lut_len);
  p.g.nmult = norm->mult;
  p.g.nshift = norm->shift;
  p.g.H = norm->out;
  p.g.ldh = kb ? 64 : norm->ld;
  p.g.kbh = kb ? norm->kb : 0;
  if (N == 128) launch_fast_norm<128, 128>(p.g, p.mul24, ctx->stream);
  else launch_fast_norm<64, 256>(p.g, p.mul24, ctx->stream);     // twice the workgroups of 128 x 256 tiles
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

extern "C" int anvil_gemm_i8(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1,
                             int M, int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut,
                             int out_dtype) {
  return anvil_gemm_i8_ex(ctx, A, Bt, C, batch0, batch1, M, N, K, strides, mult, shift, lut, out_dtype, 0);
}
