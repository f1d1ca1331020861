// Fused attention chain for proven graphs whose scores and probabilities are not returned:
//
//   scores = qmatmul(qh, kT, M_s, s_s)          (anvil/semantics.py:95-103, int8 result)
//   p      = softmax_lut(scores, lut, one)      (anvil/lower/graph_to_tensor.py:352-398, int8 result)
//   o      = qmatmul(p, vh, M_o, s_o)           (int8 result)
//
// computed per (batch, head) without writing scores or p to memory, bit-exact with the three ops. The reference
// lowers softmax_lut in three stages (row max, exp sum, normalise); the same three stages run here over score rows
// held in registers. Nothing is approximated: the LUT softmax is not invariant under rescaling, which rules out an
// online (single-pass) softmax.
//
// Workgroup: 4 waves on 32 query rows q0 .. q0 + 31; wave w takes the 32-key tiles w, w + 4, w + 8, ... up to the
// causal diagonal, so the waves share the row's keys evenly and each holds at most T / 128 tiles of scores.
//   1. S = Q K^T per tile on v_mfma_i32_32x32x32_i8, requantised to int8 and kept packed in registers: lane l holds
//      row q0 + l % 32 and, of each tile, the keys 16 (l / 32) + 4 g + e (g, e = 0..3) in dword g, byte e. A key
//      past the causal diagonal takes the lowest score. Partial row maxima meet in LDS.
//   2. Partial sums of lut[s - max + 255] (lut staged in LDS) meet in LDS; the diagonal tile's masked keys are
//      subtracted once per lane.
//   3. p = (lut[d] one + S // 2) // S, d = s - max + 255, exactly, in float64 (full rate on CDNA4): with per-row
//      A = fl(one / S) and B = fl((S // 2) / S + 2^-40), y = fma(lut[d], A, B) is within 2^-45 of n / S + 2^-40
//      (n = lut[d] one + S // 2 < 2^31, n / S < 128, three roundings of 2^-53 relative), and n / S is either an
//      integer or at least 1 / S > 2^-31 away from one, so floor(y) = n // S (taken as round(y - 1/2) by adding
//      1.5 2^52). The LUT (>= 0) is staged in LDS as doubles, and each row's p values go into a byte table indexed
//      by score. O_w = P V over the wave's tiles on MFMA, P packed in registers: lane l's 16 probabilities of a tile
//      are keys 16 (l / 32) .. + 15 (the key rows entered the score MFMA in bperm order), so its V^T fragment is one
//      contiguous 16-byte load. With a non-decreasing LUT, p = 0 below a per-row score threshold: a tile whose
//      largest kept score is below it in every lane skips its lookups and its product.
//   4. The four partial O tiles (int32) are summed through two LDS slots; o = clamp((O M_o + rnd(s_o)) >> s_o),
//      4-byte stores.
// At D = 64 the kernel fits 80 registers and 21.7 KB of LDS: six workgroups (six waves a SIMD) share a CU.
// Every product is proven to fit int32 (prove_no_overflow), so the requants run in 32 bits; with S24 the score
// requant multiply is one 24-bit multiply-add (|acc|, |M_s| < 2^23).
#include <algorithm>
#include <utility>

#include "common.h"

namespace anvil {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct AttnArgs {
  const int8_t* Q;
  const int8_t* K;
  const int8_t* V;     // V^T rows: (d, T) per (batch, head), keys contiguous
  int8_t* O;
  int batch1, T, D;
  long long sq0, sq1, ldq, sk0, sk1, ldk, sv0, sv1, ldv, so0, so1, ldo;
  int ms, ss, rnds;    // scores requant
  int clo, chi;        // the score requant's clamp in the pre-shift domain: [-128, 127] << ss, saturated to int32
  const int* lut;
  int one, causal;
  int mo, so, rndo;    // output requant
  int mo24;            // |mo| < 2^23: the output requant multiply fits 24 bits
  int clo_o, chi_o;    // the output requant's clamp in the pre-shift domain, as clo / chi
  int ldo32, obytes;   // O's row stride, and the bytes of one 32-row tile (31 ldo + D), both below 2^31
  unsigned long long mone;   // n / one as (n mone) >> (32 + kone)
  int kone;
  int nqt;             // query tiles of 32 rows per head
  unsigned long long mq, mb;   // n / nqt and n / batch1 as (n m) >> (32 + k): m = ceil(2^(32+k) / d), 2^k >= d
  int kq, kb;
  // the kept form (anvil_attention_i8_keep): scores and probabilities also stored, (batch, head, T, T) int8 with
  // strides (sc0, sc1, ldsc) and (pr0, pr1, ldpr); one 32-row tile spans 31 ld + T bytes of each (scbytes, prbytes)
  int8_t* Sc;
  int8_t* Pr;
  long long sc0, sc1, ldsc, pr0, pr1, ldpr;
  int ldsc32, ldpr32, scbytes, prbytes;
  int vrows;           // T = 16 only: V given as its (T, D) rows (strides sv0, sv1, ldv) instead of V^T
};

// n / d for a uniform n < 2^32 by one 64-bit multiply-high (scalar ALU): with m = ceil(2^(32+k) / d) and 2^k >= d,
// m < 2^33 and the error n (m d - 2^(32+k)) / (d 2^(32+k)) stays below 1 / d, so the floor is exact.
__device__ __forceinline__ unsigned udiv_magic(unsigned n, unsigned long long m, int k) {
  return (unsigned)(((unsigned long long)n * m) >> (32 + k));
}

constexpr int A_THREADS = 256;


typedef __attribute__((address_space(3))) const uint8_t lds_u8;

// 4 * (byte e of v), zero-extended: one SDWA shift, the byte offset of entry e of an int table
template <int E>
__device__ __forceinline__ unsigned byte_x4(unsigned v) {
  unsigned r;
  if constexpr (E == 0)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(r) : "v"(v));
  else if constexpr (E == 1)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(r) : "v"(v));
  else if constexpr (E == 2)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(r) : "v"(v));
  else
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(r) : "v"(v));
  return r;
}


// One 16-byte chunk of a K-contiguous operand row; zero past the head dim.
template <int D>
__device__ __forceinline__ v4i chunk16(const int8_t* row, int chunk) {
  if (chunk * 16 >= D) return v4i{0, 0, 0, 0};
  return *reinterpret_cast<const v4i*>(row + chunk * 16);
}

// 16 bytes to a buffer at a 32-bit offset
__device__ __forceinline__ void store16(v4i v, __amdgpu_buffer_rsrc_t rs, unsigned off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), rs, off,
                                         0, 0);
}

// Six workgroups a CU at D <= 64; the kept form's stores need a few more registers, five.
template <int NTW, int D, bool S24, bool KEEP>
__global__ __launch_bounds__(A_THREADS, (D <= 64 ? (KEEP ? 5 : 6) : 1)) void attention_i8(AttnArgs a) {
  constexpr int KS = (D + 31) / 32;         // 32-wide MFMA k-steps over the head dim
  constexpr int CT = (D + 31) / 32;         // 32-wide output column tiles
  constexpr int OROW = CT * 32 + 4;         // partial-O row stride in LDS (ints), padded off the bank period
  // the partial-O space (two slots of 32 rows) also holds the p tables (32 rows of 256 bytes) and the tile maxima
  constexpr int OSLOT = std::max(32 * OROW, (32 * 256 + A_THREADS * NTW) / 8);
  __shared__ __attribute__((aligned(16))) int lut_s[256];
  __shared__ double lutd_s[256];                            // the LUT as doubles, for the p tables
  __shared__ __attribute__((aligned(16))) int red_m[4][32];   // after the max: the rows' (A, B) as doubles
  __shared__ int red_s[4][32];
  __shared__ int dlow_s[32];
  __shared__ __attribute__((aligned(256))) int opart[2][OSLOT];   // 256: the p-table rows

  const int t = threadIdx.x;
  const int lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int l32 = lane & 31, half = lane >> 5;
  const int lutv = a.lut[t];       // staged in LDS after phase 1: the load's latency hides behind the score tiles

  // XCD-aware order: consecutive logical tiles on one XCD (its L2 holds the head's K and V), each head's query tiles
  // together, the longest (last) query tile of a head first
  const int nblk = gridDim.x;
  int pid = blockIdx.x;
  if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
  const int bh = (int)udiv_magic((unsigned)pid, a.mq, a.kq);
  const int qt = a.nqt - 1 - (pid - bh * a.nqt);
  const int q0 = qt * 32;
  const int b0 = (int)udiv_magic((unsigned)bh, a.mb, a.kb), b1 = bh - b0 * a.batch1;
  const int qrow = q0 + l32;
  const int ntiles = a.causal ? qt + 1 : a.nqt;

  const int8_t* Qr = a.Q + b0 * a.sq0 + b1 * a.sq1 + (long long)qrow * a.ldq;
  // key rows enter the score MFMA in bperm order: score accumulator r of lane l is then key 16 (l / 32) + r of the
  // tile, so a lane's 16 probabilities are 16 consecutive keys and its V^T fragment is one contiguous 16-byte load
  const int8_t* Vb = a.V + b0 * a.sv0 + b1 * a.sv1;

  v4i qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = chunk16<D>(Qr, 2 * ks + half);

  // The kept form stores each score and probability tile as the lanes hold it: lane l's 16 bytes of a 32-key tile
  // are keys 16 (l / 32) .. + 15 of row q0 + l % 32 (the key rows entered the score MFMA in bperm order), one
  // 16-byte store at column 32 nt + 16 (l / 32).
  const __amdgpu_buffer_rsrc_t srs =            // (unused, and dropped, in the plain form)
      uniform_rsrc(KEEP ? a.Sc + b0 * a.sc0 + b1 * a.sc1 + (long long)q0 * a.ldsc : nullptr, KEEP ? a.scbytes : 0);
  const __amdgpu_buffer_rsrc_t prs =
      uniform_rsrc(KEEP ? a.Pr + b0 * a.pr0 + b1 * a.pr1 + (long long)q0 * a.ldpr : nullptr, KEEP ? a.prbytes : 0);
  const unsigned sofs = KEEP ? (unsigned)(l32 * a.ldsc32 + 16 * half) : 0u;
  const unsigned pofs = KEEP ? (unsigned)(l32 * a.ldpr32 + 16 * half) : 0u;

  // ---- 1. scores of this wave's tiles (w + 4 i), partial row max
  // The requant clamps before its shift (clamp(x >> s) = clamp'(x) >> s with the bounds scaled by 2^s), so the
  // max runs on the clamped values and each score byte is one shift written into its byte lane.
  unsigned sc[NTW][4];
  // tile i's largest kept score of the lane (an int8 score) at tmx_s[NTW t + i], past the p tables in the partial-O
  // space (untouched until the partial O tiles)
  int8_t* tmx_s = reinterpret_cast<int8_t*>(&opart[0][0]) + 32 * 256 + NTW * t;
  int mxc = a.clo;
  // K and V^T tiles come through raw buffer loads; a tile past the causal diagonal (or a chunk past the head dim)
  // gets an offset beyond the descriptor, which loads zeros without touching memory, so every pass can issue its
  // loads whatever the wave's tile count
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(a.K + b0 * a.sk0 + b1 * a.sk1, (int)((long long)a.T * a.ldk));
  const unsigned koff = (unsigned)(bperm(l32) * a.ldk) + 16 * half;
  // Past the wave's last tile the tile part of the offset is 2^31: every lane's offset (below T ldk < 2^31 for a
  // real tile) then lands in [2^31, 2^32), beyond the descriptor, so the tile test stays on the scalar unit.
  auto kload_below = [&](int nt, int lim, v4i* kf) {     // tile nt if nt < lim, else zeros
    const unsigned tile = nt < lim ? (unsigned)(nt * 32 * a.ldk) : 0x80000000u;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const unsigned o = D >= 32 ? koff + 32 * ks + tile                    // every lane's chunk inside the head dim
                                 : (nt < lim && 32 * ks + 16 * half < D ? koff + 32 * ks + tile : OOB);
      kf[ks] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(krs, o, 0, 0));
    }
  };
  auto kload = [&](int nt, v4i* kf) { kload_below(nt, ntiles, kf); };
  // The kept form's tiles past the causal diagonal: their scores are stored like any other (the graph's scores are
  // the whole T x T product) and their probabilities are 0. The wave takes tiles ntiles + w, + 4, ... (at most NTW)
  // before its own, each pass loading the next K tile once its MFMAs have read the current one and storing after
  // that load. Passes nest as for the wave's own tiles (below): every pass has one path into it, so its wait covers
  // its own K tile and leaves the previous pass's two stores in flight.
  if constexpr (KEEP) {
    if (a.causal && ntiles + w < a.nqt) {
      v4i uf[KS];
      kload_below(ntiles + w, a.nqt, uf);
      auto upass = [&](auto self, auto ic) __attribute__((always_inline)) -> void {
        constexpr int i = decltype(ic)::value;
        const int nt = ntiles + w + 4 * i;
        v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(uf[ks], qf[ks], acc, 0, 0, 0);
        if (i + 1 < NTW) kload_below(nt + 4, a.nqt, uf);
        int x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
          x[r] = med3i(S24 ? __mul24(acc[r], a.ms) + a.rnds : acc[r] * a.ms + a.rnds, a.clo, a.chi);
        v4i sv;
#pragma unroll
        for (int g = 0; g < 4; ++g) sv[g] = (int)sra_pack4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3], a.ss);
        store16(sv, srs, sofs + 32 * nt);
        store16(v4i{0, 0, 0, 0}, prs, pofs + 32 * nt);
        if constexpr (i + 1 < NTW) {
          if (nt + 4 < a.nqt) self(self, std::integral_constant<int, i + 1>{});
        }
      };
      upass(upass, std::integral_constant<int, 0>{});
    }
  }
  // The next K tile loads into kf as soon as this pass's score MFMAs have read it, so its latency overlaps the
  // requant of this tile; one buffer (not two, loaded two tiles ahead) keeps the kernel at 80 registers, six waves a
  // SIMD. The wave's tiles are a prefix of its passes, and pass i + 1 is entered from the end of pass i only
  // (nested, not sequential, branches), each pass issuing its load unconditionally: each wait then covers exactly
  // the load one tile back, where a join of a path that loaded with one that did not would make it cover every load
  // issued so far.
  v4i kf[KS];
  kload(w, kf);
  auto pass1 = [&](auto self, auto ic) __attribute__((always_inline)) -> void {
    constexpr int i = decltype(ic)::value;
    const int nt = w + 4 * i;
    v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[ks], qf[ks], acc, 0, 0, 0);
    if (i + 1 < NTW) kload(nt + 4, kf);
    int x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int y = S24 ? __mul24(acc[r], a.ms) + a.rnds : acc[r] * a.ms + a.rnds;
      x[r] = med3i(y, a.clo, a.chi);
    }
    // the diagonal tile: a key past the row takes the lowest score (clo >> ss), which leaves the row max as it is;
    // the sums subtract its LUT term and the probabilities mask it
    if (a.causal && nt == ntiles - 1) {
      if constexpr (KEEP) {                           // the kept scores are the unmasked ones
        v4i sv;
#pragma unroll
        for (int g = 0; g < 4; ++g) sv[g] = (int)sra_pack4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3], a.ss);
        store16(sv, srs, sofs + 32 * nt);
      }
      const int lim = qrow - nt * 32 - 16 * half;     // key r of this lane is kept iff r <= lim
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = r <= lim ? x[r] : a.clo;
    }
    int tm = a.clo;                                   // the largest kept score of the lane's 16
#pragma unroll
    for (int r = 0; r < 16; ++r) tm = max(tm, x[r]);
    mxc = max(mxc, tm);
    tmx_s[i] = (int8_t)(tm >> a.ss);
#pragma unroll
    for (int g = 0; g < 4; ++g) sc[i][g] = sra_pack4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3], a.ss);
    if constexpr (KEEP) {
      if (!(a.causal && nt == ntiles - 1))
        store16(v4i{(int)sc[i][0], (int)sc[i][1], (int)sc[i][2], (int)sc[i][3]}, srs, sofs + 32 * nt);
    }

    if constexpr (i + 1 < NTW) {
      if (nt + 4 < ntiles) self(self, std::integral_constant<int, i + 1>{});
    }
  };
  if (w < ntiles) pass1(pass1, std::integral_constant<int, 0>{});
  int mx = max(mxc >> a.ss, -128);

  // the first V^T tile loads while the row maxima are reduced and the sums run
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(Vb, (int)((long long)D * a.ldv));
  auto vload = [&](int nt, v4i* vf) {                    // as for K: offsets below D ldv < 2^31, tile part 2^31 past
    const unsigned tile = nt < ntiles ? (unsigned)(nt * 32) : 0x80000000u;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const unsigned row = (unsigned)((32 * ct + l32) * a.ldv + 16 * half);
      const unsigned o = D >= 32 ? row + tile : (nt < ntiles && 32 * ct + l32 < D ? row + tile : OOB);
      vf[ct] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(vrs, o, 0, 0));
    }
  };
  v4i vf[CT];
  vload(w, vf);
  mx = max(mx, __shfl_xor(mx, 32, 64));
  if (half == 0) red_m[w][l32] = mx;
  lut_s[t] = lutv;
  lutd_s[t] = (double)lutv;
  // the p tables (8 KiB of the partial-O space, filled after the next barrier) start zeroed, 32 bytes a thread
  int8_t* ptab = reinterpret_cast<int8_t*>(&opart[0][0]);
  *reinterpret_cast<v4i*>(ptab + 32 * t) = v4i{0, 0, 0, 0};
  *reinterpret_cast<v4i*>(ptab + 32 * t + 16) = v4i{0, 0, 0, 0};
  __syncthreads();                                        // also publishes lut_s and the zeroed tables
  mx = max(max(red_m[0][l32], red_m[1][l32]), max(red_m[2][l32], red_m[3][l32]));

  // ---- 2. partial exp sums over the kept keys
  // Each score byte s becomes its LUT index d = s - max + 255, in [0, 255] for every score of the row (-128 <= s <=
  // max): in unsigned form s + 128 plus 127 - max, which no byte carries out of, so one xor-add rewrites four
  // bytes. A lookup is then one SDWA shift to the entry's byte offset, the table base folding into the LDS offset.
  const unsigned dadd = 0x01010101u * (unsigned)(127 - mx);
  const uint8_t* lutb = reinterpret_cast<const uint8_t*>(lut_s);
  int S = 0;
  static_for<NTW>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if (w + 4 * i < ntiles) {
#pragma unroll
      for (int g = 0; g < 4; ++g) sc[i][g] = (sc[i][g] ^ 0x80808080u) + dadd;
      static_for<16>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        S += *reinterpret_cast<const int*>(lutb + byte_x4<r & 3>(sc[i][r >> 2]));
      });
    }
  });
  if (a.causal && ((ntiles - 1 - w) & 3) == 0 && w < ntiles) {   // this wave holds the diagonal tile: its masked
    const int lim = l32 - 16 * half;                              // keys (those past r = lim) added lut terms of
    S -= (15 - max(-1, min(lim, 15))) * lut_s[(a.clo >> a.ss) + 255 - mx];   // the lowest score
  }
  S += __shfl_xor(S, 32, 64);
  if (half == 0) red_s[w][l32] = S;
  __syncthreads();

  // ---- 3. probabilities, O_w = P V over this wave's tiles
  // p depends on the row and the score only, so each row gets a byte table of (lut[d] one + S // 2) // S over the
  // scores s, d = s - max + 255, built in the partial-O space (free until this phase ends). With a non-decreasing table the
  // quotient is 0 below the first d where lut[d] one + S // 2 >= S, and only the entries from there up are divided;
  // otherwise every entry is.
  // The per-row constants (two float64 divisions, an integer division, a binary search) are the same for the four
  // waves of a row, so wave 0 alone forms them (lanes l and l + 32 both hold row l % 32) and passes them on in LDS:
  // the other waves' instructions go to the other workgroups on the CU.
  double* qab = reinterpret_cast<double*>(&red_m[0][0]);  // [0, 32): A, [32, 64): B; red_m is read before the last barrier
  if (w == 0) {
    S = red_s[0][l32] + red_s[1][l32] + red_s[2][l32] + red_s[3][l32];
    const v4i l4 = *reinterpret_cast<const v4i*>(lut_s + 4 * lane);      // lane l checks entries 4 l .. 4 l + 4
    const int nx = lane < 63 ? lut_s[4 * lane + 4] : INT_MAX;
    const bool mono = __all(l4[0] <= l4[1] && l4[1] <= l4[2] && l4[2] <= l4[3] && l4[3] <= nx);
    const double Sd = (double)S;                         // S >= lut[255] >= 1: the row maximum maps to d = 255
    const double qa0 = (double)a.one / Sd;
    const double qb0 = (double)(S >> 1) / Sd + 0x1p-40 - 0.5;   // the - 0.5 is exact (Sterbenz, or S = 1)
    int d0 = 0;
    if (mono) {
      // lut[d] one + S // 2 >= S  <=>  lut[d] >= e0 = ceil((S - S // 2) / one); d0 = #{d : lut[d] < e0}, by binary
      // search over the non-decreasing table (256 when even lut[255] is below e0)
      const int e0 = (int)udiv_magic((unsigned)(S - (S >> 1) + a.one - 1), a.mone, a.kone);
      int pos = 0;
#pragma unroll
      for (int step = 128; step >= 1; step >>= 1) pos += lut_s[pos + step - 1] < e0 ? step : 0;
      d0 = lut_s[255] < e0 ? 256 : pos;
    }
    if (half == 0) {
      qab[l32] = qa0;
      qab[32 + l32] = qb0;
      dlow_s[l32] = max(d0, 127 - mx);                    // d below 127 - max needs s < -128
    }
  }
  __syncthreads();
  const double qa = qab[l32], qb = qab[32 + l32];
  // The tables sit in the partial-O space, 256 bytes a row, indexed by d (the score bytes hold d since phase 2): the
  // entry of d in row r is at column d ^ 4 r, so a lookup address is the row base with its low byte replaced by the
  // swizzled byte (one v_perm), and the 32 rows' entries for one d fall in 32 different banks. The XOR keeps each
  // dword whole, so the table is written a dword at a time: dword c holds d = 4 c .. 4 c + 3.
  // An entry is y = fma(lut[d], A, B - 1/2), within 2^-45 of n / S - 1/2 + 2^-40 and never a half-integer, so
  // adding 1.5 2^52 rounds it to n // S, which is then the low dword of the sum: two full-rate float64 operations.
  // A row writes the dwords from the top one (d = 255, its max) down to the one holding d = dlow; a byte of the
  // bottom dword below dlow gets its exact quotient too (0 below d0) or belongs to a score below -128, read by no key.
  constexpr int PT = 256;
  const int cx = 4 * l32;
  int sthr;                                              // the row's scores below it have p = 0
  {
    const int part = 2 * w + half;                       // this lane's eighth of its row's dwords
    int8_t* trow = ptab + l32 * PT;
    const int dlow = dlow_s[l32];
    sthr = dlow + mx - 255;
    for (int c = 63 - part; c >= dlow >> 2; c -= 8) {
      const double* lp = lutd_s + 4 * c;
      int v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __double2loint(__builtin_fma(lp[e], qa, qb) + 0x1.8p52);
      *reinterpret_cast<unsigned*>(trow + ((4 * c) ^ cx)) = pack4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
  }
  const unsigned rbase = (unsigned)(uintptr_t)(__attribute__((address_space(3))) int8_t*)(ptab + l32 * PT);
  const unsigned swz = 0x01010101u * (unsigned)cx;
  v16i oacc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) oacc[ct] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  // A tile whose largest kept score is below its row's threshold in every lane holds p = 0 only (with a
  // non-decreasing LUT; 45 % of the causal tiles of the GPT-2 block's scores): its lookups and its product are
  // skipped. Its V^T load is still issued (made conditional too, it costs the kernel spilled registers).
  unsigned live = 0;
  static_for<NTW>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    live |= (__any(tmx_s[i] >= sthr) ? 1u : 0u) << i;
  });
  auto pass3 = [&](auto self, auto ic) __attribute__((always_inline)) -> void {   // nested passes, as for K
    constexpr int i = decltype(ic)::value;
    const int nt = w + 4 * i;
    v4i pf = {0, 0, 0, 0};                               // a dead tile's probabilities (kept form)
    if ((live >> i) & 1) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const unsigned sw = sc[i][g] ^ swz;
      int p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        p[e] = *reinterpret_cast<lds_u8*>(__builtin_amdgcn_perm(rbase, sw, 0x07060500u | e));
      pf[g] = (int)pack4(p[0], p[1], p[2], p[3]);
      if (g == 1) __builtin_amdgcn_sched_barrier(0);  // two halves of eight lookups: 8 registers fewer at the peak
    }
    if (a.causal && nt == ntiles - 1) {
      asm volatile("");                                  // keeps the masking on the diagonal tile's own path
      const int lim = qrow - nt * 32 - 16 * half;        // bytes r <= lim kept: n of dword g's four
#pragma unroll
      for (int g = 0; g < 4; ++g) pf[g] &= (int)(0xFFFFFFFFull >> (32 - 8 * min(max(lim + 1 - 4 * g, 0), 4)));
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) oacc[ct] = __builtin_amdgcn_mfma_i32_32x32x32_i8(vf[ct], pf, oacc[ct], 0, 0, 0);
    }
    // the next tile's V^T loads into vf once this pass's product has read it, so its latency overlaps the next
    // pass's lookups. Issued at the start of this pass instead (into a second buffer), the kernel ran 10 % slower
    // (115 against 104 us at config 5, with or without a register copy between the buffers).
    if (i + 1 < NTW) vload(nt + 4, vf);
    if constexpr (KEEP) store16(pf, prs, pofs + 32 * nt);   // after the prefetch: its wait need not cover the store
    if constexpr (i + 1 < NTW) {
      if (nt + 4 < ntiles) self(self, std::integral_constant<int, i + 1>{});
    }
  };
  if (w < ntiles) pass3(pass3, std::integral_constant<int, 0>{});

  // ---- 4. sum the four partial O tiles, requant, store. Lane l holds O_w[row l % 32][32 ct + 8 g + 4 (l / 32) + e].
  // Two LDS slots (half the partial-O space of one slot a wave, which lets six workgroups share a CU): waves 2 and 3
  // store theirs, waves 0 and 1 add them in and store the pair sums, and every thread adds the two slots. A lane
  // reads and then rewrites only its own chunks of a slot.
  __syncthreads();                                       // every wave is done with the p tables
  int* op = opart[w & 1] + l32 * OROW;
  auto put = [&]() {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<v4i*>(op + 32 * ct + 8 * g + 4 * half) =
            v4i{oacc[ct][4 * g], oacc[ct][4 * g + 1], oacc[ct][4 * g + 2], oacc[ct][4 * g + 3]};
  };
  if (w >= 2) put();
  __syncthreads();
  if (w < 2) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v4i x = *reinterpret_cast<const v4i*>(op + 32 * ct + 8 * g + 4 * half);
#pragma unroll
        for (int e = 0; e < 4; ++e) oacc[ct][4 * g + e] += x[e];
      }
    put();
  }
  __syncthreads();
  // |O| <= 128 (one + T / 2) < 2^17 (p >= 0 sums to at most one + T / 2 over a row), so with |m_o| < 2^23 the
  // output requant multiply is one 24-bit multiply-add. The clamp runs before the shift, as for the scores, so each
  // output byte is one shift written into its byte lane; the tile's 32 rows are stored through a buffer descriptor
  // with 32-bit offsets.
  constexpr int C4 = D / 4;                              // 4-column groups per row
  const __amdgpu_buffer_rsrc_t ors = uniform_rsrc(a.O + b0 * a.so0 + b1 * a.so1 + (long long)q0 * a.ldo, a.obytes);
  auto store = [&](auto m24) {
    for (int idx = t; idx < 32 * C4; idx += A_THREADS) {
      const int row = idx / C4, c = 4 * (idx % C4);
      v4i sum = *reinterpret_cast<const v4i*>(opart[0] + row * OROW + c);
      sum += *reinterpret_cast<const v4i*>(opart[1] + row * OROW + c);
      int x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        x[e] = med3i(decltype(m24)::value ? __mul24(sum[e], a.mo) + a.rndo : sum[e] * a.mo + a.rndo, a.clo_o, a.chi_o);
      __builtin_amdgcn_raw_buffer_store_b32(sra_pack4(x[0], x[1], x[2], x[3], a.so), ors, (unsigned)(row * a.ldo32 + c),
                                            0, 0);
    }
  };
  if (a.mo24)
    store(std::true_type{});
  else
    store(std::false_type{});
}

template <int NTW, bool S24, bool KEEP>
static void launch_attention(const AttnArgs& a, int D, unsigned grid, hipStream_t s) {
  switch (D) {
    case 16: ANVIL_LAUNCH((attention_i8<NTW, 16, S24, KEEP>), dim3(grid), dim3(A_THREADS), 0, s, a); break;
    case 32: ANVIL_LAUNCH((attention_i8<NTW, 32, S24, KEEP>), dim3(grid), dim3(A_THREADS), 0, s, a); break;
    case 64: ANVIL_LAUNCH((attention_i8<NTW, 64, S24, KEEP>), dim3(grid), dim3(A_THREADS), 0, s, a); break;
    default: ANVIL_LAUNCH((attention_i8<NTW, 128, S24, KEEP>), dim3(grid), dim3(A_THREADS), 0, s, a); break;
  }
}

template <bool S24, bool KEEP>
static void launch_attention_nt(const AttnArgs& a, int D, unsigned grid, hipStream_t s) {
  const int ntw = (a.nqt + 3) / 4;                       // key tiles per wave
  if (ntw <= 1)
    launch_attention<1, S24, KEEP>(a, D, grid, s);
  else if (ntw <= 2)
    launch_attention<2, S24, KEEP>(a, D, grid, s);
  else if (ntw <= 4)
    launch_attention<4, S24, KEEP>(a, D, grid, s);
  else
    launch_attention<8, S24, KEEP>(a, D, grid, s);
}


// ------------------------------------------------------------------------------------------------ T = 16
// The same chain for sequences of 16 tokens (the reference's frozen models: T 16, heads of 16), where a 32 x 32 tile
// is mostly empty: one lane a query row, so a wave holds four (batch, head) pairs whole and nothing crosses waves.
// Lane 16 h + i of a wave takes row i of its head h. Its q row (DC 16-byte chunks) loads into registers; its k row
// and its V^T rows (V^T row d = the 16 keys' values of dim d: rows i and 16 + i at D = 32) go to LDS, from where every
// lane of the head reads all 16 (same address across the 16 lanes: a broadcast). Then per row, in registers:
//   s_j = clamp((q . k_j) M_s + rnd) >> s_s for the 16 keys (v_dot4 on 4-byte pieces);
//   m = max(-128, max of the kept s_j) (key j kept iff j <= i when causal); e_j = lut[s_j - m + 255] (kept, else 0);
//   S = sum e_j; p_j = (e_j one + S // 2) // S exactly, as y = fma(e_j, A, B) with A = fl(one / S) and
//   B = fl((S // 2) / S + 2^-40) - 1/2, rounded by adding 1.5 2^52 (the quotient bound and error argument of the
//   long kernel's p tables, which hold for every n < 2^31 and quotient < 128);
//   o_d = clamp((p . V^T_d) M_o + rnd) >> s_o, p packed as 16 bytes (p >= 0, so the signed v_dot4 is exact).
// The kept form also stores the row's 16 scores and 16 probabilities (16-byte stores).
template <int DC, bool S24, bool KEEP>
__global__ __launch_bounds__(A_THREADS) void attention_t16(AttnArgs a, int nheads) {
  constexpr int W = A_THREADS / 64;
  __shared__ int lut_s[256];
  __shared__ __attribute__((aligned(16))) v4i kst[W][64][DC];   // lane l's k row, chunk c
  // V^T of the wave's four heads: row d of head h (the 16 keys' values of dim d) at vst[w][h][d]
  __shared__ __attribute__((aligned(16))) int8_t vst[W][4][16 * DC][16];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int hl = lane >> 4, i = lane & 15;
  const long long hh = ((long long)blockIdx.x * W + w) * 4 + hl;          // (batch, head) of this lane
  const bool live = hh < nheads;
  const int b0 = live ? (int)(hh / a.batch1) : 0, b1 = live ? (int)(hh % a.batch1) : 0;
  lut_s[t] = a.lut[t];
  v4i qv[DC];
  const int8_t* Qr = a.Q + b0 * a.sq0 + b1 * a.sq1 + (long long)i * a.ldq;
  const int8_t* Kr = a.K + b0 * a.sk0 + b1 * a.sk1 + (long long)i * a.ldk;
  const int8_t* Vr = a.V + b0 * a.sv0 + b1 * a.sv1 + (long long)i * a.ldv;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    qv[c] = live ? *reinterpret_cast<const v4i*>(Qr + 16 * c) : v4i{0, 0, 0, 0};
    kst[w][lane][c] = live ? *reinterpret_cast<const v4i*>(Kr + 16 * c) : v4i{0, 0, 0, 0};
  }
  if (a.vrows) {                                   // lane i holds V row i (key i): its D bytes go to column i
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const v4i vr = live ? *reinterpret_cast<const v4i*>(Vr + 16 * c) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int b = 0; b < 16; ++b) vst[w][hl][16 * c + b][i] = (int8_t)(vr[b >> 2] >> (8 * (b & 3)));
    }
  } else {                                         // lane i holds V^T rows i and 16 + i
#pragma unroll
    for (int c = 0; c < DC; ++c)
      *reinterpret_cast<v4i*>(vst[w][hl][i + 16 * c]) =
          live ? *reinterpret_cast<const v4i*>(Vr + 16 * c * a.ldv) : v4i{0, 0, 0, 0};
  }
  __syncthreads();
  // scores of the row, clamped in the pre-shift domain, and the row max over the kept keys
  int sc[16];
  int mx = -128;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    int acc = 0;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const v4i kj = kst[w][16 * hl + j][c];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_sdot4(qv[c][q], kj[q], acc, false);
    }
    const int y = S24 ? __mul24(acc, a.ms) + a.rnds : acc * a.ms + a.rnds;
    sc[j] = med3i(y, a.clo, a.chi) >> a.ss;
    if (!a.causal || j <= i) mx = max(mx, sc[j]);
  }
  int e[16];
  int S = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {                   // a kept score lies in [-128, mx], so its index in [0, 255]
    const bool kept = !a.causal || j <= i;
    e[j] = lut_s[kept ? sc[j] - mx + 255 : 0];
    e[j] = kept ? e[j] : 0;
    S += e[j];
  }
  S = max(S, 1);                                   // S >= lut[255] >= 1 for a live row (the entry's precondition)
  const double Sd = (double)S;
  const double qa = (double)a.one / Sd;
  const double qb = (double)(S >> 1) / Sd + 0x1p-40 - 0.5;
  int p[16];                                       // a masked key's e_j = 0 gives (S // 2) // S = 0, as it must
#pragma unroll
  for (int j = 0; j < 16; ++j) p[j] = __double2loint(__builtin_fma((double)e[j], qa, qb) + 0x1.8p52);
  v4i pp;
#pragma unroll
  for (int g = 0; g < 4; ++g) pp[g] = (int)pack4(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]);
  // O row: 16 DC dims, each the dot of p with V^T row d
  int ov[16 * DC];
#pragma unroll
  for (int d = 0; d < 16 * DC; ++d) {
    const v4i vd = *reinterpret_cast<const v4i*>(vst[w][hl][d]);
    int acc = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_sdot4(pp[q], vd[q], acc, false);
    const int y = a.mo24 ? __mul24(acc, a.mo) + a.rndo : acc * a.mo + a.rndo;
    ov[d] = med3i(y, a.clo_o, a.chi_o);
  }
  if (!live) return;
  int8_t* Or = a.O + b0 * a.so0 + b1 * a.so1 + (long long)i * a.ldo;
#pragma unroll
  for (int d = 0; d < 16 * DC; d += 4)
    *reinterpret_cast<unsigned*>(Or + d) = sra_pack4(ov[d], ov[d + 1], ov[d + 2], ov[d + 3], a.so);
  if constexpr (KEEP) {
    v4i sv;
#pragma unroll
    for (int g = 0; g < 4; ++g) sv[g] = (int)pack4(sc[4 * g], sc[4 * g + 1], sc[4 * g + 2], sc[4 * g + 3]);
    *reinterpret_cast<v4i*>(a.Sc + b0 * a.sc0 + b1 * a.sc1 + (long long)i * a.ldsc) = sv;
    *reinterpret_cast<v4i*>(a.Pr + b0 * a.pr0 + b1 * a.pr1 + (long long)i * a.ldpr) = pp;
  }
}

template <bool S24, bool KEEP>
static void launch_attention_t16(const AttnArgs& a, int D, long long nheads, hipStream_t s) {
  const unsigned grid = (unsigned)((nheads + 4 * (A_THREADS / 64) - 1) / (4 * (A_THREADS / 64)));
  if (D == 16)
    ANVIL_LAUNCH((attention_t16<1, S24, KEEP>), dim3(grid), dim3(A_THREADS), 0, s, a, (int)nheads);
  else
    ANVIL_LAUNCH((attention_t16<2, S24, KEEP>), dim3(grid), dim3(A_THREADS), 0, s, a, (int)nheads);
}

}  // namespace anvil

using namespace anvil;

static bool al(const void* p, int n) { return ((uintptr_t)p % n) == 0; }

// Both entry points: keep = false leaves S, P and strides[12..17] unread.
static int attention_entry(anvil_ctx* ctx, const int8_t* Q, const int8_t* K, const int8_t* Vt, int8_t* O, int8_t* S,
                           int8_t* P, bool keep, int batch0, int batch1, int T, int D, const int64_t* strides,
                           int32_t m_s, int s_s, const int32_t* lut, int32_t one, int causal, int32_t m_o, int s_o,
                           int flags) {
  if (!Q || !K || !Vt || !O || !strides || !lut || (keep && (!S || !P)))
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: null pointer");
  if (!(flags & ANVIL_OP_UNCHECKED) || (flags & ~(ANVIL_OP_UNCHECKED | ANVIL_ATTN_S24 | ANVIL_ATTN_V_ROWS)))
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: flags must hold ANVIL_OP_UNCHECKED (a proven graph)");
  const bool vrows = flags & ANVIL_ATTN_V_ROWS;
  if (vrows && T != 16) return set_error(ANVIL_E_VALUE, "anvil_attention_i8: ANVIL_ATTN_V_ROWS needs T = 16");
  if (batch0 < 1 || batch1 < 1 || (T != 16 && (T < 32 || T % 32 || T > 1024)))
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: T=%d must be 16 or a multiple of 32 in [32, 1024]", T);
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: head dim %d not in {16, 32, 64, 128}", D);
  if (T == 16 && D > 32)
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: T=16 takes head dims 16 and 32, not %d", D);
  if (s_s < 0 || s_s > 31 || s_o < 0 || s_o > 31) return set_error(ANVIL_E_VALUE, "shift outside [0, 31]");
  if (one < 1 || one > 127) return set_error(ANVIL_E_VALUE, "one=%d does not fit int8", one);
  if ((flags & ANVIL_ATTN_S24) && (m_s >= (1 << 23) || m_s <= -(1 << 23)))
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: ANVIL_ATTN_S24 with |m_s| >= 2^23");
  const int64_t* st = strides;
  for (int i = 0; i < 12; ++i)                     // Q, K, V^T: 16-byte loads; O: 4-byte stores
    if (st[i] < 0 || st[i] % (i < 9 ? 16 : 4))
      return set_error(ANVIL_E_VALUE, "anvil_attention_i8: stride %d (%lld) not a multiple of %d", i,
                       (long long)st[i], i < 9 ? 16 : 4);
  if (!al(Q, 16) || !al(K, 16) || !al(Vt, 16) || !al(O, 4))
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: operand not aligned");
  if ((long long)batch0 * batch1 * std::max(1, T / 32) > (1ll << 31) - 1)
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: too many heads");
  // K and V^T are read through 32-bit buffer offsets over one head: T key rows of stride ldk (each at least D
  // bytes apart), D rows of V^T of stride ldv (each at least T keys)
  if (st[5] < D || st[8] < (vrows ? D : T) || (long long)T * st[5] >= (1ll << 31) ||
      (long long)(vrows ? T : D) * st[8] >= (1ll << 31))
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: K row stride %lld / V^T row stride %lld out of range",
                     (long long)st[5], (long long)st[8]);
  if (st[11] < D || 32 * st[11] >= (1ll << 31))   // a 32-row output tile is stored through 32-bit offsets
    return set_error(ANVIL_E_VALUE, "anvil_attention_i8: O row stride %lld out of range", (long long)st[11]);
  if (keep) {                                      // S and P: 16-byte stores into 32-row tiles, 32-bit offsets
    for (int i = 12; i < 18; ++i)
      if (st[i] < 0 || st[i] % 16)
        return set_error(ANVIL_E_VALUE, "anvil_attention_i8_keep: stride %d (%lld) not a multiple of 16", i,
                         (long long)st[i]);
    if (st[14] < T || st[17] < T || 32 * st[14] >= (1ll << 31) || 32 * st[17] >= (1ll << 31))
      return set_error(ANVIL_E_VALUE, "anvil_attention_i8_keep: S / P row stride %lld / %lld out of range",
                       (long long)st[14], (long long)st[17]);
    if (!al(S, 16) || !al(P, 16)) return set_error(ANVIL_E_VALUE, "anvil_attention_i8_keep: S or P not aligned");
  }
  if (int r = check_ctx(ctx)) return r;
  AttnArgs a;
  a.Q = Q;
  a.K = K;
  a.V = Vt;
  a.O = O;
  a.batch1 = batch1;
  a.T = T;
  a.D = D;
  a.sq0 = st[0], a.sq1 = st[1], a.ldq = st[2];
  a.sk0 = st[3], a.sk1 = st[4], a.ldk = st[5];
  a.sv0 = st[6], a.sv1 = st[7], a.ldv = st[8];
  a.so0 = st[9], a.so1 = st[10], a.ldo = st[11];
  a.ms = m_s, a.ss = s_s, a.rnds = s_s ? 1 << (s_s - 1) : 0;
  a.clo = (int)std::max(-128ll * (1ll << s_s), I32_MIN);
  a.chi = (int)std::min(128ll * (1ll << s_s) - 1, I32_MAX);
  a.lut = lut;
  a.one = one, a.causal = causal ? 1 : 0;
  a.mo = m_o, a.so = s_o, a.rndo = s_o ? 1 << (s_o - 1) : 0;
  a.mo24 = m_o > -(1 << 23) && m_o < (1 << 23);
  a.clo_o = (int)std::max(-128ll * (1ll << s_o), I32_MIN);
  a.chi_o = (int)std::min(128ll * (1ll << s_o) - 1, I32_MAX);
  a.ldo32 = (int)st[11];
  a.obytes = (int)(31 * st[11] + D);
  a.nqt = T / 32;
  auto magic = [](int d, unsigned long long& m, int& k) {
    k = 0;
    while ((1 << k) < d) ++k;
    m = ((1ull << (32 + k)) + d - 1) / d;
  };
  magic(std::max(1, a.nqt), a.mq, a.kq);
  magic(batch1, a.mb, a.kb);
  magic(one, a.mone, a.kone);
  a.vrows = vrows ? 1 : 0;
  a.Sc = S;
  a.Pr = P;
  if (keep) {
    a.sc0 = st[12], a.sc1 = st[13], a.ldsc = st[14];
    a.pr0 = st[15], a.pr1 = st[16], a.ldpr = st[17];
    a.ldsc32 = (int)st[14], a.ldpr32 = (int)st[17];
    a.scbytes = (int)(31 * st[14] + T), a.prbytes = (int)(31 * st[17] + T);
  } else {
    a.sc0 = a.sc1 = a.ldsc = a.pr0 = a.pr1 = a.ldpr = 0;
    a.ldsc32 = a.ldpr32 = a.scbytes = a.prbytes = 0;
  }
  const bool s24 = flags & ANVIL_ATTN_S24;
  if (T == 16) {
    const long long nh = (long long)batch0 * batch1;
    if (keep)
      s24 ? launch_attention_t16<true, true>(a, D, nh, ctx->stream) : launch_attention_t16<false, true>(a, D, nh, ctx->stream);
    else
      s24 ? launch_attention_t16<true, false>(a, D, nh, ctx->stream) : launch_attention_t16<false, false>(a, D, nh, ctx->stream);
    ANVIL_LAUNCHED();
    return ANVIL_OK;
  }
  const unsigned grid = (unsigned)((long long)batch0 * batch1 * a.nqt);
  if (keep)
    s24 ? launch_attention_nt<true, true>(a, D, grid, ctx->stream) : launch_attention_nt<false, true>(a, D, grid, ctx->stream);
  else
    s24 ? launch_attention_nt<true, false>(a, D, grid, ctx->stream) : launch_attention_nt<false, false>(a, D, grid, ctx->stream);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

extern "C" int anvil_attention_i8(anvil_ctx* ctx, const int8_t* Q, const int8_t* K, const int8_t* Vt, int8_t* O,
                                  int batch0, int batch1, int T, int D, const int64_t* strides, int32_t m_s, int s_s,
                                  const int32_t* lut, int32_t one, int causal, int32_t m_o, int s_o, int flags) {
  return attention_entry(ctx, Q, K, Vt, O, nullptr, nullptr, false, batch0, batch1, T, D, strides, m_s, s_s, lut, one,
                         causal, m_o, s_o, flags);
}

extern "C" int anvil_attention_i8_keep(anvil_ctx* ctx, const int8_t* Q, const int8_t* K, const int8_t* Vt, int8_t* O,
                                       int8_t* S, int8_t* P, int batch0, int batch1, int T, int D,
                                       const int64_t* strides, int32_t m_s, int s_s, const int32_t* lut, int32_t one,
                                       int causal, int32_t m_o, int s_o, int flags) {
  return attention_entry(ctx, Q, K, Vt, O, S, P, true, batch0, batch1, T, D, strides, m_s, s_s, lut, one, causal, m_o,
                         s_o, flags);
}
