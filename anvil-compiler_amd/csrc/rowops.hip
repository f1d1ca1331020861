// Row reductions of the graph: rmsnorm_int and softmax_lut. One wavefront (64 lanes) per row; the row
// statistics (sum of squares, max, exp sum) are reduced across the wave with DPP-backed shuffles, so every lane
// ends with the same exact integer and the per-element pass needs no LDS round trip.
#include <algorithm>

#include "common.h"

namespace anvil {

constexpr int R_THREADS = 256, R_WAVES = R_THREADS / 64;
constexpr int ROWS_LUT_MAX = 4 * R_THREADS;   // table words rmsnorm_rows16 stages in LDS: four reads a thread

// A row kernel's table into LDS (dst: lut_len words), four reads in flight a lane; the caller synchronises.
__device__ __forceinline__ void stage_lut(int* dst, const int* __restrict__ lut, int lut_len) {
  for (int i0 = threadIdx.x; i0 < lut_len; i0 += 4 * R_THREADS) {
    int v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = i0 + j * R_THREADS < lut_len ? lut[i0 + j * R_THREADS] : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i0 + j * R_THREADS < lut_len) dst[i0 + j * R_THREADS] = v[j];
  }
}

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

__device__ __forceinline__ int wave_sum32(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int sbyte(const v4i& v, int b) {   // signed byte b (0..15) of a 16-byte chunk
  return (int)(int8_t)((unsigned)v[b >> 2] >> (8 * (b & 3)));
}

// signed byte B of x times w (|w| < 2^23) in one SDWA multiply, and a * b + c on 24-bit signed a, b: written out
// because the compiler's own lowering of these adds a shift (and a full-width multiply) per element
template <int B>
__device__ __forceinline__ int mul_sbyte(unsigned x, int w) {
  int d;
  if constexpr (B == 0)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
        : "=v"(d) : "v"(x), "v"(w));
  else if constexpr (B == 1)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:DWORD"
        : "=v"(d) : "v"(x), "v"(w));
  else if constexpr (B == 2)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2 src1_sel:DWORD"
        : "=v"(d) : "v"(x), "v"(w));
  else
    asm("v_mul_i32_i24_sdwa %0, sext(%1), %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3 src1_sel:DWORD"
        : "=v"(d) : "v"(x), "v"(w));
  return d;
}


__device__ __forceinline__ int mad_i24(int a, int b, int c) {
  int d;
  asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(b), "v"(c));
  return d;
}

// ------------------------------------------------------------------------------------- fast softmax_lut
// For proven graphs (every intermediate fits int32, lut >= 0 and lut[255] >= 1, so S >= 1) with rows of a multiple
// of 16 bytes: one wavefront per row, the row in registers as 16-byte chunks (lane l holds chunks l, l + 64, ...;
// causally masked chunks are not loaded), wave-reduced max and exp sum. The exp value of an element depends only on
// d = x - max + 255, so the 256 possible quotients (lut[d] one + S // 2) // S of a row are computed once (four exact
// integer divisions per lane) into an LDS table, and each output element is one table lookup.
template <int R, typename TO>
__global__ __launch_bounds__(R_THREADS) void softmax_fast(const int8_t* __restrict__ x, const int* __restrict__ lut,
                                                           int one, int causal, long long rows, int t1, int t2,
                                                           TO* __restrict__ out) {
  __shared__ int lut_s[256];
  __shared__ TO ptab[R_WAVES][256];
  lut_s[threadIdx.x] = lut[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  TO* pt = ptab[w];
  const int chunks = t2 >> 4;
  for (long long row = (long long)blockIdx.x * R_WAVES + w; row < rows; row += (long long)gridDim.x * R_WAVES) {
    const int i = (int)(row % t1);
    const int kept = causal ? min(i + 1, t2) : t2;
    const int8_t* xr = x + row * t2;
    v4i xv[R];
    int m = -128;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = lane + 64 * r;
      xv[r] = v4i{0, 0, 0, 0};
      if (c < chunks && 16 * c < kept) {
        xv[r] = *reinterpret_cast<const v4i*>(xr + 16 * c);
#pragma unroll
        for (int b = 0; b < 16; ++b)
          if (16 * c + b < kept) m = max(m, sbyte(xv[r], b));
      }
    }
    m = wave_max(m);
    int S = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = lane + 64 * r;
      if (c < chunks && 16 * c < kept) {
#pragma unroll
        for (int b = 0; b < 16; ++b)
          if (16 * c + b < kept) S += lut_s[sbyte(xv[r], b) - m + 255];
      }
    }
    S = wave_sum32(S);
    const unsigned us = (unsigned)S, half = us >> 1;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = lane + 64 * k;
      pt[d] = (TO)(((unsigned)lut_s[d] * (unsigned)one + half) / us);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");     // table entries written by other lanes of the wave
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = lane + 64 * r;
      if (c >= chunks) continue;
      TO* o = out + row * t2 + 16 * c;
      if (sizeof(TO) == 1) {
        unsigned wv[4] = {0, 0, 0, 0};
        if (16 * c < kept) {
#pragma unroll
          for (int b = 0; b < 16; ++b)
            if (16 * c + b < kept) wv[b >> 2] |= (unsigned)(uint8_t)pt[sbyte(xv[r], b) - m + 255] << (8 * (b & 3));
        }
        *reinterpret_cast<v4i*>(o) = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int wv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int b = 4 * q + e;
            wv[e] = 16 * c + b < kept ? (int)pt[sbyte(xv[r], b) - m + 255] : 0;
          }
          *reinterpret_cast<v4i*>(o + 4 * q) = v4i{wv[0], wv[1], wv[2], wv[3]};
        }
      }
    }
    __builtin_amdgcn_wave_barrier();                 // the table is rewritten for the wave's next row
  }
}

// ------------------------------------------------------------------------------------- fast rmsnorm_int
// For proven graphs with i8 rows (ss_shift = ss_init = 0) of a multiple of 16 bytes and at most 1024: a wavefront
// takes RMS_ROWS rows at a time, lane l holding 16 consecutive entries of each, and loads the next group while it
// requantises this one. Row loads and stores are raw buffer accesses over the group's rows: a lane past the row
// end or a row past the last gets an offset beyond the descriptor (loads 0, stores nothing), so no access sits
// under a branch and the next group's loads stay in flight across the whole group (a join of a path that loaded
// with one that did not would make the compiler wait for every load at the next use). The sum of squares is
// v_dot4 of each dword with itself; the row statistics are wave-uniform, so the rsqrt-LUT read is a scalar load.
constexpr int RMS_ROWS = 4;

// S24: every |lut[i] * mult| is below 2^23 (host-checked), so x w (lut[i] mult) + rnd -- the same integer as
// x w lut[i] mult + rnd, which is proven to fit int32 -- is one 24-bit multiply-add per element, with lut[i] mult
// formed once per row; otherwise two 32-bit multiplies per element. The requant clamps before its shift (bounds
// scaled by 2^s), so each output byte is one shift written straight into its byte lane.
template <bool S24>
__global__ __launch_bounds__(R_THREADS) void rmsnorm_fast(const int8_t* __restrict__ x, const int8_t* __restrict__ w,
                                                           const int* __restrict__ lut, int lut_len, int mult,
                                                           int shift, long long rows, int cols,
                                                           int8_t* __restrict__ out, int kbo) {
  const int lane = threadIdx.x & 63;
  const bool active = lane < (cols >> 4);
  // kbo: the output K-blocked (64-byte blocks of consecutive rows, block stride kbo bytes), stored through one buffer
  // over the whole output with rows past the end sent out of range
  const __amdgpu_buffer_rsrc_t wall = uniform_rsrc(out, kbo ? (int)(rows * cols) : 0);
  const unsigned kcol = (unsigned)((lane >> 2) * kbo + 16 * (lane & 3));
  v4i wv = {0, 0, 0, 0};
  if (active) wv = *reinterpret_cast<const v4i*>(w + 16 * lane);
  // this lane's 16 weights, sign-extended once
  int wb[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) wb[b] = sbyte(wv, b);
  unsigned off[RMS_ROWS];                                       // row j, this lane's chunk; OOB for idle lanes
#pragma unroll
  for (int j = 0; j < RMS_ROWS; ++j) off[j] = active ? (unsigned)(j * cols + 16 * lane) : OOB;
  const long long step = (long long)gridDim.x * R_WAVES * RMS_ROWS;
  auto group = [&](const int8_t* base, long long r0) {        // a raw buffer over rows r0 .. of this group
    const long long n = r0 < rows ? std::min<long long>(RMS_ROWS, rows - r0) : 0;
    return uniform_rsrc(base + (r0 < rows ? r0 : 0) * cols, (int)(n * cols));
  };
  auto load = [&](long long r0, v4i* xv) {
    const __amdgpu_buffer_rsrc_t rs = group(x, r0);
#pragma unroll
    for (int j = 0; j < RMS_ROWS; ++j)
      xv[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off[j], 0, 0));
  };
  auto process = [&](const v4i* xv, long long r0) {
    int idx[RMS_ROWS], sh[RMS_ROWS];
#pragma unroll
    for (int j = 0; j < RMS_ROWS; ++j) {
      int ss = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) ss = __builtin_amdgcn_sdot4(xv[j][q], xv[j][q], ss, false);
      ss = __builtin_amdgcn_readfirstlane(wave_sum32(ss));     // every lane holds the same sum
      const int k = rsqrt_shift(ss, lut_len, 32 - __builtin_clz((unsigned)lut_len));
      idx[j] = ss >> (2 * k);
      sh[j] = shift + k;
    }
    int r[RMS_ROWS];
#pragma unroll
    for (int j = 0; j < RMS_ROWS; ++j) r[j] = lut[idx[j]];
    const __amdgpu_buffer_rsrc_t ws = group(out, r0);
#pragma unroll
    for (int j = 0; j < RMS_ROWS; ++j) {
      const int s = sh[j];
      const int rnd = s ? (1 << (s - 1)) : 0;
      int lo = s >= 24 ? INT32_MIN : -128 * (1 << s), hi = s >= 24 ? INT32_MAX : 128 * (1 << s) - 1;
      asm("" : "+s"(lo), "+s"(hi));   // one med3 per element (a visible select becomes a v_cndmask per element)
      const int rm = S24 ? r[j] * mult : 0;
      v4i o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int y[4];
        // proven: x w r and x w r M + rnd fit int32 (S24: |x w| and |r M| below 2^23)
        if (S24) {
          const unsigned xd = (unsigned)xv[j][q];
          y[0] = med3i(mad_i24(mul_sbyte<0>(xd, wb[4 * q]), rm, rnd), lo, hi);
          y[1] = med3i(mad_i24(mul_sbyte<1>(xd, wb[4 * q + 1]), rm, rnd), lo, hi);
          y[2] = med3i(mad_i24(mul_sbyte<2>(xd, wb[4 * q + 2]), rm, rnd), lo, hi);
          y[3] = med3i(mad_i24(mul_sbyte<3>(xd, wb[4 * q + 3]), rm, rnd), lo, hi);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = med3i(sbyte(xv[j], 4 * q + e) * wb[4 * q + e] * r[j] * mult + rnd, lo, hi);
        }
        o[q] = (int)sra_pack4(y[0], y[1], y[2], y[3], s);
      }
      const unsigned ko = active && r0 + j < rows ? kcol + (unsigned)((r0 + j) * 64) : OOB;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, o),
                                             kbo ? wall : ws, kbo ? ko : off[j], 0, 0);
    }
  };
  // two row-group buffers in turn (the loop unrolled by two), so a group's rows are never copied between registers
  // and its loads stay in flight while the other group is requantised
  long long row0 = ((long long)blockIdx.x * R_WAVES + (threadIdx.x >> 6)) * RMS_ROWS;
  v4i xa[RMS_ROWS], xb[RMS_ROWS];
  load(row0, xa);
  while (row0 < rows) {
    load(row0 + step, xb);
    process(xa, row0);
    row0 += step;
    if (row0 >= rows) break;
    load(row0 + step, xa);
    process(xb, row0);
    row0 += step;
  }
}

// rmsnorm_int over rows of 256·CH bytes (the S24 form of rmsnorm_fast, every lane busy): a wave holds four rows,
// 16 lanes a row, and lane sub of row rr reads and writes chunks c·16 + sub (16 bytes each, c < CH), so each load or
// store instruction covers 256 contiguous bytes of every row. The row sums are reduced within each 16-lane DPP row,
// which leaves the row's sum in each of its lanes, and every lane forms its row's table index, requant multiplier,
// shift and clamp bounds itself, reading the table from LDS (at most ROWS_LUT_MAX words, staged once per workgroup
// while the first row group loads), so the reads do not wait behind the next group's row loads. (Formed on the
// scalar unit, read out row by row and returned to the lanes by selection, the compiler turned each row's selection
// into a branch holding that row's table load and its wait: four dependent round trips a row group.)
//
// L = 16 lanes a row as described; L = 8 takes rows of 128 CH bytes, eight rows a wave, in the same way (each load or
// store then covers 128 contiguous bytes of every row).
template <int CH, int L = 16>
__global__ __launch_bounds__(R_THREADS) void rmsnorm_rows16(const int8_t* __restrict__ x, const int8_t* __restrict__ w,
                                                             const int* __restrict__ lut, int lut_len, int mult,
                                                             int shift, long long rows, int8_t* __restrict__ out,
                                                             int kbo) {
  static_assert(L == 16 || L == 8, "16 or 8 lanes a row");
  constexpr int COLS = 16 * L * CH, R = 64 / L;               // bytes a row, rows a wave
  __shared__ int rows_lut[ROWS_LUT_MAX];
  const int lane = threadIdx.x & 63, rr = lane / L, sub = lane % L;
  // kbo: the output K-blocked, as in rmsnorm_fast; chunk L c + sub of a row is in block (L / 4) c + sub / 4
  const __amdgpu_buffer_rsrc_t wall = uniform_rsrc(out, kbo ? (int)(rows * COLS) : 0);
  const unsigned kcol = (unsigned)((sub >> 2) * kbo + 16 * (sub & 3));
  // this lane's weights, packed (each multiply selects and sign-extends its byte), through a buffer load: a plain
  // load of the read-only weights is free to sink past the table's barrier below, and then waits with the rows
  const __amdgpu_buffer_rsrc_t wr = uniform_rsrc(w, COLS);
  v4i wv[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c)
    wv[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wr, (unsigned)(16 * (L * c + sub)), 0, 0));
  unsigned off[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) off[c] = (unsigned)(rr * COLS + 16 * (L * c + sub));
  const long long step = (long long)gridDim.x * R_WAVES * R;
  auto group = [&](const int8_t* base, long long r0) {        // a raw buffer over rows r0 .. r0 + R - 1
    const long long n = r0 < rows ? std::min<long long>(R, rows - r0) : 0;
    return uniform_rsrc(base + (r0 < rows ? r0 : 0) * COLS, (int)(n * COLS));
  };
  auto load = [&](long long r0, v4i* xv) {
    const __amdgpu_buffer_rsrc_t rs = group(x, r0);
#pragma unroll
    for (int c = 0; c < CH; ++c) xv[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off[c], 0, 0));
  };
  auto process = [&](const v4i* xv, long long r0) {
    int ss = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) ss = __builtin_amdgcn_sdot4(xv[c][q], xv[c][q], ss, false);
    ss = L == 16 ? dpp_sum16(ss) : lane_group_sum<L>(ss);   // the row's sum, in each of its lanes
    const int k = rsqrt_shift(ss, lut_len, 32 - __builtin_clz((unsigned)lut_len));
    const int sh = shift + k;
    const int rm = rows_lut[ss >> (2 * k)] * mult;              // index below lut_len; proven below 2^23 in magnitude
    const int rnd = sh ? 1 << (sh - 1) : 0;
    const int lo = sh >= 24 ? INT32_MIN : -128 * (1 << sh), hi = sh >= 24 ? INT32_MAX : 128 * (1 << sh) - 1;
    const __amdgpu_buffer_rsrc_t ws = group(out, r0);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      v4i o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned xd = (unsigned)xv[c][q], wd = (unsigned)wv[c][q];
        // proven: x w r and x w r M + rnd fit int32, |x w| and |r M| below 2^23
        const int y0 = med3i(mad_i24v(mul_sbytes<0>(xd, wd), rm, rnd), lo, hi);
        const int y1 = med3i(mad_i24v(mul_sbytes<1>(xd, wd), rm, rnd), lo, hi);
        const int y2 = med3i(mad_i24v(mul_sbytes<2>(xd, wd), rm, rnd), lo, hi);
        const int y3 = med3i(mad_i24v(mul_sbytes<3>(xd, wd), rm, rnd), lo, hi);
        o[q] = (int)sra_pack4v(y0, y1, y2, y3, sh);
      }
      const unsigned ko = r0 + rr < rows ? kcol + (unsigned)((L / 4) * c * kbo + (r0 + rr) * 64) : OOB;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, o),
                                             kbo ? wall : ws, kbo ? ko : off[c], 0, 0);
    }
  };
  long long row0 = ((long long)blockIdx.x * R_WAVES + (threadIdx.x >> 6)) * R;
  v4i xa[CH], xb[CH];
  // the table's reads (words past lut_len read as zeros and are never indexed), then the first row group's, which
  // stay in flight while the table is stored
  const __amdgpu_buffer_rsrc_t lr = uniform_rsrc(lut, lut_len * 4);
  int tv[ROWS_LUT_MAX / R_THREADS];
#pragma unroll
  for (int j = 0; j < ROWS_LUT_MAX / R_THREADS; ++j)
    tv[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(lr, (unsigned)(j * R_THREADS + threadIdx.x) * 4, 0, 0);
  load(row0, xa);
#pragma unroll
  for (int j = 0; j < ROWS_LUT_MAX / R_THREADS; ++j) rows_lut[j * R_THREADS + threadIdx.x] = tv[j];
  __syncthreads();
  while (row0 < rows) {
    load(row0 + step, xb);
    process(xa, row0);
    row0 += step;
    if (row0 >= rows) break;
    load(row0 + step, xa);
    process(xb, row0);
    row0 += step;
  }
}

// rmsnorm_int over short int8 rows (16 L bytes, L = 1, 2 or 4 lanes a row, 64 / L rows a wave: the reference's
// frozen models have rows of 32), the S24 form. With so many rows a wave, the per-row values are each lane's own:
// the row sum is reduced over the row's L lanes, then every lane forms its row's table index, multiplier, shift and
// clamp bounds (the table staged in LDS, as in rmsnorm_wide_fast), and the element math is rmsnorm_rows16's.
template <int L>
__global__ __launch_bounds__(R_THREADS) void rmsnorm_narrow(const int8_t* __restrict__ x, const int8_t* __restrict__ w,
                                                             const int* __restrict__ lut, int lut_len, int mult,
                                                             int shift, long long rows, int8_t* __restrict__ out,
                                                             int kbo) {
  constexpr int COLS = 16 * L, R = 64 / L;
  extern __shared__ int narrow_lut[];
  stage_lut(narrow_lut, lut, lut_len);
  __syncthreads();
  const int lane = threadIdx.x & 63, rr = lane / L, sub = lane % L;
  const __amdgpu_buffer_rsrc_t wall = uniform_rsrc(out, kbo ? (int)(rows * COLS) : 0);
  const unsigned kcol = (unsigned)(16 * sub);                  // K-blocked output (COLS = 64): one block a row
  const v4i wv = *reinterpret_cast<const v4i*>(w + 16 * sub);
  const unsigned off = (unsigned)(rr * COLS + 16 * sub);
  const long long step = (long long)gridDim.x * R_WAVES * R;
  auto group = [&](const int8_t* base, long long r0) {        // a raw buffer over rows r0 .. r0 + R - 1
    const long long n = r0 < rows ? std::min<long long>(R, rows - r0) : 0;
    return uniform_rsrc(base + (r0 < rows ? r0 : 0) * COLS, (int)(n * COLS));
  };
  auto load = [&](long long r0) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(group(x, r0), off, 0, 0));
  };
  auto process = [&](v4i xv, long long r0) {
    int ss = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) ss = __builtin_amdgcn_sdot4(xv[q], xv[q], ss, false);
    int t = lane_group_sum<L>(ss);
    const int k = rsqrt_shift(t, lut_len, 32 - __builtin_clz((unsigned)lut_len));   // per lane: its row's sum
    t >>= 2 * k;
    const int sh = shift + k;
    const int rm = narrow_lut[t] * mult;                        // proven below 2^23 in magnitude
    const int rnd = sh ? 1 << (sh - 1) : 0;
    const int lo = sh >= 24 ? INT32_MIN : -128 * (1 << sh), hi = sh >= 24 ? INT32_MAX : 128 * (1 << sh) - 1;
    v4i o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const unsigned xd = (unsigned)xv[q], wd = (unsigned)wv[q];
      const int y0 = med3i(mad_i24v(mul_sbytes<0>(xd, wd), rm, rnd), lo, hi);
      const int y1 = med3i(mad_i24v(mul_sbytes<1>(xd, wd), rm, rnd), lo, hi);
      const int y2 = med3i(mad_i24v(mul_sbytes<2>(xd, wd), rm, rnd), lo, hi);
      const int y3 = med3i(mad_i24v(mul_sbytes<3>(xd, wd), rm, rnd), lo, hi);
      o[q] = (int)sra_pack4v(y0, y1, y2, y3, sh);
    }
    const unsigned ko = r0 + rr < rows ? kcol + (unsigned)((r0 + rr) * 64) : OOB;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, o),
                                           kbo ? wall : group(out, r0), kbo ? ko : off, 0, 0);
  };
  long long row0 = ((long long)blockIdx.x * R_WAVES + (threadIdx.x >> 6)) * R;
  v4i xa = load(row0), xb;
  while (row0 < rows) {
    xb = load(row0 + step);
    process(xa, row0);
    row0 += step;
    if (row0 >= rows) break;
    xa = load(row0 + step);
    process(xb, row0);
    row0 += step;
  }
}

// ------------------------------------------------------------------------------- fast rmsnorm_int, int16 rows
// The proven form of a wide (int16) row: ss = e + sum((x^2 + 2^(c-1)) >> c), out = requant(x w lut[i], M, s + k).
// A row of cols = 8 n entries is n chunks of 16 bytes (8 entries); L lanes (the power of two >= n, at most 64)
// take a row, so a wave holds 64 / L rows and lane sub of row rr handles chunks c L + sub (c < CH). Lanes past n
// and rows past the last get buffer offsets beyond the descriptor (loads 0, stores nothing), as in rmsnorm_fast.
// The row sum is reduced over the L lanes (DPP within 16 lanes, swizzles across), so every lane of a row holds it
// and forms that row's table index, multiplier, shift and clamp bounds itself; the table sits in LDS (lut_len words
// of dynamic LDS, staged once per workgroup), so its per-lane reads do not wait behind the next group's row loads.
// Each entry's square is one 24-bit multiply of its sign-extended half (SDWA); x w is one 24-bit multiply of that
// half by the sign-extended weight byte, |x w| <= 2^22. With s24 (every |lut[i] M| < 2^23) x w (lut[i] M) + rnd is one 24-bit multiply-add; without
// it the product wraps in 32 bits, which is exact because x w lut[i] M + rnd is proven to fit int32.
template <int H, int B>
__device__ __forceinline__ int mul_half_byte(unsigned x, unsigned w) {   // sext(half H of x) * sext(byte B of w)
  int d;
  if constexpr (H == 0 && B == 0)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:BYTE_0"
        : "=v"(d) : "v"(x), "v"(w));
  else if constexpr (H == 1 && B == 1)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:BYTE_1"
        : "=v"(d) : "v"(x), "v"(w));
  else if constexpr (H == 0 && B == 2)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:BYTE_2"
        : "=v"(d) : "v"(x), "v"(w));
  else
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:BYTE_3"
        : "=v"(d) : "v"(x), "v"(w));
  static_assert((H == 0 && (B == 0 || B == 2)) || (H == 1 && (B == 1 || B == 3)), "entry 2q + H sits in byte B");
  return d;
}

template <int H>
__device__ __forceinline__ int square_half(unsigned x) {                 // sext(half H of x)^2
  int d;
  if constexpr (H == 0)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_0"
        : "=v"(d) : "v"(x));
  else
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_1"
        : "=v"(d) : "v"(x));
  return d;
}

constexpr int WIDE_LUT_MAX = 4096;                               // table words the wide kernel stages in LDS

template <int L, int CH>
__global__ __launch_bounds__(R_THREADS) void rmsnorm_wide_fast(const int16_t* __restrict__ x,
                                                                const int8_t* __restrict__ w,
                                                                const int* __restrict__ lut, int lut_len, int mult,
                                                                int shift, int c, int e, int s24, long long rows,
                                                                int cols, int8_t* __restrict__ out, int kbo) {
  static_assert(CH == 1 || L == 64, "several chunks a lane only with a whole wave a row");
  constexpr int RW = 64 / L;                                     // rows a wave holds at once
  extern __shared__ int wide_lut[];
  stage_lut(wide_lut, lut, lut_len);
  __syncthreads();
  const int lane = threadIdx.x & 63, rr = lane / L, sub = lane % L;
  const int n = cols >> 3;                                       // 16-byte chunks of x a row
  v2i wv[CH];
  unsigned xoff[CH], ooff[CH], kcol[CH];
  const __amdgpu_buffer_rsrc_t wall = uniform_rsrc(out, kbo ? (int)(rows * cols) : 0);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int ch = k * L + sub;
    const bool on = ch < n;
    wv[k] = on ? *reinterpret_cast<const v2i*>(w + 8 * ch) : v2i{0, 0};
    xoff[k] = on ? (unsigned)(rr * 2 * cols + 16 * ch) : OOB;
    ooff[k] = on ? (unsigned)(rr * cols + 8 * ch) : OOB;
    kcol[k] = on ? (unsigned)((ch >> 3) * kbo + 8 * (ch & 7)) : OOB;   // K-blocked output: 8 chunks a block
  }
  const int rc = c ? 1 << (c - 1) : 0;
  const long long step = (long long)gridDim.x * R_WAVES * RW;
  auto group = [&](const void* base, long long r0, int row_bytes) {   // a raw buffer over rows r0 .. r0 + RW - 1
    const long long nr = r0 < rows ? std::min<long long>(RW, rows - r0) : 0;
    return uniform_rsrc((const char*)base + (r0 < rows ? r0 : 0) * row_bytes, (int)(nr * row_bytes));
  };
  auto load = [&](long long r0, v4i* xv) {
    const __amdgpu_buffer_rsrc_t rs = group(x, r0, 2 * cols);
#pragma unroll
    for (int k = 0; k < CH; ++k)
      xv[k] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, xoff[k], 0, 0));
  };
  auto process = [&](const v4i* xv, long long r0) {
    int ss = 0;
#pragma unroll
    for (int k = 0; k < CH; ++k)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned xd = (unsigned)xv[k][q];
        ss += (unsigned)(square_half<0>(xd) + rc) >> c;         // proven: x^2 + rnd and the sum fit int32
        ss += (unsigned)(square_half<1>(xd) + rc) >> c;
      }
    int t = lane_group_sum<L>(ss) + e;
    const int kk = rsqrt_shift(t, lut_len, 32 - __builtin_clz((unsigned)lut_len));  // per lane: its row's sum
    t >>= 2 * kk;
    const int sh = shift + kk;                                   // proven at most 31
    const int rm = wide_lut[t] * mult;                           // wraps unless s24; the products stay exact
    const int rnd = sh ? 1 << (sh - 1) : 0;
    const int lo = sh >= 24 ? INT32_MIN : -128 * (1 << sh), hi = sh >= 24 ? INT32_MAX : 128 * (1 << sh) - 1;
    const __amdgpu_buffer_rsrc_t ws = group(out, r0, cols);
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      int xw[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned xd = (unsigned)xv[k][q], wd = (unsigned)wv[k][q >> 1];
        if (q & 1) {
          xw[2 * q] = mul_half_byte<0, 2>(xd, wd);
          xw[2 * q + 1] = mul_half_byte<1, 3>(xd, wd);
        } else {
          xw[2 * q] = mul_half_byte<0, 0>(xd, wd);
          xw[2 * q + 1] = mul_half_byte<1, 1>(xd, wd);
        }
      }
      int y[8];
      if (s24) {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = med3i(mad_i24v(xw[j], rm, rnd), lo, hi);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = med3i((int)((unsigned)xw[j] * (unsigned)rm + (unsigned)rnd), lo, hi);
      }
      const v2i o = {(int)sra_pack4v(y[0], y[1], y[2], y[3], sh), (int)sra_pack4v(y[4], y[5], y[6], y[7], sh)};
      const unsigned ko = kcol[k] != OOB && r0 + rr < rows ? kcol[k] + (unsigned)((r0 + rr) * 64) : OOB;
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned, o),
                                            kbo ? wall : ws, kbo ? ko : ooff[k], 0, 0);
    }
  };
  long long row0 = ((long long)blockIdx.x * R_WAVES + (threadIdx.x >> 6)) * RW;
  v4i xa[CH], xb[CH];
  load(row0, xa);
  while (row0 < rows) {
    load(row0 + step, xb);
    process(xa, row0);
    row0 += step;
    if (row0 >= rows) break;
    load(row0 + step, xa);
    process(xb, row0);
    row0 += step;
  }
}

static unsigned row_grid(long long rows, int device_cus) {
  long long blocks = (rows + R_WAVES - 1) / R_WAVES;
  const long long cap = (long long)device_cus * 16;            // enough resident waves to cover HBM latency
  return (unsigned)(blocks < cap ? blocks : cap);
}

// ---------------------------------------------------------------------------------------------- rmsnorm_int
// Per row (anvil/semantics.py:164-182): ss = e + sum((x^2 + 2^(c-1)) >> c); (i, k) = rsqrt_index(ss, n);
// out = requant(x * w * lut[i], M, s + k).
template <typename T>
__global__ __launch_bounds__(R_THREADS) void rmsnorm_kernel(const T* __restrict__ x, const int8_t* __restrict__ w,
                                                             const int* __restrict__ lut, int lut_len, int mult,
                                                             int shift, int c, int e, long long rows, int cols,
                                                             int8_t* __restrict__ out, unsigned* flags, int kbo) {
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
    const int8_t y = (int8_t)requant_checked((int)xwr, mult, sh, rnd, -128, 127, bad);
    if (kbo)
      out[(long long)(j >> 6) * kbo + row * 64 + (j & 63)] = y;   // K-blocked output
    else
      o[j] = y;
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

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static bool al8(const void* p) { return ((uintptr_t)p & 7) == 0; }

extern "C" int anvil_rmsnorm_int_ex(anvil_ctx* ctx, const void* x, int x_dtype, const int8_t* w, const int32_t* lut,
                                    int lut_len, int32_t mult, int shift, int ss_shift, int32_t ss_init, int64_t rows,
                                    int cols, int8_t* out, int flags) {
  if (!x || !w || !lut || !out) return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: null pointer");
  if (rows < 0 || cols < 1 || lut_len < 1) return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: bad size");
  if (x_dtype != ANVIL_I8 && x_dtype != ANVIL_I16) return set_error(ANVIL_E_VALUE, "rmsnorm x must be i8 or i16");
  if (shift < 0 || shift > 31) return set_error(ANVIL_E_VALUE, "shift %d outside [0, 31]", shift);
  if (ss_shift < 0 || ss_shift > 30) return set_error(ANVIL_E_VALUE, "ss_shift %d outside [0, 30]", ss_shift);
  if (ss_init < 0) return set_error(ANVIL_E_VALUE, "ss_init %d negative", ss_init);
  if (flags & ~(ANVIL_OP_UNCHECKED | ANVIL_RMS_S24 | ANVIL_RMS_OUT_KBLOCK))
    return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: unknown flags %d", flags);
  if ((flags & ANVIL_RMS_OUT_KBLOCK) && (cols % 64 || rows * cols >= (1ll << 31)))
    return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: a K-blocked result needs cols %% 64 == 0 and rows x cols "
                                    "below 2^31 (cols %d)", cols);
  const int kbo = (flags & ANVIL_RMS_OUT_KBLOCK) ? (int)(rows * 64) : 0;   // block stride of a K-blocked result
  if ((flags & ANVIL_RMS_S24) && !(flags & ANVIL_OP_UNCHECKED))
    return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: ANVIL_RMS_S24 needs ANVIL_OP_UNCHECKED");
  if (int r = check_ctx(ctx)) return r;
  if (rows == 0) return ANVIL_OK;
  const long long blocks = (rows + R_WAVES - 1) / R_WAVES;
  if (blocks > (1ll << 31) - 1) return set_error(ANVIL_E_VALUE, "anvil_rmsnorm_int: too many rows");
  if ((flags & ANVIL_OP_UNCHECKED) && x_dtype == ANVIL_I8 && ss_shift == 0 && ss_init == 0 && cols % 16 == 0 &&
      cols <= 1024 && al16(x) && al16(w) && al16(out)) {
    // up to eight workgroups per CU (one row group per wave for the block shapes), a wave walking further groups with
    // the next group's loads in flight
    const long long groups = (rows + RMS_ROWS - 1) / RMS_ROWS;
    const dim3 grid((unsigned)std::min<long long>((groups + R_WAVES - 1) / R_WAVES, 8ll * ctx->num_cu));
    const int ch = cols / 256;
    if ((flags & ANVIL_RMS_S24) && cols % 256 == 0 && ch <= 4 && lut_len <= ROWS_LUT_MAX) {   // rows of 256 to 1024
      auto launch = [&](auto kernel) {
        ANVIL_LAUNCH(kernel, grid, dim3(R_THREADS), 0, ctx->stream, (const int8_t*)x, w, lut, lut_len, mult, shift,
                     (long long)rows, out, kbo);
      };
      if (ch == 1) launch(rmsnorm_rows16<1>);
      else if (ch == 2) launch(rmsnorm_rows16<2>);
      else if (ch == 3) launch(rmsnorm_rows16<3>);
      else launch(rmsnorm_rows16<4>);
    } else if ((flags & ANVIL_RMS_S24) && (cols == 16 || cols == 32 || cols == 64) && lut_len <= WIDE_LUT_MAX) {
      const int L = cols / 16;                                         // lanes a row, 64 / L rows a wave
      const long long groupsn = (rows + 64 / L - 1) / (64 / L);
      const dim3 gridn((unsigned)std::min<long long>((groupsn + R_WAVES - 1) / R_WAVES, 8ll * ctx->num_cu));
      auto launch = [&](auto kernel) {
        ANVIL_LAUNCH(kernel, gridn, dim3(R_THREADS), lut_len * sizeof(int), ctx->stream, (const int8_t*)x, w, lut,
                     lut_len, mult, shift, (long long)rows, out, kbo);
      };
      if (L == 1) launch(rmsnorm_narrow<1>);
      else if (L == 2) launch(rmsnorm_narrow<2>);
      else launch(rmsnorm_narrow<4>);
    } else if ((flags & ANVIL_RMS_S24) && cols == 128 && lut_len <= ROWS_LUT_MAX) {   // 8 lanes a row, 8 rows a wave
      const long long groups8 = (rows + 7) / 8;
      const dim3 grid8((unsigned)std::min<long long>((groups8 + R_WAVES - 1) / R_WAVES, 8ll * ctx->num_cu));
      ANVIL_LAUNCH((rmsnorm_rows16<1, 8>), grid8, dim3(R_THREADS), 0, ctx->stream, (const int8_t*)x, w, lut, lut_len,
                   mult, shift, (long long)rows, out, kbo);
    } else if (flags & ANVIL_RMS_S24)
      ANVIL_LAUNCH(rmsnorm_fast<true>, grid, dim3(R_THREADS), 0, ctx->stream, (const int8_t*)x, w, lut, lut_len,
                         mult, shift, (long long)rows, cols, out, kbo);
    else
      ANVIL_LAUNCH(rmsnorm_fast<false>, grid, dim3(R_THREADS), 0, ctx->stream, (const int8_t*)x, w, lut, lut_len,
                         mult, shift, (long long)rows, cols, out, kbo);
  } else if ((flags & ANVIL_OP_UNCHECKED) && x_dtype == ANVIL_I16 && cols % 8 == 0 && cols <= 2048 &&
             lut_len <= WIDE_LUT_MAX && al16(x) && al8(w) && al8(out)) {
    const int n = cols / 8;                                     // 16-byte chunks a row
    int L = 1;                                                  // lanes a row: the power of two >= n, at most 64
    while (L < n && L < 64) L <<= 1;
    const long long groups = (rows + 64 / L - 1) / (64 / L);
    const dim3 grid((unsigned)std::min<long long>((groups + R_WAVES - 1) / R_WAVES, 8ll * ctx->num_cu));
    const int s24 = (flags & ANVIL_RMS_S24) ? 1 : 0;
    auto launch = [&](auto kernel) {
      ANVIL_LAUNCH(kernel, grid, dim3(R_THREADS), 4 * lut_len, ctx->stream, (const int16_t*)x, w, lut, lut_len, mult,
                   shift, ss_shift, ss_init, s24, (long long)rows, cols, out, kbo);
    };
    switch (n > 64 ? 64 * ((n + 63) / 64) : L) {
      case 1: launch(rmsnorm_wide_fast<1, 1>); break;
      case 2: launch(rmsnorm_wide_fast<2, 1>); break;
      case 4: launch(rmsnorm_wide_fast<4, 1>); break;
      case 8: launch(rmsnorm_wide_fast<8, 1>); break;
      case 16: launch(rmsnorm_wide_fast<16, 1>); break;
      case 32: launch(rmsnorm_wide_fast<32, 1>); break;
      case 64: launch(rmsnorm_wide_fast<64, 1>); break;
      case 128: launch(rmsnorm_wide_fast<64, 2>); break;
      case 192: launch(rmsnorm_wide_fast<64, 3>); break;
      default: launch(rmsnorm_wide_fast<64, 4>); break;
    }
  } else if (x_dtype == ANVIL_I8) {
    ANVIL_LAUNCH(rmsnorm_kernel<int8_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream,
                       (const int8_t*)x, w, lut, lut_len, mult, shift, ss_shift, ss_init, (long long)rows, cols, out,
                       ctx->flags, kbo);
  } else {
    ANVIL_LAUNCH(rmsnorm_kernel<int16_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream,
                       (const int16_t*)x, w, lut, lut_len, mult, shift, ss_shift, ss_init, (long long)rows, cols,
                       out, ctx->flags, kbo);
  }
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

extern "C" int anvil_rmsnorm_int(anvil_ctx* ctx, const void* x, int x_dtype, const int8_t* w, const int32_t* lut,
                                 int lut_len, int32_t mult, int shift, int ss_shift, int32_t ss_init, int64_t rows,
                                 int cols, int8_t* out) {
  return anvil_rmsnorm_int_ex(ctx, x, x_dtype, w, lut, lut_len, mult, shift, ss_shift, ss_init, rows, cols, out, 0);
}

namespace anvil {

// ------------------------------------------------------------------------------ fast softmax_lut, int8 result
// The int8-result form of softmax_fast (one <= 127), with every per-element step one instruction and no integer
// division. Per 16-byte chunk a lane keeps nk bytes (its causal prefix); the others become -128, which leaves the
// row max unchanged (the reference's max starts at -128) and adds (16 - nk) lut[127 - m] to the exp sum, subtracted
// once per chunk. Byte b of a chunk becomes the table index d = x - m + 255 in [0, 255] (one SDWA add into its
// byte), then the byte offset 4 d (one SDWA shift), used for the exp table and, at the same address plus a
// constant, for the row's probability table, whose entries are the exact quotients (lut[d] one + S // 2) // S in
// float64: y = fma(lut[d], A, B) with A = fl(one fl(1 / S)), B = fl(fl((S // 2) fl(1 / S)) + 2^-40) - 1/2 lies within
// 2^-44 of n / S - 1/2 + 2^-40 (n = lut[d] one + S // 2 < 2^31, n / S < 128), and a non-integer n / S is at least
// 1 / S > 2^-31 from an integer, so y + 1.5 2^52 rounds to floor(n / S) exactly. One wavefront per row; a 64-lane
// workgroup, so both tables sit at fixed LDS addresses.

template <int B>
__device__ __forceinline__ int max_sbyte(int acc, unsigned x) {      // max(acc, signed byte B of x)
  int d;
  if constexpr (B == 0)
    asm("v_max_i32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(d) : "v"(acc), "v"(x));
  else if constexpr (B == 1)
    asm("v_max_i32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(d) : "v"(acc), "v"(x));
  else if constexpr (B == 2)
    asm("v_max_i32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(d) : "v"(acc), "v"(x));
  else
    asm("v_max_i32_sdwa %0, %1, sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(d) : "v"(acc), "v"(x));
  return d;
}

// byte B of x plus k (mod 256) written into byte B of acc, the other bytes of acc kept
template <int B>
__device__ __forceinline__ void add_byte(unsigned& acc, unsigned x, unsigned k) {
  if constexpr (B == 0)
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_0"
        : "+v"(acc) : "v"(k), "v"(x));
  else if constexpr (B == 1)
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_1"
        : "+v"(acc) : "v"(k), "v"(x));
  else if constexpr (B == 2)
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_2"
        : "+v"(acc) : "v"(k), "v"(x));
  else
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_3"
        : "+v"(acc) : "v"(k), "v"(x));
}

// 4 * (byte B of x), zero-extended
template <int B>
__device__ __forceinline__ unsigned off4(unsigned x, unsigned two) {
  unsigned d;
  if constexpr (B == 0)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(d) : "v"(two), "v"(x));
  else if constexpr (B == 1)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(d) : "v"(two), "v"(x));
  else if constexpr (B == 2)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(d) : "v"(two), "v"(x));
  else
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(d) : "v"(two), "v"(x));
  return d;
}

template <int R>
__global__ __launch_bounds__(64) void softmax_i8_fast(const int8_t* __restrict__ x, const int* __restrict__ lut,
                                                      int one, int causal, long long rows, int t1, int t2,
                                                      int8_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) int lut_s[256];
  __shared__ __attribute__((aligned(16))) int ptab[256];
  __shared__ double lutd_s[256];
  const int lane = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int v = lut[lane + 64 * k];
    lut_s[lane + 64 * k] = v;
    lutd_s[lane + 64 * k] = (double)v;
  }
  __syncthreads();
  const int chunks = t2 >> 4;
  const unsigned two = 2;
  const char* lutb = reinterpret_cast<const char*>(lut_s);
  const char* ptb = reinterpret_cast<const char*>(ptab);
  for (long long row = blockIdx.x; row < rows; row += gridDim.x) {
    const int i = (int)(row % t1);
    const int kept = causal ? min(i + 1, t2) : t2;
    const int8_t* xr = x + row * t2;
    v4i xv[R];
    unsigned mk[R][4];
    int nk[R];
    int m0 = -128, m1 = -128, m2 = -128, m3 = -128;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = lane + 64 * r;
      nk[r] = c < chunks ? min(max(kept - 16 * c, 0), 16) : 0;
      xv[r] = v4i{0, 0, 0, 0};
      if (nk[r] > 0) xv[r] = *reinterpret_cast<const v4i*>(xr + 16 * c);
#pragma unroll
      for (int q = 0; q < 4; ++q) mk[r][q] = 0xffffffffu;
      if (nk[r] < 16) {                                  // the causal edge, or a chunk past it: masked bytes -> -128
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int kq = min(max(nk[r] - 4 * q, 0), 4);
          mk[r][q] = kq >= 4 ? 0xffffffffu : (1u << (8 * kq)) - 1u;
          xv[r][q] = (int)(((unsigned)xv[r][q] & mk[r][q]) | (0x80808080u & ~mk[r][q]));
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned w = (unsigned)xv[r][q];
        m0 = max_sbyte<0>(m0, w);
        m1 = max_sbyte<1>(m1, w);
        m2 = max_sbyte<2>(m2, w);
        m3 = max_sbyte<3>(m3, w);
      }
    }
    const int m = wave_max(max(max(m0, m1), max(m2, m3)));
    const unsigned kadd = (unsigned)(255 - m);           // d = x - m + 255, in [0, 255]: byte add mod 256
    unsigned off[R][16];
    int S = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        unsigned dq = 0;
        const unsigned w = (unsigned)xv[r][q];
        add_byte<0>(dq, w, kadd);
        add_byte<1>(dq, w, kadd);
        add_byte<2>(dq, w, kadd);
        add_byte<3>(dq, w, kadd);
        off[r][4 * q + 0] = off4<0>(dq, two);
        off[r][4 * q + 1] = off4<1>(dq, two);
        off[r][4 * q + 2] = off4<2>(dq, two);
        off[r][4 * q + 3] = off4<3>(dq, two);
      }
#pragma unroll
      for (int b = 0; b < 16; ++b) S += *reinterpret_cast<const int*>(lutb + off[r][b]);
      S -= (16 - nk[r]) * lut_s[127 - m];                 // the masked bytes' share
    }
    S = wave_sum32(S);
    // the row's probability table, entry d at ptab[d] (A and B exact to 2^-52 relative; see above)
    const double inv = 1.0 / (double)S;
    const double A = (double)one * inv;
    const double Bc = (double)(S >> 1) * inv + 0x1p-40 - 0.5;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = lane + 64 * k;
      ptab[d] = __double2loint(__builtin_fma(lutd_s[d], A, Bc) + 0x1.8p52);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");     // table entries written by other lanes of the wave
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = lane + 64 * r;
      if (c >= chunks) continue;
      v4i ov;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p0 = *reinterpret_cast<const int*>(ptb + off[r][4 * q]);
        const int p1 = *reinterpret_cast<const int*>(ptb + off[r][4 * q + 1]);
        const int p2 = *reinterpret_cast<const int*>(ptb + off[r][4 * q + 2]);
        const int p3 = *reinterpret_cast<const int*>(ptb + off[r][4 * q + 3]);
        ov[q] = (int)(pack4(p0, p1, p2, p3) & mk[r][q]);  // masked keys: probability 0
      }
      *reinterpret_cast<v4i*>(out + row * t2 + 16 * c) = ov;
    }
    __builtin_amdgcn_wave_barrier();                     // the table is rewritten for the wave's next row
  }
}

}  // namespace anvil

template <typename TO>
static void launch_softmax_fast(anvil_ctx* ctx, const int8_t* x, const int32_t* lut, int one, int causal,
                                long long rows, int t1, int t2, TO* out) {
  if constexpr (sizeof(TO) == 1) {
    const long long cap = (long long)ctx->num_cu * 32;  // one 64-lane workgroup per row, grid-stride
    const unsigned grid = (unsigned)(rows < cap ? rows : cap);
    if (t2 <= 1024)
      ANVIL_LAUNCH((softmax_i8_fast<1>), dim3(grid), dim3(64), 0, ctx->stream, x, lut, one, causal, rows, t1, t2,
                   out);
    else if (t2 <= 2048)
      ANVIL_LAUNCH((softmax_i8_fast<2>), dim3(grid), dim3(64), 0, ctx->stream, x, lut, one, causal, rows, t1, t2,
                   out);
    else
      ANVIL_LAUNCH((softmax_i8_fast<4>), dim3(grid), dim3(64), 0, ctx->stream, x, lut, one, causal, rows, t1, t2,
                   out);
    return;
  }
  const unsigned grid = row_grid(rows, ctx->num_cu);
  if (t2 <= 1024)
    ANVIL_LAUNCH((softmax_fast<1, TO>), dim3(grid), dim3(R_THREADS), 0, ctx->stream, x, lut, one, causal, rows,
                       t1, t2, out);
  else if (t2 <= 2048)
    ANVIL_LAUNCH((softmax_fast<2, TO>), dim3(grid), dim3(R_THREADS), 0, ctx->stream, x, lut, one, causal, rows,
                       t1, t2, out);
  else
    ANVIL_LAUNCH((softmax_fast<4, TO>), dim3(grid), dim3(R_THREADS), 0, ctx->stream, x, lut, one, causal, rows,
                       t1, t2, out);
}

extern "C" int anvil_softmax_lut_ex(anvil_ctx* ctx, const int8_t* x, const int32_t* lut, int32_t one, int causal,
                                    int64_t batch, int t1, int t2, void* out, int out_dtype, int flags) {
  if (!x || !lut || !out) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: null pointer");
  if (batch < 0 || t1 < 1 || t2 < 1) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: bad size");
  if (out_dtype != ANVIL_I8 && out_dtype != ANVIL_I32)
    return set_error(ANVIL_E_VALUE, "softmax result must be i8 or i32");
  if (one < 1 || (out_dtype == ANVIL_I8 && one > 127))
    return set_error(ANVIL_E_VALUE, "one=%d does not fit the result dtype", one);
  if (flags & ~ANVIL_OP_UNCHECKED) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: unknown flags %d", flags);
  if (int r = check_ctx(ctx)) return r;
  const long long rows = batch * t1;
  if (rows == 0) return ANVIL_OK;
  const long long blocks = (rows + R_WAVES - 1) / R_WAVES;
  if (blocks > (1ll << 31) - 1) return set_error(ANVIL_E_VALUE, "anvil_softmax_lut: too many rows");
  if ((flags & ANVIL_OP_UNCHECKED) && t2 % 16 == 0 && t2 <= 4096 && al16(x) && al16(out)) {
    if (out_dtype == ANVIL_I8)
      launch_softmax_fast<int8_t>(ctx, x, lut, one, causal, rows, t1, t2, (int8_t*)out);
    else
      launch_softmax_fast<int32_t>(ctx, x, lut, one, causal, rows, t1, t2, (int32_t*)out);
  } else if (out_dtype == ANVIL_I8) {
    ANVIL_LAUNCH(softmax_kernel<int8_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream, x, lut, one,
                       causal, rows, t1, t2, (int8_t*)out, ctx->flags);
  } else {
    ANVIL_LAUNCH(softmax_kernel<int32_t>, dim3((unsigned)blocks), dim3(R_THREADS), 0, ctx->stream, x, lut, one,
                       causal, rows, t1, t2, (int32_t*)out, ctx->flags);
  }
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

extern "C" int anvil_softmax_lut(anvil_ctx* ctx, const int8_t* x, const int32_t* lut, int32_t one, int causal,
                                 int64_t batch, int t1, int t2, void* out, int out_dtype) {
  return anvil_softmax_lut_ex(ctx, x, lut, one, causal, batch, t1, t2, out, out_dtype, 0);
}
