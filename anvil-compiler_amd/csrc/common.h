// Shared host and device helpers of the anvil_mi355x library (gfx950 only).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../../include/anvil_mi355x.h"

// Device-side contract flags: a kernel that meets a value the reference's checked int32 semantics reject sets a
// bit here (a rare, vector-memory atomic); anvil_sync reads and clears them and returns the matching status.
enum : unsigned {
  FLAG_OVERFLOW = 1u,   // an intermediate left int32            -> OverflowError
  FLAG_SHIFT = 2u,      // rmsnorm shift s + k above 31            -> ValueError (round_term)
  FLAG_ZERODIV = 4u,    // softmax row sum 0                       -> ZeroDivisionError
  FLAG_RANGE = 8u,      // an operand outside its dtype            -> ValueError
  FLAG_NONFINITE = 16u, // a float input NaN or infinite           -> ValueError
};

constexpr int EVENT_SLOTS = 512;

struct anvil_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  unsigned* flags = nullptr;      // device word of FLAG_* bits
  hipEvent_t events[EVENT_SLOTS] = {};   // created on first use of a slot
  int num_cu = 0;
  int gemm_cfg = 0;               // ANVIL_GEMM_CFG at init: pins one GEMM tile shape (benchmarking); 0 = by problem
  // split-K workspace of anvil_gemm_i8_ex (int32 partial tiles), allocated on first use and grown as needed. A HIP
  // graph captured on the context's stream holds the workspace address of its split-K launches, so a buffer the
  // workspace outgrows is kept (ws_retired) until anvil_destroy instead of being freed under such a graph.
  int* ws = nullptr;
  long long ws_elems = 0;
  std::vector<int*> ws_retired;
};

namespace anvil {

int set_error(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
int check_ctx(anvil_ctx* ctx);
// zero `bytes` of device memory with a fill kernel on stream s (no memset node: safe inside a captured graph)
int zero_fill(hipStream_t s, void* dst, size_t bytes);
// once per device, with that device current: the device address of the GEMM's static split-K scratch
int gemm_scratch_setup(int device);
// at anvil_destroy, after the context's stream has drained: the device's static scratch is free for other contexts
void gemm_scratch_release(anvil_ctx* ctx);

#define ANVIL_HIP(call)                                        \
  do {                                                         \
    hipError_t e_ = (call);                                    \
    if (e_ != hipSuccess) return ::anvil::hip_fail(e_, #call); \
  } while (0)

// Kernel timer (anvil_time_kernels): while armed for a stream, every launch on that stream carries the timer's
// events, bound to the kernel itself (hipExtLaunchKernel): the start event to the first launch's start, the stop
// event to each launch's end, so the pair spans the kernels and no dispatch gap or event packet.
struct KernelTimer {
  hipStream_t stream;
  hipEvent_t start;   // cleared once the first timed launch has taken it
  hipEvent_t stop;
};
extern __thread KernelTimer g_timer;   // zero-initialised per thread (a trivial type: no TLS init function)

#define ANVIL_LAUNCH(kernel, grid, block, lds, strm_, ...)                                                  \
  do {                                                                                                      \
    if (::anvil::g_timer.stop && ::anvil::g_timer.stream == (strm_)) {                                      \
      hipEvent_t start_ = ::anvil::g_timer.start;                                                           \
      ::anvil::g_timer.start = nullptr;                                                                     \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, strm_, start_, ::anvil::g_timer.stop, 0, __VA_ARGS__); \
    } else {                                                                                                \
      hipLaunchKernelGGL(kernel, grid, block, lds, strm_, __VA_ARGS__);                                     \
    }                                                                                                       \
  } while (0)

#define ANVIL_LAUNCHED()                                                      \
  do {                                                                        \
    hipError_t e_ = hipGetLastError();                                        \
    if (e_ != hipSuccess) return ::anvil::hip_fail(e_, "kernel launch");      \
  } while (0)

// f(std::integral_constant<int, i>) for i = 0 .. N-1, expanded at compile time: register arrays indexed by i stay in
// registers (a loop the unroller declines would index them dynamically, through scratch).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Row order for the first operand of v_mfma_i32_32x32x32_i8 (the one whose rows become accumulator rows): feeding
// row bperm(c) at operand row c makes accumulator r of lane l hold result row 16 (l / 32) + r, so each lane owns 16
// consecutive rows of its column.
__device__ __forceinline__ int bperm(int c) { return 16 * ((c >> 2) & 1) + 4 * (c >> 3) + (c & 3); }

// the low bytes of four ints, in order, as one dword
__device__ __forceinline__ unsigned pack4(int v0, int v1, int v2, int v3) {
  const unsigned t01 = __builtin_amdgcn_perm((unsigned)v1, (unsigned)v0, 0x0c0c0400u);
  const unsigned t23 = __builtin_amdgcn_perm((unsigned)v3, (unsigned)v2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(t23, t01, 0x05040100u);
}

constexpr unsigned RSRC_DW3 = 0x00020000u;               // raw buffer, 32-bit data format (gfx9 family)
constexpr unsigned OOB = 0xFFFFFFF0u;                    // a buffer offset past any descriptor's range: loads 0

// A raw buffer resource over [base, base + bytes). Its fields pass through readfirstlane: they are uniform, and
// saying so keeps the descriptor in SGPRs (a descriptor the compiler places in VGPRs costs every buffer load a
// waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, int bytes) {
  const unsigned long long a = (unsigned long long)base;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a), hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
  void* p = (void*)(((unsigned long long)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, __builtin_amdgcn_readfirstlane(bytes), RSRC_DW3);
}

// The bytes x_e >> sh (e = 0..3) as one dword: each shift writes its low byte straight into byte lane e (SDWA
// dst_sel), so no separate pack follows. The x_e are clamped beforehand, so each shifted value is its own byte.
__device__ __forceinline__ unsigned sra_pack4(int x0, int x1, int x2, int x3, int sh) {
  unsigned d;
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
      : "=v"(d) : "s"(sh), "v"(x0));
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "s"(sh), "v"(x1));
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "s"(sh), "v"(x2));
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "s"(sh), "v"(x3));
  return d;
}

// median of three: clamp(x, lo, hi) for runtime bounds lo <= hi, written in the form that selects v_med3_i32
__device__ __forceinline__ int med3i(int x, int lo, int hi) { return max(min(x, lo), min(max(x, lo), hi)); }

// a * (byte B of x, zero-extended), a < 2^24: one full-rate SDWA multiply (a 32-bit v_mul_lo_u32 runs at a quarter
// of the rate)
template <int B>
__device__ __forceinline__ unsigned mul_u24_byte(unsigned a, unsigned x) {
  static_assert(B >= 0 && B < 4, "byte lane");
  unsigned d;
  if constexpr (B == 0)
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(d) : "s"(a), "v"(x));
  else if constexpr (B == 1)
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(d) : "s"(a), "v"(x));
  else if constexpr (B == 2)
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(d) : "s"(a), "v"(x));
  else
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(d) : "s"(a), "v"(x));
  return d;
}

// add_requant of packed int8 operands with multipliers below 2^24 in magnitude, r * m + y * n + rnd as
// u * |m| + v * |n| + c: u = r + 128 (the byte of r ^ 0x80) when m >= 0, else 127 - r (the byte of r ^ 0x7F), so that
// r * m = u * |m| - 128 m or u * |m| + 127 m; likewise v for y and n; c = rnd plus both corrections. Every product
// is below 2^32 and the sum is taken modulo 2^32, so it equals the true sum whenever that lies inside int32, as the
// proof of the add ensures.
struct PackedAdd {
  unsigned am, an, xr, xy, c;
  int clo, chi, sh;
  __host__ __device__ static bool applies(int m, int n) {
    return m > -(1 << 24) && m < (1 << 24) && n > -(1 << 24) && n < (1 << 24);
  }
  __device__ PackedAdd(int m, int n, int rnd, int shift) {
    am = m >= 0 ? (unsigned)m : (unsigned)-m;
    an = n >= 0 ? (unsigned)n : (unsigned)-n;
    xr = m >= 0 ? 0x80808080u : 0x7F7F7F7Fu;
    xy = n >= 0 ? 0x80808080u : 0x7F7F7F7Fu;
    c = (unsigned)rnd + (m >= 0 ? 0u - 128u * (unsigned)m : 127u * (unsigned)m) +
        (n >= 0 ? 0u - 128u * (unsigned)n : 127u * (unsigned)n);
    clo = (int)max(-128ll << shift, (long long)INT32_MIN);
    chi = (int)min((128ll << shift) - 1, (long long)INT32_MAX);
    sh = shift;
  }
  // four int8 results clamp((r * m + y * n + rnd) >> shift) of the bytes of r and y, packed (clamp before the shift,
  // then one SDWA shift into each byte lane)
  __device__ __forceinline__ unsigned operator()(unsigned r, unsigned y) const {
    const unsigned ur = r ^ xr, uy = y ^ xy;
    const int o0 = med3i((int)(mul_u24_byte<0>(am, ur) + mul_u24_byte<0>(an, uy) + c), clo, chi);
    const int o1 = med3i((int)(mul_u24_byte<1>(am, ur) + mul_u24_byte<1>(an, uy) + c), clo, chi);
    const int o2 = med3i((int)(mul_u24_byte<2>(am, ur) + mul_u24_byte<2>(an, uy) + c), clo, chi);
    const int o3 = med3i((int)(mul_u24_byte<3>(am, ur) + mul_u24_byte<3>(an, uy) + c), clo, chi);
    return sra_pack4(o0, o1, o2, o3, sh);
  }
};

constexpr long long I32_MIN = -(1ll << 31);
constexpr long long I32_MAX = (1ll << 31) - 1;

inline int dtype_lo(int dt) { return dt == ANVIL_I8 ? -128 : (dt == ANVIL_I16 ? -32768 : INT32_MIN); }
inline int dtype_hi(int dt) { return dt == ANVIL_I8 ? 127 : (dt == ANVIL_I16 ? 32767 : INT32_MAX); }

__device__ __forceinline__ void raise_flag(unsigned* flags, unsigned bit) { atomicOr(flags, bit); }

// requant with every step checked against int32 in the reference's order (anvil/semantics.py:146-155):
// p = acc * M, v = p + 2^(s-1); flag if either leaves int32; r = v >> s (arithmetic), clamped to [lo, hi].
__device__ __forceinline__ int requant_checked(int acc, int mult, int shift, long long rnd, int lo, int hi,
                                               unsigned& bad) {
  long long p = (long long)acc * (long long)mult;
  long long v = p + rnd;
  bad |= (p < I32_MIN) | (p > I32_MAX) | (v < I32_MIN) | (v > I32_MAX);
  long long r = v >> shift;
  r = r < lo ? lo : r;
  r = r > hi ? hi : r;
  return (int)r;
}

__device__ __forceinline__ long long round_term(int s) { return s ? (1ll << (s - 1)) : 0ll; }


// ---- row reductions and per-lane byte arithmetic shared by the row kernels and the GEMM epilogues

// signed byte B of x times signed byte B of w, both selected and sign-extended by the SDWA operands
template <int B>
__device__ __forceinline__ int mul_sbytes(unsigned x, unsigned w) {
  int d;
  if constexpr (B == 0)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:BYTE_0"
        : "=v"(d) : "v"(x), "v"(w));
  else if constexpr (B == 1)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:BYTE_1"
        : "=v"(d) : "v"(x), "v"(w));
  else if constexpr (B == 2)
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2 src1_sel:BYTE_2"
        : "=v"(d) : "v"(x), "v"(w));
  else
    asm("v_mul_i32_i24_sdwa %0, sext(%1), sext(%2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3 src1_sel:BYTE_3"
        : "=v"(d) : "v"(x), "v"(w));
  return d;
}

__device__ __forceinline__ int dpp_sum16(int v) {            // sum over the lane's 16-lane row, in every lane
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);  // row_ror:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  return v;
}

template <int L>
__device__ __forceinline__ int lane_group_sum(int v) {                   // sum over aligned groups of L lanes
  if constexpr (L > 1) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);    // quad_perm [1,0,3,2]
  if constexpr (L > 2) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);    // quad_perm [2,3,0,1]
  if constexpr (L > 4) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);   // row_half_mirror
  if constexpr (L > 8) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);   // row_mirror
  if constexpr (L > 16) v += __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 0x1F);           // lane ^ 16
  if constexpr (L > 32) v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ unsigned sra_pack4v(int x0, int x1, int x2, int x3, int sh) {   // shift per lane
  unsigned d;
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
      : "=v"(d) : "v"(sh), "v"(x0));
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "v"(sh), "v"(x1));
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "v"(sh), "v"(x2));
  asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "v"(sh), "v"(x3));
  return d;
}

__device__ __forceinline__ int mad_i24v(int a, int b, int c) {
  int d;
  asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}


// The shift count of the reference's rsqrt_index (shift the sum of squares right by 2 until it is below the table's
// length n, counting the steps): the fewest k >= 0 with ss >> 2k below n, for 0 <= ss < 2^31, nbits the bit length of
// n. With b the bit length of ss, n 4^k <= ss for k <= (b - 1 - nbits) / 2 and n 4^k > ss for k >= (b - nbits + 1) / 2,
// so k is k0 = max(0, floor((b - nbits + 1) / 2)) or k0 + 1: two compares in place of a loop of up to 15 steps.
__device__ __forceinline__ int rsqrt_shift(int ss, int n, int nbits) {
  const int b = ss == 0 ? 0 : 32 - __builtin_clz((unsigned)ss);
  const int k0 = max(0, (b - nbits + 1) >> 1);
  return k0 + ((ss >> (2 * k0)) >= n ? 1 : 0);
}

}  // namespace anvil
