/* anvil_mi355x.h: C ABI of the MI355X (gfx950) backend for Anvil's int8 graph ops.
 *
 * One entry point per graph op of the reference interpreter, plus lifecycle, memory and timing calls. Every
 * signature uses plain pointers, sizes and ints (no torch types), so a ctypes / cffi / cgo binding is a
 * one-to-one declaration. The reference is Python: these replace the numpy evaluation of each op in
 * anvil/interp/graph.py:52-91 (through anvil/semantics.py), and the backend dispatch of
 * anvil/runtime/api.py:127-141 / anvil/driver.py:305-322.
 *
 * Conventions
 *   - Every call returns ANVIL_OK (0) or an error code; anvil_last_error() returns the calling thread's message.
 *   - Device pointers come from anvil_alloc (or any HIP allocation on the context's device). Op calls are
 *     asynchronous on the context's stream; argument errors are reported at the call, int32-contract
 *     violations found on the device (the reference's OverflowError / ValueError / ZeroDivisionError) are
 *     reported by the next anvil_sync on that context.
 *   - Element strides are in elements, int64. Tensors are row-major; the last dim of every operand is
 *     contiguous unless a stride says otherwise.
 *   - dtypes: ANVIL_I8, ANVIL_I16, ANVIL_I32 (int8_t, int16_t, int32_t elements).
 *   - A context is used by one host thread at a time; distinct contexts may run concurrently.
 */
#ifndef ANVIL_MI355X_H
#define ANVIL_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum anvil_status {
  ANVIL_OK = 0,
  ANVIL_E_VALUE = 1,      /* bad argument or value outside its dtype: Python ValueError            */
  ANVIL_E_OVERFLOW = 2,   /* an int32 intermediate left int32: Python OverflowError                */
  ANVIL_E_ZERODIV = 3,    /* a softmax row summed to zero: Python ZeroDivisionError                */
  ANVIL_E_RUNTIME = 4,    /* HIP runtime failure: Python RuntimeError                              */
};

enum anvil_dtype { ANVIL_I8 = 1, ANVIL_I16 = 2, ANVIL_I32 = 4 };

typedef struct anvil_ctx anvil_ctx;

/* ------------------------------------------------------------------------------------------ lifecycle */
const char* anvil_last_error(void);
int anvil_version(void);
/* Create a context on HIP device `device` with its own stream (default priority). */
int anvil_init(int device, anvil_ctx** out);
int anvil_destroy(anvil_ctx* ctx);
/* Wait for the context's stream, then report (and clear) any device-side contract violation. */
int anvil_sync(anvil_ctx* ctx);

/* ------------------------------------------------------------------------------------------- memory */
int anvil_alloc(anvil_ctx* ctx, size_t bytes, void** dptr);
int anvil_free(anvil_ctx* ctx, void* dptr);
/* Page-locked host memory (hipHostMalloc) for downloads that go straight to it over DMA. No counterpart in the
 * reference (its values never leave the host): the read-back side of CompiledModel.run (anvil/driver.py:305-322)
 * downloads into it. anvil_host_free waits for the context's stream first. */
int anvil_host_alloc(anvil_ctx* ctx, size_t bytes, void** hptr);
int anvil_host_free(anvil_ctx* ctx, void* hptr);
/* Host <-> device copies on the context's stream; they complete before the call returns. */
int anvil_upload(anvil_ctx* ctx, void* dst, const void* src, size_t bytes);
int anvil_download(anvil_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Zero `bytes` of device memory with a fill kernel (safe inside a captured graph). */
int anvil_zero(anvil_ctx* ctx, void* dst, size_t bytes);

/* ------------------------------------------------------------------------------------------ HIP graphs */
/* No counterpart in the reference (its interpreter runs each op as it walks the graph): the device-side form of a
 * repeated CompiledModel.run forward (anvil/driver.py:305-322). anvil_graph_begin starts capturing the launches issued
 * on the context's stream (relaxed mode); the op entry points called until anvil_graph_end are recorded, not run.
 * anvil_graph_end instantiates them into *graph, an executable graph that anvil_graph_launch replays on the stream
 * (with the arguments they were recorded with), and anvil_graph_destroy frees after waiting for the stream. Between
 * begin and end, call only op entry points whose workspace is already allocated (run the same calls once first):
 * anvil_upload, anvil_download, anvil_sync and a first-use allocation end the capture with an error. The library's
 * kernels clear memory with fill kernels, never hipMemsetAsync, so a captured graph holds kernel nodes only. */
int anvil_graph_begin(anvil_ctx* ctx);
int anvil_graph_end(anvil_ctx* ctx, void** graph);
int anvil_graph_launch(anvil_ctx* ctx, void* graph);
int anvil_graph_destroy(anvil_ctx* ctx, void* graph);

/* -------------------------------------------------------------------------------------------- timing */
/* Events on the context's stream, in 512 slots: record two, then read the elapsed milliseconds between them. They
 * time work only: they are created without the system-scope fence (hipEventDisableSystemFence), so waiting on one
 * does not make device memory visible to the host (anvil_sync and the copies do). */
int anvil_event_record(anvil_ctx* ctx, int slot);
int anvil_event_elapsed(anvil_ctx* ctx, int slot0, int slot1, float* ms);
/* Kernel-bound timing (no reference counterpart: the reference times ops in simulator cycles, anvil/driver.py:
 * 313-319). Until disarmed, the kernels this host thread launches on the context's stream carry the events of
 * slot0 and slot1 inside their dispatch (hipExtLaunchKernel): slot0 marks the first such kernel's start, slot1 the
 * last one's end, so anvil_event_elapsed(slot0, slot1) spans the kernels alone, without the dispatch gap or event
 * packets that anvil_event_record brackets. anvil_time_kernels(ctx, -1, -1) disarms. */
int anvil_time_kernels(anvil_ctx* ctx, int slot0, int slot1);

/* ------------------------------------------------------------------------------------------------ ops */

/* qmatmul / qlinear (reference anvil/semantics.py:95-103 via anvil/interp/graph.py:62-64):
 *   C[b0][b1][m][n] = epilogue( sum_k A[b0][b1][m][k] * Bt[b0][b1][n][k] )
 *   epilogue: r = clamp_out((acc * mult + 2^(shift-1)) >> shift), then lut[r + 128] when lut != NULL.
 * A and Bt are int8 with their K dim contiguous (Bt is the right operand transposed: a (K, N) weight is
 * stored (N, K) once at upload; a head-batched kT operand is the K-contiguous rows of k). strides holds
 *   {sa0, sa1, lda, sb0, sb1, ldb, sc0, sc1, ldc}  (batch-0, batch-1 and row strides of A, Bt, C).
 * out_dtype ANVIL_I8 or ANVIL_I16 (no LUT with I16). mult may be negative; shift in [0, 31]. */
int anvil_gemm_i8(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1, int M,
                  int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut, int out_dtype);

/* anvil_gemm_i8 with execution flags (same reference op, anvil/semantics.py:95-103):
 *   ANVIL_GEMM_UNCHECKED    the caller has proven every acc * mult + round fits int32 (the reference quantizer's
 *                           prove_no_overflow, anvil/frontend/quantize.py:175-253): the epilogue skips the
 *                           64-bit checks. Without it, a value outside int32 is reported by anvil_sync.
 *   ANVIL_GEMM_CAUSAL_SKIP  output tiles whose every column exceeds every row (n > m) are not computed: only for a
 *                           result read by causal softmaxes alone, which never read those entries.
 *   ANVIL_GEMM_CAUSAL_K     A[m][k] is zero for k > m (a causal softmax output): the K loop of a row tile stops at
 *                           its last row, which leaves every result unchanged.
 *   ANVIL_GEMM_MUL24        (with UNCHECKED) every |acc| and |mult| is below 2^23, so the requant product is one
 *                           24-bit multiply.
 *   ANVIL_GEMM_SPLITK       (with UNCHECKED, batch 1, no causal mode) split K into up to four chunks: one launch
 *                           stores each (output tile, chunk)'s int32 partial sums in a workspace, a second one adds them
 *                           up and requantizes. Integer addition is exact, so the result is the same; the library picks
 *                           it by itself for products with few output tiles (M = 256), the flag forces it. The
 *                           workspace (one 128 x 128 int32 partial tile per output tile and chunk) belongs to the
 *                           context, allocated on first use.
 *   ANVIL_GEMM_A_KBLOCK     (with UNCHECKED) A is K-blocked: the 64-byte K block j of row r (its K bytes 64 j ..
 *                           64 j + 63) sits at A + r * 64 + j * strides[2] (plus the batch strides), so one block of
 *                           consecutive rows is contiguous and a tile's operand loads read whole cache lines.
 *   ANVIL_GEMM_B_KBLOCK     (with UNCHECKED) the same for Bt, with strides[5] the block stride.
 *   ANVIL_GEMM_C_KBLOCK     (with UNCHECKED) the result is written K-blocked, for a product that reads it as its A
 *                           operand: result (m, n) at C + (m * 64 + (n / 64) * strides[8] + n % 64) * itemsize.
 *                           Both need 16-byte aligned operands, K a multiple of 16 and a block stride that is a
 *                           multiple of 16; the results are those of the row-major operands. */
enum anvil_gemm_flags {
  ANVIL_GEMM_UNCHECKED = 1,
  ANVIL_GEMM_CAUSAL_SKIP = 2,
  ANVIL_GEMM_CAUSAL_K = 4,
  ANVIL_GEMM_MUL24 = 8,
  ANVIL_GEMM_SPLITK = 16,
  ANVIL_GEMM_A_KBLOCK = 32,
  ANVIL_GEMM_B_KBLOCK = 64,
  ANVIL_GEMM_C_KBLOCK = 128,
  ANVIL_GEMM_NORM_S24 = 256     /* anvil_gemm_i8_add_norm only: |rsqrt table entry x norm mult| < 2^23 */
};
int anvil_gemm_i8_ex(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1, int M,
                     int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut, int out_dtype,
                     int flags);

/* anvil_gemm_i8_ex that allocates nothing. It has no counterpart in the reference: it is for callers that cannot
 * allocate device memory at call time, such as code under HIP graph capture or a tight serving loop. Same arguments
 * and results as anvil_gemm_i8_ex; where anvil_gemm_i8_ex would split K into its context workspace (allocated on
 * first use), this keeps the partial tiles in a static per-device scratch of 2^22 int32 (16 MiB, held by each device
 * the library runs on until the process ends) and fails with ANVIL_E_VALUE when the split needs more (128 x 128
 * output tiles x K chunks x 16384 sums). Calls on one context run in its stream's order and never overlap; the
 * scratch of a device belongs to the first context whose call splits into it, until anvil_destroy of that context,
 * and a split-K call from any other context fails with ANVIL_E_RUNTIME instead of racing on it. */
int anvil_gemm_i8_noalloc(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1, int M,
                          int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut,
                          int out_dtype, int flags);

/* The number of int32 partial sums the context's split-K workspace holds: 0 until an anvil_gemm_i8_ex product splits
 * K, then the largest split so far (the workspace grows and is never shrunk before anvil_destroy). */
int anvil_workspace_sums(anvil_ctx* ctx, long long* sums);

/* The arguments of one anvil_gemm_i8_ex call. */
typedef struct anvil_gemm_desc {
  const int8_t* A;
  const int8_t* Bt;
  void* C;
  const int8_t* lut;
  int64_t strides[9];
  int32_t batch0, batch1, M, N, K;
  int32_t mult, shift, out_dtype, flags;
} anvil_gemm_desc;

/* 1 to 4 independent qmatmul / qlinear ops, each computed exactly as anvil_gemm_i8_ex computes it (the reference
 * evaluates them one op at a time, anvil/interp/graph.py:62-64 with anvil/semantics.py:95-103; q, k and v of one
 * attention read one input and nothing of each other). Every member is validated before anything is launched.
 * Members that all take the same kernel run as one launch (one tail instead of one per product), others one launch
 * each. No member may write memory that another member reads or writes. */
int anvil_gemm_i8_group(anvil_ctx* ctx, const anvil_gemm_desc* descs, int count);

/* The rmsnorm that follows a fused add (below), fused too (anvil_gemm_i8_add_norm): H = rmsnorm_int(D, w, lut, mult,
 * shift) over D's rows (reference anvil/semantics.py:164-182 with ss_shift = ss_init = 0). H is M x N int8, row-major
 * with row stride ld (kb = 0), or K-blocked (ld = 64, kb the 64-column block stride, kb >= 64 M). */
typedef struct anvil_norm_epilogue {
  const int8_t* w;        /* N weights */
  const int32_t* lut;     /* lut_len entries, >= 0 */
  int lut_len;
  int32_t mult;
  int shift;
  int8_t* out;
  int64_t ld;
  int64_t kb;
} anvil_norm_epilogue;

/* A qlinear / qmatmul whose int8 result y feeds an add_requant with an int8 residual R, fused in the GEMM's
 * epilogue (reference anvil/semantics.py:95-103, then add_requant :106-115):
 *   y = clamp_i8((acc * mult + 2^(shift-1)) >> shift) [-> lut];  D = clamp_i8((R * ma + y * mb + 2^(shift2-1)) >> shift2)
 * D (and R) have C's dims; rstrides = {sr0, sr1, ldr, sd0, sd1, ldd}. y is also written to C unless C is NULL.
 * flags must hold ANVIL_GEMM_UNCHECKED (every intermediate of both ops proven in int32; ANVIL_GEMM_MUL24 allowed, no
 * causal mode); A and Bt 16-byte aligned with K and their row strides multiples of 16. */
int anvil_gemm_i8_add(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, int8_t* C, int batch0, int batch1, int M,
                      int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut,
                      const int8_t* R, int32_t ma, int32_t mb, int shift2, int8_t* D, const int64_t* rstrides,
                      int flags);

/* anvil_gemm_i8_add (batch 1) whose sum D also feeds an rmsnorm_int (the block's h2 = rmsnorm(r1); reference
 * anvil/semantics.py:95-103, then add_requant :106-115, then rmsnorm_int :164-182), fused in the same epilogue: D and
 * H = rmsnorm_int(D) are written, y too unless C is NULL. Each workgroup's 128 x N tile spans whole rows, so N must be
 * 128 or 256 and M a multiple of 128. flags: ANVIL_GEMM_UNCHECKED (every intermediate of the three ops proven in
 * int32) and ANVIL_GEMM_NORM_S24 (|lut[i] x norm->mult| < 2^23 for every entry), ANVIL_GEMM_MUL24 and the K-block
 * flags allowed, no causal mode or split-K; |ma|, |mb| < 2^24; operands, results and their row strides 16-byte
 * aligned. One launch in place of the product's and the rmsnorm's. */
int anvil_gemm_i8_add_norm(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, int8_t* C, int M, int N, int K,
                           const int64_t* strides, int32_t mult, int shift, const int8_t* lut, const int8_t* R,
                           int32_t ma, int32_t mb, int shift2, int8_t* D, const int64_t* rstrides,
                           const anvil_norm_epilogue* norm, int flags);

/* anvil_gemm_i8_add with the result dtype as an argument (ADR-004's wide residual stream, reference
 * docs/decisions/ADR-004-small-inputs.md:59-82 and anvil/semantics.py:106-115): y, R and D are all out_dtype, ANVIL_I8
 * or ANVIL_I16 (no LUT with i16), D = clamp_out((R * ma + y * mb + 2^(shift2-1)) >> shift2). Same conditions as
 * anvil_gemm_i8_add. */
int anvil_gemm_i8_add_ex(anvil_ctx* ctx, const int8_t* A, const int8_t* Bt, void* C, int batch0, int batch1, int M,
                         int N, int K, const int64_t* strides, int32_t mult, int shift, const int8_t* lut, int out_dtype,
                         const void* R, int32_t ma, int32_t mb, int shift2, void* D, const int64_t* rstrides,
                         int flags);

/* rmsnorm_int over rows of `cols` elements (reference anvil/semantics.py:158-182, golden.rmsnorm_int):
 *   ss = ss_init + sum_j ((x_j^2 + 2^(ss_shift-1)) >> ss_shift); (i, k) = rsqrt_index(ss, lut_len);
 *   out_j = clamp_i8((x_j * w_j * lut[i] * mult + 2^(shift+k-1)) >> (shift + k)).
 * x is ANVIL_I8 or ANVIL_I16, contiguous rows; w int8[cols]; lut int32[lut_len]; out int8. */
int anvil_rmsnorm_int(anvil_ctx* ctx, const void* x, int x_dtype, const int8_t* w, const int32_t* lut, int lut_len,
                      int32_t mult, int shift, int ss_shift, int32_t ss_init, int64_t rows, int cols, int8_t* out);

/* Execution flags of the row ops' _ex entry points:
 *   ANVIL_OP_UNCHECKED  the caller has proven every int32 intermediate of the op in range (the reference quantizer's
 *                       prove_no_overflow, anvil/frontend/quantize.py:175-253); for softmax_lut also that every lut
 *                       entry is >= 0 and lut[255] >= 1 (so no row sums to zero). The op may then run a kernel
 *                       without the 64-bit range checks; without the flag, violations are reported by anvil_sync. */
enum anvil_op_flags { ANVIL_OP_UNCHECKED = 1 };

/* anvil_rmsnorm_int with flags (same reference op, anvil/semantics.py:158-182). ANVIL_RMS_S24 (with
 * ANVIL_OP_UNCHECKED) adds that every |lut[i] * mult| is below 2^23: each element's x w lut[i] mult + rnd is then one
 * 24-bit multiply-add. ANVIL_RMS_OUT_KBLOCK writes the result K-blocked for a GEMM that reads it as a K-blocked
 * operand (ANVIL_GEMM_A_KBLOCK / B_KBLOCK with block stride rows * 64): out_j of row r at out + (j / 64) * rows * 64 +
 * r * 64 + j % 64; cols must be a multiple of 64. */
enum anvil_rms_flags { ANVIL_RMS_S24 = 2, ANVIL_RMS_OUT_KBLOCK = 4 };
int anvil_rmsnorm_int_ex(anvil_ctx* ctx, const void* x, int x_dtype, const int8_t* w, const int32_t* lut,
                         int lut_len, int32_t mult, int shift, int ss_shift, int32_t ss_init, int64_t rows, int cols,
                         int8_t* out, int flags);

/* softmax_lut over the last axis of (batch, t1, t2) (reference anvil/lower/graph_to_tensor.py:352-398,
 * golden.softmax_lut): kept_j = (j <= i) if causal else 1; m = max(-128, max kept x);
 * e_j = lut[x_j - m + 255] (kept) else 0; S = sum e; p_j = (e_j * one + S / 2) / S.
 * x int8 contiguous; lut int32[256]; out ANVIL_I8 (one <= 127) or ANVIL_I32. */
int anvil_softmax_lut(anvil_ctx* ctx, const int8_t* x, const int32_t* lut, int32_t one, int causal, int64_t batch,
                      int t1, int t2, void* out, int out_dtype);

/* anvil_softmax_lut with flags (same reference op, anvil/lower/graph_to_tensor.py:352-398). */
int anvil_softmax_lut_ex(anvil_ctx* ctx, const int8_t* x, const int32_t* lut, int32_t one, int causal, int64_t batch,
                         int t1, int t2, void* out, int out_dtype, int flags);

/* The attention chain of a proven graph, fused (reference anvil/interp/graph.py:62-73 evaluating
 * qmatmul -> softmax_lut -> qmatmul through anvil/semantics.py:95-103 and the three-stage softmax of
 * anvil/lower/graph_to_tensor.py:352-398), per (b0, b1) of batch0 x batch1 heads:
 *   scores = clamp_i8((Q K^T * m_s + 2^(s_s-1)) >> s_s);  p = softmax_lut(scores, lut, one, causal) (int8);
 *   O      = clamp_i8((p V * m_o + 2^(s_o-1)) >> s_o)
 * bit-exact with the three ops, without writing scores or p. Q, K: (T, D) rows; Vt: V transposed, (D, T) rows;
 * O: (T, D) rows. strides = {sq0, sq1, ldq, sk0, sk1, ldk, sv0, sv1, ldv, so0, so1, ldo} in elements (bytes): the
 * first nine and Q, K, Vt multiples of 16, the O strides and O multiples of 4; ldk >= D, ldv >= T, ldo >= D, and
 * T * ldk, D * ldv, 32 * ldo below 2^31 (one head of K and of Vt is read, and 32 rows of O are written, through
 * 32-bit offsets). T a multiple of 32 in [32, 1024];
 * D in {16, 32, 64, 128}; 1 <= one <= 127; lut int32[256] with every entry >= 0 and lut[255] >= 1.
 * T may also be 16, with D 16 or 32 (one lane a query row); then ANVIL_ATTN_V_ROWS passes V itself, (T, D) rows of
 * stride ldv >= D, in place of V^T.
 * flags must hold ANVIL_OP_UNCHECKED: the caller has proven every int32 intermediate of the three ops in range;
 * ANVIL_ATTN_S24 adds that every |Q K^T| and |m_s| is below 2^23 (the score requant multiply is then 24-bit). */
enum anvil_attn_flags { ANVIL_ATTN_S24 = 2, ANVIL_ATTN_V_ROWS = 4 };
int anvil_attention_i8(anvil_ctx* ctx, const int8_t* Q, const int8_t* K, const int8_t* Vt, int8_t* O, int batch0,
                       int batch1, int T, int D, const int64_t* strides, int32_t m_s, int s_s, const int32_t* lut,
                       int32_t one, int causal, int32_t m_o, int s_o, int flags);

/* The same chain with its intermediate values kept (reference anvil/interp/graph.py:43-92 returns every value of the
 * graph, the scores of anvil/semantics.py:95-103 and the probabilities of anvil/lower/graph_to_tensor.py:352-398
 * among them): anvil_attention_i8, which also stores the whole T x T int8 score matrix into S and the probabilities
 * into P (0 for masked keys), per (b0, b1). strides = the twelve of anvil_attention_i8, then {ss0, ss1, lds} of S
 * and {sp0, sp1, ldp} of P, all multiples of 16, with lds, ldp >= T and 32 * lds, 32 * ldp below 2^31; S and P
 * 16-byte aligned. Same preconditions and flags. */
int anvil_attention_i8_keep(anvil_ctx* ctx, const int8_t* Q, const int8_t* K, const int8_t* Vt, int8_t* O, int8_t* S,
                            int8_t* P, int batch0, int batch1, int T, int D, const int64_t* strides, int32_t m_s,
                            int s_s, const int32_t* lut, int32_t one, int causal, int32_t m_o, int s_o, int flags);

/* add_requant (reference anvil/semantics.py:106-115, golden.residual_add):
 *   out = clamp_out((a * ma + b * mb + 2^(shift-1)) >> shift), a and b ANVIL_I8 or ANVIL_I16, n elements. */
int anvil_add_requant(anvil_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype, int32_t ma, int32_t mb,
                      int shift, int64_t n, void* out, int out_dtype);
/* anvil_add_requant with flags (reference anvil/semantics.py:106-115, anvil/interp/graph.py:65-66): flags 0 keeps the
 * reference's int32 checks (an overflow makes the next anvil_sync return ANVIL_E_OVERFLOW); ANVIL_OP_UNCHECKED states
 * that the caller has proven a * ma + b * mb + 2^(shift-1) inside int32 for every element (the quantizer's
 * prove_no_overflow, anvil/frontend/quantize.py:235-238), and the sum is computed in 32 bits. 16-byte aligned
 * operands run 16 elements a lane. */
int anvil_add_requant_ex(anvil_ctx* ctx, const void* a, int a_dtype, const void* b, int b_dtype, int32_t ma,
                         int32_t mb, int shift, int64_t n, void* out, int out_dtype, int flags);

/* lut (reference anvil/semantics.py:87-92): out = table[x + 128], int8, n elements. */
int anvil_lut_i8(anvil_ctx* ctx, const int8_t* x, const int8_t* table, int64_t n, int8_t* out);

/* lut_mul (golden.swiglu_lut via anvil/interp/graph.py:67-68): out = requant(table[x + 128] * y, mult, shift). */
int anvil_lut_mul(anvil_ctx* ctx, const int8_t* x, const int8_t* y, const int8_t* table, int32_t mult, int shift,
                  int64_t n, int8_t* out);
/* anvil_lut_mul with flags (same op): flags 0 keeps the reference's int32 checks; ANVIL_OP_UNCHECKED states that
 * table[x + 128] * y * mult + 2^(shift-1) is proven inside int32 (anvil/frontend/quantize.py:206-210). */
int anvil_lut_mul_ex(anvil_ctx* ctx, const int8_t* x, const int8_t* y, const int8_t* table, int32_t mult, int shift,
                     int64_t n, int8_t* out, int flags);

/* transpose / reshape (reference anvil/interp/graph.py:76-81) when a consumer needs a view laid out densely:
 * dst (contiguous, dims[0..rank)) = src viewed with element strides src_strides. elem_size 1, 2 or 4; rank <= 6. */
int anvil_copy_strided(anvil_ctx* ctx, const void* src, void* dst, int elem_size, int rank, const int64_t* dims,
                       const int64_t* src_strides);

/* CompiledModel.quantize_input (reference anvil/driver.py:233-241): out = clamp_out(rint(x / scale)), round half
 * to even, x float32 or float64 (x_is_f64), out ANVIL_I8 or ANVIL_I16. A NaN or infinite x (which the reference
 * refuses, driver.py:265-266) stores 0 and makes the next anvil_sync return ANVIL_E_VALUE. */
int anvil_quantize(anvil_ctx* ctx, const void* x, int x_is_f64, double scale, int64_t n, void* out, int out_dtype);

/* The float prelude of a token model, on the device: rows = batch * T token ids (int64), float32 tables wte
 * (vocab, C) and wpe (>= T, C); out[r][c] = clamp_out(rint((wte[ids[r]][c] + wpe[r % T][c]) / scale)) in float64,
 * round half to even, ANVIL_I8 or ANVIL_I16. It replaces the host's x = wte[ids] + wpe[positions] (float64) followed
 * by CompiledModel.quantize_input (reference anvil/driver.py:233-241). An id outside [0, vocab) is reported by
 * anvil_sync as ANVIL_E_VALUE. */
int anvil_embed_quantize(anvil_ctx* ctx, const int64_t* ids, int64_t rows, int T, int C, const float* wte, int vocab,
                         const float* wpe, double scale, void* out, int out_dtype);

#ifdef __cplusplus
}
#endif
#endif /* ANVIL_MI355X_H */
