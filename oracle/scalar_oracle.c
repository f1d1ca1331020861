/* ORACLE (test infrastructure only): scalar C restatement of the reference's graph ops, one element at a time.
 *
 * Independent of oracle/semantics.py (numpy, whole-tensor): these are the per-element loops of the reference's
 * Vortex-V code generator (anvil/vortexv/codegen.py:347-615: k_matmul, k_lut, k_lut_mul, k_add_requant,
 * k_rmsnorm, k_softmax) and of its loop-level lowering (anvil/lower/graph_to_tensor.py:243-398), with the int32
 * contract of anvil/semantics.py checked on every intermediate. Used only by tests/ to cross-check the numpy
 * oracle on the same graphs; never by the product.
 *
 * All tensors are contiguous row-major int64. Every function returns 0, or
 *   1 (ValueError: operand outside its dtype, shift outside [0, 31]), 2 (OverflowError), 3 (ZeroDivisionError).
 */
#include <stdint.h>

#define I32MIN (-2147483648LL)
#define I32MAX 2147483647LL

static int fits32(int64_t v) { return v >= I32MIN && v <= I32MAX; }

static int64_t lo_of(int dt) { return dt == 8 ? -128 : (dt == 16 ? -32768 : I32MIN); }
static int64_t hi_of(int dt) { return dt == 8 ? 127 : (dt == 16 ? 32767 : I32MAX); }

/* requant in the reference's order: chk(acc), chk(acc*M), chk(+2^(s-1)), arithmetic shift, clamp */
static int rq(int64_t acc, int64_t m, int s, int dt, int64_t* out) {
  if (s < 0 || s > 31) return 1;
  if (!fits32(acc)) return 2;
  int64_t p = acc * m;
  if (!fits32(p)) return 2;
  int64_t v = p + (s ? (1LL << (s - 1)) : 0);
  if (!fits32(v)) return 2;
  /* arithmetic shift: floor division by 2^s */
  int64_t r = v >= 0 ? (v >> s) : -((-v + (1LL << s) - 1) >> s);
  if (r < lo_of(dt)) r = lo_of(dt);
  if (r > hi_of(dt)) r = hi_of(dt);
  *out = r;
  return 0;
}

static int in_dt(int64_t v, int dt) { return v >= lo_of(dt) && v <= hi_of(dt); }

/* out[b][i][j] = rq(sum_k a[b][i][k] * w[bb][k][j]) [-> lut[. + 128]], bb = b if b_batched else 0 */
int so_qmatmul(const int64_t* a, const int64_t* w, int64_t* out, int64_t batch, int64_t M, int64_t K, int64_t N,
               int b_batched, int64_t mult, int s, const int64_t* lut, int dt) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < M; ++i)
      for (int64_t j = 0; j < N; ++j) {
        int64_t acc = 0;
        for (int64_t k = 0; k < K; ++k) {
          int64_t x = a[(b * M + i) * K + k], y = w[((b_batched ? b : 0) * K + k) * N + j];
          if (!in_dt(x, 8) || !in_dt(y, 8)) return 1;
          acc += x * y;
        }
        int64_t r;
        int e = rq(acc, mult, s, dt, &r);
        if (e) return e;
        if (lut) {
          if (dt != 8) return 1;
          r = lut[r + 128];
        }
        out[(b * M + i) * N + j] = r;
      }
  return 0;
}

int so_lut(const int64_t* x, const int64_t* table, int64_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    if (!in_dt(x[i], 8)) return 1;
    out[i] = table[x[i] + 128];
  }
  return 0;
}

int so_lut_mul(const int64_t* x, const int64_t* y, const int64_t* table, int64_t* out, int64_t n, int64_t mult,
               int s) {
  for (int64_t i = 0; i < n; ++i) {
    if (!in_dt(x[i], 8) || !in_dt(y[i], 8)) return 1;
    int e = rq(table[x[i] + 128] * y[i], mult, s, 8, &out[i]);
    if (e) return e;
  }
  return 0;
}

int so_add_requant(const int64_t* a, const int64_t* b, int64_t* out, int64_t n, int64_t ma, int64_t mb, int s,
                   int dt) {
  for (int64_t i = 0; i < n; ++i) {
    if (!in_dt(a[i], 16) || !in_dt(b[i], 16)) return 1;
    int64_t pa = a[i] * ma, pb = b[i] * mb;
    if (!fits32(pa) || !fits32(pb) || !fits32(pa + pb)) return 2;
    int e = rq(pa + pb, 1, s, dt, &out[i]);
    if (e) return e;
  }
  return 0;
}

/* per row: ss = e + sum((x^2 + 2^(c-1)) >> c); shift ss by 2 until below n (k steps); out = rq(x*w*lut[ss], M, s+k) */
int so_rmsnorm(const int64_t* x, const int64_t* w, const int64_t* lut, int64_t n, int64_t* out, int64_t rows,
               int64_t d, int64_t mult, int s, int c, int64_t e, int xdt) {
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t* xr = x + r * d;
    int64_t ss = 0;
    for (int64_t j = 0; j < d; ++j) {
      if (!in_dt(xr[j], xdt)) return 1;
      int64_t sq = xr[j] * xr[j];
      if (!fits32(sq)) return 2;
      if (c) {
        sq += 1LL << (c - 1);
        if (!fits32(sq)) return 2;
        sq >>= c;
      }
      ss += sq;
    }
    ss += e;
    if (!fits32(ss)) return 2;
    int k = 0;
    while (ss >= n) {
      ss >>= 2;
      ++k;
    }
    for (int64_t j = 0; j < d; ++j) {
      int64_t xw = xr[j] * w[j];
      if (!fits32(xw)) return 2;
      int64_t xwr = xw * lut[ss];
      if (!fits32(xwr)) return 2;
      int err = rq(xwr, mult, s + k, 8, &out[r * d + j]);
      if (err) return err;
    }
  }
  return 0;
}

static int64_t floordiv(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

/* per row i of (batch, t1, t2): kept j < min(i+1, t2) when causal; max from -128; e = lut[x - m + 255];
 * p = (e*one + S//2) // S; masked p = 0 */
int so_softmax(const int64_t* x, const int64_t* lut, int64_t* out, int64_t batch, int64_t t1, int64_t t2,
               int64_t one, int causal, int dt) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < t1; ++i) {
      const int64_t* xr = x + (b * t1 + i) * t2;
      int64_t* o = out + (b * t1 + i) * t2;
      int64_t kept = causal ? (i + 1 < t2 ? i + 1 : t2) : t2;
      int64_t m = -128;
      for (int64_t j = 0; j < kept; ++j) {
        if (!in_dt(xr[j], 8)) return 1;
        if (xr[j] > m) m = xr[j];
      }
      int64_t S = 0;
      for (int64_t j = 0; j < kept; ++j) S += lut[xr[j] - m + 255];
      if (!fits32(S)) return 2;
      if (S == 0) return 3;
      int64_t half = floordiv(S, 2);
      for (int64_t j = 0; j < t2; ++j) {
        if (j >= kept) {
          o[j] = 0;
          continue;
        }
        int64_t num = lut[xr[j] - m + 255] * one + half;
        if (!fits32(num)) return 2;
        int64_t p = floordiv(num, S);
        if (!in_dt(p, dt)) return 1;
        o[j] = p;
      }
    }
  return 0;
}
