"""nanoGPT-style int8 blocks: float weights, float calibration forward, and the quantized anvil.graph they lower to.

The graph follows the reference quantizer's recipe (anvil/frontend/quantize.py:338-493) node by node for the
block structure the reference's graph builders use (anvil/frontend/from_image.py:41-69,
tests/model/test_multihead_ir.py:17-44), with a GELU MLP in place of SwiGLU:

    h1 = rmsnorm(x); q, k, v = qlinear(h1); qh/kh/vh = split heads (reshape + transpose [1, 0, 2]);
    kT = transpose(kh, [0, 2, 1]); scores = qmatmul(qh, kT) (1/sqrt(d) folded into M); p = softmax_lut(causal);
    o = qmatmul(p, vh); om = merge heads (transpose + reshape); y = qlinear(om); r1 = add(x, y);
    h2 = rmsnorm(r1); fc = qlinear(h2, lut=GELU) (or qlinear, then lut); proj = qlinear(fc); out = add(r1, proj)

The reference IR has no LayerNorm: the "LayerNorm" of the block specs is its integer RMSNorm (rmsnorm_int), the
only normalisation anvil.interp defines. GELU is an int8 LUT built like the reference's SiLU LUT.

Scales: inputs max-abs / 127 of the calibration inputs; every other activation headroom * max-abs / 127 of its
float value on the fake-quantized calibration inputs (causal scores only where the mask keeps them); weights
max-abs / 127 per tensor; requant (M, s) from fixed_point against the worst case over all int8 inputs.
"""
from __future__ import annotations

import hashlib
import inspect
import json
import math
from dataclasses import asdict, dataclass, field
from pathlib import Path

import numpy as np

from . import ir as g
from . import quantize as Q

EPS = 1e-5


@dataclass(frozen=True)
class BlockSpec:
    n_embd: int
    n_head: int
    seq: int
    layers: int = 1
    vocab: int = 0                       # > 0: token ids -> embeddings (host) and a tied logits head
    gelu: str = "fused"                  # "fused": fc's qlinear LUT epilogue; "lut": qlinear then a lut op
    causal: bool = True
    wseed: int = 0                       # weight seed
    calib_batches: int = 8
    calib_batch: int = 1                 # sequences per calibration batch
    headroom: float = Q.HEADROOM

    @property
    def head_dim(self):
        return self.n_embd // self.n_head

    @property
    def hidden(self):
        return 4 * self.n_embd


# ----------------------------------------------------------------------------------------- float model

def init_params(spec: BlockSpec) -> dict:
    """Float weights: linears N(0, 0.02) as nn.Linear (out, in); RMSNorm weights U(0.5, 1.5); embeddings N(0, 0.02)."""
    rng = np.random.default_rng(spec.wseed)
    C, F = spec.n_embd, spec.hidden
    p = {}
    if spec.vocab:
        p["wte"] = rng.normal(0, 0.02, (spec.vocab, C)).astype(np.float32)
        p["wpe"] = rng.normal(0, 0.02, (spec.seq, C)).astype(np.float32)
    for i in range(spec.layers):
        L = f"L{i}." if spec.layers > 1 or spec.vocab else ""
        p[L + "ln1"] = rng.uniform(0.5, 1.5, C).astype(np.float32)
        for n in ("q", "k", "v", "y"):
            p[L + n] = rng.normal(0, 0.02, (C, C)).astype(np.float32)
        p[L + "ln2"] = rng.uniform(0.5, 1.5, C).astype(np.float32)
        p[L + "fc"] = rng.normal(0, 0.02, (F, C)).astype(np.float32)
        p[L + "proj"] = rng.normal(0, 0.02, (C, F)).astype(np.float32)
    if spec.vocab:
        p["lnf"] = rng.uniform(0.5, 1.5, C).astype(np.float32)
    return p


def _prefixes(spec):
    return [f"L{i}." if spec.layers > 1 or spec.vocab else "" for i in range(spec.layers)]


def embed(spec: BlockSpec, params, ids):
    """Token + position embeddings in float64 on the host (ids (N, T) ints in [0, vocab))."""
    ids = np.asarray(ids)
    return params["wte"].astype(np.float64)[ids] + params["wpe"].astype(np.float64)[None, : ids.shape[-1]]


def gelu(x):
    """GELU, erf form (torch.nn.GELU's default), in float64."""
    from scipy.special import erf
    return 0.5 * x * (1 + erf(np.asarray(x, dtype=np.float64) / math.sqrt(2)))


def _rms(x, w):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + np.float32(EPS)) * w


def float_forward_amax(spec: BlockSpec, params, x, amax: dict):
    """Float32 forward of the block stack on x (N, T, C); folds max |activation| per graph sym into amax."""
    C, H, T = spec.n_embd, spec.n_head, spec.seq
    d = C // H
    keep = np.tril(np.ones((T, T), dtype=bool))
    neg = np.float32(-np.inf)

    def rec(k, v):
        amax[k] = max(amax.get(k, 0.0), float(np.abs(v).max()))

    x = x.astype(np.float32)
    for L in _prefixes(spec):
        h1 = _rms(x, params[L + "ln1"])
        rec(L + "h1", h1)
        q, k, v = (h1 @ params[L + n].T for n in ("q", "k", "v"))
        for n, t in (("q", q), ("k", k), ("v", v)):
            rec(L + n, t)
        N = x.shape[0]
        qh = q.reshape(N, T, H, d).transpose(0, 2, 1, 3)
        kh = k.reshape(N, T, H, d).transpose(0, 2, 1, 3)
        vh = v.reshape(N, T, H, d).transpose(0, 2, 1, 3)
        sc = (qh @ kh.transpose(0, 1, 3, 2)) * np.float32(1.0 / math.sqrt(d))
        if spec.causal:
            rec(L + "scores", np.where(keep, sc, 0))
            sc = np.where(keep, sc, neg)
        else:
            rec(L + "scores", sc)
        sc = sc - sc.max(-1, keepdims=True)
        e = np.exp(sc)
        p = e / e.sum(-1, keepdims=True)
        o = p @ vh
        rec(L + "o", o)
        om = o.transpose(0, 2, 1, 3).reshape(N, T, C)
        y = om @ params[L + "y"].T
        rec(L + "y", y)
        r1 = x + y
        rec(L + "r1", r1)
        h2 = _rms(r1, params[L + "ln2"])
        rec(L + "h2", h2)
        fc = h2 @ params[L + "fc"].T
        rec(L + "fc", fc)
        ge = gelu(fc).astype(np.float32)
        rec(L + "gelu", ge)
        proj = ge @ params[L + "proj"].T
        rec(L + "proj", proj)
        x = r1 + proj
        rec(L + "out", x)
    if spec.vocab:
        hf = _rms(x, params["lnf"])
        rec("hf", hf)
        rec("logits", hf @ params["wte"].T)


def device_params(params, device):
    """The float weights on a torch device as float32: (weights, transposed 2-D weights, contiguous)."""
    import torch
    W = {k: torch.as_tensor(np.ascontiguousarray(v), dtype=torch.float32, device=device) for k, v in params.items()}
    return W, {k: v.t().contiguous() for k, v in W.items() if v.dim() == 2}      # x @ w.T as x @ (w.T, contiguous)


def float_forward_amax_torch(spec: BlockSpec, W, Wt, x, amax: dict, device):
    """float_forward_amax with the forward on a torch device (weights from device_params): float32 throughout, GELU
    in float64 as on the host. The same max-abs values up to float32 rounding of the products and reductions."""
    import torch
    C, H, T = spec.n_embd, spec.n_head, spec.seq
    d = C // H
    f32 = dict(dtype=torch.float32, device=device)
    keep = torch.ones((T, T), dtype=torch.bool, device=device).tril()
    eps = torch.tensor(np.float32(EPS), **f32)

    def rec(k, v):
        amax[k] = max(amax.get(k, 0.0), float(v.abs().max()))

    def rms(v, w):
        return v / torch.sqrt((v * v).mean(-1, keepdim=True) + eps) * w

    def heads(v):                                   # (N, T, C) -> (N, H, T, d), contiguous
        return v.reshape(v.shape[0], T, H, d).transpose(1, 2).contiguous()

    x = torch.as_tensor(np.asarray(x, dtype=np.float32), **f32)
    for L in _prefixes(spec):
        h1 = rms(x, W[L + "ln1"])
        rec(L + "h1", h1)
        q, k, v = (h1 @ Wt[L + n] for n in ("q", "k", "v"))
        for n, t in (("q", q), ("k", k), ("v", v)):
            rec(L + n, t)
        N = x.shape[0]
        qh, kh, vh = heads(q), heads(k), heads(v)
        sc = (qh @ kh.transpose(-1, -2).contiguous()) * np.float32(1.0 / math.sqrt(d))
        if spec.causal:
            rec(L + "scores", torch.where(keep, sc, torch.zeros((), **f32)))
            sc = sc.masked_fill(~keep, float("-inf"))
        else:
            rec(L + "scores", sc)
        sc = sc - sc.amax(-1, keepdim=True)
        e = torch.exp(sc)
        p = e / e.sum(-1, keepdim=True)
        o = p @ vh
        rec(L + "o", o)
        om = o.transpose(1, 2).reshape(N, T, C)
        y = om @ Wt[L + "y"]
        rec(L + "y", y)
        r1 = x + y
        rec(L + "r1", r1)
        h2 = rms(r1, W[L + "ln2"])
        rec(L + "h2", h2)
        fc = h2 @ Wt[L + "fc"]
        rec(L + "fc", fc)
        f64 = fc.double()
        ge = (0.5 * f64 * (1 + torch.erf(f64 / math.sqrt(2)))).float()
        rec(L + "gelu", ge)
        proj = ge @ Wt[L + "proj"]
        rec(L + "proj", proj)
        x = r1 + proj
        rec(L + "out", x)
    if spec.vocab:
        hf = rms(x, W["lnf"])
        rec("hf", hf)
        rec("logits", hf @ Wt["wte"])


def calibrate_on_device(spec: BlockSpec, params, tag: int, device="cuda"):
    """calibrate() with the float forward on a torch device (reference quantize.py:276-300 runs it in torch). The
    inputs, their scale and their fake quantization stay on the host, so the input scale is calibrate()'s; the
    max-abs values agree with the host forward's to float32 rounding, so a graph built from them may differ from the
    tracked calibration's in the last step of a constant. For new specs and large calibration sets; the tracked
    calibration fixes the benchmark's graphs."""
    xs = [to_float_input(spec, params, calib_inputs(spec, i, tag)) for i in range(spec.calib_batches)]
    sin = max(float(np.abs(x).max()) for x in xs) / 127
    amax = {}
    W, Wt = device_params(params, device)
    for x in xs:
        deq = (np.clip(np.rint(x / sin), -128, 127) * sin).astype(np.float32)
        for lo in range(0, len(deq), 4):
            float_forward_amax_torch(spec, W, Wt, deq[lo:lo + 4], amax, device)
    return sin, amax


# ------------------------------------------------------------------------------------------- graph build

@dataclass
class Built:
    spec: BlockSpec
    module: object
    consts: dict
    scales: dict
    params: dict = field(repr=False, default_factory=dict)


def build_graph(spec: BlockSpec, params, x_scale: float, amax: dict) -> Built:
    """The quantized graph of the block stack from float weights and calibration max-abs values."""
    C, H, T, F = spec.n_embd, spec.n_head, spec.seq, spec.hidden
    d = C // H
    b = g.GraphBuilder("block" if not spec.vocab else "model")
    consts, scales, mag = {}, {}, {}

    def const(name, data, dtype="i8", scale=None):
        data = np.asarray(data, dtype=np.int64)
        consts[name] = data
        scales[name] = scale
        return b.const(name, list(data.shape), dtype, scale)

    def act(sym):
        return spec.headroom * amax[sym] / 127

    def weight(w_io):
        sw = Q.maxabs_scale(w_io)
        return Q.to_int8(w_io, sw), sw

    def rmsnorm(sym, xv, sx, w_f):
        so = act(sym)
        wq, sw = weight(w_f)
        lut, s = Q.rsqrt_table(sx, sw, so, int(np.abs(wq).max()), C, EPS)
        v = b.rmsnorm_int(sym, xv, const(f"{sym}.w", wq, "i8", sw), const(f"{sym}.rsqrt_lut", lut, "i32"), 1, s, so)
        scales[sym], mag[sym] = so, 128
        return v, so

    def linear(sym, xv, sx, xmag, w_oi, lut=None, out_scale=None):
        so = act(sym)
        wq, sw = weight(w_oi.T.astype(np.float64))
        bound = xmag * int(np.abs(wq).sum(axis=0).max())
        (m,), s = Q.choose_shift([sx * sw / so], [bound])
        scale = so if lut is None else out_scale
        v = b.qlinear(sym, xv, const(f"{sym}.w", wq, "i8", sw), m, s, scale, lut=lut)
        scales[sym], mag[sym] = scale, 128
        return v, so

    def add(sym, av, sa, bv, sb, ma_, mb_):
        so = act(sym)
        (ma, mb), s = Q.choose_shift([sa / so, sb / so], [ma_, mb_])
        v = b.add_requant(sym, av, bv, ma, mb, s, so)
        scales[sym], mag[sym] = so, 128
        return v, so

    x = b.input("x", [T, C], "i8", x_scale)
    scales["x"], mag["x"] = x_scale, 128
    sx = x_scale
    for L in _prefixes(spec):
        h1, s_h1 = rmsnorm(L + "h1", x, sx, params[L + "ln1"])
        heads, sh = {}, {}
        for n in ("q", "k", "v"):
            t, sh[n] = linear(L + n, h1, s_h1, 128, params[L + n])
            r = b.reshape(f"{L}{n}h.r", t, [T, H, d])
            heads[n] = b.transpose(f"{L}{n}h", r, [1, 0, 2])
        kT = b.transpose(f"{L}kT", heads["k"], [0, 2, 1])
        s_sc = act(L + "scores")
        (m,), s = Q.choose_shift([sh["q"] * sh["k"] / math.sqrt(d) / s_sc], [d * 128 * 128])
        sc = b.qmatmul(L + "scores", heads["q"], kT, m, s, s_sc)
        elut = Q.exp_table(s_sc, T, Q.SOFTMAX_ONE)
        p = b.softmax_lut(L + "p", sc, const(f"{L}p.exp_lut", elut, "i32"), Q.SOFTMAX_ONE, spec.causal,
                          1 / Q.SOFTMAX_ONE)
        s_o = act(L + "o")
        (m,), s = Q.choose_shift([sh["v"] / Q.SOFTMAX_ONE / s_o], [T * Q.SOFTMAX_ONE * 128])
        o = b.qmatmul(L + "o", p, heads["v"], m, s, s_o)
        om = b.reshape(f"{L}om", b.transpose(f"{L}om.t", o, [1, 0, 2]), [T, C])
        y, s_y = linear(L + "y", om, s_o, 128, params[L + "y"])
        r1, s_r1 = add(L + "r1", x, sx, y, s_y, 128, 128)
        h2, s_h2 = rmsnorm(L + "h2", r1, s_r1, params[L + "ln2"])
        s_fc, s_ge = act(L + "fc"), act(L + "gelu")
        glut = Q.activation_table(gelu, s_fc, s_ge)
        if spec.gelu == "fused":
            ge, _ = linear(L + "fc", h2, s_h2, 128, params[L + "fc"], lut=const(f"{L}fc.gelu_lut", glut, "i8", s_ge),
                           out_scale=s_ge)
        else:
            fc, _ = linear(L + "fc", h2, s_h2, 128, params[L + "fc"])
            ge = b.lut(L + "gelu", fc, const(f"{L}gelu.lut", glut, "i8", s_ge), s_ge)
            scales[L + "gelu"] = s_ge
        pr, s_pr = linear(L + "proj", ge, s_ge, 128, params[L + "proj"])
        x, sx = add(L + "out", r1, s_r1, pr, s_pr, 128, 128)
    outs = [x]
    if spec.vocab:
        hf, s_hf = rmsnorm("hf", x, sx, params["lnf"])
        lg, _ = linear("logits", hf, s_hf, 128, params["wte"])
        outs = [lg]
    b.output(*outs)
    module = b.module()
    Q.prove_no_overflow(module, consts)
    return Built(spec, module, consts, scales, params)


# ----------------------------------------------------------------------------------------------- configs

def calib_inputs(spec: BlockSpec, i: int, tag: int):
    """Calibration batch i: float inputs N(0, 1) (or token ids -> embeddings), seeded by (tag, 1, i)."""
    rng = np.random.default_rng([tag, 1, i])
    if spec.vocab:
        return rng.integers(0, spec.vocab, (spec.calib_batch, spec.seq))
    return rng.standard_normal((spec.calib_batch, spec.seq, spec.n_embd)).astype(np.float32)


def eval_inputs(spec: BlockSpec, batch: int, tag: int, j: int = 0):
    """Evaluation inputs, seeded by (tag, 2, j): float N(0, 1) activations, or token ids for a vocab model."""
    rng = np.random.default_rng([tag, 2, j])
    if spec.vocab:
        return rng.integers(0, spec.vocab, (batch, spec.seq))
    return rng.standard_normal((batch, spec.seq, spec.n_embd)).astype(np.float32)


def to_float_input(spec, params, raw):
    return embed(spec, params, raw) if spec.vocab else np.asarray(raw, dtype=np.float32)


def calibrate(spec: BlockSpec, params, tag: int):
    """(input scale, {sym: max |float activation|}) over spec.calib_batches seeded batches: the input scale is
    max-abs / 127 of the raw inputs, activations are measured on the fake-quantized inputs (reference
    quantize.py:276-300)."""
    xs = [to_float_input(spec, params, calib_inputs(spec, i, tag)) for i in range(spec.calib_batches)]
    sin = max(float(np.abs(x).max()) for x in xs) / 127
    amax = {}
    for x in xs:
        deq = (np.clip(np.rint(x / sin), -128, 127) * sin).astype(np.float32)
        for lo in range(0, len(deq), 4):
            float_forward_amax(spec, params, deq[lo:lo + 4], amax)
    return sin, amax


CALIB_DIR = Path(__file__).resolve().parent / "calib"
_CALIB_CODE = ("init_params", "embed", "_rms", "gelu", "float_forward_amax", "calib_inputs", "to_float_input",
               "calibrate")


def calib_code_digest() -> str:
    """sha256 of the source of every function the calibration result depends on: a change to any of them gives a
    new calibration key, so a stored result can never outlive the code that produced it."""
    h = hashlib.sha256()
    for name in _CALIB_CODE:
        h.update(inspect.getsource(globals()[name]).encode())
    return h.hexdigest()


def calib_key(spec: BlockSpec, tag: int) -> str:
    return hashlib.sha256(json.dumps([tag, asdict(spec), calib_code_digest()], sort_keys=True).encode()).hexdigest()[:16]


def calib_path(spec: BlockSpec, tag: int) -> Path:
    return CALIB_DIR / f"calib-{calib_key(spec, tag)}.json"


def write_calibration(spec: BlockSpec, tag: int) -> Path:
    """Run the float calibration of (spec, tag) and store it under calib/ (a tracked file: the committed
    calibration, not the host's float arithmetic, then fixes every scale and constant of the built graph)."""
    sin, amax = calibrate(spec, init_params(spec), tag)
    path = calib_path(spec, tag)
    CALIB_DIR.mkdir(parents=True, exist_ok=True)
    body = {"key": calib_key(spec, tag), "tag": tag, "spec": asdict(spec), "sin": sin, "amax": amax}
    path.write_text(json.dumps(body, indent=1, sort_keys=True) + "\n")
    return path


def build(spec: BlockSpec, tag: int, stored: bool = True, calib_device=None) -> Built:
    """The quantized graph of `spec` (weights seed spec.wseed, calibration seed tag). With stored=True (the default)
    the calibration (input scale and max-abs values) comes from the tracked calib/ file of this spec, tag and
    calibration code when there is one, so every machine builds the same constants; otherwise it is computed here,
    on the host, or with the float forward on the torch device `calib_device` when one is given."""
    params = init_params(spec)
    path = calib_path(spec, tag)
    if calib_device is not None:
        sin, amax = calibrate_on_device(spec, params, tag, calib_device)
    elif stored and path.exists():
        body = json.loads(path.read_text())
        sin, amax = body["sin"], body["amax"]
    else:
        sin, amax = calibrate(spec, params, tag)
    return build_graph(spec, params, sin, amax)


# The block configurations of the benchmark (tags are their seeds' namespace).
CONFIGS = {
    1: (BlockSpec(n_embd=64, n_head=4, seq=32, calib_batches=8, calib_batch=1), 1, 1),
    3: (BlockSpec(n_embd=256, n_head=8, seq=256, calib_batches=16, calib_batch=64), 3, 64),
    4: (BlockSpec(n_embd=128, n_head=4, seq=128, layers=2, vocab=512, calib_batches=8, calib_batch=128), 4, 128),
    5: (BlockSpec(n_embd=768, n_head=12, seq=1024, calib_batches=8, calib_batch=32), 5, 32),
}


def config(n: int, stored: bool = True):
    """(Built, eval batch) for block config n in {1, 3, 4, 5}."""
    spec, tag, batch = CONFIGS[n]
    return build(spec, tag, stored), batch


def config_tag(n: int) -> int:
    return CONFIGS[n][1]


# ------------------------------------------------------------------------------------- config 2: linear sweep

LINEAR_SHAPES = [(m, k) for m in (256, 4096, 16384) for k in (768, 3072)]     # (M, K), N = K


@dataclass
class Linear:
    """One int8 qlinear with a per-tensor requant: x (M, K) @ w (K, N), the standalone GEMM sweep."""
    module: object
    consts: dict
    x: np.ndarray               # (M, K) int64 values in [-127, 127]
    mult: int
    shift: int


def linear_config(M: int, K: int, N: int | None = None, tag: int = 2) -> Linear:
    """Config 2 at one shape: x and w uniform integers in [-127, 127] (seeded by (tag, M, K, N)), and the requant
    (mult, shift) = choose_shift([127 / (1.5 max|acc|)], [128 max_n sum_k |w[k, n]|]): the accumulator's largest
    magnitude on these inputs maps to 127 / 1.5 (the quantizer's headroom), and the multiplier is safe for any int8
    input, as the quantizer sizes a linear's (anvil/frontend/quantize.py:401-409)."""
    N = K if N is None else N
    rng = np.random.default_rng([tag, M, K, N])
    x = rng.integers(-127, 128, (M, K))
    w = rng.integers(-127, 128, (K, N))
    acc_max = int(np.abs(x.astype(np.float64) @ w.astype(np.float64)).max())   # exact: |acc| < 2^53
    (mult,), shift = Q.choose_shift([127 / (Q.HEADROOM * acc_max)], [128 * int(np.abs(w).sum(axis=0).max())])
    b = g.GraphBuilder("linear")
    y = b.qlinear("y", b.input("x", [M, K], "i8", 1.0), b.const("w", [K, N], "i8", 1.0), mult, shift, 1.0)
    b.output(y)
    return Linear(b.module(), {"w": w}, x, mult, shift)
