"""Kernel-level checks at full model shapes.

Each decode or prefill kernel's output, captured on the GPU
(ehip_debug_capture / ehip_debug_capture_prefill), is compared with a
float64 recomputation of the reference operation on the GPU's own inputs, so
a kernel is judged on its own: differences upstream cannot cascade into it.

What is recomputed (reference file:line):
  activation Q8_0 (src/kernels.c:73-92)  exactly, in float32 arithmetic as the
      reference evaluates it; after an RMSNorm (src/model.c:50-55, a
      sequential float32 sum) likewise
  quantized products (src/kernels.c:120-220, 223-264)  in float64 from the
      dequantized weights and activation codes (every product and partial sum
      is then exact or within 1e-16), plus bias / residual / SwiGLU
      (src/model.c:382-408)
  QK-norm, RoPE, KV store, attention (src/model.c:39-80, 207-278, 386-395)
      in float64, with the RoPE angle and cos/sin taken from the host libm in
      float32 exactly as the reference computes them

Tolerances.  The GPU sums fp32 terms in another order than the reference,
so a product may differ by a few float32 roundings of its terms:
|gpu - ref| <= 1e-6 * sum_i |term_i| (+ one float32 rounding of the result;
a sum over a tree of depth 16 or a sequential one over 16 terms rounds
within that).  An attention output may differ by 1e-5 * sum_t p_t |v_t|
(exponentials on the GPU's exp2 unit, a few ulps in the probabilities).
Where the GPU normalizes an activation itself (RMSNorm prologues) its sum of
squares is taken in another order, which moves the normalized values by a
few ulps; an activation code whose scaled value x*id lies within 4e-5 of a
rounding boundary (x*id = k + 0.5) can then land on either side, and an fp16
block scale within 2e-6 relative of an fp16 rounding midpoint can round
either way.  Each such ambiguous code or scale widens the bound of the
outputs it feeds by exactly one code step (|w| * d_x) or one fp16 step of
the scale.  Everything else must agree: a wrong block scale, a dropped or
doubled row, a wrong tile or index exceeds these bounds by orders of
magnitude.
"""
import ctypes
import ctypes.util

import numpy as np

from emberllm_amd import _native

QB = 32
AMB_CODE = 4e-5      # |x*id - (k + 1/2)| below this: code ambiguous after a re-ordered norm
AMB_SCALE = 2e-6     # relative distance of d = amax/127 from an fp16 rounding midpoint
SUM_TOL = 1e-6       # relative to the sum of |terms| of a product
ATT_TOL = 1e-5       # relative to sum_t p_t |v_t| of an attention output
F32_ULP = 2.0 ** -23

_libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
for _f in ("powf", "cosf", "sinf"):
    getattr(_libm, _f).restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
_libm.cosf.argtypes = [ctypes.c_float]
_libm.sinf.argtypes = [ctypes.c_float]

Q8 = np.dtype([("d", "<f2"), ("q", "i1", (QB,))])
Q4 = np.dtype([("d", "<f2"), ("q", "u1", (QB // 2,))])


# ------------------------------------------------------------------ model file
class ModelFile:
    """Read-only numpy view of an .ember file (header, table, tensors)."""

    def __init__(self, path):
        self.raw = np.memmap(path, dtype=np.uint8, mode="r")
        self.h = _native.EmberHeader.from_buffer_copy(bytes(self.raw[:256]))
        off, n = int(self.h.tensor_table_offset), int(self.h.n_tensors)
        tab = bytes(self.raw[off:off + 88 * n])
        self.t = {}
        for i in range(n):
            e = _native.EmberTensor.from_buffer_copy(tab[88 * i:88 * (i + 1)])
            self.t[e.name.decode()] = e
        h = self.h
        self.dim, self.hid, self.L = h.dim, h.hidden_dim, h.n_layers
        self.nh, self.nkv, self.hd, self.V = h.n_heads, h.n_kv_heads, h.head_dim, h.vocab_size
        self.qd, self.kvd = self.nh * self.hd, self.nkv * self.hd
        self.eps = np.float32(h.norm_eps)
        self.theta = float(h.rope_theta)
        self.neox = h.rope_style == _native.ROPE_NEOX
        self.qk_norm = bool(h.flags & 2)
        self.tied = bool(h.flags & 1)

    def has(self, name):
        return name in self.t

    def _bytes(self, e):
        return self.raw[int(e.offset):int(e.offset) + int(e.nbytes)]

    def vec(self, name):
        if name not in self.t:
            return None
        return np.frombuffer(self._bytes(self.t[name]), dtype=np.float32).copy()

    def mat(self, names):
        """A QMat over the row-concatenation of the named matrices."""
        return QMat([self.t[n] for n in names], self)

    def layer(self, l, what):
        p = f"layers.{l}."
        return {"qkv": [p + "wq", p + "wk", p + "wv"], "wo": [p + "wo"], "w13": [p + "w1", p + "w3"],
                "w2": [p + "w2"]}[what]

    def head_names(self):
        return ["tok_embeddings"] if self.tied or "lm_head" not in self.t else ["lm_head"]

    def inv_freq(self):
        """1.0f / powf(theta, (float)(2i)/hd) with the host libm (src/model.c:69)."""
        hd = self.hd
        return np.array([np.float32(1.0) / np.float32(_libm.powf(self.theta, float(np.float32(2 * i) / np.float32(hd))))
                         for i in range(hd // 2)], dtype=np.float32)

    def rope(self, pos):
        """(cos, sin) float64 [hd/2] of the float32 angle pos * freq_i, libm cosf/sinf."""
        ang = (np.float32(pos) * self.inv_freq()).astype(np.float32)
        c = np.array([_libm.cosf(float(a)) for a in ang], dtype=np.float64)
        s = np.array([_libm.sinf(float(a)) for a in ang], dtype=np.float64)
        return c, s


class QMat:
    """Row-concatenated quantized (or F32) matrix, dequantized chunk by chunk."""

    def __init__(self, entries, mf):
        self.parts = []
        self.rows = 0
        for e in entries:
            rows, cols = int(e.shape[0]), int(e.shape[1])
            self.parts.append((e, rows, cols))
            self.rows += rows
        self.cols = self.parts[0][2]
        self.dtype = int(self.parts[0][0].dtype)
        self.mf = mf

    def chunks(self, step=16384):
        """Yield (row0, dequantized float64 [r, cols]) over all rows."""
        r0 = 0
        for e, rows, cols in self.parts:
            raw = self.mf._bytes(e)
            for a in range(0, rows, step):
                b = min(rows, a + step)
                yield r0 + a, dequant(raw, self.dtype, a, b, cols)
            r0 += rows


def dequant(raw, dtype, a, b, cols):
    nb = cols // QB
    if dtype == _native.DT_F32:
        return np.frombuffer(raw, dtype=np.float32).reshape(-1, cols)[a:b].astype(np.float64)
    if dtype == _native.DT_Q8_0:
        blk = np.frombuffer(raw, dtype=Q8).reshape(-1, nb)[a:b]
        return (blk["q"].astype(np.float64) * blk["d"].astype(np.float64)[..., None]).reshape(b - a, cols)
    blk = np.frombuffer(raw, dtype=Q4).reshape(-1, nb)[a:b]
    q = blk["q"].astype(np.int16)
    codes = np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=-1).astype(np.float64)
    return (codes * blk["d"].astype(np.float64)[..., None]).reshape(b - a, cols)


# --------------------------------------------------------------- activation
def rmsnorm_f32(x, w, eps):
    """src/model.c:50-55 in float32: sequential sum of squares, 1/sqrtf, x*r*w."""
    x = np.asarray(x, dtype=np.float32)
    ss = np.cumsum(x * x, axis=-1, dtype=np.float32)[..., -1]
    n = np.float32(x.shape[-1])
    r = (np.float32(1.0) / np.sqrt((ss / n + eps).astype(np.float32))).astype(np.float32)
    return ((x * r[..., None]).astype(np.float32) * w).astype(np.float32)


def quant_q8(x, amb_tol):
    """Q8_0 of float32 rows (src/kernels.c:73-92) in the reference's float32
    arithmetic.  Returns (dequantized activation float64 [n, cols], alts):
    alts[t] lists the ambiguous quantities of row t as (kind, index, delta):
    kind "code": element `index` may hold the neighbouring code, which moves
    its dequantized value by `delta`; kind "scale": block `index` may hold
    the neighbouring fp16 scale, which moves the scale by `delta`.  amb_tol
    is how far (in units of x*id) the GPU's own float32 input to the
    quantizer may lie from these values; 0 when the GPU quantized the very
    same float32 values (then nothing is ambiguous)."""
    x = np.asarray(x, dtype=np.float32)
    n, cols = x.shape
    xb = x.reshape(n, cols // QB, QB)
    amax = np.max(np.abs(xb), axis=-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    prod = (xb * inv[..., None]).astype(np.float32).astype(np.float64)
    mag = np.floor(np.abs(prod) + 0.5)
    q = np.clip(np.sign(prod) * mag, -127, 127)
    dq = d.astype(np.float16).astype(np.float64)
    xq = (q * dq[..., None]).reshape(n, cols)
    alts = [[] for _ in range(n)]
    if amb_tol > 0:
        frac = np.abs(prod) - np.floor(np.abs(prod))
        code_amb = (np.abs(frac - 0.5) < amb_tol) & (np.abs(prod) < 127.0)
        for t, b, k in zip(*np.nonzero(code_amb)):
            other = np.floor(np.abs(prod[t, b, k])) + (0.0 if mag[t, b, k] > np.floor(np.abs(prod[t, b, k])) else 1.0)
            alt = np.sign(prod[t, b, k]) * other
            alts[t].append(("code", b * QB + k, (alt - q[t, b, k]) * dq[t, b]))
        d64 = d.astype(np.float64)
        lo = (d64 * (1 - AMB_SCALE)).astype(np.float16).astype(np.float64)
        hi = (d64 * (1 + AMB_SCALE)).astype(np.float16).astype(np.float64)
        for t, b in zip(*np.nonzero(lo != hi)):
            other = hi[t, b] if dq[t, b] == lo[t, b] else lo[t, b]
            alts[t].append(("scale", b, other - dq[t, b]))
    return xq, alts, q.reshape(n, cols)


# ------------------------------------------------------------------ products
def qproduct(W, xq, alts=None, codes=None):
    """W @ xq^T in float64 for activation rows xq [n, cols]: returns (y, mag,
    D) with y and mag = |W| @ |xq| of shape [n, rows], and D[t] the [rows, k]
    output changes of row t's k alternatives (see quant_q8)."""
    n = xq.shape[0]
    y = np.empty((n, W.rows))
    mag = np.empty((n, W.rows))
    ax = np.abs(xq).T
    alts = alts or [[] for _ in range(n)]
    D = {t: np.empty((W.rows, len(a))) for t, a in enumerate(alts) if a}
    for r0, w in W.chunks():
        r1 = r0 + w.shape[0]
        y[:, r0:r1] = (w @ xq.T).T
        mag[:, r0:r1] = (np.abs(w) @ ax).T
        for t, dt in D.items():
            for j, (kind, idx, delta) in enumerate(alts[t]):
                if kind == "code":
                    dt[r0:r1, j] = w[:, idx] * delta
                else:   # block idx's scale moves by delta: w . codes over the block
                    cb = codes[t, idx * QB:(idx + 1) * QB]
                    dt[r0:r1, j] = (w[:, idx * QB:(idx + 1) * QB] @ cb) * delta
    return y, mag, D


MAX_ALTS = 12        # alternatives searched exhaustively per activation row


class Report:
    """Accumulates per-kernel results; `ok` is False once a bound fails."""

    def __init__(self, label):
        self.label, self.lines, self.ok = label, [], True

    def add(self, name, gpu, ref, bound, n_amb=0, n_taken=0):
        gpu = np.asarray(gpu, dtype=np.float64)
        ref = np.asarray(ref, dtype=np.float64)
        d = np.abs(gpu - ref)
        worst = float(np.max(d / np.maximum(bound, 1e-30)))
        rel = float(np.linalg.norm(gpu - ref) / max(np.linalg.norm(ref), 1e-30))
        good = bool(np.all(np.isfinite(gpu))) and worst <= 1.0
        self.ok &= good
        amb = f", ambiguous {n_amb} (the GPU took {n_taken})" if n_amb else ""
        self.lines.append(f"{self.label} {name}: rel-L2 {rel:.2e}, worst |diff|/bound {worst:.3f}{amb}"
                          f"{'' if good else '  <-- FAIL'}")
        return good

    def __str__(self):
        return "\n".join(self.lines)


def _resolve(gpu, y, mag, Dt, finish, top=4096):
    """Choose the subset of a row's alternatives (columns of Dt) that best
    explains the GPU's outputs: exhaustive over 2^k subsets on the `top`
    outputs the alternatives move most, scored by the worst |diff|/bound.
    finish(y_rows, mag_rows) -> (ref, bound) applies the epilogue.  Returns
    the chosen 0/1 vector."""
    k = Dt.shape[1]
    if k > MAX_ALTS:
        raise AssertionError(f"{k} ambiguous codes in one activation row (more than {MAX_ALTS}): "
                             "the GPU's normalization is further from the reference's than a few ulps")
    span = np.abs(Dt).sum(axis=1)
    rows = np.argsort(-span)[:top] if finish is None else None
    combos = ((np.arange(2 ** k)[:, None] >> np.arange(k)[None, :]) & 1).astype(np.float64)
    best, choice = np.inf, np.zeros(k)
    for f in combos:
        if finish is None:
            yr = y[rows] + Dt[rows] @ f
            ref, bound = yr, SUM_TOL * mag[rows] + 2 * F32_ULP * np.abs(yr) + 1e-30
            score = float(np.max(np.abs(gpu[rows] - ref) / bound))
        else:
            ref, bound = finish(y + Dt @ f, mag)
            score = float(np.max(np.abs(gpu - ref) / bound))
        if score < best:
            best, choice = score, f
    return choice


def check_product(rep, name, W, x_in, gpu_out, norm_w=None, eps=None, epi="store", pre=None,
                  bias=None, hidden=0, amb_tol=None):
    """One quantized product (decode matvec or prefill GEMM) on the GPU's own
    input rows x_in [n, cols] (the residual before the norm, or the exact
    activation for a plain prologue).  amb_tol: see quant_q8 (default AMB_CODE
    after a norm, else 0).  Ambiguous codes and scales are resolved per
    activation row: the one subset of them that explains all of the row's
    outputs is applied, then every output must lie within the product's
    rounding bound."""
    x_in = np.atleast_2d(np.asarray(x_in, dtype=np.float32))
    xa = rmsnorm_f32(x_in, norm_w, eps) if norm_w is not None else x_in
    if W.dtype == _native.DT_F32:
        raise ValueError("F32 weights are not covered by this check")
    if amb_tol is None:
        amb_tol = AMB_CODE if norm_w is not None else 0.0
    xq, alts, codes = quant_q8(xa, amb_tol)
    y, mag, D = qproduct(W, xq, alts, codes)
    gpu_out = np.atleast_2d(np.asarray(gpu_out, dtype=np.float64))
    n = x_in.shape[0]
    pre2 = None if pre is None else np.atleast_2d(pre).astype(np.float64)

    def finish_row(t):
        def fin(yt, mt):
            if epi == "swiglu":   # decode: silu(w1 row) * w3 row
                g, u = yt[:hidden], yt[hidden:]
                bg, bu = SUM_TOL * mt[:hidden], SUM_TOL * mt[hidden:]
                sg = 1.0 / (1.0 + np.exp(-g))
                ref = g * sg * u
                dsilu = sg * (1.0 + g * (1.0 - sg))
                return ref, np.abs(dsilu * u) * bg + np.abs(g * sg) * bu + 8 * F32_ULP * np.abs(ref) + 1e-30
            ref = yt.copy()
            if bias is not None:
                ref += bias.astype(np.float64)
            if epi == "resid":
                ref += pre2[t]
            return ref, SUM_TOL * mt + 2 * F32_ULP * np.abs(ref) + 1e-30
        return fin

    refs, bounds, n_amb, n_taken = [], [], 0, 0
    for t in range(n):
        yt = y[t]
        if t in D:
            simple = epi == "store" and bias is None
            f = _resolve(gpu_out[t], yt, mag[t], D[t], None if simple else finish_row(t))
            yt = yt + D[t] @ f
            n_amb += D[t].shape[1]
            n_taken += int(f.sum())
        ref, bound = finish_row(t)(yt, mag[t])
        refs.append(ref)
        bounds.append(bound)
    return rep.add(name, gpu_out, np.array(refs), np.array(bounds), n_amb, n_taken)


# ----------------------------------------------------------------- attention
def qk_rope(mf, l, vecs, which, pos):
    """QK-norm (if present) then RoPE of [n, heads*hd] q rows (which "q") or
    k rows ("k") at positions pos (array), float64 (src/model.c:66-80,
    386-392)."""
    hd = mf.hd
    n_heads = mf.nh if which == "q" else mf.nkv
    v = np.asarray(vecs, dtype=np.float64).reshape(len(pos), n_heads, hd)
    w = mf.vec(f"layers.{l}.{which}_norm") if mf.qk_norm else None
    if w is not None:
        r = 1.0 / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + float(mf.eps))
        v = v * r * w.astype(np.float64)
    out = np.empty_like(v)
    half = hd // 2
    tabs = {}
    for i, p in enumerate(pos):
        if p not in tabs:
            tabs[p] = mf.rope(p)
        c, s = tabs[p]
        if mf.neox:
            a, b = v[i, :, :half], v[i, :, half:]
            out[i, :, :half] = a * c - b * s
            out[i, :, half:] = a * s + b * c
        else:
            a, b = v[i, :, 0::2], v[i, :, 1::2]
            out[i, :, 0::2] = a * c - b * s
            out[i, :, 1::2] = a * s + b * c
    return out


def check_kv_rows(rep, name, mf, l, qkv_raw, pos, kcache, vcache, kv16):
    """The K rows (QK-normed, rotated) and V rows the kernels stored at
    positions `pos` (src/model.c:39-48) against the float64 recomputation."""
    qkv_raw = np.atleast_2d(qkv_raw)
    k = qkv_raw[:, mf.qd:mf.qd + mf.kvd]
    v = qkv_raw[:, mf.qd + mf.kvd:]
    kref = qk_rope(mf, l, k, "k", pos).reshape(len(pos), -1)
    # fp16 rounding: half an ulp relative, or half the subnormal step 2^-24
    tol, floor = (2.0 ** -11, 2.0 ** -25) if kv16 else (4 * F32_ULP, 0.0)
    ok = rep.add(name + " K rows", kcache[pos], kref,
                 tol * np.abs(kref) + 1e-6 * np.max(np.abs(kref)) + floor)
    vref = v.astype(np.float64)
    ok &= rep.add(name + " V rows", vcache[pos], vref, tol * np.abs(vref) + floor + 1e-30)
    return ok


def check_attention(rep, name, mf, l, qkv_raw, pos, kcache, vcache, gpu_o):
    """GQA attention of query rows at positions `pos` over cache rows 0..pos
    (src/model.c:207-278) in float64, on the cache the GPU holds.  Bound per
    output: ATT_TOL * sum_t p_t |v_t| (the scale of the weighted sum)."""
    qkv_raw = np.atleast_2d(qkv_raw)
    pos = np.asarray(pos)
    q = qk_rope(mf, l, qkv_raw[:, :mf.qd], "q", pos)          # [n, nh, hd]
    K = np.asarray(kcache, dtype=np.float64).reshape(kcache.shape[0], mf.nkv, mf.hd)
    V = np.asarray(vcache, dtype=np.float64).reshape(vcache.shape[0], mf.nkv, mf.hd)
    grp = mf.nh // mf.nkv
    gpu_o = np.atleast_2d(gpu_o).reshape(len(pos), mf.nh, mf.hd).astype(np.float64)
    ref = np.empty_like(gpu_o)
    scale = np.empty_like(gpu_o)
    causal = np.arange(K.shape[0])[None, :] <= pos[:, None]
    for h in range(mf.nh):
        kh, vh = K[:, h // grp, :], V[:, h // grp, :]
        s = np.where(causal, (q[:, h, :] @ kh.T) / np.sqrt(mf.hd), -np.inf)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        ref[:, h, :] = p @ vh
        scale[:, h, :] = p @ np.abs(vh)
    return rep.add(name, gpu_o, ref, ATT_TOL * scale + 1e-30)


# ------------------------------------------------------------- whole layers
AMB_SWIGLU = 1e-4    # SwiGLU computed on the GPU with its own expf: a few ulps


def swiglu_f32(h13, hid):
    """silu(g) * u of [n, 2*hid] rows in float64 (the GPU's float32 values lie
    within a few ulps: AMB_SWIGLU covers the codes that can move)."""
    g = h13[:, :hid].astype(np.float64)
    u = h13[:, hid:].astype(np.float64)
    return (g / (1.0 + np.exp(-g)) * u).astype(np.float32)


def check_decode_layer(rep, mf, l, slots, pos, kcache, vcache, kv16):
    """Every kernel of decode layer l at position pos, from its captured
    vectors (slots 0..5 of ehip_debug_capture / orc_capture) and the layer's
    cache rows [0, pos]."""
    xin, qkv, o, xmid, h, xout = (np.asarray(v, dtype=np.float32).reshape(-1) for v in slots)
    p = f"layers.{l}."
    bias = None
    if mf.has(p + "wq_bias"):
        bias = np.concatenate([mf.vec(p + "wq_bias"), mf.vec(p + "wk_bias"), mf.vec(p + "wv_bias")])
    check_product(rep, f"L{l} qkv", mf.mat(mf.layer(l, "qkv")), xin, qkv, norm_w=mf.vec(p + "attn_norm"),
                  eps=mf.eps, bias=bias)
    check_kv_rows(rep, f"L{l} kv store", mf, l, qkv[None], np.array([pos]), kcache, vcache, kv16)
    check_attention(rep, f"L{l} attention", mf, l, qkv[None], np.array([pos]), kcache[:pos + 1],
                    vcache[:pos + 1], o)
    check_product(rep, f"L{l} wo", mf.mat(mf.layer(l, "wo")), o, xmid, epi="resid", pre=xin)
    check_product(rep, f"L{l} w1|w3 swiglu", mf.mat(mf.layer(l, "w13")), xmid, h,
                  norm_w=mf.vec(p + "ffn_norm"), eps=mf.eps, epi="swiglu", hidden=mf.hid)
    check_product(rep, f"L{l} w2", mf.mat(mf.layer(l, "w2")), h, xout, epi="resid", pre=xmid)


def check_head(rep, mf, x_final, logits):
    """final RMSNorm + lm_head (src/model.c:411-412) on the last layer's output."""
    check_product(rep, "final norm + lm_head", mf.mat(mf.head_names()), x_final, logits,
                  norm_w=mf.vec("final_norm"), eps=mf.eps)


def check_prefill_layer(rep, mf, l, slots, pos0, kcache, vcache, kv16):
    """Every kernel of prefill layer l over the captured pass: rows [n][width]
    of slots 0..5 (slot 4 the w1|w3 products), tokens at pos0.., the layer's
    cache rows [0, pos0 + n)."""
    xin, qkv, o, xmid, h13, xout = (np.asarray(v, dtype=np.float32) for v in slots)
    n = xin.shape[0]
    pos = pos0 + np.arange(n)
    p = f"layers.{l}."
    bias = None
    if mf.has(p + "wq_bias"):
        bias = np.concatenate([mf.vec(p + "wq_bias"), mf.vec(p + "wk_bias"), mf.vec(p + "wv_bias")])
    check_product(rep, f"L{l} qkv", mf.mat(mf.layer(l, "qkv")), xin, qkv, norm_w=mf.vec(p + "attn_norm"),
                  eps=mf.eps, bias=bias)
    check_kv_rows(rep, f"L{l} kv store", mf, l, qkv, pos, kcache, vcache, kv16)
    check_attention(rep, f"L{l} attention", mf, l, qkv, pos, kcache[:pos0 + n], vcache[:pos0 + n], o)
    check_product(rep, f"L{l} wo", mf.mat(mf.layer(l, "wo")), o, xmid, epi="resid", pre=xin)
    check_product(rep, f"L{l} w1|w3", mf.mat(mf.layer(l, "w13")), xmid, h13,
                  norm_w=mf.vec(p + "ffn_norm"), eps=mf.eps)
    check_product(rep, f"L{l} w2", mf.mat(mf.layer(l, "w2")), swiglu_f32(h13, mf.hid), xout, epi="resid",
                  pre=xmid, amb_tol=AMB_SWIGLU)


def cache_rows(raw, mf, kv16):
    """One layer's cache bytes as float64 rows [n_pos][kv_dim]."""
    dt = np.float16 if kv16 else np.float32
    return np.frombuffer(np.ascontiguousarray(raw).tobytes(), dtype=dt).reshape(-1, mf.kvd).astype(np.float64)
