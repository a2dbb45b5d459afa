"""The kernel-level checker (tests/kernel_check.py) pinned on the CPU.

The GPU tests judge each kernel by recomputing it in float64 from the
model file.  Before that recomputation is trusted it must (1) accept the
oracle's own intermediate vectors (the reference's arithmetic, captured by
orc_capture) for every kernel, on every variant of the forward pass, and
(2) reject the plausible mistakes a kernel could make, planted into those
vectors here on the CPU: a wrong block scale, a dropped or shifted row, one
position missing from the attention, swapped RoPE pairs, the residual
omitted, SwiGLU's factors exchanged.
"""
import numpy as np
import pytest

import kernel_check as kc
import oracle
from emberllm_amd import configs

PINNED = ["t_llama", "t_gqa", "t_bias", "t_qwen3", "t_q4", "t_g7"]


def _cache(orc, mf, l, kv16):
    esize = 2 if kv16 else 4
    per_layer = orc.ctx * mf.kvd * esize
    out = []
    for which in (0, 1):
        raw = orc.kv(which)[l * per_layer:(l + 1) * per_layer]
        out.append(kc.cache_rows(raw, mf, kv16))
    return out


def _decode_run(name, kv16, layer):
    path = configs.model_path(name)
    mf = kc.ModelFile(path)
    orc = oracle.Oracle(path, kv_fp16=kv16)
    ids = (np.arange(11) * 37 + 5) % mf.V
    orc.prefill(ids)
    slots = orc.capture(layer)
    pos = len(ids)
    logits = orc.forward(int(ids[3]), pos)
    slots = [s.copy() for s in slots]
    # the head check needs the last layer's output
    orc.capture(mf.L - 1)
    orc.close()
    orc = oracle.Oracle(path, kv_fp16=kv16)
    orc.prefill(ids)
    last = orc.capture(mf.L - 1)
    logits2 = orc.forward(int(ids[3]), pos)
    assert np.array_equal(logits, logits2)
    k, v = _cache(orc, mf, layer, kv16)
    x_final = last[5][0].copy()
    orc.close()
    return mf, slots, pos, k, v, logits, x_final


@pytest.mark.parametrize("kv16", [False, True])
@pytest.mark.parametrize("name", PINNED)
def test_checker_accepts_the_oracle_decode(name, kv16):
    mf = kc.ModelFile(configs.model_path(name))
    for layer in range(mf.L):
        mf, slots, pos, k, v, logits, xf = _decode_run(name, kv16, layer)
        rep = kc.Report(f"{name} kv16={kv16}")
        kc.check_decode_layer(rep, mf, layer, slots, pos, k, v, kv16)
        kc.check_head(rep, mf, xf, logits)
        assert rep.ok, str(rep)


@pytest.mark.parametrize("name", PINNED)
def test_checker_accepts_the_oracle_prefill(name):
    path = configs.model_path(name)
    mf = kc.ModelFile(path)
    ids = (np.arange(40) * 53 + 1) % mf.V
    for layer in range(mf.L):
        orc = oracle.Oracle(path)
        orc.prefill(ids[:7])                   # a continuation: the pass starts at position 7
        slots = orc.capture(layer, n_tok=len(ids) - 7, prefill=True)
        orc.prefill(ids[7:], start=7)
        k, v = _cache(orc, mf, layer, False)
        rep = kc.Report(f"{name} prefill")
        kc.check_prefill_layer(rep, mf, layer, slots, 7, k, v, False)
        orc.close()
        assert rep.ok, str(rep)


def _planted(name="t_qwen3"):
    mf, slots, pos, k, v, logits, xf = _decode_run(name, False, 1)
    return mf, slots, pos, k, v


def _fails(fn):
    rep = kc.Report("planted")
    fn(rep)
    return not rep.ok


def test_checker_rejects_planted_mistakes():
    mf, slots, pos, k, v = _planted()
    xin, qkv, o, xmid, h, xout = [s.reshape(-1).copy() for s in slots]
    l = 1
    p = "layers.1."

    def qkv_check(rep, out):
        kc.check_product(rep, "qkv", mf.mat(mf.layer(l, "qkv")), xin, out, norm_w=mf.vec(p + "attn_norm"),
                         eps=mf.eps)

    assert not _fails(lambda r: qkv_check(r, qkv))
    # one output row off by one block's worth (a wrong block scale): 1/(cols/32) of the row
    bad = qkv.copy()
    bad[5] *= 1.0 + 1.0 / (mf.dim // 32)
    assert _fails(lambda r: qkv_check(r, bad))
    # a row shifted (output written to its neighbour)
    bad = qkv.copy()
    bad[7], bad[8] = qkv[8], qkv[7]
    assert _fails(lambda r: qkv_check(r, bad))
    # one relative ulp-scale error far above fp32 noise: 1e-4
    bad = qkv.copy()
    bad[100] += 1e-4 * abs(qkv[100]) + 1e-4 * np.abs(qkv).mean()
    assert _fails(lambda r: qkv_check(r, bad))

    # attention: the newest position dropped, or the oldest
    def att(rep, kk, vv, out):
        kc.check_attention(rep, "att", mf, l, qkv[None], np.array([pos]), kk, vv, out)

    assert not _fails(lambda r: att(r, k[:pos + 1], v[:pos + 1], o))
    trunc = k[:pos + 1].copy()
    trunc[pos] = trunc[pos - 1]
    assert _fails(lambda r: att(r, trunc, v[:pos + 1], o))
    vv = v[:pos + 1].copy()
    vv[0] *= 0.0
    assert _fails(lambda r: att(r, k[:pos + 1], vv, o))

    # KV store with the interleaved pairing instead of NEOX
    def kvs(rep, kk):
        kc.check_kv_rows(rep, "kv", mf, l, qkv[None], np.array([pos]), kk, v, False)

    assert not _fails(lambda r: kvs(r, k))
    swapped = k.copy()
    hd = mf.hd
    row = swapped[pos].reshape(-1, hd)
    row[:, :hd // 2], row[:, hd // 2:] = row[:, hd // 2:].copy(), row[:, :hd // 2].copy()
    swapped[pos] = row.reshape(-1)
    assert _fails(lambda r: kvs(r, swapped))

    # wo without the residual, w2 with it applied twice, SwiGLU factors exchanged
    assert _fails(lambda r: kc.check_product(r, "wo", mf.mat(mf.layer(l, "wo")), o, xmid - xin, epi="resid",
                                             pre=xin))
    assert _fails(lambda r: kc.check_product(r, "w2", mf.mat(mf.layer(l, "w2")), h, xout + xmid, epi="resid",
                                             pre=xmid))
    w13 = mf.mat(mf.layer(l, "w13"))
    assert not _fails(lambda r: kc.check_product(r, "w13", w13, xmid, h, norm_w=mf.vec(p + "ffn_norm"),
                                                 eps=mf.eps, epi="swiglu", hidden=mf.hid))
    xq, _, _ = kc.quant_q8(kc.rmsnorm_f32(xmid[None], mf.vec(p + "ffn_norm"), mf.eps), 0.0)
    y, _, _ = kc.qproduct(w13, xq)
    g, u = y[0, :mf.hid], y[0, mf.hid:]
    exchanged = (u / (1 + np.exp(-u)) * g).astype(np.float32)
    assert _fails(lambda r: kc.check_product(r, "w13", w13, xmid, exchanged, norm_w=mf.vec(p + "ffn_norm"),
                                             eps=mf.eps, epi="swiglu", hidden=mf.hid))


class _RandomQ8:
    """A random Q8_0 matrix with the QMat interface (rows x cols)."""

    def __init__(self, rows, cols, seed):
        rng = np.random.default_rng(seed)
        self.rows, self.cols, self.dtype = rows, cols, 1
        codes = rng.integers(-127, 128, (rows, cols)).astype(np.float64)
        d = (rng.uniform(0.5, 1.5, (rows, cols // 32)) * 0.02 / 127).astype(np.float16).astype(np.float64)
        self.w = (codes.reshape(rows, -1, 32) * d[..., None]).reshape(rows, cols)

    def chunks(self, step=16384):
        yield 0, self.w


def _tree_norm(x, w, eps):
    """RMSNorm with the sum of squares taken as 64 lane partials combined by
    a butterfly, the order of a wave reduction."""
    x = x.astype(np.float32)
    part = np.zeros(64, dtype=np.float32)
    for i in range(0, len(x), 64):
        part = (part + x[i:i + 64] * x[i:i + 64]).astype(np.float32)
    while len(part) > 1:
        part = (part[: len(part) // 2] + part[len(part) // 2:]).astype(np.float32)
    r = np.float32(1.0) / np.sqrt(np.float32(part[0] / np.float32(len(x)) + eps))
    return ((x * r).astype(np.float32) * w).astype(np.float32)


def test_ambiguity_bound_covers_a_reordered_norm():
    """A norm whose sum of squares is taken in another order (as the GPU's
    wave reductions do) moves the normalized values by a few ulps and can
    flip activation codes that sit near a rounding boundary.  Over many
    random 1024-wide activations, the checker must accept every product
    computed from such re-ordered codes (some codes do flip), and must still
    reject a wrong block scale in them."""
    rng = np.random.default_rng(3)
    W = _RandomQ8(256, 1024, 4)
    w = np.ones(1024, dtype=np.float32)
    eps = np.float32(1e-6)
    flipped = 0
    for _ in range(300):
        x = rng.standard_normal(1024).astype(np.float32)
        xg, _, _ = kc.quant_q8(_tree_norm(x, w, eps)[None], 0.0)
        xr, _, _ = kc.quant_q8(kc.rmsnorm_f32(x[None], w, eps), 0.0)
        flipped += int(np.count_nonzero(xg != xr))
        y = (W.w @ xg[0])
        rep = kc.Report("reordered norm")
        kc.check_product(rep, "random", W, x, y, norm_w=w, eps=eps)
        assert rep.ok, str(rep)
        bad = xg.copy()
        bad[0, 64:96] *= 1.001      # one block scale off by 1e-3 (an fp16 step is ~1e-3)
        rep = kc.Report("wrong scale")
        kc.check_product(rep, "random", W, x, W.w @ bad[0], norm_w=w, eps=eps)
        assert not rep.ok
        # one code off by one step where the rounding was not in doubt
        xn = kc.rmsnorm_f32(x[None], w, eps)[0].reshape(-1, 32)
        prod = np.abs(xn / (np.abs(xn).max(axis=1, keepdims=True) / 127))
        far = int(np.argmax(np.abs(prod - np.floor(prod) - 0.5).reshape(-1) * (prod.reshape(-1) < 120)))
        bad = xg.copy()
        bad[0, far] += np.sign(bad[0, far] or 1.0) * np.abs(xg[0, far // 32 * 32:far // 32 * 32 + 32]).max() / 127
        rep = kc.Report("one code off")
        kc.check_product(rep, "random", W, x, W.w @ bad[0], norm_w=w, eps=eps)
        assert not rep.ok
    assert flipped > 0, "no code moved: the test exercises nothing"
