"""CPU tests of the product's host library (libember.so without a GPU):
the exported ABI, the bit-exact quantizers and fp16 conversions, the
sampler, the tokenizers, the loader's error handling, the requantizer's
failure without a GPU and the synthetic model generator.
"""
import ctypes
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import oracle
from emberllm_amd import _native, configs
from quant_rows import edge_rows

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLD = os.path.join(HERE, "golden")
L = _native.lib()
HAVE_REF = os.path.exists(oracle.reference_path(True))


# ------------------------------------------------------------------- ABI ---
def declared_functions():
    names = set()
    for h in ("ember.h", "ehip.h", "ember_synth.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b((?:ember|ehip)_\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 21 + 14
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) <= set(_native.PROTOTYPES)


def test_struct_layouts():
    assert ctypes.sizeof(_native.EmberHeader) == 256
    assert ctypes.sizeof(_native.EmberTensor) == 88
    assert _native.EmberHeader.tensor_table_offset.offset == 112
    assert _native.EmberTensor.offset.offset == 72
    # EmberSampler is caller-allocated (main.c:180): natural C layout
    assert ctypes.sizeof(_native.EmberSampler) == 64
    assert _native.EmberSampler.rng_state.offset == 32 and _native.EmberSampler.history.offset == 40


def test_no_gpu_means_loud_failure():
    """Without a GPU, creating a state exits with an error; nothing falls back to the CPU."""
    if L.ehip_device_count() > 0:
        pytest.skip("a GPU is visible")
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from emberllm_amd import configs, emberllm\n"
            "emberllm.Engine(configs.model_path('t_llama'))\n") % ROOT
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "ember: no GPU" in r.stderr


# ----------------------------------------------------- fp16 / quantizers ---
def test_half_conversions_exhaustive_and_rne():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.ember_half_to_float(int(v)) for v in h], np.float32)
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    rng = np.random.default_rng(9)
    x = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        want16 = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(np.array([L.ember_float_to_half(float(v)) for v in x], np.uint16), want16)
    g = np.load(os.path.join(GOLD, "f16.npz"))
    assert np.array_equal(np.array([L.ember_float_to_half(float(v)) for v in g["x"]], np.uint16), g["h"])


def test_quantizers_match_reference_golden():
    g = np.load(os.path.join(GOLD, "quant.npz"))
    for i, row in enumerate(g["x"]):
        row = np.ascontiguousarray(row)
        q8 = np.zeros(68, np.uint8)
        q4 = np.zeros(36, np.uint8)
        L.ember_quant_q8_row(row.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), q8.ctypes.data, 64)
        L.ember_quant_q4_row(row.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), q4.ctypes.data, 64)
        assert np.array_equal(q8, g["q8"][i]) and np.array_equal(q4, g["q4"][i]), i


def test_quantizers_match_reference_on_edge_rows():
    """The host row quantizers and the oracle's against the reference's own
    ember_quantize_q8_0 / q4_0 (src/kernels.c:73-115, its deterministic
    build in oracle/_ref) on rows that reach every branch: zero blocks,
    subnormal and overflowing scales, ties, infinities, NaNs and blocks whose
    inverse scale overflows (NaN and infinite products, which the reference's
    (int)lroundf maps to code 0)."""
    import oracle
    x = edge_rows()
    n = x.shape[1]
    fp = ctypes.POINTER(ctypes.c_float)
    refl = oracle.reference_lib(debug=True) if os.path.exists(oracle.reference_path(True)) else None
    orc = oracle.oracle_lib()
    for bs, host, orcf, reff in ((34, L.ember_quant_q8_row, orc.orc_quantize_q8_0, "ember_quantize_q8_0"),
                                 (18, L.ember_quant_q4_row, orc.orc_quantize_q4_0, "ember_quantize_q4_0")):
        for i, row in enumerate(x):
            row = np.ascontiguousarray(row)
            got = np.zeros(n // 32 * bs, np.uint8)
            via_orc = np.zeros_like(got)
            host(row.ctypes.data_as(fp), got.ctypes.data, n)
            orcf(row.ctypes.data_as(fp), via_orc.ctypes.data, n)
            assert np.array_equal(got, via_orc), (bs, i, got, via_orc)
            if refl is not None:
                want = np.zeros_like(got)
                getattr(refl, reff)(row.ctypes.data_as(fp), want.ctypes.data, n)
                assert np.array_equal(got, want), (bs, i, got, want)
    # the case the reference maps to 0: codes of a block whose 1/d overflows
    q8 = np.zeros(68, np.uint8)
    row = np.ascontiguousarray(x[12])
    L.ember_quant_q8_row(row.ctypes.data_as(fp), q8.ctypes.data, 64)
    assert not q8[2:34].any() and not q8[36:68].any()


def test_quantize_file_without_gpu_fails_loudly(tmp_path):
    """ember_quantize_file encodes its blocks on the GPU (its parity with the
    reference's requantizer is a GPU test); without one it reports an error
    and writes nothing.  Nothing falls back to the CPU."""
    if L.ehip_device_count() > 0:
        pytest.skip("a GPU is visible")
    f32 = configs.model_path("hq_f32", dict(configs.TINY["t_qwen3"], dtype=_native.DT_F32))
    out = tmp_path / "q.ember"
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from emberllm_amd import _native\n"
            "sys.exit(_native.lib().ember_quantize_file(%r, %r, 1))\n") % (ROOT, f32.encode(), str(out).encode())
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "ember: no GPU" in r.stderr, (r.returncode, r.stderr)
    assert not out.exists()


def test_quantize_file_rejects_shape_beyond_payload(tmp_path, capfd):
    """A 2-D fp32 tensor whose [rows, cols] needs more bytes than its payload
    holds is rejected before any row is read (the encoder would otherwise
    read past the tensor, and past the mapping for the last one)."""
    f32 = configs.model_path("hq_f32", dict(configs.TINY["t_qwen3"], dtype=_native.DT_F32))
    raw = bytearray(open(f32, "rb").read())
    tab, n = struct.unpack_from("<Q", raw, 112)[0], struct.unpack_from("<i", raw, 76)[0]
    for i in range(n):
        e = tab + 88 * i
        if raw[e:e + 48].rstrip(b"\0") == b"layers.1.w2":
            rows = struct.unpack_from("<i", raw, e + 56)[0]
            struct.pack_into("<i", raw, e + 56, rows * 1000)
            break
    else:
        raise AssertionError("layers.1.w2 not in the table")
    bad, out = tmp_path / "bad.ember", tmp_path / "q.ember"
    bad.write_bytes(bytes(raw))
    assert L.ember_quantize_file(str(bad).encode(), str(out).encode(), _native.DT_Q8_0) == 1
    err = capfd.readouterr().err
    assert "layers.1.w2" in err and "fewer than its" in err, err
    assert not out.exists()


# ---------------------------------------------------------------- sampler ---
def test_sampler_matches_reference_golden():
    g = np.load(os.path.join(GOLD, "sampler.npz"))
    V = g["logits"].shape[1]
    for k, (t, p, topk, seed, rp, ln, pr, fr, mp) in enumerate(g["settings"]):
        s = _native.EmberSampler()
        L.ember_sampler_init(ctypes.byref(s), t, p, int(topk), int(seed))
        L.ember_sampler_set_penalties(ctypes.byref(s), rp, int(ln), pr, fr, mp)
        for i in range(g["logits"].shape[0]):
            row = np.ascontiguousarray(g["logits"][i].copy())
            c = L.ember_sample(ctypes.byref(s), row.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V)
            assert c == g["chosen"][k, i] and s.rng_state == g["states"][k, i], (k, i)
        L.ember_sampler_free(ctypes.byref(s))


def test_sampler_matches_oracle_on_vocab_sized_logits():
    rng = np.random.default_rng(5)
    O = oracle.oracle_lib()
    for trial in range(12):
        V = 151936 if trial < 4 else 4096
        lg = rng.normal(0, 3, V).astype(np.float32)
        lg[rng.integers(0, V, 50)] = lg[7]                      # ties
        for temp, top_p, top_k in ((0.8, 0.9, 40), (1.0, 0.95, 0), (0.5, 1.0, 3), (0.0, 0.9, 0)):
            a, b = _native.EmberSampler(), oracle.Sampler()
            L.ember_sampler_init(ctypes.byref(a), temp, top_p, top_k, 1000 + trial)
            O.orc_sampler_init(ctypes.byref(b), temp, top_p, top_k, 1000 + trial)
            x, y = lg.copy(), lg.copy()
            assert L.ember_sample(ctypes.byref(a), x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V) == \
                O.orc_sample(ctypes.byref(b), oracle.f32p(y), V)
            assert np.array_equal(x, y)                          # same in-place mutation


def test_sampler_history_ring():
    s = _native.EmberSampler()
    L.ember_sampler_init(ctypes.byref(s), 0.0, 1.0, 0, 1)
    L.ember_sampler_set_penalties(ctypes.byref(s), 2.0, 3, 0.0, 0.0, 0.0)
    for t in (4, 5, 6, 7):
        L.ember_sampler_accept(ctypes.byref(s), t)
    assert s.hist_len == 3 and s.hist_pos == 1 and [s.history[i] for i in range(3)] == [7, 5, 6]
    lg = np.zeros(10, np.float32)
    lg[5], lg[7], lg[2] = 3.0, 2.9, 1.6
    # 5 and 7 are in the window: 3.0/2 = 1.5 and 2.9/2 = 1.45, so 2 wins
    assert L.ember_sample(ctypes.byref(s), lg.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 10) == 2
    L.ember_sampler_reset(ctypes.byref(s))
    assert s.hist_len == 0
    L.ember_sampler_free(ctypes.byref(s))
    assert not s.history


# -------------------------------------------------------------- tokenizer ---
def write_tok_model(path, tok_type, blob, vocab, bos=1, eos=2):
    """A header + tokenizer blob + empty table: enough for the tokenizer API."""
    h = _native.EmberHeader()
    h.magic = b"EMBR"
    h.version = 1
    h.dim, h.hidden_dim, h.n_layers, h.n_heads, h.n_kv_heads, h.head_dim = 32, 32, 1, 1, 1, 32
    h.vocab_size, h.max_seq_len = vocab, 16
    h.bos_token_id, h.eos_token_id, h.eos_token_id2 = bos, eos, -1
    h.tokenizer_type = tok_type
    h.tokenizer_offset, h.tokenizer_size = 256, len(blob)
    h.tensor_table_offset = (256 + len(blob) + 7) // 8 * 8
    h.tensor_table_size = 0
    h.header_bytes = (h.tensor_table_offset + 63) // 64 * 64
    with open(path, "wb") as f:
        f.write(bytes(h) + blob + b"\0" * (h.header_bytes - 256 - len(blob)))


def sp_blob():
    pieces = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    extra = [" ", "h", "e", "l", "o", "w", "r", "d", "he", "ll", "hell", "hello", " h", " hello",
             "wor", "world", " w", " world", "lo", "el"]
    pieces += extra
    out = struct.pack("<i", max(len(p.encode()) for p in pieces))
    for i, p in enumerate(pieces):
        b = p.encode()
        score = -float(i) if i < 259 else float(len(b)) - 0.01 * i
        out += struct.pack("<fi", score, len(b)) + b
    return out, len(pieces)


def gpt2_bytes():
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cs, n = bs[:], 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return {b: chr(c) for b, c in zip(bs, cs)}


def bpe_blob():
    m = gpt2_bytes()
    vocab = [m[b] for b in range(256)]
    merges = [("h", "e"), ("l", "l"), ("he", "ll"), ("hell", "o"), ("Ġ", "w"), ("o", "r"),
              ("Ġw", "or"), ("Ġwor", "ld"), ("Ġ", "t"), ("Ġt", "h"), ("Ġth", "e"), ("'", "s"),
              ("1", "2"), ("Ċ", "Ċ"), ("Ġ", "Ġ"), ("l", "d")]
    for a, b in merges:
        vocab.append(a + b)
    specials = ["<|im_start|>", "<|im_end|>"]
    out = struct.pack("<III", len(vocab) + len(specials), len(merges), len(specials))
    for s in vocab:
        e = s.encode()
        out += struct.pack("<BI", 0, len(e)) + e
    for s in specials:
        e = s.encode()
        out += struct.pack("<BI", 1, len(e)) + e
    for a, b in merges:
        ea, eb = a.encode(), b.encode()
        out += struct.pack("<I", len(ea)) + ea + struct.pack("<I", len(eb)) + eb
    for i, s in enumerate(specials):
        e = s.encode()
        out += struct.pack("<II", len(vocab) + i, len(e)) + e
    return out, len(vocab) + len(specials)


TEXTS = ["hello world", "hello", "", "Hello, world! 123", "  multiple   spaces\n\nnew lines\n",
         "<|im_start|>user\nhello<|im_end|>", "it's the world's", "héllo wörld 日本語 ✓",
         "12345 6789", "...!?;", "tab\there", "the the the", " hello world ", "x"]


def encode(lib, tok, text, bos=1):
    out = ctypes.POINTER(ctypes.c_int)()
    n = lib.ember_encode(tok, text.encode(), bos, ctypes.byref(out))
    ids = [out[i] for i in range(n)]
    ctypes.CDLL(None).free(ctypes.cast(out, ctypes.c_void_p))
    return ids


@pytest.mark.parametrize("kind", ["sp", "bpe"])
def test_tokenizer(tmp_path, kind):
    blob, vocab = sp_blob() if kind == "sp" else bpe_blob()
    path = str(tmp_path / f"{kind}.ember")
    write_tok_model(path, 0 if kind == "sp" else 1, blob, vocab, bos=1 if kind == "sp" else -1)
    m = L.ember_model_load(path.encode())
    assert m
    t = L.ember_tokenizer_new(m)
    got = {s: encode(L, t, s) for s in TEXTS}
    if kind == "bpe":
        ids = got["hello world"]
        assert [L.ember_decode(t, 0, i) for i in ids] == [b"hello", b" world"]
        assert got["<|im_start|>user\nhello<|im_end|>"][0] == vocab - 2
    # decoding the ids restores the text (byte fallback included)
    for s, ids in got.items():
        pieces, prev = [], -1
        for i in ids[(1 if kind == "sp" and ids and ids[0] == 1 else 0):]:
            pieces.append(L.ember_decode(t, prev, i))
            prev = i
        text = b"".join(pieces).decode("utf-8", "replace")
        assert text.strip() == s.strip() or kind == "sp" and text == " " + s, (s, text)
    if HAVE_REF:
        R = oracle.reference_lib()
        rm = R.ember_model_load(path.encode())
        rt = R.ember_tokenizer_new(rm)
        for s in TEXTS:
            assert encode(R, rt, s) == got[s], s
            for i in got[s]:
                assert R.ember_decode(rt, 1, i) == L.ember_decode(t, 1, i)
        R.ember_tokenizer_free(rt)
        R.ember_model_free(rm)
    L.ember_tokenizer_free(t)
    L.ember_model_free(m)


# ------------------------------------------------------------------ loader ---
def test_loader_rejects_malformed_files(tmp_path):
    good = configs.model_path("t_llama")
    raw = bytearray(open(good, "rb").read())
    cases = {
        "random": os.urandom(4096),
        "short": raw[:100],
        "magic": b"XXXX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 2) + raw[8:],
        "table": raw[:112] + struct.pack("<Q", len(raw) + 8) + raw[120:],
        "tokenizer": raw[:96] + struct.pack("<Q", len(raw) - 10) + struct.pack("<Q", 1000) + raw[112:],
        "dims": raw[:16] + struct.pack("<i", 0) + raw[20:],
    }
    for name, data in cases.items():
        p = str(tmp_path / name)
        open(p, "wb").write(bytes(data))
        assert not L.ember_model_load(p.encode()), name
    assert not L.ember_model_load(str(tmp_path / "absent").encode())
    m = L.ember_model_load(good.encode())
    assert m and L.ember_model_tensor(m, b"layers.1.w2") and not L.ember_model_tensor(m, b"layers.9.w2")
    t = L.ember_model_tensor(m, b"final_norm")
    norm = np.ctypeslib.as_array(ctypes.cast(L.ember_model_data(m, ctypes.cast(t, ctypes.c_void_p)),
                                             ctypes.POINTER(ctypes.c_float)), shape=(128,))
    assert np.all(norm == 1.0)
    L.ember_model_free(m)


def test_missing_tensor_exits_cleanly(tmp_path):
    """A file without layers.0.w2 fails state creation with an ember: message
    and exit status 1 (model.c:163-170), not a signal."""
    good = configs.model_path("t_llama")
    raw = bytearray(open(good, "rb").read())
    off = struct.unpack_from("<Q", raw, 112)[0]
    n = struct.unpack_from("<i", raw, 76)[0]
    for i in range(n):
        name = raw[off + 88 * i: off + 88 * i + 48].rstrip(b"\0")
        if name == b"layers.0.w2":
            raw[off + 88 * i: off + 88 * i + 11] = b"layers.0.wX"
    p = str(tmp_path / "missing.ember")
    open(p, "wb").write(bytes(raw))
    code = ("import sys; sys.path.insert(0, %r)\nfrom emberllm_amd import emberllm\n"
            "emberllm.Engine(%r)\n") % (ROOT, p)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "missing a required tensor in layer 0" in r.stderr


# --------------------------------------------------------------- generator ---
def splitmix(state):
    state = (state + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return state, z ^ (z >> 31)


def test_generator_follows_its_documented_spec():
    """ember_synth_fill_row = splitmix64 streams + Box-Muller (synth.c header)."""
    name, seed, row, std = b"layers.3.wq", 1234, 17, float(np.float32(0.02))
    h = 1469598103934665603
    for c in name:
        h = ((h ^ c) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    _, key = splitmix(seed ^ h)
    st = (key + (row + 1) * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    assert L.ember_synth_row_state(seed, name, row) == st
    want = []
    for _ in range(8):
        st, a = splitmix(st)
        st, b = splitmix(st)
        u1, u2 = ((a >> 11) + 1) * 2.0 ** -53, (b >> 11) * 2.0 ** -53
        r = np.sqrt(-2.0 * np.log(u1))
        want += [np.float32(std * r * np.cos(2 * np.pi * u2)), np.float32(std * r * np.sin(2 * np.pi * u2))]
    got = np.zeros(16, np.float32)
    L.ember_synth_fill_row(seed, name, row, std, got.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 16)
    assert np.array_equal(got, np.array(want, np.float32))


def test_generator_is_deterministic_and_shaped(tmp_path):
    cfg = configs.TINY["t_bias"]
    a, b = str(tmp_path / "a.ember"), str(tmp_path / "b.ember")
    for p, th in ((a, 1), (b, 5)):
        assert L.ember_synth_write(p.encode(), ctypes.byref(configs.synth_config(cfg, th))) == 0
    assert open(a, "rb").read() == open(b, "rb").read()       # thread count does not matter
    m = L.ember_model_load(a.encode())
    hd = L.ember_model_header(m).contents
    assert (hd.dim, hd.n_layers, hd.vocab_size, hd.flags) == (128, 2, 448, _native.FLAG_TIED_EMBED)
    t = L.ember_model_tensor(m, b"layers.1.wq_bias").contents
    assert t.dtype == _native.DT_F32 and t.ndim == 1 and t.shape[0] == 256
    t = L.ember_model_tensor(m, b"layers.0.w2").contents
    assert t.dtype == _native.DT_Q8_0 and list(t.shape)[:2] == [128, 256] and t.offset % 64 == 0
    L.ember_model_free(m)


def test_libm_expf_restatement_equals_the_c_library():
    """The expf the reference-order kernels use (emberllm_amd/csrc/hip/
    libm_expf.h, evaluated on the host through ehip_libm_expf) equals the
    host C library's expf, the function the reference's softmax and SwiGLU
    call (src/model.c:61, 405), bit for bit: every 61st float bit pattern
    (about 70 million inputs, both signs, every exponent, NaN and the
    infinities) plus the edges of the special-case ranges."""
    import oracle
    lib = _native.lib()
    olib = oracle.oracle_lib()
    bits = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0x42b00000, 0xc2b00000, 0x42b17217, 0x42b17218, 0xc2cff1b4, 0xc2cff1b5, 0x7f800000,
                      0xff800000, 0x7fc00000, 0x00000001, 0x80000001, 0x3f800000, 0xbf800000], dtype=np.uint32)
    x = np.concatenate([bits, edges]).view(np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    got = np.empty_like(x)
    want = np.empty_like(x)
    lib.ehip_libm_expf(x.ctypes.data_as(fp), got.ctypes.data_as(fp), len(x))
    olib.orc_expf_n(x.ctypes.data_as(fp), want.ctypes.data_as(fp), len(x))
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same)
    assert bad.size == 0, [(hex(int(x.view(np.uint32)[i])), float(got[i]), float(want[i])) for i in bad[:8]]
    # against the correctly rounded exponential it differs now and then: the
    # reason the restatement exists
    fin = np.isfinite(x) & (np.abs(x) < 80)
    cr = np.exp(x[fin].astype(np.float64)).astype(np.float32)
    assert np.mean(cr != want[fin]) > 1e-5   # 7.5e-5 of these bit patterns (6e-4 of uniform [-20, 0])
