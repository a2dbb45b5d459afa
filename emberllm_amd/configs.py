"""Model shapes of the benchmark workloads and of the small parity models,
plus a cache of their seeded synthetic .ember files.

Real shapes (weights drawn N(0, 0.02), norms 1.0, encoded by the package's
bit-exact quantizer; see csrc/host/synth.c for the generator):
  stories110m   dim 768, 12 layers, 12/12 heads of 64, FFN 2048, vocab 32000,
                interleaved RoPE theta 1e4, max_seq 1024, eps 1e-5
  smollm2_135m  dim 576, 30 layers, 9/3 heads of 64, FFN 1536, vocab 49152,
                tied, NEOX RoPE theta 1e5, eps 1e-5
  qwen25_05b    dim 896, 24 layers, 14/2 heads of 64, FFN 4864, vocab 151936,
                QKV bias, tied, NEOX theta 1e6, eps 1e-6
  qwen3_06b     dim 1024, 28 layers, 16/8 heads of 128, FFN 3072, vocab
                151936, QK-norm, tied, NEOX theta 1e6, eps 1e-6 (Q8_0 and Q4_0)
All are tied, which matches the reference's published file sizes.
"""
import ctypes
import hashlib
import os
import tempfile

from . import _native

SEED = 20240601


def _cfg(dim, hidden, layers, heads, kv, hd, vocab, max_seq, theta, eps, rope, *,
         qk_norm=0, bias=0, tied=1, dtype=_native.DT_Q8_0, seed=SEED, std=0.02):
    return dict(dim=dim, hidden_dim=hidden, n_layers=layers, n_heads=heads, n_kv_heads=kv,
                head_dim=hd, vocab_size=vocab, max_seq_len=max_seq, rope_theta=theta,
                norm_eps=eps, rope_style=rope, qk_norm=qk_norm, qkv_bias=bias, tied=tied,
                dtype=dtype, seed=seed, std=std)


I, N = _native.ROPE_INTERLEAVED, _native.ROPE_NEOX

REAL = {
    "stories110m": _cfg(768, 2048, 12, 12, 12, 64, 32000, 1024, 1e4, 1e-5, I),
    "smollm2_135m": _cfg(576, 1536, 30, 9, 3, 64, 49152, 8192, 1e5, 1e-5, N),
    "qwen25_05b": _cfg(896, 4864, 24, 14, 2, 64, 151936, 32768, 1e6, 1e-6, N, bias=1),
    "qwen3_06b": _cfg(1024, 3072, 28, 16, 8, 128, 151936, 40960, 1e6, 1e-6, N, qk_norm=1),
    "qwen3_06b_q4": _cfg(1024, 3072, 28, 16, 8, 128, 151936, 40960, 1e6, 1e-6, N, qk_norm=1,
                         dtype=_native.DT_Q4_0),
}

# Small models that exercise every variant of the forward pass.
TINY = {
    "t_llama": _cfg(128, 256, 2, 2, 2, 64, 512, 64, 1e4, 1e-5, I),
    "t_gqa": _cfg(192, 320, 2, 3, 1, 64, 384, 64, 1e5, 1e-5, N),
    "t_bias": _cfg(128, 256, 2, 4, 2, 64, 448, 64, 1e6, 1e-6, N, bias=1),
    "t_qwen3": _cfg(128, 384, 2, 4, 2, 128, 640, 96, 1e6, 1e-6, N, qk_norm=1, tied=0),
    "t_q4": _cfg(128, 384, 2, 4, 2, 128, 640, 96, 1e6, 1e-6, N, qk_norm=1, dtype=_native.DT_Q4_0),
    "t_f32": _cfg(96, 192, 2, 2, 1, 48, 320, 64, 1e4, 1e-5, I, dtype=_native.DT_F32),
    "t_g7": _cfg(128, 256, 2, 7, 1, 64, 384, 320, 1e6, 1e-6, N, bias=1),
}

# Qwen3-0.6B width and heads with 2 layers and a small vocabulary: reaches the
# prefill GEMM tiles of the real shape (64- and 128-token MFMA tiles) and a
# second 2048-token prefill pass while the oracle stays fast.
WIDE = {
    "w_qwen3": _cfg(1024, 3072, 2, 16, 8, 128, 4096, 4608, 1e6, 1e-6, N, qk_norm=1),
    "w_qwen3_q4": _cfg(1024, 3072, 2, 16, 8, 128, 4096, 4608, 1e6, 1e-6, N, qk_norm=1,
                       dtype=_native.DT_Q4_0),
}

ALL = dict(REAL, **TINY, **WIDE)


def synth_config(cfg, threads=0):
    c = _native.EmberSynthConfig()
    for k, v in cfg.items():
        setattr(c, k, v)
    c.threads = threads
    return c


def cache_dir():
    d = os.environ.get("EMBER_MODEL_CACHE") or os.path.join(tempfile.gettempdir(), "ember_models")
    os.makedirs(d, exist_ok=True)
    return d


def key(cfg):
    return hashlib.sha1(repr(sorted(cfg.items())).encode()).hexdigest()[:12]


def model_path(name, cfg=None, threads=0):
    """Path of the synthetic model `name` (generated on first use)."""
    cfg = cfg or ALL[name]
    path = os.path.join(cache_dir(), f"{name}-{key(cfg)}.ember")
    if not os.path.exists(path):
        tmp = f"{path}.{os.getpid()}.tmp"
        rc = _native.lib().ember_synth_write(tmp.encode(), ctypes.byref(synth_config(cfg, threads)))
        if rc != 0:
            raise RuntimeError(f"writing {tmp} failed")
        os.replace(tmp, path)
    return path


def file_sha1(path):
    h = hashlib.sha1()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 22), b""):
            h.update(chunk)
    return h.hexdigest()
