"""ctypes binding of libmatmul_decoder.so (the C ABI of this package).

Plumbing for Python callers, tests and the benchmark: it loads the in-tree
library built by build.py and exposes the functions of matmul_decoder.h,
rknn_matmul_parallel.h and mdx_ext.h with numpy-friendly wrappers.  Loading
fails loudly when the library has not been built; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmatmul_decoder.so")

QUANT = {"fp16": 0, "int8": 1, "int4": 2, "int4_g128": 3}

_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int)
_U16 = C.POINTER(C.c_uint16)
_I8 = C.POINTER(C.c_int8)


class MatmulDecoderConfig(C.Structure):
    """Mirror of MatmulDecoderConfig (include/matmul_decoder.h)."""
    _fields_ = [
        ("name", C.c_char_p),
        ("hidden_dim", C.c_int), ("num_q_heads", C.c_int), ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("ffn_dim", C.c_int), ("num_layers", C.c_int),
        ("vocab_size", C.c_int), ("max_seq_len", C.c_int),
        ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("tie_word_embeddings", C.c_int),
        ("rope_scaling_factor", C.c_float), ("rope_scaling_type", C.c_int),
        ("norm_type", C.c_int), ("rope_style", C.c_int), ("ffn_act_type", C.c_int),
        ("has_qk_norm", C.c_int), ("num_lm_heads", C.c_int), ("lm_head_vocab_size", C.c_int),
        ("context_pool_mode", C.c_int), ("iommu_domain_id", C.c_int), ("exec_mode", C.c_int),
        ("disable_npu_lm_head", C.c_int), ("max_batch_prefill", C.c_int),
    ]


class MatmulDecoderStats(C.Structure):
    _fields_ = [("total_ms", C.c_float), ("matmul_ms", C.c_float), ("rebind_ms", C.c_float),
                ("convert_ms", C.c_float), ("cpu_ops_ms", C.c_float), ("lm_head_ms", C.c_float),
                ("n_steps", C.c_int)]


class SamplingParams(C.Structure):
    """Mirror of SamplingParams (include/matmul_decoder.h)."""
    _fields_ = [("top_k", C.c_int), ("top_p", C.c_float), ("temperature", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_tokens", _I), ("n_repeat_tokens", C.c_int)]


def sampling_params(top_k=1, top_p=1.0, temperature=1.0, repeat_penalty=1.0, repeat_tokens=()):
    """SamplingParams plus the int32 array its repeat_tokens points into (keep
    both alive for the call)."""
    toks = np.ascontiguousarray(np.asarray(repeat_tokens, dtype=np.int32).ravel())
    p = SamplingParams(top_k=int(top_k), top_p=float(top_p), temperature=float(temperature),
                       repeat_penalty=float(repeat_penalty),
                       repeat_tokens=_p(toks, _I) if toks.size else None, n_repeat_tokens=toks.size)
    return p, toks


class RmpConfig(C.Structure):
    _fields_ = [("M", C.c_int), ("K", C.c_int), ("N", C.c_int), ("type", C.c_int),
                ("layout", C.c_int), ("n_workers", C.c_int)]


def qwen3_0_6b_config(**overrides) -> MatmulDecoderConfig:
    """matmul_decoder_config_qwen3_0_6b() with field overrides."""
    c = MatmulDecoderConfig(
        name=b"qwen3-asr-0.6b", hidden_dim=1024, num_q_heads=16, num_kv_heads=8, head_dim=128,
        ffn_dim=3072, num_layers=28, vocab_size=151936, max_seq_len=4096, rms_eps=1e-6,
        rope_theta=1e6, tie_word_embeddings=1, rope_scaling_factor=1.0, rope_scaling_type=0,
        norm_type=0, rope_style=0, ffn_act_type=0, has_qk_norm=1, num_lm_heads=0,
        lm_head_vocab_size=0, context_pool_mode=0, iommu_domain_id=1, exec_mode=1,
        disable_npu_lm_head=0, max_batch_prefill=64)
    for k, v in overrides.items():
        if k == "name" and isinstance(v, str):
            v = v.encode()
        setattr(c, k, v)
    return c


def config_dict(c: MatmulDecoderConfig) -> dict:
    return {n: getattr(c, n) for n, _ in MatmulDecoderConfig._fields_ if n != "name"}


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run build.py (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        sig = {
            "matmul_decoder_create": (P, [C.c_char_p, C.POINTER(MatmulDecoderConfig), C.c_int, C.c_int]),
            "matmul_decoder_destroy": (None, [P]),
            "matmul_decoder_step": (C.c_int, [P, C.c_int, _F, _F]),
            "matmul_decoder_step_get_logits": (C.c_int, [P, C.c_int, _F, _F]),
            "matmul_decoder_step_head": (C.c_int, [P, C.c_int, _F, C.c_int, _F]),
            "matmul_decoder_prefill_batch": (C.c_int, [P, _F, C.c_int]),
            "matmul_decoder_clear_kv_cache": (None, [P]),
            "matmul_decoder_get_seq_len": (C.c_int, [P]),
            "matmul_decoder_get_config": (C.POINTER(MatmulDecoderConfig), [P]),
            "matmul_decoder_get_stats": (None, [P, C.POINTER(MatmulDecoderStats)]),
            "matmul_decoder_load_config": (C.c_int, [C.c_char_p, C.POINTER(MatmulDecoderConfig)]),
            "matmul_sample_token": (C.c_int, [_F, C.c_int, P]),
            "matmul_kv_cache_create": (P, [C.c_int, C.c_int, C.c_int, C.c_int]),
            "matmul_kv_cache_clear": (None, [P]),
            "matmul_kv_cache_get_seq_len": (C.c_int, [P]),
            "matmul_kv_cache_destroy": (None, [P]),
            "rmp_create": (P, [C.POINTER(RmpConfig), P, _F]),
            "rmp_run": (C.c_int, [P, _U16, _F]),
            "rmp_destroy": (None, [P]),
            "rmp_benchmark": (C.c_float, [P, C.c_int]),
            "rmp_get_single_core_time": (C.c_float, [P]),
            "mdx_version": (C.c_char_p, []),
            "mdx_device_count": (C.c_int, []),
            "mdx_copy_probe": (C.c_int, [C.c_size_t, C.c_int]),
            "mdx_last_error": (C.c_char_p, []),
            "mdx_step_token": (C.c_int, [P, C.c_int, _F]),
            "mdx_decode_path": (C.c_int, [P]),
            "mdx_debug_persist_spin_limit": (C.c_int, [P, C.c_uint]),
            "mdx_debug_persist_kv_stream": (C.c_int, [P, C.c_int]),
            "mdx_debug_persist_local_exchange": (C.c_int, [P, C.c_int]),
            "mdx_debug_persist_poison_retry": (C.c_int, [P]),
            "mdx_trace_step": (C.c_int, [P, C.c_int, C.POINTER(C.c_uint64), C.c_int]),
            "mdx_kv_fill_normal": (C.c_int, [P, C.c_int, C.c_uint64]),
            "mdx_kv_read": (C.c_int, [P, C.c_int, C.c_int, C.c_int, _F, _F]),
            "mdx_prefill_logits": (C.c_int, [P, _F, C.c_int, _F]),
            "mdx_generate_greedy": (C.c_int, [P, C.c_int, C.c_int, _I, _F]),
            "mdx_time_projection": (C.c_int, [P, C.c_char_p, C.c_int, _F, C.POINTER(C.c_double)]),
            "mdx_time_prefill": (C.c_int, [P, _F, C.c_int, C.c_int, _F]),
            "mdx_time_gemv": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F]),
            "mdx_sample_topk_noalloc": (C.c_int, [P, C.c_int, C.c_float, C.c_int, C.c_float, C.c_float,
                                                  P, P, P, P]),
            "mdx_device_malloc": (C.c_int, [C.POINTER(C.c_void_p), C.c_size_t]),
            "mdx_device_free": (C.c_int, [P]),
            "mdx_memcpy_h2d": (C.c_int, [P, P, C.c_size_t]),
            "mdx_memcpy_d2h": (C.c_int, [P, P, C.c_size_t]),
            "mdx_device_synchronize": (C.c_int, []),
            "mdx_debug_gemv": (C.c_int, [C.c_int, C.c_int, C.c_int, P, _F, _F, _F]),
            "mdx_debug_gemm": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, P, _F, _F, _F]),
            "mdx_debug_gemm_splits": (C.c_int, [C.c_int, C.c_int, C.c_int, _I]),
            "mdx_debug_persist_kv_rows": (C.c_longlong, [C.c_int, C.c_int, C.POINTER(C.c_longlong)]),
            "mdx_debug_gemm_residual": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, P, _F, _F, _F,
                                                  _F, C.c_float, C.POINTER(C.c_uint16)]),
            "mdx_debug_attn_decode": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                C.c_float, _F, _F, _F, _U16, _U16, _F, _U16, _U16]),
            "mdx_debug_attn_prefill": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F, _U16,
                                                 _U16, _F]),
            "mdx_debug_qk_rope": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                            C.c_float, _F, _F, _F, _F, _U16, _U16]),
            "mdx_debug_lmhead": (C.c_int, [C.c_int, C.c_int, C.c_int, P, _F, _F, _F, C.c_float, _F]),
            "mdx_debug_sample": (C.c_int, [_F, C.c_int, C.POINTER(SamplingParams), C.c_float, _I, _I, _F]),
            "matmul_decoder_step_sample": (C.c_int, [P, C.c_int, _F, C.POINTER(SamplingParams), C.c_float,
                                                     _F]),
            "mdx_quantize_lm_head": (None, [_I8, _F, _U16, C.c_int, C.c_int]),
            "mdx_f32_to_f16": (C.c_uint16, [C.c_float]),
            "mdx_f16_to_f32": (C.c_float, [C.c_uint16]),
            "mdx_synth_seed": (C.c_uint64, [C.c_uint64, C.c_char_p]),
            "mdx_synth_fill_normal": (None, [_F, C.c_size_t, C.c_uint64, C.c_double, C.c_double]),
            "matmul_decoder_export_hf_model": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int]),
            "mdx_synth_write_model": (C.c_int, [C.c_char_p, C.POINTER(MatmulDecoderConfig), C.c_int,
                                                C.c_uint64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def device_count() -> int:
    return lib().mdx_device_count()


def last_error() -> str:
    return lib().mdx_last_error().decode(errors="replace")


# ---- host helpers --------------------------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    x = _f32(x).ravel()
    f = lib().mdx_f32_to_f16
    return np.array([f(float(v)) for v in x], np.uint16)


def synth_seed(base: int, name: str) -> int:
    return lib().mdx_synth_seed(base, name.encode())


def synth_fill_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().mdx_synth_fill_normal(_p(out, _F), n, seed, mean, std)
    return out


def quantize_lm_head(lm16, V: int, K: int):
    lm16 = np.ascontiguousarray(lm16, np.uint16)
    q = np.empty(V * K, np.int8)
    s = np.empty(V, np.float32)
    lib().mdx_quantize_lm_head(_p(q, _I8), _p(s, _F), _p(lm16, _U16), V, K)
    return q.reshape(V, K), s


QUANT_NAMES = {"fp16": 0, "int8": 1, "int4": 2, "int4_g128": 3}


def export_hf_model(hf_dir: str, out_dir: str, quant: str = "fp16") -> None:
    """matmul_decoder_export_hf_model: a local HuggingFace checkpoint
    (config.json + *.safetensors) to the reference on-disk format."""
    rc = lib().matmul_decoder_export_hf_model(hf_dir.encode(), out_dir.encode(), QUANT_NAMES[quant])
    if rc != 0:
        raise RuntimeError(f"matmul_decoder_export_hf_model failed ({rc})")


def write_model(path: str, cfg: MatmulDecoderConfig, quant: int, seed: int) -> None:
    rc = lib().mdx_synth_write_model(path.encode(), C.byref(cfg), quant, seed)
    if rc != 0:
        raise RuntimeError(f"mdx_synth_write_model failed ({rc})")


def load_config(path: str) -> MatmulDecoderConfig:
    c = MatmulDecoderConfig()
    rc = lib().matmul_decoder_load_config(path.encode(), C.byref(c))
    if rc != 0:
        raise RuntimeError(f"load_config failed ({rc})")
    return c


# ---- single-kernel entry points -------------------------------------------------

def _check(rc: int, what: str) -> int:
    if rc < 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")
    return rc


def gemv(kind: int, K: int, N: int, w: np.ndarray, scales, x) -> np.ndarray:
    w = np.ascontiguousarray(w)
    y = np.empty(N, np.float32)
    s, x = _f32(scales), _f32(x)
    _check(lib().mdx_debug_gemv(kind, K, N, w.ctypes.data, _p(s, _F), _p(x, _F), _p(y, _F)), "gemv")
    return y


def gemm(kind: int, M: int, K: int, N: int, w: np.ndarray, scales, x) -> np.ndarray:
    w = np.ascontiguousarray(w)
    y = np.empty(M * N, np.float32)
    s, x = _f32(scales), _f32(x)
    _check(lib().mdx_debug_gemm(kind, M, K, N, w.ctypes.data, _p(s, _F), _p(x, _F), _p(y, _F)),
           "gemm")
    return y.reshape(M, N)


def gemm_residual(kind: int, M: int, K: int, N: int, w: np.ndarray, scales, x, hidden, norm_w,
                  eps: float = 1e-6):
    """Prefill residual projection: (hidden + fp16(x) . W * scale, fp16 normed rows or None)."""
    w = np.ascontiguousarray(w)
    s, x = _f32(scales), _f32(x)
    h = np.array(_f32(hidden), dtype=np.float32, copy=True).reshape(M, N)
    nw = _f32(norm_w)
    out = np.zeros((M, N), np.uint16) if norm_w is not None else None
    _check(lib().mdx_debug_gemm_residual(kind, M, K, N, w.ctypes.data, _p(s, _F), _p(x, _F),
                                         _p(h, _F), _p(nw, _F), eps,
                                         out.ctypes.data_as(C.POINTER(C.c_uint16)) if out is not None
                                         else None), "gemm_residual")
    return h, out


def attn_decode(nq, nkv, hd, pos, style, theta, eps, q_norm, k_norm, qkv, k16, v16):
    """Fused decode attention at position pos; returns (out fp32, k_new16, v_new16)."""
    qkv = _f32(qkv)
    qn, kn = _f32(q_norm), _f32(k_norm)
    k16 = np.ascontiguousarray(k16, np.uint16) if pos > 0 else None
    v16 = np.ascontiguousarray(v16, np.uint16) if pos > 0 else None
    out = np.empty(nq * hd, np.float32)
    kn16 = np.empty(nkv * hd, np.uint16)
    vn16 = np.empty(nkv * hd, np.uint16)
    _check(lib().mdx_debug_attn_decode(nq, nkv, hd, pos, style, theta, eps, _p(qn, _F), _p(kn, _F),
                                       _p(qkv, _F), _p(k16, _U16), _p(v16, _U16), _p(out, _F),
                                       _p(kn16, _U16), _p(vn16, _U16)), "attn_decode")
    return out, kn16, vn16


def attn_prefill(nq, nkv, hd, S, M, q, k16, v16) -> np.ndarray:
    q = _f32(q)
    k16 = np.ascontiguousarray(k16, np.uint16)
    v16 = np.ascontiguousarray(v16, np.uint16)
    out = np.empty(M * nq * hd, np.float32)
    _check(lib().mdx_debug_attn_prefill(nq, nkv, hd, S, M, _p(q, _F), _p(k16, _U16), _p(v16, _U16),
                                        _p(out, _F)), "attn_prefill")
    return out.reshape(M, nq * hd)


def qk_rope(nq, nkv, hd, pos, style, theta, eps, q_norm, k_norm, qkv):
    qkv = _f32(qkv)
    qn, kn = _f32(q_norm), _f32(k_norm)
    q = np.empty(nq * hd, np.float32)
    k = np.empty(nkv * hd, np.uint16)
    v = np.empty(nkv * hd, np.uint16)
    _check(lib().mdx_debug_qk_rope(nq, nkv, hd, pos, style, theta, eps, _p(qn, _F), _p(kn, _F),
                                   _p(qkv, _F), _p(q, _F), _p(k, _U16), _p(v, _U16)), "qk_rope")
    return q, k, v


def time_gemv(kind: int, K: int, N: int, copies: int, iters: int) -> float:
    """Average device microseconds of one GEMV launch over rotated weight copies."""
    us = C.c_float(0.0)
    _check(lib().mdx_time_gemv(kind, K, N, copies, iters, C.byref(us)), "time_gemv")
    return float(us.value)


def lmhead(kind: int, K: int, N: int, w_rows, scales, hidden, norm_w, eps: float):
    w = np.ascontiguousarray(w_rows)
    s, h, nw = _f32(scales), _f32(hidden), _f32(norm_w)
    out = np.empty(N, np.float32)
    tok = _check(lib().mdx_debug_lmhead(kind, K, N, w.ctypes.data, _p(s, _F), _p(h, _F),
                                        _p(nw, _F), eps, _p(out, _F)), "lmhead")
    return tok, out


def sample(logits, top_k=1, temperature=1.0, top_p=1.0, u=0.0, repeat_tokens=(), repeat_penalty=1.0):
    """The device sampler on host logits: (token, candidate indices, candidate
    values after temperature, kept after top-p)."""
    x = _f32(logits).ravel()
    p, toks = sampling_params(top_k, top_p, temperature, repeat_penalty, repeat_tokens)
    k = max(1, min(int(top_k), x.size))
    out = np.zeros(2, np.int32)
    idx = np.zeros(k, np.int32)
    val = np.zeros(k, np.float32)
    _check(lib().mdx_debug_sample(_p(x, _F), x.size, C.byref(p), float(u), _p(out, _I), _p(idx, _I),
                                  _p(val, _F)), "sample")
    return int(out[0]), idx, val, int(out[1])


# ---- decoder ---------------------------------------------------------------------

class Decoder:
    """matmul_decoder_* on one context."""

    def __init__(self, model_dir: str, cfg: MatmulDecoderConfig | None, quant: str | int,
                 max_seq_len: int):
        q = QUANT[quant] if isinstance(quant, str) else quant
        self.h = lib().matmul_decoder_create(model_dir.encode(),
                                             C.byref(cfg) if cfg is not None else None, q, max_seq_len)
        if not self.h:
            raise RuntimeError(f"matmul_decoder_create failed: {last_error()}")
        c = lib().matmul_decoder_get_config(self.h).contents
        self.V = c.vocab_size
        self.d = c.hidden_dim
        self.kvd = c.num_kv_heads * c.head_dim
        self.n_lm = c.num_lm_heads
        self.lm_vocab = c.lm_head_vocab_size if c.num_lm_heads > 1 else c.vocab_size

    def trace_step(self, token: int) -> np.ndarray:
        """One traced one-launch step: [256 workgroups][events] timestamps."""
        cap = 256 * (16 * 64 + 4)
        out = np.zeros(cap, np.uint64)
        ev = lib().mdx_trace_step(self.h, token, out.ctypes.data_as(C.POINTER(C.c_uint64)), cap)
        _check(ev if ev < 0 else 0, "trace_step")
        return out[:256 * ev].reshape(256, ev)

    @property
    def path(self) -> int:
        """1: one launch per step; 0: per-stage kernels."""
        return lib().mdx_decode_path(self.h)

    def poison_next_retry(self):
        """Plant stale epoch-tagged exchange words before the next retry."""
        _check(lib().mdx_debug_persist_poison_retry(self.h), "poison_retry")

    def force_spin_limit(self, rounds: int):
        """Next one-launch step gives up a wait after `rounds` polls (test hook)."""
        _check(lib().mdx_debug_persist_spin_limit(self.h, rounds), "spin_limit")

    def force_kv_stream(self, mode: int):
        """K/V load policy of the one-launch step: -1 auto, 0 ordinary, 1 non-temporal."""
        _check(lib().mdx_debug_persist_kv_stream(self.h, mode), "kv_stream")

    def force_local_exchange(self, mode: int):
        """Per-head exchanges of the one-launch step: -1 auto, 0 through memory, 1 in the L2."""
        _check(lib().mdx_debug_persist_local_exchange(self.h, mode), "local_exchange")

    def close(self):
        if self.h:
            lib().matmul_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def step(self, token: int = 0, embedding=None, logits: bool = True):
        e = _f32(embedding)
        out = np.empty(self.V, np.float32) if logits else None
        tok = lib().matmul_decoder_step(self.h, token, _p(e, _F), _p(out, _F))
        return tok, out

    def step_into(self, token: int, out: np.ndarray, embedding=None) -> int:
        """matmul_decoder_step writing the logits into a caller-owned float32 buffer
        (reused across steps, as a C caller would)."""
        assert out.dtype == np.float32 and out.flags.c_contiguous and out.size >= self.V
        e = _f32(embedding)
        return lib().matmul_decoder_step(self.h, token, _p(e, _F), _p(out, _F))

    def step_sample(self, token: int, u: float, top_k=1, temperature=1.0, top_p=1.0, repeat_tokens=(),
                    repeat_penalty=1.0, embedding=None, logits: bool = False):
        """matmul_decoder_step_sample: one step, then sampling on the device.
        Returns (token or negative error, logits or None)."""
        e = _f32(embedding)
        p, toks = sampling_params(top_k, top_p, temperature, repeat_penalty, repeat_tokens)
        out = np.empty(self.V, np.float32) if logits else None
        tok = lib().matmul_decoder_step_sample(self.h, token, _p(e, _F), C.byref(p), float(u), _p(out, _F))
        return tok, out

    def step_token(self, token: int = 0, embedding=None) -> int:
        e = _f32(embedding)
        return lib().mdx_step_token(self.h, token, _p(e, _F))

    def step_head(self, token: int, head: int, embedding=None):
        e = _f32(embedding)
        out = np.empty(self.lm_vocab, np.float32)
        tok = lib().matmul_decoder_step_head(self.h, token, _p(e, _F), head, _p(out, _F))
        return tok, out

    def prefill_batch(self, emb) -> int:
        e = _f32(emb)
        return lib().matmul_decoder_prefill_batch(self.h, _p(e, _F), e.shape[0])

    def prefill_logits(self, emb):
        e = _f32(emb)
        out = np.empty(self.V, np.float32)
        tok = lib().mdx_prefill_logits(self.h, _p(e, _F), e.shape[0], _p(out, _F))
        return tok, out

    def clear(self):
        lib().matmul_decoder_clear_kv_cache(self.h)

    @property
    def seq_len(self) -> int:
        return lib().matmul_decoder_get_seq_len(self.h)

    def stats(self) -> dict:
        s = MatmulDecoderStats()
        lib().matmul_decoder_get_stats(self.h, C.byref(s))
        return {n: getattr(s, n) for n, _ in MatmulDecoderStats._fields_}

    def kv_fill_normal(self, n_pos: int, seed: int) -> None:
        _check(lib().mdx_kv_fill_normal(self.h, n_pos, seed), "kv_fill_normal")

    def kv_read(self, layer: int, pos0: int, n: int):
        k = np.empty(n * self.kvd, np.float32)
        v = np.empty_like(k)
        _check(lib().mdx_kv_read(self.h, layer, pos0, n, _p(k, _F), _p(v, _F)), "kv_read")
        return k.reshape(n, self.kvd), v.reshape(n, self.kvd)

    def generate_greedy(self, first_token: int, n: int):
        toks = np.empty(n, np.int32)
        ms = C.c_float(0.0)
        _check(lib().mdx_generate_greedy(self.h, first_token, n, _p(toks, _I), C.byref(ms)),
               "generate_greedy")
        return toks.tolist(), ms.value

    def time_projection(self, which: str, iters: int):
        us = C.c_float(0.0)
        b = C.c_double(0.0)
        _check(lib().mdx_time_projection(self.h, which.encode(), iters, C.byref(us), C.byref(b)),
               "time_projection")
        return us.value, b.value

    def time_prefill(self, emb, iters: int) -> float:
        e = _f32(emb)
        ms = C.c_float(0.0)
        _check(lib().mdx_time_prefill(self.h, _p(e, _F), e.shape[0], iters, C.byref(ms)),
               "time_prefill")
        return ms.value
