"""ctypes binding of the oracle (oracle/ref_cpu.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product never imports it.  Every function here forwards to the C restatement
of the reference CPU path; see ref_cpu.h for the reference file:line each one
follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_F = C.POINTER(C.c_float)
_U16 = C.POINTER(C.c_uint16)
_I8 = C.POINTER(C.c_int8)
_U8 = C.POINTER(C.c_uint8)
_I32 = C.POINTER(C.c_int32)


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden_dim", "num_q_heads", "num_kv_heads", "head_dim", "ffn_dim", "num_layers",
        "vocab_size")] + [("rms_eps", C.c_float), ("rope_theta", C.c_float)] + [
        (n, C.c_int) for n in ("tie_word_embeddings", "rope_style", "has_qk_norm", "num_lm_heads",
                               "lm_head_vocab_size", "disable_npu_lm_head", "max_batch_prefill")]


def build() -> str:
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_vec_f32_to_f16": (None, [_U16, _F, C.c_size_t]),
            "orc_vec_f16_to_f32": (None, [_F, _U16, C.c_size_t]),
            "orc_seed_for": (C.c_uint64, [C.c_uint64, C.c_char_p]),
            "orc_fill_normal_f32": (None, [_F, C.c_size_t, C.c_uint64, C.c_double, C.c_double]),
            "orc_rms_norm": (None, [_F, _F, _F, C.c_int, C.c_float]),
            "orc_rope_tables": (None, [_F, _F, C.c_int, C.c_int, C.c_float]),
            "orc_apply_rope": (None, [_F, _F, _F, C.c_int, C.c_int, C.c_int]),
            "orc_apply_rope_batch": (None, [_F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int]),
            "orc_attention": (None, [_F, _F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int]),
            "orc_attention_batch_causal": (None, [_F, _F, _F, _F, _F, _F, C.c_int, C.c_int, C.c_int,
                                                  C.c_int, C.c_int]),
            "orc_silu_mul": (None, [_F, _F, _F, C.c_int]),
            "orc_vec_add": (None, [_F, _F, C.c_int]),
            "orc_argmax": (C.c_int, [_F, C.c_int]),
            "orc_sample_topk": (C.c_int, [_F, C.c_int, _I32, C.c_int, C.c_float, C.c_int, C.c_float,
                                          C.c_float, C.c_float, _I32, _F, _I32]),
            "orc_matmul_f16": (None, [_F, _F, _U16, C.c_int, C.c_int, C.c_int]),
            "orc_set_accum_order": (None, [C.c_int]),
            "orc_matmul_i8": (None, [_F, _F, _I8, _F, C.c_int, C.c_int, C.c_int]),
            "orc_matmul_i4": (None, [_F, _F, _U8, _F, C.c_int, C.c_int, C.c_int]),
            "orc_gemv_rows_f16": (None, [_F, _F, _U16, C.c_int, C.c_int]),
            "orc_gemv_rows_f32": (None, [_F, _F, _F, C.c_int, C.c_int]),
            "orc_quantize_lm_head": (None, [_I8, _F, _U16, C.c_int, C.c_int]),
            "orc_model_open": (C.c_void_p, [C.c_char_p, C.POINTER(OrcConfig), C.c_int, C.c_int, C.c_int]),
            "orc_model_close": (None, [C.c_void_p]),
            "orc_model_step": (C.c_int, [C.c_void_p, C.c_int, _F, _F]),
            "orc_model_step_head": (C.c_int, [C.c_void_p, C.c_int, _F, C.c_int, _F]),
            "orc_model_prefill_batch": (C.c_int, [C.c_void_p, _F, C.c_int]),
            "orc_model_seq_len": (C.c_int, [C.c_void_p]),
            "orc_model_set_seq_len": (None, [C.c_void_p, C.c_int]),
            "orc_model_kv_fill_normal": (C.c_int, [C.c_void_p, C.c_int, C.c_uint64]),
            "orc_model_kv_read": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, _F, _F]),
            "orc_model_last_normed": (None, [C.c_void_p, _F]),
            "orc_model_lm_q": (_I8, [C.c_void_p]),
            "orc_model_lm_scales": (_F, [C.c_void_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- element-wise ops ------------------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_vec_f32_to_f16(_p(out, _U16), _p(x, _F), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().orc_vec_f16_to_f32(_p(out, _F), _p(h, _U16), h.size)
    return out


def seed_for(base: int, name: str) -> int:
    return lib().orc_seed_for(base, name.encode())


def fill_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(_p(out, _F), n, seed, mean, std)
    return out


def rms_norm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().orc_rms_norm(_p(out, _F), _p(x, _F), _p(w, _F), x.size, eps)
    return out


def rope_tables(max_seq: int, head_dim: int, theta: float):
    c = np.empty((max_seq, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_tables(_p(c, _F), _p(s, _F), max_seq, head_dim, theta)
    return c, s


def apply_rope(x, cos_row, sin_row, num_heads: int, head_dim: int, style: int) -> np.ndarray:
    x = _f32(x).copy()
    c, s = _f32(cos_row), _f32(sin_row)
    lib().orc_apply_rope(_p(x, _F), _p(c, _F), _p(s, _F), num_heads, head_dim, style)
    return x


def apply_rope_batch(x, M, start, num_heads, head_dim, theta, style) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_apply_rope_batch(_p(x, _F), M, start, num_heads, head_dim, theta, style)
    return x


def attention(q, kc, vc, nq: int, nkv: int, hd: int, L: int) -> np.ndarray:
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    out = np.empty(nq * hd, np.float32)
    lib().orc_attention(_p(out, _F), _p(q, _F), _p(kc, _F), _p(vc, _F), nq, nkv, hd, L)
    return out


def attention_batch_causal(qb, kb, vb, kc, vc, M, nq, nkv, hd, S) -> np.ndarray:
    qb, kb, vb = _f32(qb), _f32(kb), _f32(vb)
    kc = _f32(kc) if S > 0 else np.zeros(1, np.float32)
    vc = _f32(vc) if S > 0 else np.zeros(1, np.float32)
    out = np.empty(M * nq * hd, np.float32)
    lib().orc_attention_batch_causal(_p(out, _F), _p(qb, _F), _p(kb, _F), _p(vb, _F), _p(kc, _F),
                                     _p(vc, _F), M, nq, nkv, hd, S)
    return out


def silu_mul(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().orc_silu_mul(_p(out, _F), _p(g, _F), _p(u, _F), g.size)
    return out


def argmax(x) -> int:
    x = _f32(x)
    return lib().orc_argmax(_p(x, _F), x.size)


def sample_topk(logits, top_k=1, temperature=1.0, top_p=1.0, u=0.0, repeat_tokens=(),
                repeat_penalty=1.0):
    """Top-k sampling with the given uniform (src/cpu_ops.c:593-648 with u in
    place of rand()/RAND_MAX); top_k is clamped to [1, V].  Returns (token,
    candidate indices, candidate values after temperature, kept after top-p)."""
    x = np.array(logits, dtype=np.float32, copy=True).ravel()
    k = max(1, min(int(top_k), x.size))
    rep = np.ascontiguousarray(np.asarray(repeat_tokens, dtype=np.int32).ravel())
    idx = np.zeros(k, np.int32)
    val = np.zeros(k, np.float32)
    kept = np.zeros(1, np.int32)
    tok = lib().orc_sample_topk(_p(x, _F), x.size, _p(rep, _I32), rep.size, float(repeat_penalty), k,
                                float(temperature), float(top_p), float(u), _p(idx, _I32),
                                _p(val, _F), _p(kept, _I32))
    return tok, idx, val, int(kept[0])


# ---- projections -------------------------------------------------------------

def matmul(kind: int, x, w, scale, M: int, K: int, N: int) -> np.ndarray:
    """kind 0 fp16 [K,N] bits, 1 int8 [K,N], 2 int4 [K,N/2]; x fp32 [M,K]."""
    x = _f32(x)
    y = np.empty(M * N, np.float32)
    sp = None
    if scale is not None:
        scale = _f32(scale)
        sp = _p(scale, _F)
    if kind == 0:
        w = np.ascontiguousarray(w, np.uint16)
        lib().orc_matmul_f16(_p(y, _F), _p(x, _F), _p(w, _U16), M, K, N)
    elif kind == 1:
        w = np.ascontiguousarray(w, np.int8)
        lib().orc_matmul_i8(_p(y, _F), _p(x, _F), _p(w, _I8), sp, M, K, N)
    else:
        w = np.ascontiguousarray(w, np.uint8)
        lib().orc_matmul_i4(_p(y, _F), _p(x, _F), _p(w, _U8), sp, M, K, N)
    return y.reshape(M, N)


def gemv_rows_f16(x, w16, N: int, K: int) -> np.ndarray:
    x = _f32(x)
    w16 = np.ascontiguousarray(w16, np.uint16)
    out = np.empty(N, np.float32)
    lib().orc_gemv_rows_f16(_p(out, _F), _p(x, _F), _p(w16, _U16), N, K)
    return out


def gemv_rows_f32(x, w, N: int, K: int) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty(N, np.float32)
    lib().orc_gemv_rows_f32(_p(out, _F), _p(x, _F), _p(w, _F), N, K)
    return out


def quantize_lm_head(lm16, V: int, K: int):
    lm16 = np.ascontiguousarray(lm16, np.uint16)
    q = np.empty(V * K, np.int8)
    s = np.empty(V, np.float32)
    lib().orc_quantize_lm_head(_p(q, _I8), _p(s, _F), _p(lm16, _U16), V, K)
    return q.reshape(V, K), s


# ---- the decoder ---------------------------------------------------------------

def config_from_dict(d: dict) -> OrcConfig:
    c = OrcConfig()
    for name, _ in OrcConfig._fields_:
        if name in d:
            setattr(c, name, type(getattr(c, name))(d[name]))
    if "max_batch_prefill" not in d:
        c.max_batch_prefill = 64
    return c


class Model:
    """The oracle decoder over a model directory in the reference format."""

    def __init__(self, model_dir: str, cfg: dict, quant: int, max_seq: int, kv_fp16: bool = True):
        self.cfg = dict(cfg)
        self._c = config_from_dict(cfg)
        self.h = lib().orc_model_open(model_dir.encode(), C.byref(self._c), quant, max_seq,
                                      1 if kv_fp16 else 0)
        if not self.h:
            raise RuntimeError(f"oracle could not open {model_dir}")
        self.V = cfg["vocab_size"]
        self.d = cfg["hidden_dim"]
        self.kvd = cfg["num_kv_heads"] * cfg["head_dim"]

    def close(self):
        if self.h:
            lib().orc_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def step(self, token: int = 0, embedding=None, logits: bool = True):
        e = _f32(embedding) if embedding is not None else None
        out = np.empty(self.V, np.float32) if logits else None
        tok = lib().orc_model_step(self.h, token, _p(e, _F) if e is not None else None,
                                   _p(out, _F) if out is not None else None)
        return tok, out

    def step_head(self, token: int, head: int, embedding=None, n_logits: int | None = None):
        e = _f32(embedding) if embedding is not None else None
        out = np.empty(n_logits or self.V, np.float32)
        tok = lib().orc_model_step_head(self.h, token, _p(e, _F) if e is not None else None, head,
                                        _p(out, _F))
        return tok, out

    def prefill_batch(self, emb) -> int:
        e = _f32(emb)
        return lib().orc_model_prefill_batch(self.h, _p(e, _F), e.shape[0])

    @property
    def seq_len(self) -> int:
        return lib().orc_model_seq_len(self.h)

    @seq_len.setter
    def seq_len(self, n: int):
        lib().orc_model_set_seq_len(self.h, n)

    def kv_fill_normal(self, n_pos: int, seed: int) -> int:
        return lib().orc_model_kv_fill_normal(self.h, n_pos, seed)

    def kv_read(self, layer: int, pos0: int, n: int):
        k = np.empty(n * self.kvd, np.float32)
        v = np.empty_like(k)
        rc = lib().orc_model_kv_read(self.h, layer, pos0, n, _p(k, _F), _p(v, _F))
        if rc:
            raise ValueError("kv_read out of range")
        return k.reshape(n, self.kvd), v.reshape(n, self.kvd)

    def last_normed(self) -> np.ndarray:
        out = np.empty(self.d, np.float32)
        lib().orc_model_last_normed(self.h, _p(out, _F))
        return out

    def lm_head_q(self):
        q = lib().orc_model_lm_q(self.h)
        s = lib().orc_model_lm_scales(self.h)
        if not q:
            return None, None
        qa = np.ctypeslib.as_array(q, shape=(self.V * self.d,)).copy().reshape(self.V, self.d)
        sa = np.ctypeslib.as_array(s, shape=(self.V,)).copy()
        return qa, sa

    def greedy(self, first_token: int, n: int) -> tuple[list[int], list[float]]:
        """n greedy steps feeding each argmax back; returns tokens and the
        top-1 minus top-2 logit margin of every step."""
        toks, margins = [], []
        t = first_token
        for _ in range(n):
            t, lg = self.step(t)
            top2 = np.partition(lg, -2)[-2:]
            margins.append(float(top2[1] - top2[0]))
            toks.append(int(t))
        return toks, margins
