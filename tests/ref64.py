"""A float64 numpy restatement of the reference decoder's forward pass, used to
pin the oracle's layer composition.

It reads a model directory in the reference on-disk format directly (no call
into the oracle or the product) and follows:
  - the decode step src/matmul_decoder.c:1430-1634 (embedding, per layer
    RMSNorm -> q/k/v -> per-head QK-norm -> RoPE -> KV append -> GQA
    attention -> o -> residual -> RMSNorm -> gate/up -> SiLU*up -> down ->
    residual; final norm; INT8 lm_head tiles; argmax),
  - the multi-head step src/matmul_decoder.c:1636-1742 (fp32 lm_head rows,
    fp32 activations),
  - the batch prefill src/matmul_decoder.c:1901-2065 (row-wise the same
    layer with positions start+t and causal attention over the cache and the
    batch rows before it),
  - tests/generate_reference.py:60-217 for the same layer order.

Arithmetic is float64 everywhere except at the points where the reference
changes precision on purpose: fp32 activations rounded to fp16 at every NPU
projection input (vec_fp32_to_fp16, src/cpu_ops.c:383-395), K/V rounded to
fp16 when the cache is fp16, and the INT8 lm_head quantiser
(src/matmul_decoder.c:1216-1244), which is restated in float32 because its
bytes must match.  Projection outputs are not rounded (NPU type 1 and 5 write
fp32, include/rknn_matmul_api.h:71-85).

`faults` plants one composition mistake at a time (used by the tests to show
that a wrong composition is rejected).
"""
from __future__ import annotations

import json
import os

import numpy as np

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def f16(x) -> np.ndarray:
    """fp32 value rounded to fp16 (RNE), returned as float64."""
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def _read(path, dtype, n):
    a = np.fromfile(path, dtype=dtype)
    if a.size != n:
        raise ValueError(f"{path}: {a.size} elements, want {n}")
    return a


def _first(dirpath, names, n):
    for nm in names:
        p = os.path.join(dirpath, nm)
        if os.path.exists(p):
            return _read(p, np.float32, n).astype(np.float64)
    return None


def load_projection(layer_dir: str, name: str, K: int, N: int, quant: int) -> np.ndarray:
    """Dequantised [K, N] float64 weights in the on-disk semantic (the loader
    src/matmul_decoder.c:778-808): fp16 <name>.bin, or int8 / int4
    <name>_weight.bin with per-column fp32 <name>_scales.bin.  The int4 bytes
    hold column 2j in the low and 2j+1 in the high nibble, two's complement."""
    wpath = os.path.join(layer_dir, f"{name}_weight.bin")
    if quant != 0 and os.path.exists(wpath):
        s = _read(os.path.join(layer_dir, f"{name}_scales.bin"), np.float32, N).astype(np.float64)
        if quant == 1:
            q = _read(wpath, np.int8, K * N).reshape(K, N).astype(np.float64)
        else:
            b = _read(wpath, np.uint8, K * N // 2).reshape(K, N // 2)
            lo = (b & 0xF).astype(np.int16)
            hi = (b >> 4).astype(np.int16)
            lo = np.where(lo >= 8, lo - 16, lo)
            hi = np.where(hi >= 8, hi - 16, hi)
            q = np.empty((K, N), np.float64)
            q[:, 0::2] = lo
            q[:, 1::2] = hi
        return q * s[None, :]
    w = _read(os.path.join(layer_dir, f"{name}.bin"), np.float16, K * N)
    return w.reshape(K, N).astype(np.float64)


def quantize_lm_head_f32(lm16: np.ndarray):
    """Per vocab row: scale = max|v|/127, q = clamp((int)roundf(v * (127/max)),
    -128, 127), in float32 as src/matmul_decoder.c:1216-1244."""
    v = lm16.astype(np.float32)
    mx = np.max(np.abs(v), axis=1).astype(np.float32)
    scale = (mx / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(mx > 0, np.float32(127.0) / mx, np.float32(0.0)).astype(np.float32)
    prod = (v * inv[:, None]).astype(np.float32)
    # roundf: half away from zero
    r = np.sign(prod) * np.floor(np.abs(prod).astype(np.float64) + 0.5)
    q = np.clip(r, -128, 127).astype(np.int8)
    return q, scale


class Ref64:
    def __init__(self, model_dir: str, cfg: dict, quant: int, max_seq: int, kv_fp16: bool = True,
                 faults: frozenset = frozenset()):
        self.c = dict(cfg)
        self.kv_fp16 = kv_fp16
        self.faults = frozenset(faults)
        c = self.c
        d, V, hd = c["hidden_dim"], c["vocab_size"], c["head_dim"]
        nq, nkv, F = c["num_q_heads"], c["num_kv_heads"], c["ffn_dim"]
        qd, kvd = nq * hd, nkv * hd
        self.d, self.V, self.hd, self.nq, self.nkv, self.F = d, V, hd, nq, nkv, F
        self.qd, self.kvd = qd, kvd
        self.eps = float(np.float32(c.get("rms_eps", 1e-6)))
        self.theta = float(np.float32(c.get("rope_theta", 1e6)))
        self.style = int(c.get("rope_style", 0))
        self.emb = _read(os.path.join(model_dir, "embeddings.bin"), np.float32, V * d).reshape(V, d)
        n_lm = int(c.get("num_lm_heads", 0) or 0)
        self.lm_heads = None
        if n_lm > 1:
            lv = int(c.get("lm_head_vocab_size", 0) or 0) or V
            self.lm_heads = [
                _read(os.path.join(model_dir, f"lm_head_{i:02d}.bin"), np.float32, lv * d)
                .reshape(lv, d).astype(np.float64) for i in range(n_lm)]
        else:
            p = os.path.join(model_dir, "lm_head.bin")
            lm = _read(p, np.float32, V * d).reshape(V, d) if os.path.exists(p) else self.emb
            lm16 = lm.astype(np.float16)
            if c.get("disable_npu_lm_head", 0):
                self.lm_f16 = lm16.astype(np.float64)
                self.lm_q = None
            else:
                q, s = quantize_lm_head_f32(lm16)
                self.lm_q, self.lm_s = q.astype(np.float64), s.astype(np.float64)
        self.layers = []
        Ks = (d, d, d, qd, d, d, F)
        Ns = (qd, kvd, kvd, d, F, F, d)
        for l in range(c["num_layers"]):
            ld = os.path.join(model_dir, "layers", f"layer_{l:02d}")
            if not os.path.isdir(ld):
                ld = os.path.join(model_dir, f"layer_{l:02d}")
            L = {n: load_projection(ld, n, K, N, quant) for n, K, N in zip(PROJ, Ks, Ns)}
            L["in"] = _first(ld, ("input_norm.bin", "input_norm_weight.bin"), d)
            L["post"] = _first(ld, ("post_attn_norm.bin", "post_norm.bin", "post_attn_norm_weight.bin"), d)
            if c.get("has_qk_norm", 0):
                L["qn"] = _first(ld, ("q_norm.bin", "q_norm_weight.bin"), hd)
                L["kn"] = _first(ld, ("k_norm.bin", "k_norm_weight.bin"), hd)
            self.layers.append(L)
        fn = _first(model_dir, ("final_norm.bin", "model_norm.bin"), d)
        self.final_norm = fn if fn is not None else self.layers[-1]["post"]
        nl = c["num_layers"]
        self.kc = np.zeros((nl, max_seq, kvd))
        self.vc = np.zeros((nl, max_seq, kvd))
        self.max_seq = max_seq
        self.seq_len = 0

    # ---- element-wise pieces (float64) ----
    def rms(self, x, w):
        x = np.asarray(x, np.float64)
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * w

    def proj(self, name, L, x):
        """NPU projection: fp16 input, exact products, float64 sum, fp32 out."""
        return f16(x) @ L[name]

    def rope(self, x, pos, nh):
        hd, half = self.hd, self.hd // 2
        i = np.arange(half, dtype=np.float64)
        ang = pos * (1.0 / self.theta ** (2.0 * i / hd))
        cs, sn = np.cos(ang), np.sin(ang)
        x = x.reshape(nh, hd).copy()
        style = (1 - self.style) if "rope_style" in self.faults else self.style
        if style == 0:
            a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
            x[:, 0::2] = a * cs - b * sn
            x[:, 1::2] = b * cs + a * sn
        else:
            a, b = x[:, :half].copy(), x[:, half:].copy()
            x[:, :half] = a * cs - b * sn
            x[:, half:] = b * cs + a * sn
        return x.reshape(-1)

    def attend(self, q, K, V):
        """GQA attention of one query row over K/V rows [L, kvd]."""
        hd, g = self.hd, self.nq // self.nkv
        out = np.empty(self.qd)
        for h in range(self.nq):
            kh = (h % self.nkv) if "gqa" in self.faults else h // g
            s = K[:, kh * hd:(kh + 1) * hd] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[h * hd:(h + 1) * hd] = p @ V[:, kh * hd:(kh + 1) * hd]
        return out

    # ---- the layer stack ----
    def layer(self, l, h, pos, kv_rows=None):
        """One layer for one row at position pos; K/V of this row are appended
        to the cache at pos (the cache holds rows [0, pos) already)."""
        L = self.layers[l]
        n_in, n_post = (L["post"], L["in"]) if "norms" in self.faults else (L["in"], L["post"])
        res = h
        x = self.rms(h, n_in)
        q, k, v = self.proj("q_proj", L, x), self.proj("k_proj", L, x), self.proj("v_proj", L, x)
        if self.c.get("has_qk_norm", 0) and "qk_norm" not in self.faults:
            q = self.rms(q.reshape(self.nq, self.hd), L["qn"]).reshape(-1)
            k = self.rms(k.reshape(self.nkv, self.hd), L["kn"]).reshape(-1)
        q, k = self.rope(q, pos, self.nq), self.rope(k, pos, self.nkv)
        if self.kv_fp16:
            k, v = f16(k), f16(v)
        self.kc[l, pos], self.vc[l, pos] = k, v
        a = self.attend(q, self.kc[l, :pos + 1], self.vc[l, :pos + 1])
        h = self.proj("o_proj", L, a) + (0.0 if "residual" in self.faults else res)
        x = self.rms(h, n_post)
        g, u = self.proj("gate_proj", L, x), self.proj("up_proj", L, x)
        act = g / (1.0 + np.exp(-g)) * u
        return h + self.proj("down_proj", L, act)

    def hidden_after(self, token: int = 0, embedding=None) -> np.ndarray:
        h = np.asarray(embedding if embedding is not None else self.emb[token], np.float64)
        pos = self.seq_len
        for l in range(len(self.layers)):
            h = self.layer(l, h, pos)
        return h

    def head(self, h) -> np.ndarray:
        x = self.rms(h, self.final_norm)
        if self.lm_q is not None:
            return (self.lm_q @ f16(x)) * self.lm_s
        return self.lm_f16 @ x

    def step(self, token: int = 0, embedding=None, logits: bool = True):
        h = self.hidden_after(token, embedding)
        self.seq_len += 1
        if not logits:
            return 0, None
        lg = self.head(h)
        return int(np.argmax(lg)), lg

    def step_head(self, token: int, head: int, embedding=None):
        h = self.hidden_after(token, embedding)
        self.seq_len += 1
        x = self.rms(h, self.final_norm)
        lg = self.lm_heads[head] @ x
        return int(np.argmax(lg)), lg

    def prefill_batch(self, emb):
        """Rows t at positions seq_len + t; causal attention over the cache and
        the earlier batch rows, which is row-wise the decode layer."""
        emb = np.asarray(emb, np.float64)
        for t in range(emb.shape[0]):
            self.step(0, emb[t], logits=False)
        return 0


def read_config(model_dir: str) -> dict:
    with open(os.path.join(model_dir, "config.json")) as f:
        return json.load(f)
