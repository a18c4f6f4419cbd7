"""Pins the oracle's decoder composition against an independent float64
restatement of the reference forward pass (tests/ref64.py, which reads the
model files itself and calls nothing in the oracle or the product).

The element-wise pieces of the oracle are pinned one by one elsewhere; this
pins the order in which they are composed: the decode step
(src/matmul_decoder.c:1464-1546 and the head :1563-1628), the batch prefill
(:1901-2065) and the multi-head step (:1636-1742), over fp16 / int8 / int4
weights, both RoPE styles, fp16 and fp32 KV, with random norm weights so
that every norm vector matters.  Each planted composition mistake in the
float64 restatement (norms swapped, the other RoPE style, the wrong GQA
head map, QK-norm skipped, the attention residual dropped) must be rejected
by the same comparison.  CPU only.
"""
import os

import numpy as np
import pytest

from conftest import tiny_config
from ref64 import Ref64

# max |oracle - float64| / max |float64| over the logits.  The fp32 oracle and
# the float64 restatement round the same fp16 projection inputs; a value that
# lies within its fp32 error of an fp16 rounding midpoint rounds the other way
# in one of them, which moves the logits by ~1e-4 (measured on these models).
TOL = 1e-3
KV_TOL = 2e-3       # relative, per K/V row (fp16 rounding flips allowed)
CHECK_AT = (0, 1, 5, 30)
TOKENS = [int(t) for t in np.random.default_rng(77).integers(0, 512, 40)]


def _randomise_norms(path, d, hd, n_layers, seed):
    rng = np.random.default_rng(seed)
    for l in range(n_layers):
        ld = os.path.join(path, "layers", f"layer_{l:02d}")
        if not os.path.isdir(ld):
            ld = os.path.join(path, f"layer_{l:02d}")
        for name, n in (("input_norm.bin", d), ("post_attn_norm.bin", d), ("q_norm.bin", hd),
                        ("k_norm.bin", hd)):
            rng.uniform(0.5, 1.5, n).astype(np.float32).tofile(os.path.join(ld, name))
    rng.uniform(0.5, 1.5, d).astype(np.float32).tofile(os.path.join(path, "final_norm.bin"))


@pytest.fixture(scope="module")
def models(mdx, workdir):
    out = {}
    for quant in (0, 1, 2):
        for style in (0, 1):
            cfg, d = tiny_config(mdx, rope_style=style)
            path = os.path.join(workdir, f"comp_q{quant}_s{style}")
            mdx.write_model(path, cfg, quant, 4000 + 10 * quant + style)
            _randomise_norms(path, d["hidden_dim"], d["head_dim"], d["num_layers"], 91 + quant)
            out[(quant, style)] = (path, d)
    return out


def _rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def _run_steps(o, r, n):
    """Teacher-forced steps; returns the largest relative logit error at the
    checked positions and the argmax agreement away from near ties."""
    worst = 0.0
    for i in range(n):
        to, lo = o.step(TOKENS[i])
        tr, lr = r.step(TOKENS[i])
        if i in CHECK_AT:
            e = _rel(lo, lr)
            worst = max(worst, e)
            top2 = np.sort(lr)[-2:]
            if top2[1] - top2[0] > 10 * e * np.max(np.abs(lr)):
                assert to == tr, f"step {i}: oracle token {to}, float64 token {tr}"
    return worst


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("kv_fp16", [True, False])
def test_step_composition(oracle_lib, models, quant, style, kv_fp16):
    path, d = models[(quant, style)]
    o = oracle_lib.Model(path, d, quant, 64, kv_fp16)
    r = Ref64(path, d, quant, 64, kv_fp16)
    assert _run_steps(o, r, max(CHECK_AT) + 1) < TOL
    o.close()


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("kv_fp16", [True, False])
def test_prefill_composition(oracle_lib, models, quant, kv_fp16):
    """KV rows after a 9-row batch prefill and the logits of the step after it."""
    path, d = models[(quant, 1)]
    emb = np.random.default_rng(5 + quant).standard_normal((9, d["hidden_dim"])).astype(np.float32)
    o = oracle_lib.Model(path, d, quant, 64, kv_fp16)
    r = Ref64(path, d, quant, 64, kv_fp16)
    assert o.prefill_batch(emb) == 0 and r.prefill_batch(emb) == 0
    for layer in range(d["num_layers"]):
        ko, vo = o.kv_read(layer, 0, 9)
        for t in range(9):
            assert _rel(ko[t], r.kc[layer, t]) < KV_TOL
            assert _rel(vo[t], r.vc[layer, t]) < KV_TOL
    to, lo = o.step(11)
    tr, lr = r.step(11)
    assert _rel(lo, lr) < TOL and to == tr
    o.close()


def test_step_head_composition(oracle_lib, mdx, workdir):
    cfg, d = tiny_config(mdx, num_lm_heads=3, lm_head_vocab_size=300, tie_word_embeddings=0)
    path = os.path.join(workdir, "comp_multihead")
    mdx.write_model(path, cfg, 1, 4100)
    _randomise_norms(path, d["hidden_dim"], d["head_dim"], d["num_layers"], 4101)
    o = oracle_lib.Model(path, d, 1, 32)
    r = Ref64(path, d, 1, 32)
    for i, head in enumerate((0, 2, 1, 2, 0, 1)):
        to, lo = o.step_head(TOKENS[i], head, n_logits=300)
        tr, lr = r.step_head(TOKENS[i], head)
        assert _rel(lo, lr) < TOL and to == tr
    o.close()


def test_fp16_lm_head_composition(oracle_lib, mdx, workdir):
    """disable_npu_lm_head: the CPU fp16 GEMV with fp32 activations."""
    cfg, d = tiny_config(mdx, disable_npu_lm_head=1)
    path = os.path.join(workdir, "comp_f16head")
    mdx.write_model(path, cfg, 0, 4200)
    _randomise_norms(path, d["hidden_dim"], d["head_dim"], d["num_layers"], 4201)
    o = oracle_lib.Model(path, d, 0, 32)
    r = Ref64(path, d, 0, 32)
    assert _run_steps(o, r, 6) < TOL
    o.close()


@pytest.mark.parametrize("fault", ["norms", "rope_style", "gqa", "qk_norm", "residual"])
def test_planted_composition_mistakes_are_rejected(oracle_lib, models, fault):
    """The comparison above must fail for a float64 restatement with one
    composition mistake planted (each changes the logits well beyond TOL)."""
    path, d = models[(0, 1)]
    o = oracle_lib.Model(path, d, 0, 64, True)
    r = Ref64(path, d, 0, 64, True, faults={fault})
    worst = 0.0
    for i in range(max(CHECK_AT) + 1):
        _, lo = o.step(TOKENS[i])
        _, lr = r.step(TOKENS[i])
        if i in CHECK_AT:
            worst = max(worst, _rel(lo, lr))
    assert worst > 20 * TOL, f"planted mistake '{fault}' went unnoticed (rel err {worst:.2e})"
    o.close()
