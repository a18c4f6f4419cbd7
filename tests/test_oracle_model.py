"""Pins the oracle decoder (reference: src/matmul_decoder.c:1430-2065) on a tiny
model: internal invariants of the reference that any correct restatement must
keep (batch prefill == the same tokens stepped one by one, chunked prefill ==
one batch, embedding input == token input, the error returns) and the INT8
lm_head the model builds.  CPU only."""
import os

import numpy as np
import pytest

from conftest import tiny_config


@pytest.fixture(scope="module")
def tiny_dirs(mdx, workdir):
    out = {}
    for quant, name in ((0, "fp16"), (1, "int8"), (2, "int4")):
        cfg, d = tiny_config(mdx)
        path = os.path.join(workdir, f"oracle_tiny_{name}")
        mdx.write_model(path, cfg, quant, 2024)
        out[quant] = (path, d)
    return out


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("kv_fp16", [True, False])
def test_prefill_batch_equals_sequential_steps(oracle_lib, tiny_dirs, quant, kv_fp16):
    path, d = tiny_dirs[quant]
    rng = np.random.default_rng(quant)
    emb = rng.standard_normal((9, d["hidden_dim"])).astype(np.float32)
    a = oracle_lib.Model(path, d, quant, 64, kv_fp16)
    b = oracle_lib.Model(path, d, quant, 64, kv_fp16)
    assert a.prefill_batch(emb) == 0
    for t in range(9):
        assert b.step(0, emb[t], logits=False)[0] == 0
    assert a.seq_len == b.seq_len == 9
    for layer in range(d["num_layers"]):
        ka, va = a.kv_read(layer, 0, 9)
        kb, vb = b.kv_read(layer, 0, 9)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    ta, la = a.step(7)
    tb, lb = b.step(7)
    assert ta == tb and np.array_equal(la, lb)


def test_chunked_prefill_equals_one_batch(oracle_lib, tiny_dirs):
    path, d = tiny_dirs[1]
    emb = np.random.default_rng(3).standard_normal((10, d["hidden_dim"])).astype(np.float32)
    small = dict(d, max_batch_prefill=4)
    a = oracle_lib.Model(path, small, 1, 64)
    b = oracle_lib.Model(path, d, 1, 64)
    assert a.prefill_batch(emb) == 0 and b.prefill_batch(emb) == 0
    assert np.array_equal(a.kv_read(1, 0, 10)[0], b.kv_read(1, 0, 10)[0])


def test_embedding_input_equals_token_input(oracle_lib, tiny_dirs):
    path, d = tiny_dirs[0]
    table = np.fromfile(os.path.join(path, "embeddings.bin"), np.float32).reshape(d["vocab_size"], -1)
    a = oracle_lib.Model(path, d, 0, 64)
    b = oracle_lib.Model(path, d, 0, 64)
    for tok in (5, 300, 17):
        ta, la = a.step(tok)
        tb, lb = b.step(0, table[tok])
        assert ta == tb and np.array_equal(la, lb)


def test_error_returns(oracle_lib, tiny_dirs):
    path, d = tiny_dirs[0]
    m = oracle_lib.Model(path, d, 0, 3)
    assert m.step(-1)[0] == -1 and m.step(d["vocab_size"])[0] == -1
    for _ in range(3):
        assert m.step(1, logits=False)[0] == 0
    assert m.step(1)[0] == -1                      # KV cache full
    e = np.zeros((2, d["hidden_dim"]), np.float32)
    m.seq_len = 2
    assert m.prefill_batch(e) == -1                # 2 + 2 > 3


def test_lm_head_is_the_quantised_tied_embedding(oracle_lib, tiny_dirs):
    path, d = tiny_dirs[0]
    m = oracle_lib.Model(path, d, 0, 16)
    table = np.fromfile(os.path.join(path, "embeddings.bin"), np.float32).reshape(d["vocab_size"], -1)
    q, s = m.lm_head_q()
    q2, s2 = oracle_lib.quantize_lm_head(oracle_lib.f32_to_f16(table), *table.shape)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    # logits[v] = scale[v] * sum_k fp16(normed_k) q[v,k]: check against float64
    tok, lg = m.step(3)
    x16 = oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(m.last_normed())).astype(np.float64)
    want = (q.astype(np.float64) @ x16) * s
    assert np.max(np.abs(lg - want)) < 1e-5 * np.max(np.abs(want))
    assert tok == int(np.argmax(lg))


def test_kv_fill_hook(oracle_lib, tiny_dirs):
    path, d = tiny_dirs[0]
    m = oracle_lib.Model(path, d, 0, 32, kv_fp16=True)
    assert m.kv_fill_normal(20, 99) == 0 and m.seq_len == 20
    k, v = m.kv_read(1, 0, 20)
    kvd = d["num_kv_heads"] * d["head_dim"]
    want = oracle_lib.fill_normal(20 * kvd, oracle_lib.seed_for(99, "kv/k/01"))
    assert np.array_equal(k.ravel(), oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(want)))
