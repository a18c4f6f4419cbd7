"""The device sampler (k_repeat_penalty + k_topk_sample) against the oracle's
restatement of src/cpu_ops.c:593-648 (given uniform in place of rand()).

Bars:
- candidate indices and tempered values bit-exact (the temperature is an IEEE
  division on both sides; the selection is an exact order);
- the kept count after top-p and the drawn token equal to the oracle's,
  except where the draw or the top-p threshold falls within 1e-5 (relative)
  of a boundary of the running sum: the device's expf and the host's may
  differ in the last bit, which moves a boundary by about 1e-7;
- through the decoder: matmul_decoder_step_sample draws what the oracle
  draws from the logits that the same step returns, and leaves the context
  where matmul_decoder_step does."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V_FULL = 151936


def _logits(V, seed, scale=3.0, quant=None):
    x = (np.random.default_rng(seed).standard_normal(V) * scale).astype(np.float32)
    if quant:
        x = (np.round(x * quant) / quant).astype(np.float32)
    return x


def _near_boundary(val, kept, u, top_p):
    """True when u * sum or the top-p threshold lies within 1e-5 of a running
    sum of the candidates (then a last-bit difference in expf may move it)."""
    e = np.exp((val.astype(np.float64) - float(val[0])))
    run = np.cumsum(e)
    near = lambda t: np.any(np.abs(run - t) <= 1e-5 * run[-1])  # noqa: E731
    lim = top_p * run[-1] if top_p < 1.0 else None
    return near(u * run[kept - 1]) or (lim is not None and near(lim))


def _check(mdx, oracle_lib, x, **kw):
    tok, idx, val, kept = mdx.sample(x, **kw)
    rtok, ridx, rval, rkept = oracle_lib.sample_topk(x, **kw)
    assert np.array_equal(idx, ridx), kw
    assert np.array_equal(val.view(np.uint32), rval.view(np.uint32)), kw
    if kept != rkept or tok != rtok:
        assert _near_boundary(rval, rkept, kw.get("u", 0.0), kw.get("top_p", 1.0)), (kw, tok, rtok)
    return tok


@pytest.mark.parametrize("k", [1, 2, 40, 64, 65, 1000, 1024])
def test_top_k_full_vocab(mdx, gpu, oracle_lib, k):
    # k <= 64 runs the two-launch path (per-range top-64 lists, one merging
    # workgroup), k >= 65 the radix-select path: both sides of the switch
    x = _logits(V_FULL, 100 + k)
    for u in (0.0, 0.37, 0.999):
        tok = _check(mdx, oracle_lib, x, top_k=k, u=u)
        if u == 0.0 or k == 1:
            assert tok == int(np.argmax(x))


@pytest.mark.parametrize("T", [0.7, 1.3])
@pytest.mark.parametrize("top_p", [1.0, 0.9, 0.5])
def test_temperature_and_top_p(mdx, gpu, oracle_lib, T, top_p):
    x = _logits(V_FULL, 7)
    for u in (0.1, 0.55, 0.93):
        _check(mdx, oracle_lib, x, top_k=50, temperature=T, top_p=top_p, u=u)


def test_repeat_penalty(mdx, gpu, oracle_lib):
    x = _logits(V_FULL, 8)
    order = np.argsort(-x, kind="stable")
    toks = [int(order[0]), int(order[0]), int(order[2]), int(order[-1]), int(order[5]), int(order[5]),
            12345, 12345]
    for p in (1.3, 0.8):
        _check(mdx, oracle_lib, x, top_k=30, u=0.4, repeat_tokens=toks, repeat_penalty=p)
    # greedy under a penalty: the argmax of the penalised logits
    tok, _, _, _ = mdx.sample(x, top_k=1, repeat_tokens=toks, repeat_penalty=5.0)
    assert tok == oracle_lib.sample_topk(x, top_k=1, repeat_tokens=toks, repeat_penalty=5.0)[0]


@pytest.mark.parametrize("V", [V_FULL, 151669, 1001, 5, 300001])
def test_ties_signed_zeros_and_ragged_vocab(mdx, gpu, oracle_lib, V):
    # 300001 values exceed what the two-launch small-k path covers (256
    # ranges of at most 1024), so every k there takes the radix-select path
    # values on a coarse grid: long runs of equal values at the threshold, and
    # both +0 and -0 (np.round keeps the sign)
    x = _logits(V, V, scale=1.0, quant=2)
    assert np.any(np.signbit(x) & (x == 0)) or V < 100
    for k in sorted({1, 3, min(V, 64), min(V, 257), min(V, 1024)}):
        _check(mdx, oracle_lib, x, top_k=k, u=0.6)
    # every value equal: the first k indices
    z = np.zeros(V, np.float32)
    _, idx, _, _ = mdx.sample(z, top_k=min(V, 64), u=0.5)
    assert np.array_equal(idx, np.arange(min(V, 64)))


def test_rejects_bad_parameters(mdx, gpu):
    x = _logits(4096, 9)
    for kw in (dict(top_k=1025), dict(temperature=0.0), dict(u=1.5), dict(u=-0.1),
               dict(repeat_tokens=[4096], repeat_penalty=1.2), dict(repeat_penalty=0.0)):
        args = dict(top_k=4, u=0.5)
        args.update(kw)
        with pytest.raises(RuntimeError):
            mdx.sample(x, **args)
    # top_k beyond the vocabulary is clamped to it
    _, idx, _, _ = mdx.sample(x[:16], top_k=5000, u=0.5)
    assert idx.size == 16


def test_step_sample_through_the_decoder(mdx, gpu, oracle_lib, workdir):
    d = dict(hidden_dim=128, num_q_heads=4, num_kv_heads=2, head_dim=64, ffn_dim=256,
             num_layers=2, vocab_size=4096, max_seq_len=64, rms_eps=1e-6, rope_theta=1e6,
             tie_word_embeddings=1, has_qk_norm=1, rope_style=1, max_batch_prefill=64)
    cfg = mdx.qwen3_0_6b_config(name="sample", **d)
    path = os.path.join(workdir, "model_sample_i8")
    if not os.path.exists(os.path.join(path, "config.json")):
        mdx.write_model(path, cfg, 1, 4242)
    a = mdx.Decoder(path, cfg, "int8", 64)      # sampled on the device
    b = mdx.Decoder(path, cfg, "int8", 64)      # plain steps, same tokens
    rng = np.random.default_rng(3)
    ta = tb = 11
    history = []
    for i in range(12):
        u = float(rng.random())
        kw = dict(top_k=[1, 8, 40][i % 3], temperature=[1.0, 0.8][i % 2], top_p=[1.0, 0.9][i % 2],
                  repeat_tokens=history[-6:], repeat_penalty=1.2)
        tok, lg = a.step_sample(ta, u, logits=True, **kw)
        assert tok >= 0
        greedy, ref_lg = b.step(tb)
        assert np.array_equal(lg, ref_lg)               # same step, same logits
        rtok, _, rval, rkept = oracle_lib.sample_topk(ref_lg, u=u, **kw)
        assert tok == rtok or _near_boundary(rval, rkept, u, kw["top_p"]), (i, tok, rtok)
        if kw["top_k"] == 1 and not history:
            assert tok == greedy
        history.append(tok)
        ta = tb = tok
    assert a.seq_len == b.seq_len == 12
    a.close()
    b.close()


@pytest.mark.parametrize("k", [1, 8, 300])
def test_top_k_floor_and_nan_as_the_reference(mdx, gpu, oracle_lib, k):
    """Only values above -1e30 become candidates (the reference's slots start
    at (0, -1e30) and take a value only when it is strictly greater; NaN
    never is); missing slots stay (0, -1e30).  Checked bit-exact against the
    oracle with -inf, -1e30, NaN and, in the last case, fewer real values
    than k."""
    V = 5000
    x = _logits(V, 900 + k)
    x[[3, 17, 4000]] = -np.inf
    x[[5, 4001]] = np.nan
    x[[9, 2500]] = -1e30
    x[[11]] = -2e30
    for u in (0.0, 0.5, 0.999):
        _check(mdx, oracle_lib, x, top_k=k, u=u)
    y = np.full(V, -np.inf, np.float32)
    y[[7, 70, 700]] = [1.0, 2.0, -3.0]
    y[[8, 80]] = np.nan
    y[90] = -1e30
    for u in (0.0, 0.4, 0.999):
        _check(mdx, oracle_lib, y, top_k=k, u=u)
    z = np.full(V, np.nan, np.float32)
    z[[10, 20]] = -np.inf
    tok = _check(mdx, oracle_lib, z, top_k=k, u=0.3)
    assert tok == 0
