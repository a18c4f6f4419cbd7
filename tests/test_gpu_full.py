"""Full-size parity on the Qwen3-0.6B shape (28 layers, d=1024, 16Q/8KV x 128,
FFN 3072, vocab 151936, INT8 lm_head, split-half RoPE theta 1e6):

- 28-layer greedy decode, FP16 layers, fp16 KV prefilled to 512 N(0,1)
  positions, 64 greedy steps;
- the same with INT8 layers;
- M=60 batch prefill through 28 INT8, FP16 or INT4 layers from an empty
  cache, then the lm_head on the last token: cosine >= 0.9999, same argmax;
- W4A16 decode at long context (KV 4096, max_seq 4224), 128 greedy steps.

Greedy parity.  The reference runs the projections on an NPU whose fp32
accumulation order is unspecified, so the oracle fixes one order (increasing
k).  Other, equally valid orders (four or sixteen interleaved sums combined
as a pairwise tree, the oracle's orders 1 and 2) already move the step-0
logits by about 2e-3 of their range and make the oracle runs pick different
tokens wherever the top-2 margin is that small (with random-init weights
this happens within 64 steps).  The decode tests therefore measure that
order sensitivity B (the largest max |logit difference| at step 0 between
two of the oracle's three orders) and require:
  1. the GPU's step-0 logits within 2*B of the oracle's, cosine >= 0.9999;
  2. teacher forcing (both fed the oracle's tokens): the GPU argmax equals
     the oracle's at every step whose oracle top-1/top-2 margin is >= 2*B,
     and is one of the oracle's candidates within 2*B of the top otherwise;
  3. free-running greedy tokens identical to the oracle's up to the first
     step whose margin is below 2*B (all of them when there is none).

Model files are written at test time by the seeded synthetic writer (seed
1000 + config number)."""
import os

import numpy as np
import pytest

from conftest import cosine, rel_err

pytestmark = pytest.mark.gpu

FULL = dict(hidden_dim=1024, num_q_heads=16, num_kv_heads=8, head_dim=128, ffn_dim=3072,
            num_layers=28, vocab_size=151936, max_seq_len=4224, rms_eps=1e-6, rope_theta=1e6,
            tie_word_embeddings=1, has_qk_norm=1, rope_style=1, max_batch_prefill=64)
START = 151644


@pytest.fixture(scope="module")
def full(mdx, workdir):
    cfg = mdx.qwen3_0_6b_config(name="qwen3-0.6b-synthetic", **FULL)
    made = {}

    def get(quant, seed):
        key = (quant, seed)
        if key not in made:
            path = os.path.join(workdir, f"full_q{quant}_s{seed}")
            mdx.write_model(path, cfg, quant, seed)
            made[key] = path
        return made[key]
    return cfg, get


def _first_divergence(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return i
    return None


def _order_sensitivity(oracle_lib, path, quant, max_seq, n_pos, seed):
    """The largest max |logit difference| at the first step between two of
    the oracle's three projection accumulation orders, and the step-0 logits
    of each order."""
    out = []
    for order in (0, 1, 2):
        oracle_lib.lib().orc_set_accum_order(order)
        try:
            m = oracle_lib.Model(path, FULL, quant, max_seq, kv_fp16=True)
            assert m.kv_fill_normal(n_pos, seed) == 0
            out.append(m.step(START)[1])
            m.close()
        finally:
            oracle_lib.lib().orc_set_accum_order(0)
    pairs = [(a, b) for a in range(3) for b in range(a + 1, 3)]
    return max(float(np.max(np.abs(out[a] - out[b]))) for a, b in pairs), out


def _greedy_parity(mdx, oracle_lib, g, o, path, quant, max_seq, n_pos, seed, n_steps):
    bound, orders = _order_sensitivity(oracle_lib, path, quant, max_seq, n_pos, seed)
    lo0 = orders[0]
    delta = 2.0 * bound
    # oracle free-running greedy: tokens, logits and margins
    assert o.kv_fill_normal(n_pos, seed) == 0
    toks_o, logits_o, margins = [], [], []
    t = START
    for _ in range(n_steps):
        t, lg = o.step(t)
        top2 = np.partition(lg, -2)[-2:]
        toks_o.append(int(t))
        logits_o.append(lg)
        margins.append(float(top2[1] - top2[0]))
    assert np.array_equal(logits_o[0], lo0)
    # GPU teacher-forced on the oracle's inputs
    g.kv_fill_normal(n_pos, seed)
    inputs = [START] + toks_o[:-1]
    worst_cos, errs, near = 1.0, [], 0
    for i, tok_in in enumerate(inputs):
        tg, lg = g.step(tok_in)
        lo = logits_o[i]
        errs.append(float(np.max(np.abs(lg - lo))))
        if i == 0:
            gpu_to = [float(np.max(np.abs(lg - orders[k]))) for k in range(3)]
        worst_cos = min(worst_cos, cosine(lg, lo))
        if margins[i] >= delta:
            assert tg == toks_o[i], (f"step {i}: gpu {tg} oracle {toks_o[i]} margin {margins[i]:.3g} "
                                     f">= {delta:.3g}")
        else:
            near += 1
            assert lo[tg] >= lo.max() - delta, f"step {i}: gpu {tg} is not an oracle near-tie candidate"
    # GPU free-running
    g.kv_fill_normal(n_pos, seed)
    toks_g, _ = g.generate_greedy(START, n_steps)
    first_tie = next((i for i, m in enumerate(margins) if m < delta), None)
    div = _first_divergence(toks_g, toks_o)
    dist = [float(np.max(np.abs(orders[a] - orders[b]))) for a, b in ((0, 1), (0, 2), (1, 2))]
    print(f"oracle orders 0-1 {dist[0]:.3g}, 0-2 {dist[1]:.3g}, 1-2 {dist[2]:.3g}; "
          f"gpu to orders 0/1/2 {gpu_to[0]:.3g}/{gpu_to[1]:.3g}/{gpu_to[2]:.3g}")
    print(f"order sensitivity B {bound:.3g}; gpu step-0 error {errs[0]:.3g} = {errs[0] / bound:.2f} B "
          f"(max {max(errs):.3g}); "
          f"worst cos {worst_cos:.7f}; near-tie steps {near}/{n_steps}; first near tie {first_tie}; "
          f"first free-running divergence {div}")
    assert errs[0] <= 2.0 * bound and worst_cos >= 0.9999
    if div is not None:
        assert first_tie is not None and div >= first_tie, (
            f"free-running token {div} differs (gpu {toks_g[div]} oracle {toks_o[div]}) before the "
            f"first near tie {first_tie}")


@pytest.mark.timeout(400)
def test_decode_28_layers_fp16_greedy_parity(mdx, gpu, oracle_lib, full):
    cfg, get = full
    path = get(0, 1003)
    max_seq = 512 + 64 + 8
    g = mdx.Decoder(path, cfg, "fp16", max_seq)
    o = oracle_lib.Model(path, FULL, 0, max_seq, kv_fp16=True)
    _greedy_parity(mdx, oracle_lib, g, o, path, 0, max_seq, 512, 1003, 64)


@pytest.mark.timeout(400)
def test_decode_28_layers_int8_greedy_parity(mdx, gpu, oracle_lib, full):
    """The same 64-step greedy parity with INT8 layer weights (the one-launch
    step's int8 kernel)."""
    cfg, get = full
    path = get(1, 1006)
    max_seq = 512 + 64 + 8
    g = mdx.Decoder(path, cfg, "int8", max_seq)
    o = oracle_lib.Model(path, FULL, 1, max_seq, kv_fp16=True)
    _greedy_parity(mdx, oracle_lib, g, o, path, 1, max_seq, 512, 1006, 64)


@pytest.mark.timeout(400)
@pytest.mark.parametrize("quant", [1, 0, 2])
def test_prefill_m60_then_lm_head_matches_oracle(mdx, gpu, oracle_lib, full, quant):
    """M=60 batch prefill through 28 layers (INT8, FP16 and INT4 weights)."""
    cfg, get = full
    path = get(quant, 1004)
    emb = mdx.synth_fill_normal(60 * 1024, mdx.synth_seed(1004, "prefill/emb")).reshape(60, 1024)
    g = mdx.Decoder(path, cfg, ["fp16", "int8", "int4"][quant], 128)
    o = oracle_lib.Model(path, FULL, quant, 128, kv_fp16=True)
    tok, lg = g.prefill_logits(emb)
    assert o.prefill_batch(emb) == 0
    x16 = oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(o.last_normed())).astype(np.float64)
    q, s = o.lm_head_q()
    ref = (q.astype(np.float64) @ x16) * s
    tref = int(np.argmax(ref))
    err = float(np.max(np.abs(lg - ref)))
    print(f"prefill lm_head q{quant}: gpu {tok} oracle {tref} cos {cosine(lg, ref):.7f} "
          f"margin-to-gpu {ref[tref] - ref[tok]:.3g} err {err:.3g}")
    # same argmax, or a near tie within twice the largest logit error
    assert cosine(lg, ref) >= 0.9999 and (tok == tref or ref[tref] - ref[tok] <= 2 * err)
    for layer in (0, 13, 27):
        kg, vg = g.kv_read(layer, 0, 60)
        ko, vo = o.kv_read(layer, 0, 60)
        assert rel_err(kg, ko) < 2e-3 and rel_err(vg, vo) < 2e-3
    # the decode that follows the prefill agrees too (both fed the oracle's token)
    tg, lg2 = g.step(tref)
    to, lo2 = o.step(tref)
    err2 = float(np.max(np.abs(lg2 - lo2)))
    assert cosine(lg2, lo2) >= 0.9999 and (tg == to or lo2[to] - lo2[tg] <= 2 * err2)


@pytest.mark.timeout(600)
def test_w4a16_long_context_128_steps(mdx, gpu, oracle_lib, full):
    cfg, get = full
    path = get(2, 1005)
    max_seq = 4224
    g = mdx.Decoder(path, cfg, "int4", max_seq)
    o = oracle_lib.Model(path, FULL, 2, max_seq, kv_fp16=True)
    _greedy_parity(mdx, oracle_lib, g, o, path, 2, max_seq, 4096, 1005, 128)
