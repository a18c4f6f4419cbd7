"""The one-launch decode step (all layers, the lm_head and the argmax in one
cooperative launch) on the 0.6B layer shape: d=1024, 16Q/8KV heads of 128,
FFN 3072, with 2 layers and a 5000-row INT8 lm_head (not a multiple of the
256 workgroups, so the row ranges are ragged).

Checked against the oracle on the same seeded model files and KV contents,
and against the per-stage kernel path of the same library (MDX_PERSIST=0 at
context creation):
- logits cosine >= 0.9999 and max relative error <= 2e-3, same argmax;
- the K/V row appended at the step's position;
- cache lengths that exercise every attention chunking case: 0 (only the new
  position), 1, 33, 511, 600, 2100 (chunks longer than the 64 prefetched
  positions) and 4100 (129 positions per split: with int8 and int4 layers
  the launch takes rounds of 80 positions), and for int4 and int8 layers
  4095 and 4096 (128 and 129 per split, either side of the switch to
  rounds of 80), 5500 (172 per split: three rounds of 64, the third
  requested while the first is computed) and 6200 (194 per split: three
  rounds of 80);
- an uploaded embedding instead of a token, a step without the lm_head, and
  16 greedy steps fed back on the device.
"""
import os

import numpy as np
import pytest

from conftest import cosine, rel_err
from test_gpu_sample import _near_boundary

pytestmark = pytest.mark.gpu

SHAPE = dict(hidden_dim=1024, num_q_heads=16, num_kv_heads=8, head_dim=128, ffn_dim=3072,
             num_layers=2, vocab_size=5000, max_seq_len=4224, rms_eps=1e-6, rope_theta=1e6,
             tie_word_embeddings=1, has_qk_norm=1, rope_style=1, max_batch_prefill=64)
QUANTS = {0: "fp16", 1: "int8", 2: "int4"}
MAX_SEQ = 4224


@pytest.fixture(scope="module")
def models(mdx, workdir):
    cfg = mdx.qwen3_0_6b_config(name="persist-2l", **SHAPE)
    made = {}

    def get(quant):
        if quant not in made:
            path = os.path.join(workdir, f"persist_q{quant}")
            mdx.write_model(path, cfg, quant, 2000 + quant)
            made[quant] = path
        return made[quant]
    return cfg, get


def _pair(mdx, oracle_lib, cfg, path, quant, persist=True, shape=SHAPE, want_path=1, max_seq=MAX_SEQ):
    old = os.environ.get("MDX_PERSIST")
    os.environ["MDX_PERSIST"] = "1" if persist else "0"
    try:
        g = mdx.Decoder(path, cfg, QUANTS[quant], max_seq)
    finally:
        if old is None:
            del os.environ["MDX_PERSIST"]
        else:
            os.environ["MDX_PERSIST"] = old
    assert g.path == (want_path if persist else 0)
    o = oracle_lib.Model(path, shape, quant, max_seq, kv_fp16=True)
    return g, o


@pytest.mark.parametrize("quant,n_pos", [(q, n) for q in (0, 1, 2)
                                          for n in (0, 1, 33, 511, 600, 2100, 4100)]
                         + [(2, 4095), (2, 4096), (1, 5500), (2, 5500), (1, 6200), (2, 6200)])
def test_step_matches_oracle(mdx, gpu, oracle_lib, models, quant, n_pos):
    cfg, get = models
    path = get(quant)
    g, o = _pair(mdx, oracle_lib, cfg, path, quant, max_seq=max(MAX_SEQ, n_pos + 8))
    seed = 77 + n_pos
    if n_pos:
        g.kv_fill_normal(n_pos, seed)
        assert o.kv_fill_normal(n_pos, seed) == 0
    tok = 4321
    tg, lg = g.step(tok)
    to, lo = o.step(tok)
    c, r = cosine(lg, lo), rel_err(lg, lo)
    print(f"q{quant} pos {n_pos}: gpu {tg} oracle {to} cos {c:.7f} rel {r:.2e}")
    assert c >= 0.9999 and r <= 2e-3
    assert tg == to == int(np.argmax(lo))
    for layer in range(2):
        kg, vg = g.kv_read(layer, n_pos, 1)
        ko, vo = o.kv_read(layer, n_pos, 1)
        assert np.allclose(kg, ko, rtol=4e-3, atol=4e-3), f"layer {layer} K row {n_pos}"
        assert np.allclose(vg, vo, rtol=4e-3, atol=4e-3), f"layer {layer} V row {n_pos}"
    assert g.seq_len == n_pos + 1


@pytest.mark.parametrize("quant,n_pos", [(0, 0), (0, 33), (0, 600), (2, 600), (1, 4100), (2, 4100)])
def test_local_exchange_is_bit_identical(mdx, gpu, oracle_lib, models, quant, n_pos):
    """The per-head exchanges of the one-launch step (qkv rows to attention,
    partial records to the merge) through the XCD's L2 (the default) or
    through the uncached words like the other exchanges: only the transport
    differs, so three steps give the same logits, tokens and K/V rows, and
    the local path matches the oracle."""
    cfg, get = models
    path = get(quant)
    runs = []
    for mode in (1, 0):
        g, o = _pair(mdx, oracle_lib, cfg, path, quant)
        g.force_local_exchange(mode)
        g.kv_fill_normal(n_pos, 61)
        out = []
        tok = 777
        for _ in range(3):
            tok, lg = g.step(tok)
            out.append((tok, lg.copy()))
        k, v = g.kv_read(1, n_pos, 3)
        runs.append((out, k.copy(), v.copy()))
        if mode == 1:
            assert o.kv_fill_normal(n_pos, 61) == 0
            to, lo = o.step(777)
            assert cosine(out[0][1], lo) >= 0.9999 and rel_err(out[0][1], lo) <= 2e-3
        g.close()
    (a, ka, va), (b, kb, vb) = runs
    for (ta, la), (tb, lb) in zip(a, b):
        assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)


@pytest.mark.parametrize("n_pos", [33, 600, 4100])
def test_kv_load_policy_is_bit_identical(mdx, gpu, oracle_lib, models, n_pos):
    """The K/V rows read with ordinary or with non-temporal loads (the policy
    the host picks by cache size) give the same bits: logits, token and the
    appended K/V row, over three steps. With fp16 layers the policy also moves
    the first K/V round of each layer: requested at the end of the previous
    layer's gate|up stage (ordinary loads) or in the layer's own qkv stage
    (non-temporal loads)."""
    cfg, get = models
    path = get(0)
    runs = []
    # ordinary loads, non-temporal loads, and the policy switched between the
    # steps of one decoder (each launch decides on its own)
    for modes in ((0, 0, 0), (1, 1, 1), (0, 1, 0)):
        g, _ = _pair(mdx, oracle_lib, cfg, path, 0)
        g.kv_fill_normal(n_pos, 91)
        out = []
        tok = 1234
        for mode in modes:
            g.force_kv_stream(mode)
            tok, lg = g.step(tok)
            out.append((tok, lg.copy()))
        k, v = g.kv_read(1, n_pos, 3)
        runs.append((out, k.copy(), v.copy()))
        g.close()
    a, ka, va = runs[0]
    for b, kb, vb in runs[1:]:
        for (ta, la), (tb, lb) in zip(a, b):
            assert ta == tb and np.array_equal(la, lb)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_one_launch_matches_per_stage_path(mdx, gpu, oracle_lib, models, quant):
    cfg, get = models
    path = get(quant)
    g1, _ = _pair(mdx, oracle_lib, cfg, path, quant, persist=True)
    g0, _ = _pair(mdx, oracle_lib, cfg, path, quant, persist=False)
    for g in (g0, g1):
        g.kv_fill_normal(700, 5)
    for tok in (17, 4999, 0):
        t1, l1 = g1.step(tok)
        t0, l0 = g0.step(tok)
        print(f"q{quant} tok {tok}: cos {cosine(l1, l0):.8f} rel {rel_err(l1, l0):.2e}")
        assert t1 == t0 and cosine(l1, l0) >= 0.99999 and rel_err(l1, l0) <= 1e-3


def test_uploaded_embedding_and_headless_step(mdx, gpu, oracle_lib, models):
    cfg, get = models
    path = get(1)
    g, o = _pair(mdx, oracle_lib, cfg, path, 1)
    g.kv_fill_normal(64, 9)
    assert o.kv_fill_normal(64, 9) == 0
    emb = mdx.synth_fill_normal(1024, mdx.synth_seed(9, "persist/emb")) * 0.05
    # a step without the lm_head only appends K/V and advances the position
    tg, lg = g.step(12, logits=False)
    to, _ = o.step(12, logits=False)
    assert lg is None and g.seq_len == 65
    tg, lg = g.step(0, embedding=emb)
    to, lo = o.step(0, embedding=emb)
    print(f"embedding step: gpu {tg} oracle {to} cos {cosine(lg, lo):.7f} rel {rel_err(lg, lo):.2e}")
    assert cosine(lg, lo) >= 0.9999 and rel_err(lg, lo) <= 2e-3 and tg == to
    kg, _ = g.kv_read(1, 64, 2)
    ko, _ = o.kv_read(1, 64, 2)
    assert np.allclose(kg, ko, rtol=4e-3, atol=4e-3)


@pytest.mark.parametrize("quant", [0, 2])
def test_greedy_tokens_match_oracle(mdx, gpu, oracle_lib, models, quant):
    cfg, get = models
    path = get(quant)
    g, o = _pair(mdx, oracle_lib, cfg, path, quant)
    g.kv_fill_normal(300, 31)
    assert o.kv_fill_normal(300, 31) == 0
    toks_g, _ = g.generate_greedy(100, 16)
    toks_o, margins = o.greedy(100, 16)
    print(f"q{quant}: gpu {toks_g}\n    oracle {toks_o}\n    min margin {min(margins):.3g}")
    assert list(toks_g) == list(toks_o)
    assert g.seq_len == 316


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_multi_head_layers_in_one_launch(mdx, gpu, oracle_lib, workdir, quant):
    """Several lm_heads (the Code Predictor form): the layers run as one launch
    and step_head's head as a per-stage GEMV after it.  Checked against the
    oracle and the per-stage path per step, with a token and an uploaded
    embedding as input and heads chosen out of order."""
    shape = dict(SHAPE, num_lm_heads=3, lm_head_vocab_size=512, vocab_size=1000,
                 tie_word_embeddings=0)
    cfg = mdx.qwen3_0_6b_config(name="persist-multihead", **shape)
    path = os.path.join(workdir, f"persist_multihead_q{quant}")
    mdx.write_model(path, cfg, quant, 3100 + quant)
    g1, o = _pair(mdx, oracle_lib, cfg, path, quant, shape=shape, want_path=2)
    g0, _ = _pair(mdx, oracle_lib, cfg, path, quant, persist=False, shape=shape)
    for m in (g1, g0):
        m.kv_fill_normal(300, 12)
    assert o.kv_fill_normal(300, 12) == 0
    emb = mdx.synth_fill_normal(1024, mdx.synth_seed(12, "persist/mh-emb")) * 0.05
    for i, head in enumerate((0, 2, 1, 2)):
        e = emb if i == 1 else None
        t1, l1 = g1.step_head(10 + i, head, embedding=e)
        t0, l0 = g0.step_head(10 + i, head, embedding=e)
        to, lo = o.step_head(10 + i, head, embedding=e, n_logits=512)
        print(f"head {head}: one-launch {t1} per-stage {t0} oracle {to} "
              f"cos {cosine(l1, lo):.7f} rel {rel_err(l1, lo):.2e}")
        assert cosine(l1, lo) >= 0.9999 and rel_err(l1, lo) <= 2e-3
        # same argmax, or a near tie: when the GPU ranks t1 above the
        # oracle's token, the oracle's gap between them is at most twice the
        # largest logit error
        err = float(np.max(np.abs(l1 - lo)))
        assert t1 == to or lo[to] - lo[t1] <= 2 * err, (t1, to, float(lo[to] - lo[t1]), err)
        assert t1 == t0 and cosine(l1, l0) >= 0.99999 and rel_err(l1, l0) <= 1e-3
    assert g1.seq_len == g0.seq_len == 304
    kg, vg = g1.kv_read(1, 300, 4)
    ko, vo = o.kv_read(1, 300, 4)
    assert np.allclose(kg, ko, rtol=4e-3, atol=4e-3) and np.allclose(vg, vo, rtol=4e-3, atol=4e-3)


def test_fp16_lm_head_layers_in_one_launch(mdx, gpu, oracle_lib, models):
    """disable_npu_lm_head (the fp16 lm_head): layers in one launch, then the
    fp16 head; steps and the device greedy loop against the oracle."""
    shape = dict(SHAPE, disable_npu_lm_head=1)
    _, get = models
    path = get(0)
    cfg = mdx.qwen3_0_6b_config(name="persist-fp16-head", **shape)
    g, o = _pair(mdx, oracle_lib, cfg, path, 0, shape=shape, want_path=2)
    g.kv_fill_normal(200, 4)
    assert o.kv_fill_normal(200, 4) == 0
    for tok in (4321, 7):
        tg, lg = g.step(tok)
        to, lo = o.step(tok)
        print(f"fp16 head tok {tok}: gpu {tg} oracle {to} cos {cosine(lg, lo):.7f}")
        assert cosine(lg, lo) >= 0.9999 and rel_err(lg, lo) <= 2e-3 and tg == to
    toks_g, _ = g.generate_greedy(100, 12)
    toks_o, margins = o.greedy(100, 12)
    print(f"fp16 head greedy: gpu {toks_g}\n    oracle {toks_o}\n    min margin {min(margins):.3g}")
    assert list(toks_g) == list(toks_o)
    assert g.seq_len == 214


def test_create_destroy_cycles_release_device_memory(mdx, gpu, oracle_lib, models):
    """Contexts of the one-launch shape created, stepped (token, greedy loop,
    prefill) and destroyed ten times: the device's free memory returns to
    where it started (within 64 MiB of runtime caching)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    free_b, total_b = ctypes.c_size_t(0), ctypes.c_size_t(0)

    def free_now():
        assert hip.hipMemGetInfo(ctypes.byref(free_b), ctypes.byref(total_b)) == 0
        return free_b.value

    cfg, get = models
    path = get(1)
    g = mdx.Decoder(path, cfg, "int8", 256)     # first context: runtime set-up outside the count
    g.step(3)
    g.close()
    before = free_now()
    emb = np.random.default_rng(3).standard_normal((20, 1024)).astype(np.float32)
    for i in range(10):
        g = mdx.Decoder(path, cfg, "int8", 256)
        assert g.path == 1
        g.step(3 + i)
        g.generate_greedy(5, 4)
        assert g.prefill_batch(emb) == 0
        g.close()
    after = free_now()
    print(f"free before {before >> 20} MiB, after {after >> 20} MiB")
    assert before - after < (64 << 20)


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("M", [60, 64, 17, 1])
def test_prefill_full_width_matches_oracle(mdx, gpu, oracle_lib, models, quant, M):
    """Batch prefill on the 0.6B layer shape (the split-K MFMA projections
    with the SwiGLU finished by the last split, the RoPE/append and residual
    kernels summing the splits): K/V rows of both layers and the lm_head on
    the last row against the oracle, then a second chunk on top of a
    non-empty cache."""
    cfg, get = models
    g, o = _pair(mdx, oracle_lib, cfg, get(quant), quant)
    rng = np.random.default_rng(100 + M + 7 * quant)
    for chunk in range(2):
        emb = rng.standard_normal((M, 1024)).astype(np.float32)
        tok, lg = g.prefill_logits(emb)
        assert o.prefill_batch(emb) == 0
        x16 = oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(o.last_normed())).astype(np.float64)
        q, sc = o.lm_head_q()
        ref = (q.astype(np.float64) @ x16) * sc
        err = float(np.max(np.abs(lg - ref)))
        assert rel_err(lg, ref) < 2e-3 and cosine(lg, ref) > 0.9999
        tref = int(np.argmax(ref))
        assert tok == tref or ref[tref] - ref[tok] <= 2 * err
        n = (chunk + 1) * M
        for layer in (0, 1):
            kg, vg = g.kv_read(layer, 0, n)
            ko, vo = o.kv_read(layer, 0, n)
            assert rel_err(kg, ko) < 2e-3 and rel_err(vg, vo) < 2e-3
    assert g.seq_len == o.seq_len == 2 * M


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_prefill_panel_gemm_is_bit_identical(mdx, gpu, oracle_lib, models, quant):
    """The batch-prefill projections with the activation panel staged in LDS
    (k_gemm_p, the default where a K split fits 1024) against the GEMM that
    loads its fragments per wave in rounds (k_gemm, selected by the test
    hook): the same K partition and summation order, so the logits and every
    K/V row are the same bits, over M = 60, 17 and 1 on top of each other."""
    cfg, get = models
    rng = np.random.default_rng(900 + quant)
    embs = [rng.standard_normal((m, 1024)).astype(np.float32) for m in (60, 17, 1)]
    runs = []
    for rounds in (0, 1):
        prev = mdx.lib().mdx_debug_gemm_rounds(rounds)
        try:
            g, _ = _pair(mdx, oracle_lib, cfg, get(quant), quant)
            out = [g.prefill_logits(e) for e in embs]
            kv = [g.kv_read(layer, 0, 78) for layer in (0, 1)]
            g.close()
        finally:
            mdx.lib().mdx_debug_gemm_rounds(prev)
        runs.append((out, kv))
    (oa, ka), (ob, kb) = runs
    for (ta, la), (tb, lb) in zip(oa, ob):
        assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    for (k1, v1), (k2, v2) in zip(ka, kb):
        assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def test_timed_out_launch_is_retried_cooperatively(mdx, gpu, oracle_lib, models, capfd):
    """A one-launch step whose waits give up (forced here with a 1-round spin
    limit, as a grid that is not co-resident would) reports the timeout in the
    state; the host runs the step again as a cooperative launch, and the
    result equals an undisturbed context's."""
    cfg, get = models
    path = get(1)
    g_ref, _ = _pair(mdx, oracle_lib, cfg, path, 1)
    g, _ = _pair(mdx, oracle_lib, cfg, path, 1)
    for d in (g_ref, g):
        d.kv_fill_normal(200, 13)
    t_ref, l_ref = g_ref.step(321)
    g.force_spin_limit(1)
    t, lg = g.step(321)
    err = capfd.readouterr().err
    print(err)
    assert "retrying with cooperative launches" in err
    assert t == t_ref and np.array_equal(lg, l_ref)
    assert g.seq_len == g_ref.seq_len == 201
    for tok in (7, 4000):   # later steps (cooperative now) still agree
        t_ref, l_ref = g_ref.step(tok)
        t, lg = g.step(tok)
        assert t == t_ref and np.array_equal(lg, l_ref)


def test_retry_ignores_stale_exchange_words(mdx, gpu, oracle_lib, models, capfd):
    """A timed-out launch whose late workgroups left words tagged with the
    epochs the retry would use (planted by a test hook between the failed
    launch and the retry): the retry clears the exchange words first, so its
    result still equals an undisturbed context's."""
    cfg, get = models
    path = get(1)
    g_ref, _ = _pair(mdx, oracle_lib, cfg, path, 1)
    g, _ = _pair(mdx, oracle_lib, cfg, path, 1)
    for d in (g_ref, g):
        d.kv_fill_normal(150, 17)
    t_ref, l_ref = g_ref.step(555)
    g.force_spin_limit(1)
    g.poison_next_retry()
    t, lg = g.step(555)
    assert "retrying with cooperative launches" in capfd.readouterr().err
    assert t == t_ref and np.array_equal(lg, l_ref)
    t_ref, l_ref = g_ref.step(t_ref)
    t, lg = g.step(t)
    assert t == t_ref and np.array_equal(lg, l_ref)


def test_stats_breakdown_with_profile(mdx, gpu, oracle_lib, models, monkeypatch):
    """MatmulDecoderStats (src/matmul_decoder.c:1616-1623): without
    MDX_PROFILE the one launch counts as matmul_ms; with MDX_PROFILE=1 it is
    split over matmul / cpu_ops / rebind (waits) / lm_head from the step's
    own timestamps.  Every field is >= 0 and the parts add up to total_ms;
    prefill-mode steps report no lm_head time.  The profiled step computes
    the same logits."""
    cfg, get = models
    path = get(0)
    plain, _ = _pair(mdx, oracle_lib, cfg, path, 0)
    monkeypatch.setenv("MDX_PROFILE", "1")
    prof, _ = _pair(mdx, oracle_lib, cfg, path, 0)
    monkeypatch.delenv("MDX_PROFILE")
    for d in (plain, prof):
        d.kv_fill_normal(300, 21)
    fields = ("matmul_ms", "rebind_ms", "convert_ms", "cpu_ops_ms", "lm_head_ms")
    for i, tok in enumerate((12, 3456, 78)):
        t0, l0 = plain.step(tok)
        t1, l1 = prof.step(tok)
        assert t0 == t1 and np.array_equal(l0, l1)
        a, b = plain.stats(), prof.stats()
        for st in (a, b):
            assert st["n_steps"] == i + 1 and st["total_ms"] > 0
            assert all(st[f] >= 0 for f in fields), st
            parts = sum(st[f] for f in fields)
            assert abs(parts - st["total_ms"]) <= 1e-3 + 1e-4 * st["total_ms"], st
        assert a["cpu_ops_ms"] == a["rebind_ms"] == a["lm_head_ms"] == 0 and a["matmul_ms"] > 0
        assert min(b["matmul_ms"], b["cpu_ops_ms"], b["rebind_ms"], b["lm_head_ms"]) > 0, b
    # prefill mode: no logits, no lm_head
    assert prof.step(5, logits=False)[0] == 0
    st = prof.stats()
    assert st["lm_head_ms"] == 0 and st["matmul_ms"] > 0 and st["n_steps"] == 4


def test_two_contexts_in_two_threads(mdx, gpu, oracle_lib, models, capfd):
    """Two contexts stepping at the same time from two threads: their one-launch
    steps are serialised inside the library, so neither grid is crowded out
    (no timeout, no cooperative retry) and each produces what it produces alone."""
    import threading
    cfg, get = models
    path = get(2)
    ref = []
    for seed in (3, 4):
        g, _ = _pair(mdx, oracle_lib, cfg, path, 2)
        g.kv_fill_normal(100, seed)
        ref.append(g.generate_greedy(11, 24)[0])
        g.close()
    ctx = []
    for seed in (3, 4):
        g, _ = _pair(mdx, oracle_lib, cfg, path, 2)
        g.kv_fill_normal(100, seed)
        ctx.append(g)
    out = [None, None]

    def run(i):
        out[i] = ctx[i].generate_greedy(11, 24)[0]

    th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    err = capfd.readouterr().err
    assert "retrying with cooperative launches" not in err
    assert out[0] == ref[0] and out[1] == ref[1]


def test_step_sample_after_one_launch_step(mdx, gpu, oracle_lib, models):
    """matmul_decoder_step_sample on the one-launch path: the sampler is
    enqueued after the persistent step and draws what the oracle's sampler
    (src/cpu_ops.c:593-648 with the same uniform) draws from the logits the
    same step returns; a plain-step twin fed the same tokens sees the same
    logits at every step."""
    cfg, get = models
    path = get(1)
    a, _ = _pair(mdx, oracle_lib, cfg, path, 1)
    b, _ = _pair(mdx, oracle_lib, cfg, path, 1)
    a.kv_fill_normal(40, 9)
    b.kv_fill_normal(40, 9)
    rng = np.random.default_rng(5)
    tok = 4321
    hist = []
    for i in range(8):
        u = float(rng.random())
        kw = dict(top_k=[2, 50, 1000][i % 3], temperature=0.9, top_p=[1.0, 0.8][i % 2],
                  repeat_tokens=hist[-4:], repeat_penalty=1.3)
        ts, ls = a.step_sample(tok, u, logits=True, **kw)
        _, lb = b.step(tok)
        assert np.array_equal(ls, lb), i
        rt, _, rval, rkept = oracle_lib.sample_topk(lb, u=u, **kw)
        # equal, except where a last-bit expf difference can move a boundary
        assert ts == rt or _near_boundary(rval, rkept, u, kw["top_p"]), (i, ts, rt)
        hist.append(ts)
        tok = ts
    assert a.seq_len == b.seq_len == 48
    a.close()
    b.close()


@pytest.mark.parametrize("quant", [0, 1])
def test_reference_python_callers_call_sequences(mdx, gpu, oracle_lib, models, quant):
    """The two reference Python callers' call sequences through the pybind
    module, on the one-launch path, against the oracle:
    - python/matmul_decoder.py:196-203 (run_embed): step_get_token(token_id=-1,
      embedding=row) for every embedding row, then step_get_token(token_id=-1,
      embedding=None), which the reference's C step rejects (no embedding and
      token -1: src/matmul_decoder.c:1447-1452), so the module returns -1 and
      the cache does not advance;
    - examples/qwen3_asr/matmul_decoder.py:186-201 (run_embed):
      prefill(token_id=-1, embedding=row) for all rows but the last (a step
      without the lm_head), step_get_token(token_id=-1, embedding=last row),
      then step_get_token(token_id=prev) fed back for the generated tokens.
    The oracle runs the same calls, fed the tokens the module returned (the
    caller's own feedback), and every returned token is the oracle's argmax
    for that step, or within the step tests' logit bar of it (2e-3 of the
    largest |logit|: a near tie, where two valid accumulation orders may
    pick either)."""
    import matmul_decoder as md     # the pybind module, beside mdx_lib on the test path
    cfg, get = models
    path = get(quant)
    dec = md.MatmulDecoder(path, max_seq_len=256, quant_type=QUANTS[quant])
    rng = np.random.default_rng(77 + quant)
    n = 6
    emb = (rng.standard_normal((n, SHAPE["hidden_dim"])) * 0.5).astype(np.float32)

    # python/matmul_decoder.py: every row through step_get_token
    def same_choice(t, to, lo, what):
        assert 0 <= t < SHAPE["vocab_size"], what
        assert t == to or lo[to] - lo[t] <= 2e-3 * float(np.abs(lo).max()), f"{what}: {t} vs {to}"

    dec.clear_kv_cache()
    o = oracle_lib.Model(path, SHAPE, quant, 256, kv_fp16=True)
    for i in range(n):
        t = dec.step_get_token(token_id=-1, embedding=emb[i])
        to, lo = o.step(-1, emb[i])
        same_choice(t, to, lo, f"row {i}")
    assert dec.seq_len == n
    for _ in range(3):
        assert dec.step_get_token(token_id=-1, embedding=None) == -1
        assert o.step(-1, None)[0] == -1
    assert dec.seq_len == n and o.seq_len == n

    # examples/qwen3_asr/matmul_decoder.py: prefill rows, last row with the head, then greedy
    dec.clear_kv_cache()
    o = oracle_lib.Model(path, SHAPE, quant, 256, kv_fp16=True)
    for i in range(n - 1):
        dec.prefill(token_id=-1, embedding=emb[i])
        o.step(-1, emb[i], logits=False)
    first = dec.step_get_token(token_id=-1, embedding=emb[n - 1])
    to, lo = o.step(-1, emb[n - 1])
    same_choice(first, to, lo, "first token")
    prev, exact = first, int(first == to)
    for i in range(12):
        t = dec.step_get_token(token_id=prev)
        to, lo = o.step(prev)
        same_choice(t, to, lo, f"generated token {i + 1}")
        exact += int(t == to)
        prev = t
    assert exact >= 11, f"only {exact} of 13 tokens equal to the oracle's argmax"
    assert dec.seq_len == n + 12
