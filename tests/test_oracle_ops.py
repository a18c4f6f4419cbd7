"""Pins the oracle's element-wise ops and projections (CPU only).

Each check is chosen so that a plausible mistake in the restatement of the
reference (src/cpu_ops.c, src/matmul_decoder.c) fails it: closed forms,
special cases that reduce to exact arithmetic, float64 brute force, and the
invariants that the reference's own fixtures (tests/golden/reference_data,
copied from the reference's tests/reference_data) fix.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_err

RD = os.path.join(GOLDEN, "reference_data")


def test_fp16_round_trip_all_patterns(oracle_lib):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_lib.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _rounding_cases():
    rng = np.random.default_rng(7)
    vals = [rng.standard_normal(20000) * s for s in (1e-7, 1e-5, 1e-3, 1.0, 100.0, 3e4)]
    # exact midpoints between adjacent halves: ties must go to even
    base = rng.integers(0x0400, 0x7bff, 5000).astype(np.uint16)
    lo = base.view(np.float16).astype(np.float64)
    hi = (base + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    sub = (np.arange(1, 2048) * 2.0 ** -25).astype(np.float32)       # subnormal ties
    edge = np.array([0.0, -0.0, 65504, 65519.996, 65520, 65536, 1e9, -1e9, np.inf, -np.inf,
                     2 ** -24, 2 ** -25, 3 * 2 ** -26, 6.1e-5, 6.103515625e-05], np.float32)
    return np.concatenate([*[v.astype(np.float32) for v in vals], mids, -mids, sub, edge])


def test_fp16_rne_matches_numpy(oracle_lib):
    x = _rounding_cases()
    got = oracle_lib.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_rng_streams_match_product(oracle_lib, mdx):
    for name, n in (("a", 1), ("kv/k/00", 5), ("x", 3 * (1 << 20) + 7)):
        s1 = oracle_lib.seed_for(1234, name)
        s2 = mdx.synth_seed(1234, name)
        assert s1 == s2
        a = oracle_lib.fill_normal(n, s1)
        b = mdx.synth_fill_normal(n, s2)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    big = oracle_lib.fill_normal(1 << 21, oracle_lib.seed_for(5, "stats"))
    assert abs(big.mean()) < 5e-3 and abs(big.std() - 1.0) < 5e-3


# ---- RMSNorm (reference: src/cpu_ops.c:18-55) ------------------------------------

def test_rms_norm_closed_forms(oracle_lib):
    eps = 1e-6
    for d in (8, 13, 128, 1024):
        c = 0.37
        x = np.full(d, c, np.float32)
        w = np.linspace(0.5, 1.5, d).astype(np.float32)
        want = w * c / np.sqrt(c * c + eps)
        assert rel_err(oracle_lib.rms_norm(x, w, eps), want) < 2e-6
    # eps dominates for tiny inputs: a dropped eps would give |out| = 1
    x = np.full(64, 1e-4, np.float32)
    out = oracle_lib.rms_norm(x, np.ones(64, np.float32), eps)
    assert abs(out[0] - 1e-4 / np.sqrt(1e-8 + 1e-6)) < 1e-6


def test_rms_norm_float64(oracle_lib):
    rng = np.random.default_rng(1)
    for d in (7, 100, 1024, 3072):
        x = rng.standard_normal(d).astype(np.float32) * 3
        w = rng.standard_normal(d).astype(np.float32)
        xd = x.astype(np.float64)
        want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
        assert rel_err(oracle_lib.rms_norm(x, w, 1e-6), want) < 3e-6


# ---- RoPE (reference: src/matmul_decoder.c:620-631, src/cpu_ops.c:109-155) -------

def test_rope_tables_formula(oracle_lib):
    c, s = oracle_lib.rope_tables(300, 128, 1e6)
    i = np.arange(64)
    ang = np.arange(300)[:, None] * (1e6 ** (-2.0 * i / 128))[None, :]
    # fp32 angle: relative error of a few ulp of the angle itself
    tol = 4e-7 * ang + 2e-6
    assert np.all(np.abs(c - np.cos(ang)) < tol)
    assert np.all(np.abs(s - np.sin(ang)) < tol)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)


@pytest.mark.parametrize("style", [0, 1])
def test_rope_identity_norm_and_direction(oracle_lib, style):
    rng = np.random.default_rng(2)
    c, s = oracle_lib.rope_tables(64, 128, 1e6)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    assert np.array_equal(oracle_lib.apply_rope(x, c[0], s[0], 4, 128, style), x)
    y = oracle_lib.apply_rope(x, c[37], s[37], 4, 128, style)
    pairs = (lambda v: v.reshape(4, 64, 2)) if style == 0 else \
        (lambda v: np.stack([v.reshape(4, 2, 64)[:, 0], v.reshape(4, 2, 64)[:, 1]], -1))
    assert np.allclose(np.linalg.norm(pairs(y), axis=-1), np.linalg.norm(pairs(x), axis=-1),
                       rtol=1e-6)
    # pair 0 has frequency 1: (1, 0) rotates to (cos p, sin p)
    e = np.zeros(128, np.float32)
    e[0] = 1.0
    r = oracle_lib.apply_rope(e, c[1], s[1], 1, 128, style)
    i1 = 1 if style == 0 else 64
    assert abs(r[0] - np.cos(1.0)) < 1e-6 and abs(r[i1] - np.sin(1.0)) < 1e-6


def test_rope_composition_and_styles(oracle_lib):
    rng = np.random.default_rng(3)
    c, s = oracle_lib.rope_tables(128, 64, 1e4)
    x = rng.standard_normal(64).astype(np.float32)
    two = oracle_lib.apply_rope(oracle_lib.apply_rope(x, c[20], s[20], 1, 64, 1), c[33], s[33], 1, 64, 1)
    one = oracle_lib.apply_rope(x, c[53], s[53], 1, 64, 1)
    assert np.max(np.abs(two - one)) < 2e-5
    # style 0 on interleaved data == style 1 on the de-interleaved data
    perm = np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)])
    a = oracle_lib.apply_rope(x, c[9], s[9], 1, 64, 0)
    b = oracle_lib.apply_rope(x[perm], c[9], s[9], 1, 64, 1)
    assert np.array_equal(a[perm], b)


def test_rope_batch_equals_tables(oracle_lib):
    rng = np.random.default_rng(4)
    M, nh, hd = 5, 3, 128
    x = rng.standard_normal(M * nh * hd).astype(np.float32)
    c, s = oracle_lib.rope_tables(200, hd, 1e6)
    got = oracle_lib.apply_rope_batch(x, M, 150, nh, hd, 1e6, 1)
    for t in range(M):
        row = oracle_lib.apply_rope(x[t * nh * hd:(t + 1) * nh * hd], c[150 + t], s[150 + t], nh, hd, 1)
        assert np.array_equal(got[t * nh * hd:(t + 1) * nh * hd], row)


# ---- attention (reference: src/cpu_ops.c:202-264, :459-571) ------------------------

def _attn64(q, kc, vc, nq, nkv, hd, L):
    q = q.reshape(nq, hd).astype(np.float64)
    k = kc.reshape(-1, nkv, hd)[:L].astype(np.float64)
    v = vc.reshape(-1, nkv, hd)[:L].astype(np.float64)
    out = np.empty((nq, hd))
    for h in range(nq):
        g = h // (nq // nkv)
        sc = k[:, g] @ q[h] / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ v[:, g]
    return out.ravel()


def test_attention_single_position_is_gqa_copy(oracle_lib):
    rng = np.random.default_rng(5)
    nq, nkv, hd = 16, 8, 128
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    out = oracle_lib.attention(q, k, v, nq, nkv, hd, 1)
    assert np.array_equal(out, np.repeat(v.reshape(nkv, hd), nq // nkv, axis=0).ravel())


def test_attention_special_cases_and_float64(oracle_lib):
    rng = np.random.default_rng(6)
    nq, nkv, hd, L = 8, 2, 64, 37
    q = rng.standard_normal(nq * hd).astype(np.float32)
    v = rng.standard_normal(L * nkv * hd).astype(np.float32)
    kc = np.tile(rng.standard_normal(nkv * hd).astype(np.float32), L)   # identical keys
    out = oracle_lib.attention(q, kc, v, nq, nkv, hd, L)
    mean_v = np.repeat(v.reshape(L, nkv, hd).mean(0), nq // nkv, axis=0).ravel()
    assert np.max(np.abs(out - mean_v)) < 1e-5
    k = rng.standard_normal(L * nkv * hd).astype(np.float32)
    assert rel_err(oracle_lib.attention(q, k, v, nq, nkv, hd, L), _attn64(q, k, v, nq, nkv, hd, L)) < 1e-5
    # one dominant key selects its value row
    k2 = np.zeros((L, nkv, hd), np.float32)
    k2[11, :, :] = 50.0 * q.reshape(nq, hd)[::nq // nkv] / np.linalg.norm(q.reshape(nq, hd)[::nq // nkv], axis=1, keepdims=True)
    o2 = oracle_lib.attention(q, k2.ravel(), v, nq, nkv, hd, L).reshape(nq, hd)
    assert np.max(np.abs(o2[::nq // nkv] - v.reshape(L, nkv, hd)[11])) < 1e-3


def test_batch_causal_equals_per_token(oracle_lib):
    rng = np.random.default_rng(8)
    nq, nkv, hd, S, M = 4, 2, 64, 9, 6
    kvd = nkv * hd
    kc = rng.standard_normal(S * kvd).astype(np.float32)
    vc = rng.standard_normal(S * kvd).astype(np.float32)
    qb = rng.standard_normal(M * nq * hd).astype(np.float32)
    kb = rng.standard_normal(M * kvd).astype(np.float32)
    vb = rng.standard_normal(M * kvd).astype(np.float32)
    out = oracle_lib.attention_batch_causal(qb, kb, vb, kc, vc, M, nq, nkv, hd, S).reshape(M, -1)
    for t in range(M):
        k_all = np.concatenate([kc, kb[:(t + 1) * kvd]])
        v_all = np.concatenate([vc, vb[:(t + 1) * kvd]])
        row = oracle_lib.attention(qb[t * nq * hd:(t + 1) * nq * hd], k_all, v_all, nq, nkv, hd, S + t + 1)
        assert np.array_equal(out[t], row)


# ---- SiLU, argmax ------------------------------------------------------------------

def test_silu_mul(oracle_lib):
    rng = np.random.default_rng(9)
    for n in (3072, 6):                       # 6: two tail elements use the division form
        g = (rng.standard_normal(n) * 4).astype(np.float32)
        u = rng.standard_normal(n).astype(np.float32)
        gd = g.astype(np.float64)
        want = gd / (1 + np.exp(-gd)) * u
        assert rel_err(oracle_lib.silu_mul(g, u), want) < 2e-6
    assert oracle_lib.silu_mul(np.zeros(4, np.float32), np.ones(4, np.float32)).tolist() == [0, 0, 0, 0]


def test_argmax_first_index_wins(oracle_lib):
    x = np.array([1, 5, 3, 5, 5, -1], np.float32)
    assert oracle_lib.argmax(x) == 1
    assert oracle_lib.argmax(np.full(100, -2.0, np.float32)) == 0


def _argmax_strict(x):
    """argmax_f32 (src/cpu_ops.c:575-586) as written: the running maximum
    starts at x[0] and moves only on a strict '>'."""
    mv, mi = x[0], 0
    for i in range(1, len(x)):
        if x[i] > mv:
            mv, mi = x[i], i
    return mi


def test_argmax_signed_zero_and_nan(oracle_lib):
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    cases = [
        [-0.0, 0.0, -1.0],          # -0 and +0 are equal: the first index
        [0.0, -0.0, -3.0],
        [-5.0, -0.0, 0.0, -0.0],
        [nan, 3.0, 7.0],            # NaN at 0: no later value compares greater
        [1.0, nan, 2.0, nan],       # NaN elsewhere never wins
        [-inf, nan, nan],
        [nan, nan],
        [-inf, -inf, -1e30],
    ]
    for c in cases:
        x = np.array(c, np.float32)
        assert oracle_lib.argmax(x) == _argmax_strict(x), c


# ---- projections ---------------------------------------------------------------------

def test_matmul_f16_float64(oracle_lib):
    rng = np.random.default_rng(10)
    M, K, N = 3, 96, 40
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float16)
    y = oracle_lib.matmul(0, x, w.view(np.uint16), None, M, K, N)
    want = x.astype(np.float16).astype(np.float64) @ w.astype(np.float64)
    assert rel_err(y, want) < 1e-5
    # integer-valued operands: every partial sum is exact
    xi = rng.integers(-16, 17, (M, K)).astype(np.float32)
    wi = rng.integers(-100, 101, (K, N)).astype(np.float16)
    yi = oracle_lib.matmul(0, xi, wi.view(np.uint16), None, M, K, N)
    assert np.array_equal(yi, (xi.astype(np.int64) @ wi.astype(np.int64)).astype(np.float32))


def test_matmul_accumulation_orders(oracle_lib):
    """Order 1 (four interleaved sums) is a second valid accumulation order:
    exact on integer-valued operands like order 0, within fp32 rounding of
    the float64 product on general data, different from order 0 in the last
    bits, and order 0 is what the oracle uses unless switched."""
    rng = np.random.default_rng(11)
    M, K, N = 2, 1024, 256
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    want = x.astype(np.float16).astype(np.float64) @ w.astype(np.float64)
    xi = rng.integers(-16, 17, (M, K)).astype(np.float32)
    exact = (xi.astype(np.int64) @ q.astype(np.int64)).astype(np.float32)
    ys = {}
    try:
        for order in (0, 1, 2):
            oracle_lib.lib().orc_set_accum_order(order)
            ys[order] = oracle_lib.matmul(0, x, w.view(np.uint16), None, M, K, N)
            assert rel_err(ys[order], want) < 1e-5
            assert np.array_equal(oracle_lib.matmul(1, xi, q, None, M, K, N), exact)
    finally:
        oracle_lib.lib().orc_set_accum_order(0)
    assert not np.array_equal(ys[0], ys[1]) and not np.array_equal(ys[0], ys[2])
    assert not np.array_equal(ys[1], ys[2])
    # order 2 by hand: 16 sums of k mod 16 in increasing k, then a pairwise tree
    x16 = x.astype(np.float16).astype(np.float32)
    wf = w.astype(np.float32)
    sums = np.zeros((16, M, N), np.float32)
    for k in range(K):
        sums[k % 16] = sums[k % 16] + np.outer(x16[:, k], wf[k]).astype(np.float32)
    while len(sums) > 1:
        sums = np.stack([sums[2 * j] + sums[2 * j + 1] for j in range(len(sums) // 2)])
    assert np.array_equal(sums[0], ys[2])
    assert np.array_equal(oracle_lib.matmul(0, x, w.view(np.uint16), None, M, K, N), ys[0])


@pytest.mark.parametrize("K,N", [(1024, 4096), (3072, 64), (48, 1000)])
def test_matmul_i8_known_answer_bit_exact(oracle_lib, K, N):
    rng = np.random.default_rng(K + N)
    x = rng.integers(-16, 17, K).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    exact = x.astype(np.int64) @ q.astype(np.int64)
    y = oracle_lib.matmul(1, x, q, None, 1, K, N)[0]
    assert np.array_equal(y, exact.astype(np.float32))
    s = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    ys = oracle_lib.matmul(1, x, q, s, 1, K, N)[0]
    assert np.array_equal(ys, exact.astype(np.float32) * s)


def _pack_i4(q):
    """[K,N] int in [-8,7] -> [K,N/2] bytes, column 2j in the low nibble."""
    u = (q & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def test_matmul_i4_all_codes(oracle_lib):
    K, N = 32, 64
    q = ((np.arange(K)[:, None] * 3 + np.arange(N)[None, :]) % 16 - 8).astype(np.int64)
    packed = _pack_i4(q)
    s = np.linspace(0.5, 2.0, N).astype(np.float32)
    for k in (0, 5, 31):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = oracle_lib.matmul(2, x, packed, s, 1, K, N)[0]
        assert np.array_equal(y, q[k].astype(np.float32) * s)
    assert set(np.unique(q)) == set(range(-8, 8))


def test_gemv_rows(oracle_lib):
    rng = np.random.default_rng(11)
    for K in (1024, 30):
        N = 77
        x = rng.standard_normal(K).astype(np.float32)
        w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        assert rel_err(oracle_lib.gemv_rows_f32(x, w, N, K), w.astype(np.float64) @ x) < 1e-5
        w16 = w.astype(np.float16)
        assert rel_err(oracle_lib.gemv_rows_f16(x, w16.view(np.uint16), N, K),
                       w16.astype(np.float64) @ x) < 1e-5


def test_lm_head_quantiser_matches_product_and_bounds(oracle_lib, mdx):
    rng = np.random.default_rng(12)
    V, K = 300, 128
    lm = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    lm[17] = 0.0                                  # zero row: scale 0, q 0
    lm16 = lm.astype(np.float16)
    q1, s1 = oracle_lib.quantize_lm_head(lm16.view(np.uint16), V, K)
    q2, s2 = mdx.quantize_lm_head(lm16.view(np.uint16), V, K)
    assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    amax = np.abs(lm16.astype(np.float32)).max(1)
    assert np.array_equal(s1, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q1).max(1)[amax > 0] == 127) and np.all(q1[17] == 0)
    err = np.abs(q1 * s1[:, None] - lm16.astype(np.float32))
    assert np.all(err <= s1[:, None] * 0.5 + 1e-7)


# ---- invariants fixed by the reference's own fixtures --------------------------------

def _npy(name):
    return np.load(os.path.join(RD, name + ".npy"), allow_pickle=False)


@pytest.mark.parametrize("layer", ["00", "27"])
def test_fixture_gqa_attention_at_pos0(oracle_lib, layer):
    v = _npy(f"layer_{layer}_v_proj")
    k = _npy(f"layer_{layer}_k_proj")
    q = _npy(f"layer_{layer}_after_rope_q")
    out = oracle_lib.attention(q, k, v, 16, 8, 128, 1)
    assert np.array_equal(out, _npy(f"layer_{layer}_attn_out"))


@pytest.mark.parametrize("layer", ["00", "27"])
def test_fixture_qk_norm_and_rope_pos0(oracle_lib, layer):
    q = _npy(f"layer_{layer}_q_proj").reshape(16, 128)
    after = _npy(f"layer_{layer}_after_rope_q").reshape(16, 128)
    unit = q / np.sqrt(np.mean(q.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
    w = after / unit                              # the q_norm weight, seen through every head
    assert np.max(np.abs(w - w[0])) < 1e-3 * np.max(np.abs(w[0]))
    w0 = np.median(w, axis=0).astype(np.float32)
    c, s = oracle_lib.rope_tables(1, 128, 1e6)
    got = np.stack([oracle_lib.apply_rope(oracle_lib.rms_norm(q[h], w0, 1e-6), c[0], s[0], 1, 128, 0)
                    for h in range(16)])
    assert rel_err(got, after) < 1e-4


def test_fixture_projections_are_fp16_values(oracle_lib):
    for name in ("layer_00_q_proj", "layer_00_k_proj", "layer_00_v_proj", "layer_27_q_proj"):
        a = _npy(name)
        assert np.array_equal(oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(a)), a)
