"""The oracle's sampler (src/cpu_ops.c:593-648 restated, with a given uniform in
place of rand()/RAND_MAX), pinned on the CPU by methods independent of its
insertion sort:
- candidates: a stable numpy lexsort on (value desc, index asc), so ties go to
  the lower index as the reference's strict '>' insertion keeps them;
- temperature: the candidate values equal float32 x / T;
- repetition penalty: numpy's rule on the distinct listed tokens (a listed
  duplicate is penalised once);
- the draw is the inverse CDF of the softmax over the candidates: u = 0 gives
  the argmax, u = 1 the last candidate, and a grid of N uniforms hits each
  candidate N * p_i times to within one;
- top-p keeps the shortest prefix whose float32 running sum reaches
  top_p * sum (numpy's cumsum is sequential), and a tiny top_p is greedy.
The device sampler is checked against this oracle in tests/test_gpu_sample.py."""
import numpy as np
import pytest


def _brute(x, k):
    order = np.lexsort((np.arange(x.size), -x))
    return order[:k]


def _logits(V, seed, scale=3.0, quant=None):
    x = (np.random.default_rng(seed).standard_normal(V) * scale).astype(np.float32)
    if quant:
        x = (np.round(x * quant) / quant).astype(np.float32)
    return x


@pytest.mark.parametrize("k", [1, 2, 7, 64, 500])
@pytest.mark.parametrize("quant", [None, 2])
def test_candidates_match_stable_sort(oracle_lib, k, quant):
    x = _logits(5003, 11 + k, quant=quant)
    tok, idx, val, kept = oracle_lib.sample_topk(x, top_k=k, u=0.0)
    ref = _brute(x, k)
    assert np.array_equal(idx, ref)
    assert np.array_equal(val, x[ref])
    assert kept == k
    assert tok == int(np.argmax(x))          # u = 0: the first maximum


def test_temperature_divides(oracle_lib):
    x = _logits(4096, 3)
    for T in (0.7, 1.3, 2.0):
        _, idx, val, _ = oracle_lib.sample_topk(x, top_k=50, temperature=T, u=0.5)
        xt = (x / np.float32(T)).astype(np.float32)
        ref = _brute(xt, 50)
        assert np.array_equal(idx, ref) and np.array_equal(val, xt[ref])


def test_repeat_penalty_once_per_token(oracle_lib):
    x = _logits(2048, 4)
    top = _brute(x, 6)
    neg = np.argsort(x)[:2]
    toks = [int(top[0]), int(top[0]), int(top[3]), int(neg[0]), int(neg[1]), int(neg[1])]
    p = np.float32(1.7)
    xp = x.copy()
    for t in set(toks):
        xp[t] = xp[t] / p if xp[t] > 0 else xp[t] * p
    _, idx, val, _ = oracle_lib.sample_topk(x, top_k=20, u=0.2, repeat_tokens=toks, repeat_penalty=1.7)
    ref = _brute(xp, 20)
    assert np.array_equal(idx, ref) and np.array_equal(val, xp[ref])


def test_draw_is_the_inverse_cdf(oracle_lib):
    x = _logits(1000, 5, scale=1.0)
    k = 8
    ref = _brute(x, k)
    e = np.exp((x[ref] - x[ref[0]]).astype(np.float64))
    p = e / e.sum()
    N = 4000
    counts = np.zeros(k, np.int64)
    for j in range(N):
        tok, idx, _, _ = oracle_lib.sample_topk(x, top_k=k, u=(j + 0.5) / N)
        counts[list(idx).index(tok)] += 1
    assert np.all(np.abs(counts - N * p) <= 1.5), (counts, N * p)
    assert oracle_lib.sample_topk(x, top_k=k, u=1.0)[0] == ref[-1]
    assert oracle_lib.sample_topk(x, top_k=k, u=0.0)[0] == ref[0]


@pytest.mark.parametrize("top_p", [0.3, 0.6, 0.9, 0.999])
def test_top_p_prefix(oracle_lib, top_p):
    x = _logits(3000, 6, scale=1.5)
    k = 40
    ref = _brute(x, k)
    e = np.exp((x[ref] - x[ref[0]]).astype(np.float32)).astype(np.float32)
    run = np.cumsum(e, dtype=np.float32)
    m = int(np.argmax(run >= np.float32(top_p) * run[-1])) + 1
    toks = set()
    for u in np.linspace(0.0, 1.0, 97):
        tok, _, _, kept = oracle_lib.sample_topk(x, top_k=k, top_p=top_p, u=float(u))
        assert kept == m
        toks.add(tok)
    assert toks <= set(ref[:m].tolist()) and ref[m - 1] in toks
    assert oracle_lib.sample_topk(x, top_k=k, top_p=1e-9, u=0.9)[0] == ref[0]
