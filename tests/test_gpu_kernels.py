"""GPU parity of each hand-written kernel against the oracle, through the C ABI
single-kernel entry points (mdx_ext.h).  Bars: INT8 dot products bit-exact on
integer-valued known-answer inputs; floating point within 1e-3 of the
oracle measured as max|gpu - oracle| / max|oracle| ("rel"), with the
tolerance written at each check."""
import numpy as np
import pytest

from conftest import cosine, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3          # bound per projection


def _f16_bits(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def _pack_i4(q):
    u = (q & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


# ---- M = 1 projections -------------------------------------------------------------

LAYER_SHAPES = [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 3072), (3072, 1024)]


@pytest.mark.parametrize("K,N", LAYER_SHAPES)
def test_gemv_fp16_layer_projection(mdx, gpu, oracle_lib, K, N):
    rng = np.random.default_rng(K * 7 + N)
    x = rng.standard_normal(K).astype(np.float32)
    w = _f16_bits(rng.standard_normal((K, N)) * 0.02)
    y = mdx.gemv(0, K, N, w, None, x)
    ref = oracle_lib.matmul(0, x, w, None, 1, K, N)[0]
    assert rel_err(y, ref) < TOL * 0.1


def test_gemv_int8_lm_head_tile(mdx, gpu, oracle_lib):
    """1 x 1024 x 4096 INT8 tile: int8 U[-127,127], fp32 scales U[1e-3,1e-2], x ~N(0,1)."""
    rng = np.random.default_rng(1001)
    K, N = 1024, 4096
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    y = mdx.gemv(1, K, N, q, s, x)
    ref = oracle_lib.matmul(1, x, q, s, 1, K, N)[0]
    assert rel_err(y, ref) < TOL * 0.1


@pytest.mark.parametrize("K,N", [(1024, 4096), (3072, 1024), (2048, 96)])
def test_gemv_int8_known_answer_bit_exact(mdx, gpu, oracle_lib, K, N):
    rng = np.random.default_rng(K + 3 * N)
    x = rng.integers(-16, 17, K).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    exact = (x.astype(np.int64) @ q.astype(np.int64)).astype(np.float32)
    assert np.array_equal(mdx.gemv(1, K, N, q, None, x), exact)
    s = np.ones(N, np.float32)
    assert np.array_equal(mdx.gemv(1, K, N, q, s, x), exact)


def test_gemv_int4_all_codes_and_random(mdx, gpu, oracle_lib):
    K, N = 1024, 256
    q = ((np.arange(K)[:, None] * 5 + np.arange(N)[None, :]) % 16 - 8).astype(np.int64)
    packed = _pack_i4(q)
    s = np.linspace(0.25, 2.0, N).astype(np.float32)
    for k in (0, 1, 7, 8, 31, 1023):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        assert np.array_equal(mdx.gemv(2, K, N, packed, s, x), q[k].astype(np.float32) * s)
    rng = np.random.default_rng(5)
    xi = rng.integers(-16, 17, K).astype(np.float32)
    assert np.array_equal(mdx.gemv(2, K, N, packed, None, xi),
                          (xi.astype(np.int64) @ q).astype(np.float32))
    for K2, N2 in ((1024, 2048), (3072, 1024)):
        qr = rng.integers(-8, 8, (K2, N2))
        sr = _f16_bits(rng.uniform(1e-3, 3e-3, N2)).view(np.float16).astype(np.float32)
        x = rng.standard_normal(K2).astype(np.float32)
        y = mdx.gemv(2, K2, N2, _pack_i4(qr), sr, x)
        ref = oracle_lib.matmul(2, x, _pack_i4(qr), sr, 1, K2, N2)[0]
        assert rel_err(y, ref) < TOL * 0.1


def test_gemv_fp32_activation_rows(mdx, gpu, oracle_lib):
    rng = np.random.default_rng(6)
    K, N = 1024, 2048
    x = rng.standard_normal(K).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    assert rel_err(mdx.gemv(3, K, N, w, None, x), oracle_lib.gemv_rows_f32(x, w, N, K)) < 1e-5
    w16 = _f16_bits(w)
    assert rel_err(mdx.gemv(4, K, N, w16, None, x), oracle_lib.gemv_rows_f16(x, w16, N, K)) < 1e-5


# ---- M <= 64 MFMA projections ------------------------------------------------------------

@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("M,K,N", [(60, 1024, 4096), (60, 3072, 1024), (1, 1024, 1024),
                                   (64, 2048, 1024), (7, 1024, 6144), (64, 352, 96), (3, 96, 64)])
def test_gemm_matches_oracle(mdx, gpu, oracle_lib, kind, M, K, N):
    rng = np.random.default_rng(M * 31 + K + N + kind)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if kind == 0:
        w, s = _f16_bits(rng.standard_normal((K, N)) * 0.02), None
    elif kind == 1:
        w, s = rng.integers(-127, 128, (K, N)).astype(np.int8), rng.uniform(1e-4, 2e-4, N).astype(np.float32)
    else:
        w, s = _pack_i4(rng.integers(-8, 8, (K, N))), rng.uniform(1e-3, 3e-3, N).astype(np.float32)
    y = mdx.gemm(kind, M, K, N, w, s, x)
    ref = oracle_lib.matmul(kind, x, w, s, M, K, N)
    assert rel_err(y, ref) < TOL * 0.1


# The o / down stages of the prefill: split-K over 256-K blocks with the block
# order grouped per XCD (N/64 x K/256 a multiple of 8: (60,2048,1024),
# (60,3072,1024), (5,4096,192), (33,1024,4096)), the plain order otherwise
# ((17,768,960): 45 blocks; (64,256,64): one block), and K not a multiple of
# 256 (the k_gemm path: (9,320,128), whose last K-block is partial for int8
# and int4, and (11,2592,128), where ten requested splits of 81 fp16
# K-blocks would leave the last one empty).  hidden += x.W*s is checked
# against the oracle's projection; the fp16 normed rows against numpy on the
# returned hidden (one fp16 ulp).
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("M,K,N", [(60, 2048, 1024), (60, 3072, 1024), (5, 4096, 192), (33, 1024, 4096),
                                   (17, 768, 960), (64, 256, 64), (9, 320, 128), (11, 2592, 128)])
def test_gemm_residual_norm_matches_oracle(mdx, gpu, oracle_lib, kind, M, K, N):
    rng = np.random.default_rng(M * 7 + K * 3 + N + kind)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if kind == 0:
        w, s = _f16_bits(rng.standard_normal((K, N)) * 0.02), None
    elif kind == 1:
        w, s = rng.integers(-127, 128, (K, N)).astype(np.int8), rng.uniform(1e-4, 2e-4, N).astype(np.float32)
    else:
        w, s = _pack_i4(rng.integers(-8, 8, (K, N))), rng.uniform(1e-3, 3e-3, N).astype(np.float32)
    h0 = rng.standard_normal((M, N)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, N).astype(np.float32)
    h, x16 = mdx.gemm_residual(kind, M, K, N, w, s, x, h0, nw)
    y = oracle_lib.matmul(kind, x, w, s, M, K, N)
    assert rel_err(h - h0, y) < TOL * 0.1, f"projection rel err {rel_err(h - h0, y):.2e}"
    assert np.allclose(h, h0 + y, rtol=1e-5, atol=1e-5 * float(np.abs(y).max()))
    rms = 1.0 / np.sqrt((h.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    ref16 = ((h * rms) * nw).astype(np.float16).view(np.uint16).astype(np.int32)
    ulp = np.abs(x16.astype(np.int32) - ref16)
    assert ulp.max() <= 1, f"normed rows differ by {ulp.max()} fp16 ulp"
    h2, none = mdx.gemm_residual(kind, M, K, N, w, s, x, h0, None)
    assert none is None and np.array_equal(h2, h)


def test_gemm_int8_known_answer_bit_exact(mdx, gpu):
    rng = np.random.default_rng(77)
    M, K, N = 60, 3072, 256
    x = rng.integers(-16, 17, (M, K)).astype(np.float32)
    q = rng.integers(-127, 128, (K, N)).astype(np.int8)
    exact = (x.astype(np.int64) @ q.astype(np.int64)).astype(np.float32)
    assert np.array_equal(mdx.gemm(1, M, K, N, q, None, x), exact)


# ---- attention -----------------------------------------------------------------------

def _kv(rng, L, kvd):
    k = rng.standard_normal(L * kvd).astype(np.float16)
    v = rng.standard_normal(L * kvd).astype(np.float16)
    return k, v


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("pos", [0, 1, 16, 17, 512, 575, 1023, 4096])
def test_attention_decode_fused(mdx, gpu, oracle_lib, pos, style):
    """QK-norm + RoPE + K/V append + split-K GQA attention + merge, one kernel."""
    rng = np.random.default_rng(pos * 2 + style)
    nq, nkv, hd = 16, 8, 128
    qd, kvd = nq * hd, nkv * hd
    qkv = (rng.standard_normal(qd + 2 * kvd) * 2).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    k, v = _kv(rng, pos, kvd)
    out, k_new, v_new = mdx.attn_decode(nq, nkv, hd, pos, style, 1e6, 1e-6, qn, kn, qkv,
                                        k.view(np.uint16), v.view(np.uint16))
    c, s = oracle_lib.rope_tables(pos + 1, hd, 1e6)
    q = np.concatenate([oracle_lib.rms_norm(qkv[h * hd:(h + 1) * hd], qn, 1e-6) for h in range(nq)])
    kr = np.concatenate([oracle_lib.rms_norm(qkv[qd + h * hd:qd + (h + 1) * hd], kn, 1e-6)
                         for h in range(nkv)])
    q = oracle_lib.apply_rope(q, c[pos], s[pos], nq, hd, style)
    kr = oracle_lib.apply_rope(kr, c[pos], s[pos], nkv, hd, style)
    k16 = kr.astype(np.float16)
    v16 = qkv[qd + kvd:].astype(np.float16)
    assert rel_err(k_new.view(np.float16).astype(np.float32), k16.astype(np.float32)) < 1e-3
    assert np.array_equal(v_new, v16.view(np.uint16))
    kc = np.concatenate([k.astype(np.float32), k_new.view(np.float16).astype(np.float32)])
    vc = np.concatenate([v.astype(np.float32), v16.astype(np.float32)])
    ref = oracle_lib.attention(q, kc, vc, nq, nkv, hd, pos + 1)
    assert rel_err(out, ref.astype(np.float16).astype(np.float32)) < TOL
    if pos == 0:
        assert np.array_equal(out, np.repeat(v16.astype(np.float32).reshape(nkv, hd), 2, axis=0).ravel())


@pytest.mark.parametrize("S,M", [(0, 60), (0, 1), (100, 33), (4000, 64)])
@pytest.mark.parametrize("nq,nkv,hd", [(16, 8, 128), (8, 2, 64), (4, 2, 256)])
def test_attention_prefill(mdx, gpu, oracle_lib, S, M, nq, nkv, hd):
    rng = np.random.default_rng(S + M + hd)
    kvd = nkv * hd
    q = rng.standard_normal(M * nq * hd).astype(np.float32)
    k, v = _kv(rng, S + M, kvd)
    out = mdx.attn_prefill(nq, nkv, hd, S, M, q, k.view(np.uint16), v.view(np.uint16))
    kf, vf = k.astype(np.float32), v.astype(np.float32)
    ref = oracle_lib.attention_batch_causal(q, kf[S * kvd:], vf[S * kvd:], kf[:S * kvd], vf[:S * kvd],
                                            M, nq, nkv, hd, S).reshape(M, -1)
    assert rel_err(out, ref.astype(np.float16).astype(np.float32)) < TOL


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("pos", [0, 1, 4000])
def test_qk_norm_rope_append(mdx, gpu, oracle_lib, style, pos):
    rng = np.random.default_rng(pos * 2 + style)
    nq, nkv, hd = 16, 8, 128
    qkv = rng.standard_normal(nq * hd + 2 * nkv * hd).astype(np.float32) * 2
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    q, k16, v16 = mdx.qk_rope(nq, nkv, hd, pos, style, 1e6, 1e-6, qn, kn, qkv)
    c, s = oracle_lib.rope_tables(pos + 1, hd, 1e6)
    qd = nq * hd
    qref = np.concatenate([oracle_lib.rms_norm(qkv[h * hd:(h + 1) * hd], qn, 1e-6) for h in range(nq)])
    kref = np.concatenate([oracle_lib.rms_norm(qkv[qd + h * hd:qd + (h + 1) * hd], kn, 1e-6)
                           for h in range(nkv)])
    qref = oracle_lib.apply_rope(qref, c[pos], s[pos], nq, hd, style)
    kref = oracle_lib.apply_rope(kref, c[pos], s[pos], nkv, hd, style)
    assert rel_err(q, qref) < 1e-5
    k = k16.view(np.float16).astype(np.float32)
    assert rel_err(k, kref.astype(np.float16).astype(np.float32)) < 1e-3
    assert np.array_equal(v16, qkv[qd + nkv * hd:].astype(np.float16).view(np.uint16))


# ---- lm_head + argmax ------------------------------------------------------------------

@pytest.mark.parametrize("V", [151936, 5000])
def test_lm_head_int8_argmax(mdx, gpu, oracle_lib, V):
    rng = np.random.default_rng(V)
    K = 1024
    lm = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    q, s = oracle_lib.quantize_lm_head(oracle_lib.f32_to_f16(lm), V, K)
    h = rng.standard_normal(K).astype(np.float32)
    nw = np.ones(K, np.float32)
    tok, lg = mdx.lmhead(1, K, V, q, s, h, nw, 1e-6)
    x16 = oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(oracle_lib.rms_norm(h, nw, 1e-6)))
    ref = (q.astype(np.float64) @ x16.astype(np.float64)) * s
    assert rel_err(lg, ref) < TOL * 0.1 and cosine(lg, ref) > 0.9999
    assert tok == int(np.argmax(lg))
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 1e-4 * np.abs(ref).max():
        assert tok == int(np.argmax(ref))


@pytest.mark.parametrize("K,V,ties", [(64, 4096, [10, 700, 3000]),
                                      # the streaming K=1024 kernel: ties within one
                                      # block's rows and across blocks
                                      (1024, 16384, [4100, 4101, 9000, 16383])])
def test_lm_head_argmax_ties_pick_lowest_index(mdx, gpu, K, V, ties):
    q = np.zeros((V, K), np.int8)
    q[ties, 0] = 5                                  # equal maxima
    s = np.ones(V, np.float32)
    h = np.zeros(K, np.float32)
    h[0] = 1.0
    tok, lg = mdx.lmhead(1, K, V, q, s, h, np.ones(K, np.float32), 1e-6)
    assert tok == ties[0] and all(lg[i] == lg[ties[0]] for i in ties)


@pytest.mark.parametrize("K,V", [(64, 4096), (1024, 16384)])
def test_lm_head_argmax_signed_zero_and_nan(mdx, gpu, oracle_lib, K, V):
    """The fused argmax follows argmax_f32 (src/cpu_ops.c:575-586) where a
    sort key could differ: -0 and +0 tie (first index wins), a NaN at index 0
    wins, a NaN elsewhere never does.  Logits are scale * dot with exact
    integer dots, so the signs of the zeros are the scales' signs."""
    h = np.zeros(K, np.float32)
    h[0] = 1.0                                         # x16[0] = fp16(sqrt(K)), the rest 0
    q = np.zeros((V, K), np.int8)
    q[:, 0] = 1
    far = V - 5                                        # another block of the streaming kernel
    zero_rows = [0, 1, 2, far]
    q[zero_rows, 0] = 0

    def run(s):
        tok, lg = mdx.lmhead(1, K, V, q, s, h, np.ones(K, np.float32), 1e-6)
        return tok, lg

    # every other row is negative; rows 0, 1 are -0.0, rows 2 and far +0.0
    s = -np.ones(V, np.float32)
    s[[2, far]] = 1.0
    tok, lg = run(s)
    assert np.signbit(lg[0]) and not np.signbit(lg[2]) and lg[2] == 0.0
    assert tok == oracle_lib.argmax(lg) == 0
    # a +0 first, then -0 rows: still the first
    s = -np.ones(V, np.float32)
    s[1] = 1.0
    tok, lg = run(s)
    assert tok == oracle_lib.argmax(lg) == 0
    # NaN at index 0 wins over a larger value later
    s = -np.ones(V, np.float32)
    s[0] = np.nan
    s[far - 10] = 2.0
    tok, lg = run(s)
    assert np.isnan(lg[0]) and tok == oracle_lib.argmax(lg) == 0
    # NaN elsewhere is skipped
    s = -np.ones(V, np.float32)
    s[[5, far - 10]] = np.nan
    s[700] = 3.0
    tok, lg = run(s)
    assert tok == oracle_lib.argmax(lg) == 700


@pytest.mark.parametrize("K", [2080, 3072, 4096])
@pytest.mark.parametrize("kind", [1, 3, 4])
def test_lm_head_wide_rows_norm_staging(mdx, gpu, oracle_lib, kind, K):
    """Hidden sizes above one staging batch of the GEMV (2048 values for 256
    threads): the RMSNorm's sum of squares and the staged activations span
    two batches, the second one partial at K = 2080.  INT8 rows multiply the
    fp16-rounded normed activations, fp32 and fp16 rows the fp32 ones."""
    rng = np.random.default_rng(K + 17 * kind)
    V = 640
    h = rng.standard_normal(K).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    x = oracle_lib.rms_norm(h, nw, 1e-6)
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    if kind == 1:
        q, s = oracle_lib.quantize_lm_head(oracle_lib.f32_to_f16(w), V, K)
        tok, lg = mdx.lmhead(1, K, V, q, s, h, nw, 1e-6)
        x16 = oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(x))
        ref = (q.astype(np.float64) @ x16.astype(np.float64)) * s
        assert rel_err(lg, ref) < TOL * 0.1 and cosine(lg, ref) > 0.9999
    elif kind == 3:
        tok, lg = mdx.lmhead(3, K, V, w, None, h, nw, 1e-6)
        assert rel_err(lg, oracle_lib.gemv_rows_f32(x, w, V, K)) < 1e-5
    else:
        w16 = _f16_bits(w)
        tok, lg = mdx.lmhead(4, K, V, w16, None, h, nw, 1e-6)
        assert rel_err(lg, oracle_lib.gemv_rows_f16(x, w16, V, K)) < 1e-5
    assert tok == int(np.argmax(lg))


def test_lm_head_fp32_and_fp16_rows(mdx, gpu, oracle_lib):
    rng = np.random.default_rng(11)
    K, V = 1024, 2048
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    h = rng.standard_normal(K).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    x = oracle_lib.rms_norm(h, nw, 1e-6)
    tok, lg = mdx.lmhead(3, K, V, w, None, h, nw, 1e-6)
    assert rel_err(lg, oracle_lib.gemv_rows_f32(x, w, V, K)) < 1e-5 and tok == int(np.argmax(lg))
    w16 = _f16_bits(w)
    tok, lg = mdx.lmhead(4, K, V, w16, None, h, nw, 1e-6)
    assert rel_err(lg, oracle_lib.gemv_rows_f16(x, w16, V, K)) < 1e-5 and tok == int(np.argmax(lg))
