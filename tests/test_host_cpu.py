"""Host-side checks of the product library that need no GPU: the exported
C ABI, struct layouts, config.json parsing, the synthetic model writer and
its quantisers, the host KV-cache object, the pybind module surface, and
that creating a decoder without a GPU fails loudly (no CPU fallback)."""
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import PKG, ROOT, tiny_config

INCLUDE = os.path.join(ROOT, "include")
REF_INCLUDE = "/root/reference/include"


def _declared_functions():
    names = set()
    for h in ("matmul_decoder.h", "rknn_matmul_parallel.h", "mdx_ext.h"):
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        inline = set(re.findall(r"static inline [\w\s\*]+?\b(\w+)\s*\(", text))
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\(", text, flags=re.M):
            name = m.group(1)
            if name in inline or m.group(0).lstrip().startswith(("typedef", "static", "return", "if")):
                continue
            names.add(name)
    return names


def test_library_exports_every_declared_symbol(mdx):
    declared = _declared_functions()
    assert "matmul_decoder_step" in declared and "rmp_run" in declared and "mdx_debug_gemv" in declared
    out = subprocess.run(["nm", "-D", "--defined-only", mdx.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = sorted(declared - exported)
    assert not missing, f"declared but not exported: {missing}"


_LAYOUT_C = r"""
#include <stdio.h>
#include <stddef.h>
#include "matmul_decoder.h"
#include "rknn_matmul_parallel.h"
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m));
int main(void) {
  printf("MatmulDecoderConfig %zu\n", sizeof(MatmulDecoderConfig));
  F(MatmulDecoderConfig, name) F(MatmulDecoderConfig, max_seq_len) F(MatmulDecoderConfig, rms_eps)
  F(MatmulDecoderConfig, rope_style) F(MatmulDecoderConfig, has_qk_norm)
  F(MatmulDecoderConfig, num_lm_heads) F(MatmulDecoderConfig, context_pool_mode)
  F(MatmulDecoderConfig, exec_mode) F(MatmulDecoderConfig, disable_npu_lm_head)
  F(MatmulDecoderConfig, max_batch_prefill)
  printf("ProjectionWeight %zu\n", sizeof(ProjectionWeight));
  printf("LayerWeights %zu\n", sizeof(LayerWeights)); F(LayerWeights, k_norm_weight)
  printf("MatmulDecoderStats %zu\n", sizeof(MatmulDecoderStats)); F(MatmulDecoderStats, n_steps)
  printf("SamplingParams %zu\n", sizeof(SamplingParams)); F(SamplingParams, n_repeat_tokens)
  printf("RmpConfig %zu\n", sizeof(RmpConfig)); F(RmpConfig, n_workers)
  MatmulDecoderConfig c = matmul_decoder_config_qwen3_0_6b();
  printf("qwen3 %d %d %d %d %d %g %g %d %d %d %d\n", c.hidden_dim, c.num_q_heads, c.num_kv_heads,
         c.num_layers, c.vocab_size, c.rms_eps, c.rope_theta, c.iommu_domain_id, c.exec_mode,
         c.max_batch_prefill, c.rope_style);
  MatmulDecoderConfig t = matmul_decoder_config_qwen3_tts_cp();
  printf("tts %d %d %d %d %d %d\n", t.num_layers, t.vocab_size, t.max_seq_len, t.num_lm_heads,
         t.lm_head_vocab_size, t.tie_word_embeddings);
  printf("enums %d %d %d %d %d\n", QUANT_INT4_G128, MATMUL_DECODER_ERR_UNSUPPORTED, EXEC_DUAL_CORE,
         RMP_TYPE_FP16_INT8, RMP_LAYOUT_NATIVE);
  return 0;
}
"""


def _layout(include_dir, tmp_path, tag):
    src = tmp_path / f"layout_{tag}.c"
    exe = tmp_path / f"layout_{tag}"
    src.write_text(_LAYOUT_C)
    subprocess.run(["gcc", "-std=gnu11", "-I", include_dir, str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout


def test_struct_layout_and_inline_helpers(tmp_path):
    ours = _layout(INCLUDE, tmp_path, "ours")
    assert "MatmulDecoderConfig 104" in ours and "MatmulDecoderConfig.max_batch_prefill 100" in ours
    assert "qwen3 1024 16 8 28 151936 1e-06 1e+06 1 1 64 0" in ours
    if os.path.isdir(REF_INCLUDE):
        assert ours == _layout(REF_INCLUDE, tmp_path, "ref")


def test_load_config_parses_reference_keys_and_exponents(mdx, tmp_path):
    p = tmp_path / "config.json"
    p.write_text(json.dumps({"model": {"hidden_dim": 64, "num_layers": 3}, "num_q_heads": 4,
                             "num_kv_heads": 2, "head_dim": 16, "ffn_dim": 96, "vocab_size": 300,
                             "rms_eps": 1e-06, "rope_theta": 10000.0, "has_qk_norm": False,
                             "tie_word_embeddings": False, "rope_style": 1, "name": "x",
                             "max_batch_prefill": 16, "hidden": 7}))
    c = mdx.load_config(str(p))
    assert (c.hidden_dim, c.num_layers, c.num_q_heads, c.num_kv_heads, c.head_dim) == (64, 3, 4, 2, 16)
    assert (c.ffn_dim, c.vocab_size, c.has_qk_norm, c.tie_word_embeddings) == (96, 300, 0, 0)
    assert abs(c.rms_eps - 1e-6) < 1e-12 and c.rope_theta == 10000.0
    assert c.rope_style == 1 and c.max_batch_prefill == 16
    assert c.iommu_domain_id == 1 and c.exec_mode == 1       # defaults kept
    with pytest.raises(RuntimeError):
        mdx.load_config(str(tmp_path / "missing.json"))


def test_synth_writer_formats(mdx, oracle_lib, tmp_path):
    cfg, d = tiny_config(mdx)
    for quant in (0, 1, 2):
        path = str(tmp_path / f"m{quant}")
        mdx.write_model(path, cfg, quant, 7)
        L0 = os.path.join(path, "layers", "layer_00")
        K, N = d["hidden_dim"], d["ffn_dim"]
        w32 = oracle_lib.fill_normal(K * N, oracle_lib.seed_for(7, "layer_00/gate_proj"), 0, 0.02)
        w32 = w32.reshape(K, N)
        if quant == 0:
            w = np.fromfile(os.path.join(L0, "gate_proj.bin"), np.uint16).reshape(K, N)
            assert np.array_equal(w, oracle_lib.f32_to_f16(w32).reshape(K, N))
        else:
            s = np.fromfile(os.path.join(L0, "gate_proj_scales.bin"), np.float32)
            raw = np.fromfile(os.path.join(L0, "gate_proj_weight.bin"), np.uint8)
            amax = np.abs(w32).max(0)
            if quant == 1:
                q = raw.view(np.int8).reshape(K, N).astype(np.int64)
                assert np.array_equal(s, (amax / np.float32(127)).astype(np.float32))
                assert np.all(np.abs(q).max(0) == 127)
            else:
                b = raw.reshape(K, N // 2)
                lo, hi = (b & 0xF).astype(np.int64), (b >> 4).astype(np.int64)
                q = np.empty((K, N), np.int64)
                q[:, 0::2], q[:, 1::2] = lo, hi
                q[q >= 8] -= 16
                assert np.array_equal(oracle_lib.f16_to_f32(oracle_lib.f32_to_f16(s)), s)
                assert q.min() >= -8 and q.max() <= 7
            assert np.all(np.abs(q * s - w32) <= s * (0.5 if quant == 1 else 1.0) + 1e-6)
        assert os.path.getsize(os.path.join(path, "embeddings.bin")) == d["vocab_size"] * K * 4
        c = mdx.load_config(os.path.join(path, "config.json"))
        assert c.rope_style == 1 and abs(c.rms_eps - 1e-6) < 1e-12


def test_host_kv_cache_object(mdx):
    L = mdx.lib()
    c = L.matmul_kv_cache_create(2, 2, 64, 16)
    assert c and L.matmul_kv_cache_get_seq_len(c) == 0
    L.matmul_kv_cache_clear(c)
    L.matmul_kv_cache_destroy(c)
    assert not L.matmul_kv_cache_create(0, 2, 64, 16)
    L.matmul_kv_cache_destroy(None)


def test_no_gpu_means_no_decoder(mdx, tmp_path):
    if mdx.device_count() > 0:
        pytest.skip("a GPU is visible")
    cfg, _ = tiny_config(mdx)
    path = str(tmp_path / "m")
    mdx.write_model(path, cfg, 0, 1)
    with pytest.raises(RuntimeError):
        mdx.Decoder(path, cfg, "fp16", 64)
    L = mdx.lib()
    rc = mdx.RmpConfig(M=1, K=64, N=64, type=0, layout=0, n_workers=2)
    w = np.zeros(64 * 64, np.uint16)
    import ctypes
    assert not L.rmp_create(ctypes.byref(rc), w.ctypes.data, None)
    assert mdx.lib().mdx_debug_gemv(0, 64, 64, w.ctypes.data, None,
                                    np.zeros(64, np.float32).ctypes.data_as(mdx._F),
                                    np.zeros(64, np.float32).ctypes.data_as(mdx._F)) < 0


def test_pybind_module_surface(mdx):
    sys.path.insert(0, PKG)
    import matmul_decoder as md
    assert md.__version__ == "1.0.0"
    for name in ("step", "prefill", "prefill_batch", "step_get_token", "clear_kv_cache", "generate",
                 "step_sample"):
        assert hasattr(md.MatmulDecoder, name)
    for prop in ("seq_len", "config", "stats"):
        assert isinstance(getattr(md.MatmulDecoder, prop), property)
    c = md.config_qwen3_0_6b()
    assert c["hidden_dim"] == 1024 and c["exec_mode"] == "dual_core"
    assert md.config_qwen3_0_6b_single_core()["exec_mode"] == "single_core"
    if mdx.device_count() == 0:
        with pytest.raises(RuntimeError):
            md.MatmulDecoder("/nonexistent", max_seq_len=16, quant_type="fp16")


def test_sampler_parameter_checks_run_before_any_device_call(mdx):
    """md_sample_prepare rejects out-of-range SamplingParams with INVALID_ARG
    (-1) before touching a device; valid ones reach the device (UNSUPPORTED,
    -5, where there is none)."""
    import ctypes
    if mdx.device_count() != 0:
        pytest.skip("checks the no-device return code")
    L = mdx.lib()
    x = np.zeros(2048, np.float32)        # top_k is clamped to V first, then limited to 1024
    out = np.zeros(2, np.int32)

    def call(u=0.5, **kw):
        p, toks = mdx.sampling_params(**kw)
        return L.mdx_debug_sample(x.ctypes.data_as(mdx._F), x.size, ctypes.byref(p), u,
                                  out.ctypes.data_as(mdx._I), None, None)

    for kw in (dict(top_k=1025), dict(temperature=0.0), dict(temperature=float("inf")),
               dict(repeat_penalty=-1.0), dict(top_p=float("nan")), dict(repeat_tokens=[2048], repeat_penalty=1.1),
               dict(repeat_tokens=[-1], repeat_penalty=1.1), dict(repeat_tokens=list(range(64)) * 65)):
        assert call(**kw) == -1, kw
    assert call(u=1.01) == -1 and call(u=-0.01) == -1
    assert call(top_k=1000, top_p=0.9, temperature=0.7, repeat_tokens=[1, 1, 2], repeat_penalty=1.3) == -5


def test_gemm_splits_are_never_empty(mdx):
    """The K-split count of a split prefill projection (host arithmetic,
    mdx_debug_gemm_splits) leaves no split empty for any kind and shape the
    config check admits (K, N multiples of 32 up to 16384), the case where
    an empty split once reached the kernels (fp16 K=2592, N=128: 81
    K-blocks, 10 requested splits of 9) included."""
    import ctypes
    L = mdx.lib()
    per = ctypes.c_int(0)
    blocks = {0: 32, 1: 64, 2: 128}
    checked = 0
    for kind, kb in blocks.items():
        for K in list(range(32, 4097, 32)) + [6144, 8192, 12288, 16384]:
            for N in (32, 64, 96, 128, 160, 192, 256, 480, 1024, 2048, 4096, 6144):
                ns = L.mdx_debug_gemm_splits(kind, N, K, ctypes.byref(per))
                nkb = -(-K // kb)
                assert 1 <= ns <= 16, (kind, K, N, ns)
                assert per.value == -(-nkb // ns), (kind, K, N)
                assert (ns - 1) * per.value < nkb, f"empty split: kind {kind} K {K} N {N} ns {ns}"
                assert ns * per.value >= nkb
                checked += 1
    assert L.mdx_debug_gemm_splits(0, 128, 2592, ctypes.byref(per)) == 9 and per.value == 9
    assert L.mdx_debug_gemm_splits(5, 128, 256, None) == -1
    assert checked > 4000


def test_persist_kv_rows_stay_in_the_written_cache(mdx):
    """Every K/V row address the one-launch decode step forms (the kernel's
    own kv_split / kv_row functions, enumerated on the host over every
    position of a 6400-row cache, every split, pass row and requested round,
    for rounds of 4 and of 5 passes) lies in rows [0, pos]."""
    import ctypes
    L = mdx.lib()
    n = ctypes.c_longlong(0)
    for pp in (4, 5):
        assert L.mdx_debug_persist_kv_rows(6400, pp, ctypes.byref(n)) == 0, pp
        assert n.value > 6400 * 32 * 16 * pp
    assert L.mdx_debug_persist_kv_rows(100, 3, None) == -1
