"""matmul_decoder_export_hf_model (a local HuggingFace safetensors checkpoint to
the reference on-disk format) on the CPU: a tiny Qwen3-shaped checkpoint in
BF16, written with safetensors and sharded over two files, is exported as
fp16, int8 and int4 and every file is checked against numpy:
- config.json carries the dimensions, eps, theta, QK norm and tying;
- embeddings, norms and an untied lm_head are the exact fp32 values of the
  BF16 tensors;
- fp16 projections are fp16(W^T) bit for bit, W being HF's [N, K];
- int8/int4 files follow the documented quantiser (per-column max|w| / 127 or
  fp16(max|w| / 7), C roundf, clamp, two nibbles per byte low-first),
  restated here in numpy;
- a multimodal layout (text model under "thinker.model.", an audio tower with
  layers of its own) exports the text model's tensors.
The loader side (the GPU decoder reading these files) is checked in
tests/test_gpu_decoder.py."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import PKG

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")

HF = dict(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
          intermediate_size=96, num_hidden_layers=2, vocab_size=160, rms_norm_eps=1e-6,
          rope_theta=1000000.0, max_position_embeddings=4096)


def _tensors(hf, prefix="model.", tied=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    d, hd = hf["hidden_size"], hf["head_dim"]
    qd, kvd = hf["num_attention_heads"] * hd, hf["num_key_value_heads"] * hd
    F, V = hf["intermediate_size"], hf["vocab_size"]

    def rnd(*shape, scale=0.05):
        return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)

    t = {f"{prefix}embed_tokens.weight": rnd(V, d, scale=0.5), f"{prefix}norm.weight": rnd(d, scale=1.0)}
    for l in range(hf["num_hidden_layers"]):
        p = f"{prefix}layers.{l}."
        t[p + "input_layernorm.weight"] = rnd(d, scale=1.0)
        t[p + "post_attention_layernorm.weight"] = rnd(d, scale=1.0)
        t[p + "self_attn.q_norm.weight"] = rnd(hd, scale=1.0)
        t[p + "self_attn.k_norm.weight"] = rnd(hd, scale=1.0)
        for name, (n, k) in dict(q_proj=(qd, d), k_proj=(kvd, d), v_proj=(kvd, d), o_proj=(d, qd)).items():
            t[p + f"self_attn.{name}.weight"] = rnd(n, k)
        for name, (n, k) in dict(gate_proj=(F, d), up_proj=(F, d), down_proj=(d, F)).items():
            t[p + f"mlp.{name}.weight"] = rnd(n, k)
    if not tied:
        outer = prefix[:-len("model.")] if prefix.endswith("model.") else prefix
        t[f"{outer}lm_head.weight"] = rnd(V, d)
    return t


def _write_checkpoint(path, tensors, hf, tied=True, shards=2, nest=False):
    os.makedirs(path, exist_ok=True)
    cfg = dict(hf, tie_word_embeddings=tied)
    if nest:
        cfg = {"model_type": "qwen3_asr", "audio_config": {"hidden_size": 17, "num_hidden_layers": 9},
               "text_config": cfg}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    names = sorted(tensors)
    for i in range(shards):
        part = {n: tensors[n].contiguous() for n in names[i::shards]}
        st_torch.save_file(part, os.path.join(path, f"model-{i + 1:05d}-of-{shards:05d}.safetensors"))


def _f32(t):
    return t.to(torch.float32).numpy()


def _roundf(x):
    return np.sign(x) * np.floor(np.abs(x) + np.float32(0.5))


def _quant_int8(wt):
    amax = np.max(np.abs(wt), axis=0)
    scale = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    q = np.clip(_roundf((wt * inv).astype(np.float32)), -128, 127).astype(np.int8)
    return q, scale


def _quant_int4(wt):
    amax = np.max(np.abs(wt), axis=0)
    scale = (amax / np.float32(7)).astype(np.float16).astype(np.float32)
    safe = np.where(scale > 0, scale, 1).astype(np.float32)
    q = np.where(scale > 0, np.clip(_roundf((wt / safe).astype(np.float32)), -8, 7), 0).astype(np.int8)
    u = (q & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8), scale


def _check_export(out, tensors, hf, quant, prefix="model.", tied=True):
    d, hd = hf["hidden_size"], hf["head_dim"]
    cfg = json.load(open(os.path.join(out, "config.json")))
    assert cfg["hidden_dim"] == d and cfg["num_q_heads"] == hf["num_attention_heads"]
    assert cfg["num_kv_heads"] == hf["num_key_value_heads"] and cfg["head_dim"] == hd
    assert cfg["ffn_dim"] == hf["intermediate_size"] and cfg["num_layers"] == hf["num_hidden_layers"]
    assert cfg["vocab_size"] == hf["vocab_size"] and abs(cfg["rms_eps"] - 1e-6) < 1e-12
    assert cfg["rope_theta"] == 1e6 and cfg["has_qk_norm"] is True and cfg["rope_style"] == 1
    assert cfg["tie_word_embeddings"] is tied and cfg["quant_type"] == quant

    def f32file(*p):
        return np.fromfile(os.path.join(out, *p), np.float32)

    assert np.array_equal(f32file("embeddings.bin"), _f32(tensors[f"{prefix}embed_tokens.weight"]).ravel())
    assert np.array_equal(f32file("final_norm.bin"), _f32(tensors[f"{prefix}norm.weight"]))
    if tied:
        assert not os.path.exists(os.path.join(out, "lm_head.bin"))
    else:
        outer = prefix[:-len("model.")] if prefix.endswith("model.") else prefix
        assert np.array_equal(f32file("lm_head.bin"), _f32(tensors[f"{outer}lm_head.weight"]).ravel())
    for l in range(hf["num_hidden_layers"]):
        p, ld = f"{prefix}layers.{l}.", f"layer_{l:02d}"
        for src, dst in [("input_layernorm", "input_norm"), ("post_attention_layernorm", "post_attn_norm"),
                         ("self_attn.q_norm", "q_norm"), ("self_attn.k_norm", "k_norm")]:
            assert np.array_equal(f32file(ld, dst + ".bin"), _f32(tensors[p + src + ".weight"])), (l, dst)
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            w = _f32(tensors[p + ("self_attn." if name[0] in "qkvo" else "mlp.") + name + ".weight"])
            wt = np.ascontiguousarray(w.T)                       # [K, N]
            if quant == "fp16":
                got = np.fromfile(os.path.join(out, ld, name + ".bin"), np.float16)
                assert np.array_equal(got.view(np.uint16), wt.astype(np.float16).ravel().view(np.uint16)), name
                continue
            qref, sref = _quant_int8(wt) if quant == "int8" else _quant_int4(wt)
            got_q = np.fromfile(os.path.join(out, ld, name + "_weight.bin"), np.uint8)
            got_s = np.fromfile(os.path.join(out, ld, name + "_scales.bin"), np.float32)
            assert np.array_equal(got_s, sref), (l, name)
            assert np.array_equal(got_q, qref.ravel().view(np.uint8)), (l, name)


@pytest.mark.parametrize("quant", ["fp16", "int8", "int4"])
def test_export_qwen3_checkpoint(mdx, workdir, quant):
    hf_dir = os.path.join(workdir, "hf_qwen3")
    tensors = _tensors(HF, seed=1)
    if not os.path.exists(os.path.join(hf_dir, "config.json")):
        _write_checkpoint(hf_dir, tensors, HF)
    out = os.path.join(workdir, f"export_{quant}")
    mdx.export_hf_model(hf_dir, out, quant)
    _check_export(out, tensors, HF, quant)


def test_export_untied_multimodal_layout(mdx, workdir):
    hf_dir = os.path.join(workdir, "hf_asr_like")
    tensors = _tensors(HF, prefix="thinker.model.", tied=False, seed=2)
    # an audio tower with layers of its own, which the exporter must not pick
    g = torch.Generator().manual_seed(3)
    tensors["thinker.audio_tower.layers.0.self_attn.q_proj.weight"] = torch.randn(17, 17, generator=g).to(torch.bfloat16)
    tensors["thinker.audio_tower.layers.0.input_layernorm.weight"] = torch.randn(17, generator=g).to(torch.bfloat16)
    _write_checkpoint(hf_dir, tensors, HF, tied=False, shards=3, nest=True)
    out = os.path.join(workdir, "export_asr_like")
    mdx.export_hf_model(hf_dir, out, "int8")
    _check_export(out, tensors, HF, "int8", prefix="thinker.model.", tied=False)


def test_export_errors_and_cli(mdx, workdir):
    empty = os.path.join(workdir, "hf_empty")
    os.makedirs(empty, exist_ok=True)
    with open(os.path.join(empty, "config.json"), "w") as f:
        json.dump(HF, f)
    with pytest.raises(RuntimeError):
        mdx.export_hf_model(empty, os.path.join(workdir, "export_empty"), "fp16")
    # a checkpoint that lacks one projection
    broken = os.path.join(workdir, "hf_broken")
    tensors = _tensors(HF, seed=4)
    del tensors["model.layers.1.mlp.down_proj.weight"]
    _write_checkpoint(broken, tensors, HF, shards=1)
    with pytest.raises(RuntimeError):
        mdx.export_hf_model(broken, os.path.join(workdir, "export_broken"), "fp16")
    # a dimension out of range, and a header with a negative data offset
    huge = os.path.join(workdir, "hf_huge")
    _write_checkpoint(huge, _tensors(HF, seed=6), dict(HF, hidden_size=1 << 40), shards=1)
    with pytest.raises(RuntimeError):
        mdx.export_hf_model(huge, os.path.join(workdir, "export_huge"), "fp16")
    bad = os.path.join(workdir, "hf_bad_header")
    os.makedirs(bad, exist_ok=True)
    with open(os.path.join(bad, "config.json"), "w") as f:
        json.dump(HF, f)
    hdr = json.dumps({"model.embed_tokens.weight": {"dtype": "F32", "shape": [1, 1],
                                                    "data_offsets": [-8, 4]}}).encode()
    with open(os.path.join(bad, "model.safetensors"), "wb") as f:
        f.write(len(hdr).to_bytes(8, "little") + hdr + bytes(4))
    with pytest.raises(RuntimeError):
        mdx.export_hf_model(bad, os.path.join(workdir, "export_bad_header"), "fp16")
    # the command line
    hf_dir = os.path.join(workdir, "hf_cli")
    tensors = _tensors(HF, seed=5)
    _write_checkpoint(hf_dir, tensors, HF, shards=1)
    out = os.path.join(workdir, "export_cli")
    r = subprocess.run([sys.executable, os.path.join(PKG, "export_weights.py"), "--model", hf_dir,
                        "--output-dir", out, "--quant", "int4"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    _check_export(out, tensors, HF, "int4")
