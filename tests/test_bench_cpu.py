"""bench.py's host-side figures, on synthetic inputs (no GPU): the stage
split read from a traced step, the algorithmic bytes of a decode step, and the
committed counter summaries it reports as traffic."""
from __future__ import annotations

import importlib.util
import os

import numpy as np

from conftest import ROOT


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_layer_stage_split_reads_the_event_offsets():
    """A trace whose layer l has event e at 1000 l + off[e] ticks (100 MHz),
    the same for every workgroup, gives each segment as its offset difference
    in microseconds; the previous layer's last event starts the h wait."""
    b = _bench()
    L = 28
    off = np.array([0, 170, 255, 400, 432, 480, 560, 600, 790, 866, 1000 - 60, 1000 - 12,
                    420, 460, 450, 1000 - 70])     # events 0..15 of a layer
    ev = 16 * L + 4
    tr = np.zeros((256, ev), np.uint64)
    for lay in range(L):
        tr[:, 16 * lay:16 * lay + 16] = 1000 * lay + off
    r = b.layer_stage_split([tr, tr, tr], L)
    us = lambda a, c: (c - a) * 0.01
    assert np.isclose(r["qkv"], us(off[1], off[2]))
    assert np.isclose(r["o"], us(off[6], off[7]))
    assert np.isclose(r["gate_up"], us(off[8], off[9]))
    assert np.isclose(r["down"], us(off[10], off[11]))
    assert np.isclose(r["wait_attn_before_o"], us(off[5], off[6]))
    assert np.isclose(r["wait_h_before_gate_up"], us(off[7], off[8]))
    assert np.isclose(r["wait_act_before_down"], us(off[9], off[10]))
    assert np.isclose(r["wait_h_before_qkv"], us(off[11], 1000 + off[1]))
    assert np.isclose(r["layer"], 10.0)
    assert np.isclose(r["projections_sum"], r["qkv"] + r["o"] + r["gate_up"] + r["down"])


def test_layer_stage_split_takes_the_median_workgroup():
    b = _bench()
    L = 8
    tr = np.zeros((256, 16 * L + 4), np.uint64)
    for lay in range(L):
        tr[:, 16 * lay:16 * lay + 16] = 1000 * lay + np.arange(16) * 10
    tr[:3, 16 * 3 + 2] += 500          # three slow workgroups in layer 3's qkv stage
    r = b.layer_stage_split([tr], L)
    assert np.isclose(r["qkv"], 0.1)


def test_step_bytes_closed_form():
    """fp16: 2 bytes per weight; int4: half a byte plus an fp32 scale per output
    row; the INT8 lm_head with its scales; K and V rows of every layer."""
    b = _bench()
    d = dict(hidden_dim=1024, num_q_heads=16, num_kv_heads=8, head_dim=128, ffn_dim=3072,
             num_layers=28, vocab_size=151936)
    elems = 1024 * 4096 + 2048 * 1024 + 2 * 1024 * 3072 + 3072 * 1024
    rows = 4096 + 1024 + 6144 + 1024
    norms = 4.0 * (2 * 1024 + 2 * 128)
    lm = 151936 * 1024 + 151936 * 4.0
    kv = 28 * 513 * 1024 * 2 * 2.0
    assert b.step_bytes(d, [512], 0) == 28 * (2.0 * elems + norms) + lm + kv + 4.0 * 1024
    assert b.step_bytes(d, [512], 2) == 28 * (0.5 * elems + 4.0 * rows + norms) + lm + kv + 4.0 * 1024
    # the mean over positions is the K/V term at the mean position
    assert np.isclose(b.step_bytes(d, [512, 514], 0), b.step_bytes(d, [513], 0))


def test_committed_traffic_summaries_are_consistent():
    """Each profiles/*_traffic.json: scaled FETCH_SIZE plus WRITE_SIZE gives the
    bytes it states, and its ratio to the algorithmic bytes matches."""
    b = _bench()
    for name in ("k_persist_step_fp16_decode_kv512", "k_persist_step_int4_decode_kv4096"):
        t = b.profile_traffic(name)
        assert t is not None, name
        total = (t["fetch_kib_per_dispatch"] * t["fetch_scale"]
                 + t["write_kib_per_dispatch"] * t["write_scale"]) * 1024
        assert abs(total - t["hbm_bytes_per_launch"]) < 2048, name
        assert np.isclose(t["hbm_bytes_per_launch"] / t["algorithmic_bytes_per_launch"],
                          t["traffic_over_algorithmic"], rtol=2e-3), name
    t = b.profile_traffic("k_gemm_prefill_m60_int8")
    per_layer = (t["fetch_kib_per_layer_scaled"] + t["write_kib_per_layer"]) * 1024
    assert abs(28 * per_layer - t["hbm_bytes_per_prefill"]) < 2048
    assert np.isclose(t["hbm_bytes_per_prefill"] / t["algorithmic_bytes_per_prefill"],
                      t["traffic_over_algorithmic"], rtol=2e-3)
    assert b.profile_traffic("no_such_kernel") is None
