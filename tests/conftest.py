"""Shared pytest setup.

Markers: `gpu` tests need a visible MI355X and call the HIP path through the
C ABI; everything else runs on the CPU (oracle checks, host logic, ABI
surface).  Libraries are built in-tree: the CPU session builds whatever is
missing (the oracle with make, the decoder with build.py); GPU sessions only
load what was built beforehand.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rknn-matmul-parallel_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP path through the C ABI)")
    config.addinivalue_line("markers", "slow: full-size configuration (minutes)")


def _gpu_session(config) -> bool:
    expr = config.getoption("-m") or ""
    return "gpu" in expr and "not gpu" not in expr


@pytest.fixture(scope="session")
def oracle_lib(request):
    import oracle as orc
    if not os.path.exists(orc.LIB_PATH):
        orc.build()
    return orc


@pytest.fixture(scope="session")
def mdx(request):
    import mdx_lib
    if not os.path.exists(mdx_lib.LIB_PATH):
        if _gpu_session(request.config):
            pytest.fail("libmatmul_decoder.so is not built; build before running GPU tests")
        import build as pkg_build
        pkg_build.build()
    return mdx_lib


@pytest.fixture(scope="session")
def gpu(mdx):
    n = mdx.device_count()
    if n <= 0:
        pytest.fail("no GPU visible to the HIP runtime")
    return n


@pytest.fixture(scope="session")
def workdir():
    base = os.environ.get("MDX_TEST_TMP") or tempfile.gettempdir()
    d = tempfile.mkdtemp(prefix="mdx_tests_", dir=base)
    yield d
    shutil.rmtree(d, ignore_errors=True)


# Tiny decoder shape used by the end-to-end tests: every kernel path at a
# size the oracle finishes in milliseconds.
TINY = dict(hidden_dim=128, num_q_heads=4, num_kv_heads=2, head_dim=64, ffn_dim=256,
            num_layers=2, vocab_size=512, max_seq_len=128, rms_eps=1e-6, rope_theta=1e6,
            tie_word_embeddings=1, has_qk_norm=1, rope_style=1, max_batch_prefill=64)


def tiny_config(mdx_lib, **over):
    cfg = dict(TINY)
    cfg.update(over)
    return mdx_lib.qwen3_0_6b_config(name="tiny", **cfg), cfg


def rel_err(a, b) -> float:
    """max |a-b| / max |b| (the per-projection error measure)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / (den if den > 0 else 1.0))


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
