"""Shared fixtures: import paths, the `gpu` marker and cached seeded archives.

Archives are written by libchpe_pack.so into $CHPE_ARCHIVE_DIR (default /tmp/chpe_archives)
and reused while the generator sources are unchanged (the file name carries a hash of them).
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "chpe-qwen-engine_amd"
for p in (PKG, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import chpe_amd  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP engine)")


def archive_path(kind, seed=0):
    return chpe_amd.ensure_archive(kind, seed, threads=int(os.environ.get("CHPE_PACK_THREADS", "0")))


@pytest.fixture(scope="session")
def w4_archive():
    return archive_path(chpe_amd.PACK_3B_W4)


@pytest.fixture(scope="session")
def fp16_archive():
    return archive_path(chpe_amd.PACK_3B_FP16_RAW)


@pytest.fixture(scope="session")
def bf16_archive():
    return archive_path(chpe_amd.PACK_3B_BF16_RAW)
