"""Shared test setup: import paths, the `gpu` marker, model fixtures."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("ane-training_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: minutes of CPU work")


# Tiny model shapes used across tests: every kernel family at a small size.
TINY = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=512, seq_len=128)
TINY_GQA = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=500, seq_len=128)
TINY_HD128 = dict(dim=512, hidden_dim=1024, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=1000, seq_len=160)


def cfg7(d):
    return (d["dim"], d["hidden_dim"], d["n_layers"], d["n_heads"], d["n_kv_heads"], d["vocab_size"], d["seq_len"])


@pytest.fixture(scope="session")
def lm():
    import stories_lm
    stories_lm.lib()
    return stories_lm


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle
