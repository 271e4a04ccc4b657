import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import __graft_entry__ as graft  # noqa: E402

graft.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def pkg():
    import parakeet_amd
    return parakeet_amd


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    oracle.lib()
    return oracle


def small_tdt(path, **kw):
    """A small TDT decoder (shapes scaled down from TDT-0.6b-v3)."""
    from parakeet_amd import synth
    cfg = dict(kind="tdt", H=64, L=2, J=96, D=128, vocab=61, durations=[0, 1, 2, 3, 4], quant="q8_0")
    cfg.update(kw)
    return synth.make_decoder_gguf(path, **cfg)


def small_eou(path, **kw):
    from parakeet_amd import synth
    cfg = dict(kind="eou", H=64, L=1, J=96, D=64, vocab=35, eou_id=33, eob_id=34, max_symbols=5,
               quant="q8_0")
    cfg.update(kw)
    return synth.make_decoder_gguf(path, **cfg)


@pytest.fixture(scope="session")
def tmpdir_session(tmp_path_factory):
    return tmp_path_factory.mktemp("pk")


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
