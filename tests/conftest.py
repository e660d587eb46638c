import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def native_lib():
    """The built C-ABI library (built here if it is missing)."""
    from jangq_amd import _lib, build

    if not _lib.LIB_PATH.exists():
        build.build()
    return _lib.lib()


@pytest.fixture(scope="session")
def c_oracle():
    """ctypes handle of the C oracle (oracle/jq_oracle.c)."""
    import ctypes

    from oracle import build_oracle

    h = ctypes.CDLL(str(build_oracle.build()))
    P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    h.jqo_unpack.argtypes = [P, I, L, L, P]
    h.jqo_pack.argtypes = [P, I, L, L, P]
    h.jqo_dequant.argtypes = [P, P, P, I, I, L, L, P]
    h.jqo_gemm_f64.argtypes = [P, P, L, L, L, P]
    return h
