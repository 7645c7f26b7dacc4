"""Shared test configuration.

Markers: ``gpu`` tests need a gfx950 GPU and the built libavey_hip.so; they are
the parity tests proper. Everything else runs on a CPU-only host.
"""

import ctypes
import json
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

GOLDEN = os.path.join(REPO, 'tests', 'golden')


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a gfx950 GPU and the built HIP library')


def load_kats():
    with open(os.path.join(GOLDEN, 'kats.json')) as fh:
        return json.load(fh)


_c_oracle = None


def c_oracle():
    """ctypes handle to oracle/build/libavey_oracle.so (built on demand)."""
    global _c_oracle
    if _c_oracle is None:
        from oracle import build as oracle_build
        if not os.path.exists(oracle_build.LIB_PATH):
            oracle_build.build(verbose=False)
        lib = ctypes.CDLL(oracle_build.LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.avey_oracle_f64.restype = ctypes.c_int
        lib.avey_oracle_f64.argtypes = [dp, dp, dp, dp, ctypes.POINTER(ctypes.c_uint8), dp,
                                        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double]
        _c_oracle = lib
    return _c_oracle


ACT_IDS = {'identity': 0, 'relu': 1, 'relu2': 2, 'silu': 3, 'gelu': 4}


def c_contextualize(z_tr, v=None, z_tl=None, bias=None, valid=None, *, eps, norm_eps, causal,
                    normalize, activation):
    """Run the C restatement on float64 numpy inputs."""
    lib = c_oracle()
    dp = ctypes.POINTER(ctypes.c_double)
    z = np.ascontiguousarray(z_tr, dtype=np.float64)
    out = np.empty_like(z)
    # Keep the converted arrays alive until the call returns.
    keep = [None if a is None else np.ascontiguousarray(a, dtype=np.float64) for a in (v, z_tl, bias)]
    vp, gp, bp = [None if a is None else a.ctypes.data_as(dp) for a in keep]
    valid_u8 = None if valid is None else np.ascontiguousarray(valid, dtype=np.uint8)
    valp = None if valid_u8 is None else valid_u8.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
    st = lib.avey_oracle_f64(z.ctypes.data_as(dp), vp, gp, bp, valp, out.ctypes.data_as(dp),
                             z.shape[0], z.shape[1], z.shape[2], int(causal), int(normalize),
                             ACT_IDS[activation], float(eps), float(norm_eps))
    assert st == 0
    return out


def gpu_available():
    try:
        import torch
    except ImportError:
        return False
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    props = torch.cuda.get_device_properties(0)
    return getattr(props, 'gcnArchName', '').startswith('gfx950')
