"""ctypes wrapper of the optimizer restatement in optim.c (part of liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from oracle import lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def sr_hash(x: int) -> int:
    f = lib().or_sr_hash
    f.restype = C.c_uint32
    f.argtypes = [C.c_uint32]
    return int(f(x))


def bf16_sr(values: np.ndarray, rnd: np.ndarray) -> np.ndarray:
    f = lib().or_bf16_sr
    f.restype = C.c_uint16
    f.argtypes = [C.c_float, C.c_uint32]
    return np.array([f(float(v), int(r)) for v, r in zip(values.ravel(), rnd.ravel())], np.uint16)


def adam_step(grad, param, exp_avg, exp_avg_sq, step, lr, beta1=0.9, beta2=0.999, eps=1e-15, visibility=None):
    """In place on numpy arrays (float32; moments float32 or uint16 bfloat16 bits). The first
    dimension of param is the primitive count."""
    assert param.dtype == np.float32 and param.flags.c_contiguous and grad.dtype == np.float32
    lowp = exp_avg.dtype == np.uint16
    n = param.size
    n_prim = param.shape[0] if param.ndim else 1
    vis = None if visibility is None else np.ascontiguousarray(visibility, np.int32)
    lib().or_adam_step(_p(np.ascontiguousarray(grad)), _p(param), _p(exp_avg), _p(exp_avg_sq), C.c_int(int(lowp)),
                       C.c_int64(n), C.c_int64(n_prim), _p(vis), C.c_int(step), C.c_double(lr),
                       C.c_double(beta1), C.c_double(beta2), C.c_double(eps))
