"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle
(oracle/liboracle_eigen.so, a restatement of KataGo's Eigen backend).

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_LIB = None
_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liboracle_eigen.so")


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(_PATH):
            raise RuntimeError(f"{_PATH} is not built; run python -m katago_amd.build")
        l = ctypes.CDLL(_PATH)
        c = ctypes
        l.oracle_load_model.restype = c.c_void_p
        l.oracle_load_model.argtypes = [c.c_char_p, c.c_int, c.c_int, c.c_char_p, c.c_int]
        l.oracle_load_model_ex.restype = c.c_void_p
        l.oracle_load_model_ex.argtypes = [c.c_char_p, c.c_int, c.c_int, c.c_int, c.c_char_p, c.c_int]
        l.oracle_free_model.argtypes = [c.c_void_p]
        l.oracle_forward.argtypes = [c.c_void_p, c.c_int] + [c.c_void_p] * 8 + [c.c_char_p, c.c_int]
        l.oracle_test_evaluate.argtypes = [c.c_int, c.c_char_p, c.c_int, c.c_int, c.c_int, c.c_void_p, c.c_void_p,
                                           c.c_void_p, c.c_char_p, c.c_int]
        l.oracle_direct_conv_f64.argtypes = [c.c_int] * 4 + [c.c_void_p, c.c_int, c.c_int, c.c_int, c.c_void_p,
                                                              c.c_void_p]
        l.oracle_copy_with_symmetry.argtypes = [c.c_void_p, c.c_void_p] + [c.c_int] * 7
        l.oracle_set_layer_dump.argtypes = [c.c_void_p, c.c_int]
        l.oracle_layer_dump.argtypes = [c.c_void_p, c.c_char_p, c.c_int]
        _LIB = l
    return _LIB


class OracleModel:
    def __init__(self, path: str, nn_x: int = 19, nn_y: int = 19, load_time_transforms: bool = True):
        """load_time_transforms=False skips transformToReduceActivations."""
        err = ctypes.create_string_buffer(4096)
        self.nn_x, self.nn_y = nn_x, nn_y
        self._ptr = lib().oracle_load_model_ex(path.encode(), nn_x, nn_y, int(load_time_transforms), err, len(err))
        if not self._ptr:
            raise RuntimeError(err.value.decode())

    def forward(self, spatial, global_in, symmetry=None, policy_optimism=None):
        n = int(np.asarray(global_in).shape[0])
        hw = self.nn_x * self.nn_y
        spatial = np.ascontiguousarray(spatial, dtype=np.float32).reshape(n, -1)
        global_in = np.ascontiguousarray(global_in, dtype=np.float32).reshape(n, -1)
        sym = np.ascontiguousarray(np.zeros(n) if symmetry is None else symmetry, dtype=np.int32)
        opt = np.ascontiguousarray(np.zeros(n) if policy_optimism is None else policy_optimism, dtype=np.float32)
        out = {"policy": np.zeros((n, hw + 1), np.float32), "value": np.zeros((n, 3), np.float32),
               "score": np.zeros((n, 6), np.float32), "ownership": np.zeros((n, hw), np.float32)}
        err = ctypes.create_string_buffer(4096)
        rc = lib().oracle_forward(self._ptr, n, spatial.ctypes.data, global_in.ctypes.data, sym.ctypes.data,
                                  opt.ctypes.data, out["policy"].ctypes.data, out["value"].ctypes.data,
                                  out["score"].ctypes.data, out["ownership"].ctypes.data, err, len(err))
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return out

    def set_layer_dump(self, enabled: bool):
        """Per-block trunk summary lines of the following forwards."""
        lib().oracle_set_layer_dump(self._ptr, int(enabled))

    def layer_dump(self) -> str:
        buf = ctypes.create_string_buffer(1 << 20)
        if lib().oracle_layer_dump(self._ptr, buf, len(buf)) != 0:
            raise RuntimeError("oracle layer dump does not fit the buffer")
        return buf.value.decode()

    def close(self):
        if getattr(self, "_ptr", None):
            lib().oracle_free_model(self._ptr)
            self._ptr = None

    def __del__(self):
        self.close()


def test_evaluate(kind: int, desc_text: str, batch: int, nn_x: int, nn_y: int, inputs, mask=None, out_channels=0):
    """NHWC fp32 layer evaluation (kind 0 conv, 1 BN, 2 residual, 3 gpool residual)."""
    inp = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32).reshape(-1)
    out = np.zeros(batch * nn_x * nn_y * out_channels, np.float32)
    err = ctypes.create_string_buffer(4096)
    rc = lib().oracle_test_evaluate(kind, desc_text.encode(), batch, nn_x, nn_y, inp.ctypes.data,
                                    None if m is None else m.ctypes.data, out.ctypes.data, err, len(err))
    if rc < 0:
        raise RuntimeError(err.value.decode())
    return out


def direct_conv_f64(w_oiyx, inputs_nhwc, ky, kx, cin, cout, batch, nn_x, nn_y):
    w = np.ascontiguousarray(w_oiyx, dtype=np.float32)
    x = np.ascontiguousarray(inputs_nhwc, dtype=np.float32)
    out = np.zeros(batch * nn_y * nn_x * cout, np.float64)
    lib().oracle_direct_conv_f64(ky, kx, cin, cout, w.ctypes.data, batch, nn_x, nn_y, x.ctypes.data, out.ctypes.data)
    return out


def copy_with_symmetry(src, n, h, w, c, nhwc, symmetry, outputs):
    s = np.ascontiguousarray(src, dtype=np.float32)
    d = np.zeros_like(s)
    lib().oracle_copy_with_symmetry(s.ctypes.data, d.ctypes.data, n, h, w, c, int(nhwc), symmetry, int(outputs))
    return d
