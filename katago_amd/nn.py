"""Python binding of the HIP backend's NeuralNet interface (include/katago_nn.h).

Mirrors KataGo's backend API (/root/reference/cpp/neuralnet/nninterface.h):
``LoadedModel`` (loadModelFile / getModelDesc), ``ComputeContext``
(createComputeContext) and ``ComputeHandle`` (createComputeHandle,
getOutput, isUsingFP16), plus the layer-level ``test_evaluate`` hooks.
Errors raise ``StringError``, the reference's error type.

The native libraries must have been built (``python -m katago_amd.build``);
there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from dataclasses import dataclass

import numpy as np

_LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
_host = None
_hip = None


class StringError(RuntimeError):
    """Error raised by the backend (KataGo's StringError); code is the C
    library's status (KGH_ERR_*), 0 where there is none."""

    def __init__(self, message: str, code: int = 0):
        super().__init__(message)
        self.code = code


def _f32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _i32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def hip_library() -> ctypes.CDLL:
    """libkatago_hip.so (the C ABI of include/katago_hip.h)."""
    global _hip
    if _hip is None:
        path = os.path.join(_LIB_DIR, "libkatago_hip.so")
        if not os.path.exists(path):
            raise StringError(f"{path} is not built; run python -m katago_amd.build")
        lib = ctypes.CDLL(path)
        lib.kgh_last_error.restype = ctypes.c_char_p
        lib.kgh_output_row_floats.restype = ctypes.c_int32
        lib.kgh_output_row_floats.argtypes = [ctypes.c_int32] * 3
        lib.kgh_device_alloc.argtypes = [ctypes.c_int32, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]
        lib.kgh_device_free.argtypes = [ctypes.c_void_p]
        lib.kgh_memcpy_htod.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        lib.kgh_memcpy_dtoh.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        lib.kgh_device_info.argtypes = [ctypes.c_int32, ctypes.c_char_p, ctypes.c_int32]
        lib.kgh_selftest_mfma.argtypes = [ctypes.c_int32]
        _hip = lib
    return _hip


def host_library() -> ctypes.CDLL:
    """libkatago_host.so (the C ABI of include/katago_nn.h)."""
    global _host
    if _host is None:
        hip_library()
        path = os.path.join(_LIB_DIR, "libkatago_host.so")
        if not os.path.exists(path):
            raise StringError(f"{path} is not built; run python -m katago_amd.build")
        lib = ctypes.CDLL(path)
        c = ctypes
        lib.kgn_load_model.restype = c.c_void_p
        lib.kgn_load_model.argtypes = [c.c_char_p, c.c_char_p, c.c_char_p, c.c_int32]
        lib.kgn_free_model.argtypes = [c.c_void_p]
        lib.kgn_model_info.argtypes = [c.c_void_p, c.POINTER(c.c_int32), c.POINTER(c.c_float), c.c_char_p, c.c_int32]
        lib.kgn_create_context.restype = c.c_void_p
        lib.kgn_create_context.argtypes = [c.c_void_p, c.c_int32, c.c_int32, c.c_int32, c.c_char_p, c.c_int32]
        lib.kgn_free_context.argtypes = [c.c_void_p]
        lib.kgn_create_context_cfg.restype = c.c_void_p
        lib.kgn_create_context_cfg.argtypes = [c.c_void_p, c.c_int32, c.c_int32, c.c_int32, c.c_char_p, c.c_char_p, c.c_char_p,
                                               c.c_int32]
        lib.kgn_create_context_ex.restype = c.c_void_p
        lib.kgn_create_context_ex.argtypes = [c.c_void_p, c.c_int32, c.c_int32, c.c_int32, c.c_char_p, c.c_int32, c.c_char_p,
                                              c.c_char_p, c.c_int32]
        lib.kgn_handle_tuning.argtypes = [c.c_void_p, c.c_char_p, c.c_int32]
        lib.kgn_handle_set_tuning.argtypes = [c.c_void_p, c.c_char_p, c.c_char_p, c.c_int32]
        lib.kgn_create_handle.restype = c.c_void_p
        lib.kgn_create_handle.argtypes = [c.c_void_p, c.c_void_p, c.c_int32, c.c_int32, c.c_int32, c.c_int32, c.c_char_p,
                                          c.c_int32]
        lib.kgn_free_handle.argtypes = [c.c_void_p]
        lib.kgn_is_using_fp16.argtypes = [c.c_void_p]
        lib.kgn_get_output.argtypes = [c.c_void_p, c.c_void_p, c.c_int32, c.c_int32, c.c_int32] + [c.c_void_p] * 8 + [
            c.c_char_p, c.c_int32]
        lib.kgn_test_evaluate.argtypes = [c.c_int32, c.c_char_p, c.c_int32, c.c_int32, c.c_int32, c.c_int32, c.c_int32,
                                          c.c_void_p, c.c_void_p, c.c_void_p, c.c_int64, c.c_char_p, c.c_int32]
        lib.kgn_get_output_post.argtypes = [c.c_void_p, c.c_void_p, c.c_int32, c.c_int32, c.c_int32] + [c.c_void_p] * 10 + [
            c.c_char_p, c.c_int32]
        lib.kgn_evaluator_create.restype = c.c_void_p
        lib.kgn_evaluator_create.argtypes = [c.c_void_p] + [c.c_int32] * 7 + [c.c_char_p, c.c_int32]
        lib.kgn_evaluator_free.argtypes = [c.c_void_p]
        lib.kgn_evaluator_evaluate.argtypes = [c.c_void_p, c.c_void_p, c.c_int32, c.c_void_p, c.c_int32, c.c_int32, c.c_int32,
                                               c.c_int32, c.c_float] + [c.c_void_p] * 4 + [c.c_char_p, c.c_int32]
        lib.kgn_evaluator_stats.argtypes = [c.c_void_p, c.POINTER(c.c_uint64), c.POINTER(c.c_uint64)]
        lib.kgn_evaluator_clear_stats.argtypes = [c.c_void_p]
        lib.kgn_evaluator_run_clients.argtypes = [c.c_void_p, c.c_int32, c.c_int32, c.c_int32, c.c_void_p, c.c_int32,
                                                  c.c_void_p, c.c_int32, c.c_int32, c.c_int32, c.c_void_p,
                                                  c.POINTER(c.c_double), c.c_char_p, c.c_int32]
        _host = lib
    return _host


def _as_rows(a, n: int):
    """a as a contiguous float32 [n, row] array; an empty batch stays empty
    (reshape cannot infer a row length from zero rows)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a.reshape(n, a.size // n if n else 0)


def _errbuf():
    return ctypes.create_string_buffer(4096)


def _raise(err) -> None:
    raise StringError(err.value.decode(errors="replace"))


@dataclass
class ModelInfo:
    name: str
    model_version: int
    num_input_channels: int
    num_input_global_channels: int
    num_policy_channels: int
    num_value_channels: int
    num_score_value_channels: int
    num_ownership_channels: int
    trunk_num_channels: int
    num_input_meta_channels: int
    output_scale_multiplier: float


class LoadedModel:
    """NeuralNet::loadModelFile: parses the file, applies the load-time
    transforms (reduce-activations and scale8)."""

    def __init__(self, path: str, expected_sha256: str = ""):
        lib = host_library()
        err = _errbuf()
        self._ptr = lib.kgn_load_model(path.encode(), expected_sha256.encode(), err, len(err))
        if not self._ptr:
            _raise(err)
        info = (ctypes.c_int32 * 9)()
        osm = ctypes.c_float()
        name = ctypes.create_string_buffer(256)
        lib.kgn_model_info(self._ptr, info, ctypes.byref(osm), name, len(name))
        self.info = ModelInfo(name.value.decode(), *list(info), float(osm.value))

    def close(self):
        if getattr(self, "_ptr", None):
            host_library().kgn_free_model(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # at interpreter exit the library may already be gone
            pass


class ComputeContext:
    """NeuralNet::createComputeContext. use_fp16: True, False or None (auto).
    auto_tune: None keeps the backend default (on), True/False sets
    hipAutoTune; home_data_dir is homeDataDirOverride (tuning tables under
    <dir>/hiptuning); tuner_file sets hipTunerFile; low_latency sets
    hipLowLatency (split-K 3x3 convs for handles of max_batch <= 16)."""

    def __init__(self, model: LoadedModel, nn_x: int = 19, nn_y: int = 19, use_fp16=None, auto_tune=None,
                 home_data_dir: str = "", tuner_file: str = "", low_latency=None):
        lib = host_library()
        err = _errbuf()
        mode = 2 if use_fp16 is None else (1 if use_fp16 else 0)
        self.model = model
        self.nn_x, self.nn_y = nn_x, nn_y
        self._handles = weakref.WeakSet()
        cfg = []
        if auto_tune is not None:
            cfg.append(f"hipAutoTune = {'true' if auto_tune else 'false'}")
        if tuner_file:
            cfg.append(f"hipTunerFile = {tuner_file}")
        if low_latency is not None:
            cfg.append(f"hipLowLatency = {'true' if low_latency else 'false'}")
        self._ptr = lib.kgn_create_context_cfg(model._ptr, nn_x, nn_y, mode, home_data_dir.encode(), "\n".join(cfg).encode(),
                                               err, len(err))
        if not self._ptr:
            _raise(err)

    def close(self):
        """Frees the context; its live handles are closed first, since a
        handle cannot run without its context. (Handles the garbage collector
        finalizes after the context are still freed safely: they share the
        context's model table.)"""
        if getattr(self, "_ptr", None):
            for h in list(getattr(self, "_handles", ())):
                h.close()
            host_library().kgn_free_context(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # at interpreter exit the library may already be gone
            pass


class ComputeHandle:
    """NeuralNet::createComputeHandle + getOutput."""

    def __init__(self, context: ComputeContext, max_batch: int, require_exact_nn_len: bool = False,
                 inputs_use_nhwc: bool = True, gpu_idx: int = 0):
        lib = host_library()
        err = _errbuf()
        self.context = context
        self.model = context.model
        self.max_batch = max_batch
        self.inputs_use_nhwc = inputs_use_nhwc
        self._ptr = lib.kgn_create_handle(context._ptr, context.model._ptr, max_batch, int(require_exact_nn_len),
                                          int(inputs_use_nhwc), gpu_idx, err, len(err))
        if not self._ptr:
            _raise(err)
        context._handles.add(self)

    @property
    def using_fp16(self) -> bool:
        return bool(host_library().kgn_is_using_fp16(self._ptr))

    def tuning(self):
        """(source, table): source 0 built-in choices, 1 loaded from a tuning
        file, 2 tuned at creation; table as saved."""
        buf = ctypes.create_string_buffer(1 << 16)
        src = host_library().kgn_handle_tuning(self._ptr, buf, len(buf))
        if src < 0:
            raise StringError(buf.value.decode(errors="replace"))
        return src, buf.value.decode()

    def set_tuning(self, table: str):
        err = _errbuf()
        if host_library().kgn_handle_set_tuning(self._ptr, table.encode(), err, len(err)) != 0:
            _raise(err)

    def get_output(self, spatial, global_in, symmetry=None, policy_optimism=None):
        """Returns raw outputs as a dict of arrays: policy [n, HW+1] (pass last),
        value [n, 3], score [n, 6], ownership [n, HW]."""
        lib = host_library()
        n = int(np.asarray(global_in).shape[0])
        hw = self.context.nn_x * self.context.nn_y
        spatial = _as_rows(spatial, n)
        global_in = _as_rows(global_in, n)
        sym = np.ascontiguousarray(np.zeros(n) if symmetry is None else symmetry, dtype=np.int32)
        opt = np.ascontiguousarray(np.zeros(n) if policy_optimism is None else policy_optimism, dtype=np.float32)
        policy = np.zeros((n, hw + 1), np.float32)
        value = np.zeros((n, 3), np.float32)
        score = np.zeros((n, 6), np.float32)
        own = np.zeros((n, hw), np.float32)
        err = _errbuf()
        rc = lib.kgn_get_output(self._ptr, self.model._ptr, self.context.nn_x, self.context.nn_y, n,
                                spatial.ctypes.data, global_in.ctypes.data, sym.ctypes.data, opt.ctypes.data,
                                policy.ctypes.data, value.ctypes.data, score.ctypes.data, own.ctypes.data, err, len(err))
        if rc != 0:
            _raise(err)
        return {"policy": policy, "value": value, "score": score, "ownership": own}

    def get_output_post(self, spatial, global_in, legal, row_info, temperature=None, symmetry=None, policy_optimism=None):
        """getOutput with device post-processing of the rows whose row_info
        has POST_ENABLED: returns policy [n, HW+1], values [n, 9], ownership
        [n, HW] (see kgn_get_output_post)."""
        lib = host_library()
        n = int(np.asarray(global_in).shape[0])
        hw = self.context.nn_x * self.context.nn_y
        spatial = _as_rows(spatial, n)
        global_in = _as_rows(global_in, n)
        legal = np.ascontiguousarray(legal, dtype=np.uint8).reshape(n, hw + 1)
        info = np.ascontiguousarray(row_info, dtype=np.int32)
        temp = np.ascontiguousarray(np.ones(n) if temperature is None else temperature, dtype=np.float32)
        sym = np.ascontiguousarray(np.zeros(n) if symmetry is None else symmetry, dtype=np.int32)
        opt = np.ascontiguousarray(np.zeros(n) if policy_optimism is None else policy_optimism, dtype=np.float32)
        policy = np.zeros((n, hw + 1), np.float32)
        values = np.zeros((n, 9), np.float32)
        own = np.zeros((n, hw), np.float32)
        err = _errbuf()
        rc = lib.kgn_get_output_post(self._ptr, self.model._ptr, self.context.nn_x, self.context.nn_y, n, spatial.ctypes.data,
                                     global_in.ctypes.data, sym.ctypes.data, opt.ctypes.data, legal.ctypes.data,
                                     info.ctypes.data, temp.ctypes.data, policy.ctypes.data, values.ctypes.data,
                                     own.ctypes.data, err, len(err))
        if rc != 0:
            _raise(err)
        return {"policy": policy, "values": values, "ownership": own}

    def close(self):
        if getattr(self, "_ptr", None):
            host_library().kgn_free_handle(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # at interpreter exit the library may already be gone
            pass


class Evaluator:
    """NNEvaluator's batching server loop (nneval.cpp:549-739) over this
    backend: server threads with one compute handle each, batches of whatever
    rows are queued up to max_batch. evaluate() is thread-safe and blocks.
    With model=None and debug_skip_nn the threads answer without a device."""

    def __init__(self, model, nn_x: int = 19, nn_y: int = 19, max_batch: int = 256, use_fp16=True,
                 num_server_threads: int = 1, gpu: int = 0, debug_skip_nn: bool = False):
        lib = host_library()
        err = _errbuf()
        self.model = model
        self.nn_x, self.nn_y = nn_x, nn_y
        fp16 = 2 if use_fp16 is None else int(bool(use_fp16))
        self._ptr = lib.kgn_evaluator_create(model._ptr if model is not None else None, nn_x, nn_y, max_batch, fp16,
                                             num_server_threads, gpu, int(debug_skip_nn), err, len(err))
        if not self._ptr:
            _raise(err)

    def evaluate(self, spatial, global_in, board_x: int = None, board_y: int = None, symmetry: int = 0,
                 policy_optimism: float = 0.0, include_owner_map: bool = True):
        """One featurized row (NHWC spatial, globals) -> raw outputs dict."""
        lib = host_library()
        hw = self.nn_x * self.nn_y
        spatial = np.ascontiguousarray(spatial, dtype=np.float32).reshape(-1)
        global_in = np.ascontiguousarray(global_in, dtype=np.float32).reshape(-1)
        policy = np.zeros(hw + 1, np.float32)
        value = np.zeros(3, np.float32)
        score = np.zeros(6, np.float32)
        own = np.zeros(hw, np.float32) if include_owner_map else None
        err = _errbuf()
        rc = lib.kgn_evaluator_evaluate(self._ptr, spatial.ctypes.data, spatial.size, global_in.ctypes.data, global_in.size,
                                        board_x or self.nn_x, board_y or self.nn_y, symmetry, policy_optimism,
                                        policy.ctypes.data, value.ctypes.data, score.ctypes.data,
                                        own.ctypes.data if own is not None else None, err, len(err))
        if rc != 0:
            _raise(err)
        return {"policy": policy, "value": value, "score": score, "ownership": own}

    def stats(self):
        rows, batches = ctypes.c_uint64(0), ctypes.c_uint64(0)
        host_library().kgn_evaluator_stats(self._ptr, ctypes.byref(rows), ctypes.byref(batches))
        return rows.value, batches.value

    def clear_stats(self):
        host_library().kgn_evaluator_clear_stats(self._ptr)

    def run_clients(self, spatial_rows, global_rows, num_clients: int, evals_per_client: int, board_x: int = None,
                    board_y: int = None, want_policy: bool = False):
        """Native client threads evaluating rows in a loop; returns (seconds,
        policy of each client's first row or None)."""
        lib = host_library()
        spatial_rows = np.ascontiguousarray(spatial_rows, dtype=np.float32)
        global_rows = np.ascontiguousarray(global_rows, dtype=np.float32)
        n = global_rows.shape[0]
        spatial_rows = spatial_rows.reshape(n, -1)
        global_rows = global_rows.reshape(n, -1)
        hw = self.nn_x * self.nn_y
        policy = np.zeros((min(num_clients, n), hw + 1), np.float32) if want_policy else None
        secs = ctypes.c_double(0.0)
        err = _errbuf()
        rc = lib.kgn_evaluator_run_clients(self._ptr, num_clients, evals_per_client, n, spatial_rows.ctypes.data,
                                           spatial_rows.shape[1], global_rows.ctypes.data, global_rows.shape[1],
                                           board_x or self.nn_x, board_y or self.nn_y,
                                           policy.ctypes.data if policy is not None else None, ctypes.byref(secs), err,
                                           len(err))
        if rc != 0:
            _raise(err)
        return secs.value, policy

    def close(self):
        if getattr(self, "_ptr", None):
            host_library().kgn_evaluator_free(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # at interpreter exit the library may already be gone
            pass


TEST_CONV, TEST_BATCHNORM, TEST_RESIDUAL, TEST_GPOOL = 0, 1, 2, 3


def test_evaluate(kind: int, desc_text: str, batch: int, nn_x: int, nn_y: int, use_fp16: bool, use_nhwc: bool,
                  inputs, mask=None, out_channels: int = 0):
    """NeuralNet::testEvaluate{Conv,BatchNorm,ResidualBlock,GlobalPoolingResidualBlock}.
    Returns the output array, or None when the combination is unsupported."""
    lib = host_library()
    inp = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32).reshape(-1)
    out = np.zeros(batch * nn_x * nn_y * max(out_channels, 1) * 4 + inp.size, np.float32)
    err = _errbuf()
    rc = lib.kgn_test_evaluate(kind, desc_text.encode(), batch, nn_x, nn_y, int(use_fp16), int(use_nhwc), inp.ctypes.data,
                               None if m is None else m.ctypes.data, out.ctypes.data, out.size, err, len(err))
    if rc < 0:
        _raise(err)
    if rc == 0:
        return None
    return out[: batch * nn_x * nn_y * out_channels]


HIP_ERROR_OUT_OF_MEMORY = 2
HIP_ERROR_LAUNCH_FAILURE = 719
FAULT_ANY_CALL, FAULT_ALLOCATION, FAULT_KERNEL_LAUNCH = 0, 1, 2


def inject_fault(site: int, countdown: int, hip_error: int = HIP_ERROR_LAUNCH_FAILURE) -> None:
    """kgh_debug_inject_fault: the countdown-th checked HIP call at the site
    reports hip_error (one-shot); countdown 0 disarms."""
    lib = hip_library()
    lib.kgh_debug_inject_fault.argtypes = [ctypes.c_int32] * 3
    hip_check(lib.kgh_debug_inject_fault(site, countdown, hip_error))


def peek_last_error() -> int:
    """kgh_debug_peek_last_error: the runtime's pending HIP error code."""
    v = ctypes.c_int32()
    hip_check(hip_library().kgh_debug_peek_last_error(ctypes.byref(v)))
    return v.value


def fault_pending() -> bool:
    v = ctypes.c_int32()
    hip_check(hip_library().kgh_debug_fault_pending(ctypes.byref(v)))
    return bool(v.value)


def hip_check(status: int) -> None:
    if status != 0:
        # Raised without a local name: a frame holding the exception that
        # holds the frame would keep every caller's locals alive until the
        # cycle collector runs.
        raise StringError(hip_library().kgh_last_error().decode(errors="replace"), status)


def device_count() -> int:
    c = ctypes.c_int32(0)
    hip_check(hip_library().kgh_device_count(ctypes.byref(c)))
    return int(c.value)


# ---------------------------------------------------------------------------
# Direct use of the device library's C ABI (include/katago_hip.h).

LAYER_DTYPE = np.dtype([("op", "<i4"), ("i", "<i4", 7), ("f", "<f4", 2), ("w", "<i8", 2), ("wn", "<i8", 2)])


class _ModelDescC(ctypes.Structure):
    _fields_ = [("model_version", ctypes.c_int32), ("num_input_channels", ctypes.c_int32),
                ("num_input_global_channels", ctypes.c_int32), ("num_input_meta_channels", ctypes.c_int32),
                ("num_policy_channels", ctypes.c_int32), ("num_value_channels", ctypes.c_int32),
                ("num_score_value_channels", ctypes.c_int32), ("num_ownership_channels", ctypes.c_int32),
                ("num_layers", ctypes.c_int32), ("layers", ctypes.c_void_p), ("weights", ctypes.c_void_p),
                ("num_weights", ctypes.c_int64)]


def flatten_model(model: LoadedModel):
    """The layer program (LAYER_DTYPE records) and weights that the backend
    passes to kgh_model_create for this model (kgn_model_flatten)."""
    lib = host_library()
    lib.kgn_model_flatten.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64),
                                      ctypes.c_void_p, ctypes.c_void_p]
    nl = ctypes.c_int32()
    nw = ctypes.c_int64()
    if lib.kgn_model_flatten(model._ptr, ctypes.byref(nl), ctypes.byref(nw), None, None) != 0:
        raise StringError("kgn_model_flatten failed")
    layers = np.zeros(nl.value, LAYER_DTYPE)
    weights = np.zeros(nw.value, np.float32)
    if lib.kgn_model_flatten(model._ptr, ctypes.byref(nl), ctypes.byref(nw), layers.ctypes.data, weights.ctypes.data) != 0:
        raise StringError("kgn_model_flatten failed")
    return layers, weights


class DeviceModel:
    """kgh_model: a model's weights uploaded to one device."""

    def __init__(self, model: LoadedModel, use_fp16: bool, device: int = 0):
        lib = hip_library()
        self.layers, self.weights = flatten_model(model)
        info = model.info
        d = _ModelDescC(info.model_version, info.num_input_channels, info.num_input_global_channels,
                        info.num_input_meta_channels, info.num_policy_channels, info.num_value_channels,
                        info.num_score_value_channels, info.num_ownership_channels, len(self.layers),
                        self.layers.ctypes.data, self.weights.ctypes.data, len(self.weights))
        self.info = info
        self._handles = weakref.WeakSet()
        self._ptr = ctypes.c_void_p()
        lib.kgh_model_create.argtypes = [ctypes.c_int32, ctypes.POINTER(_ModelDescC), ctypes.c_int32,
                                         ctypes.POINTER(ctypes.c_void_p)]
        hip_check(lib.kgh_model_create(device, ctypes.byref(d), int(use_fp16), ctypes.byref(self._ptr)))

    def forward_device_noalloc(self, n, nn_x, nn_y, d_spatial, d_global, d_sym, d_opt, d_out, stream=None):
        """kgh_forward_device_noalloc: a forward in the library's static device
        scratch, on `stream` (a hipStream_t as an int, None for the null
        stream); asynchronous."""
        lib = hip_library()
        lib.kgh_forward_device_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32] + \
            [ctypes.c_void_p] * 6
        hip_check(lib.kgh_forward_device_noalloc(self._ptr, n, nn_x, nn_y, d_spatial, d_global, d_sym, d_opt, d_out, stream))

    def close(self):
        """Frees the model; its live handles are closed first, since a handle
        cannot run without the weights. (kgh_handle_free does not read the
        model, so handles finalized after it are still freed safely.)"""
        if getattr(self, "_ptr", None) and self._ptr.value:
            for h in list(getattr(self, "_handles", ())):
                h.close()
            hip_library().kgh_model_free(self._ptr)
            self._ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:  # at interpreter exit the library may already be gone
            pass


class DeviceHandle:
    """kgh_handle: stream and buffers for device-memory forwards."""

    def __init__(self, model: DeviceModel, max_batch: int, nn_x: int = 19, nn_y: int = 19):
        lib = hip_library()
        self.model = model
        self.nn_x, self.nn_y = nn_x, nn_y
        self._ptr = ctypes.c_void_p()
        lib.kgh_handle_create.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.POINTER(ctypes.c_void_p)]
        hip_check(lib.kgh_handle_create(model._ptr, max_batch, nn_x, nn_y, 0, ctypes.byref(self._ptr)))
        model._handles.add(self)
        lib.kgh_forward_device.argtypes = [ctypes.c_void_p, ctypes.c_int32] + [ctypes.c_void_p] * 5
        lib.kgh_handle_synchronize.argtypes = [ctypes.c_void_p]
        lib.kgh_handle_set_profiling.argtypes = [ctypes.c_void_p, ctypes.c_int32]
        lib.kgh_handle_set_graphs.argtypes = [ctypes.c_void_p, ctypes.c_int32]
        lib.kgh_handle_profile.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_double)]
        self.row_floats = lib.kgh_output_row_floats(nn_x, nn_y, model.info.num_score_value_channels)

    def forward_device(self, n, d_spatial, d_global, d_sym, d_opt, d_out):
        hip_check(hip_library().kgh_forward_device(self._ptr, n, d_spatial, d_global, d_sym, d_opt, d_out))

    def postprocess_device(self, n, d_raw, d_legal, d_info, d_temp, params: "PostParams", d_post):
        lib = hip_library()
        lib.kgh_postprocess_device.argtypes = [ctypes.c_void_p, ctypes.c_int32] + [ctypes.c_void_p] * 4 + [
            ctypes.POINTER(PostParams), ctypes.c_void_p]
        hip_check(lib.kgh_postprocess_device(self._ptr, n, d_raw, d_legal, d_info, d_temp, ctypes.byref(params), d_post))

    def synchronize(self):
        hip_check(hip_library().kgh_handle_synchronize(self._ptr))

    def autotune(self, reps: int = 3) -> str:
        """kgh_handle_autotune: returns the table (one line per conv shape)."""
        lib = hip_library()
        lib.kgh_handle_autotune.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_char_p, ctypes.c_int32]
        buf = ctypes.create_string_buffer(1 << 16)
        hip_check(lib.kgh_handle_autotune(self._ptr, reps, buf, len(buf)))
        return buf.value.decode()

    def set_tuning(self, table: str):
        """kgh_handle_set_tuning: kernel choices per conv shape, in the format
        autotune() returns."""
        lib = hip_library()
        lib.kgh_handle_set_tuning.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        hip_check(lib.kgh_handle_set_tuning(self._ptr, table.encode()))

    def set_profiling(self, on: bool):
        hip_check(hip_library().kgh_handle_set_profiling(self._ptr, int(on)))

    def set_graphs(self, on: bool):
        """Enables (default) or disables HIP graph replay of repeated forwards."""
        hip_check(hip_library().kgh_handle_set_graphs(self._ptr, int(on)))

    def set_low_latency(self, on: bool):
        """kgh_handle_set_low_latency: split-K 3x3 convs (max_batch <= 16)."""
        lib = hip_library()
        lib.kgh_handle_set_low_latency.argtypes = [ctypes.c_void_p, ctypes.c_int32]
        hip_check(lib.kgh_handle_set_low_latency(self._ptr, int(on)))

    def profile(self, kind: int):
        ms = ctypes.c_double()
        cnt = ctypes.c_int32()
        fl = ctypes.c_double()
        hip_check(hip_library().kgh_handle_profile(self._ptr, kind, ctypes.byref(ms), ctypes.byref(cnt), ctypes.byref(fl)))
        return ms.value, cnt.value, fl.value

    def set_layer_dump(self, on: bool, value_scale: float = 1.0):
        """kgh_handle_set_layer_dump: per-block trunk summary lines of the
        following forwards, values times value_scale."""
        lib = hip_library()
        lib.kgh_handle_set_layer_dump.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_float]
        hip_check(lib.kgh_handle_set_layer_dump(self._ptr, int(on), value_scale))

    def layer_dump(self) -> str:
        lib = hip_library()
        lib.kgh_handle_layer_dump.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int32]
        buf = ctypes.create_string_buffer(1 << 20)
        hip_check(lib.kgh_handle_layer_dump(self._ptr, buf, len(buf)))
        return buf.value.decode()

    def profile_kernels(self):
        """kgh_handle_profile_kernels: [(kind, launches, total_ms, flops,
        kernel)] per kernel that ran, in order of first launch."""
        lib = hip_library()
        lib.kgh_handle_profile_kernels.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int32]
        buf = ctypes.create_string_buffer(1 << 16)
        hip_check(lib.kgh_handle_profile_kernels(self._ptr, buf, len(buf)))
        rows = []
        for line in buf.value.decode().splitlines():
            kind, launches, ms, flops, name = line.split("\t", 4)
            rows.append((int(kind), int(launches), float(ms), float(flops), name))
        return rows

    def close(self):
        if getattr(self, "_ptr", None) and self._ptr.value:
            hip_library().kgh_handle_free(self._ptr)
            self._ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:  # at interpreter exit the library may already be gone
            pass


POST_ENABLED, POST_WHITE_TO_MOVE, POST_NO_RESULT_DISABLED, POST_PASSING_HACKS = 1, 2, 4, 8


def post_info(enabled=True, white_to_move=False, no_result_disabled=False, passing_hacks=False, board_x=19, board_y=19):
    """The per-row info word of the device post-processing (katago_hip.h)."""
    return ((POST_ENABLED if enabled else 0) | (POST_WHITE_TO_MOVE if white_to_move else 0) |
            (POST_NO_RESULT_DISABLED if no_result_disabled else 0) | (POST_PASSING_HACKS if passing_hacks else 0) |
            (board_x << 8) | (board_y << 16))


class PostParams(ctypes.Structure):
    """kgh_post_params (ModelPostProcessParams, desc.h:468-481)."""
    _fields_ = [("output_scale_multiplier", ctypes.c_float), ("score_mean_multiplier", ctypes.c_double),
                ("score_stdev_multiplier", ctypes.c_double), ("lead_multiplier", ctypes.c_double),
                ("variance_time_multiplier", ctypes.c_double), ("shortterm_value_error_multiplier", ctypes.c_double),
                ("shortterm_score_error_multiplier", ctypes.c_double)]


class DeviceBuffer:
    """Device memory from kgh_device_alloc, filled from / read into numpy."""

    def __init__(self, nbytes: int, device: int = 0):
        self.nbytes = nbytes
        self.ptr = ctypes.c_void_p()
        hip_check(hip_library().kgh_device_alloc(device, nbytes, ctypes.byref(self.ptr)))

    @classmethod
    def from_array(cls, a: np.ndarray, device: int = 0):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, device)
        hip_check(hip_library().kgh_memcpy_htod(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype)
        hip_check(hip_library().kgh_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr.value:
            hip_library().kgh_device_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        self.free()


# ---------------------------------------------------------------------------
# Position featurizer (include/katago_featurize.h).

class KgnPosition(ctypes.Structure):
    """kgn_position."""
    _fields_ = [("x_size", ctypes.c_int32), ("y_size", ctypes.c_int32), ("next_player", ctypes.c_int32),
                ("colors", ctypes.c_void_p * 3), ("ko_point", ctypes.c_int32 * 3),
                ("chain_head", ctypes.c_void_p * 3), ("chain_next", ctypes.c_void_p * 3),
                ("super_ko_banned", ctypes.c_void_p), ("ko_recap_blocked", ctypes.c_void_p),
                ("second_encore_start_colors", ctypes.c_void_p),
                ("num_moves", ctypes.c_int32), ("move_point", ctypes.c_int32 * 5), ("move_player", ctypes.c_int32 * 5),
                ("num_approx_valid_turns_this_phase", ctypes.c_int32), ("encore_phase", ctypes.c_int32),
                ("ko_rule", ctypes.c_int32), ("scoring_rule", ctypes.c_int32), ("tax_rule", ctypes.c_int32),
                ("multi_stone_suicide_legal", ctypes.c_int32), ("has_button", ctypes.c_int32),
                ("self_komi", ctypes.c_float),
                ("pass_would_end_game", ctypes.c_uint8), ("pass_would_end_phase", ctypes.c_uint8),
                ("suppress_end_game_from_friendly_pass", ctypes.c_uint8), ("is_game_finished", ctypes.c_uint8),
                ("is_past_normal_phase_end", ctypes.c_uint8), ("conservative_pass_and_is_root", ctypes.c_uint8),
                ("enable_passing_hacks", ctypes.c_uint8), ("playout_doubling_advantage", ctypes.c_double),
                ("max_history", ctypes.c_int32)]


_POSITION_SCALARS = ["num_approx_valid_turns_this_phase", "encore_phase", "ko_rule", "scoring_rule", "tax_rule",
                     "multi_stone_suicide_legal", "has_button", "self_komi", "pass_would_end_game", "pass_would_end_phase",
                     "suppress_end_game_from_friendly_pass", "is_game_finished", "is_past_normal_phase_end",
                     "conservative_pass_and_is_root", "enable_passing_hacks", "playout_doubling_advantage", "max_history"]


class Positions:
    """An array of kgn_position built from dicts with the struct's field
    names (colors, chain_head and chain_next as lists of three per-point
    lists); keeps the arrays the structs point into alive."""

    def __init__(self, dicts, with_chain_order: bool = True):
        self.n = len(dicts)
        self.array = (KgnPosition * max(self.n, 1))()
        self._keep = []
        for i, d in enumerate(dicts):
            p = self.array[i]
            p.x_size, p.y_size, p.next_player = d["x_size"], d["y_size"], d["next_player"]
            for k in range(3):
                p.colors[k] = self._ptr(d["colors"][k], np.int8)
                p.ko_point[k] = d["ko_point"][k]
                if with_chain_order and "chain_head" in d:
                    p.chain_head[k] = self._ptr(d["chain_head"][k], np.int16)
                    p.chain_next[k] = self._ptr(d["chain_next"][k], np.int16)
            p.super_ko_banned = self._ptr(d.get("super_ko_banned"), np.uint8)
            p.ko_recap_blocked = self._ptr(d.get("ko_recap_blocked"), np.uint8)
            p.second_encore_start_colors = self._ptr(d.get("second_encore_start_colors"), np.int8)
            p.num_moves = d["num_moves"]
            for k in range(5):
                p.move_point[k] = d["move_point"][k]
                p.move_player[k] = d["move_player"][k]
            for f in _POSITION_SCALARS:
                if f in d:
                    setattr(p, f, d[f])

    def _ptr(self, values, dtype):
        if values is None:
            return None
        a = np.ascontiguousarray(values, dtype=dtype)
        self._keep.append(a)
        return a.ctypes.data


KGN_FEATURIZE_MAX_CACHE = 64  # include/katago_featurize.h


def featurize_set_cache(entries: int) -> int:
    """kgn_featurize_set_cache: ladder results kept per thread for boards
    that come again (0 turns it off); returns the previous setting."""
    lib = host_library()
    lib.kgn_featurize_set_cache.restype = ctypes.c_int32
    lib.kgn_featurize_set_cache.argtypes = [ctypes.c_int32]
    prev = lib.kgn_featurize_set_cache(entries)
    if prev < 0:
        raise StringError(f"kgn_featurize_set_cache: {entries} entries is out of range")
    return prev


def featurize(positions: Positions, nn_x: int = 19, nn_y: int = 19, use_nhwc: bool = True, num_threads: int = 0):
    """kgn_featurize: returns spatial [n, nn_y*nn_x*22] (NHWC or NCHW per
    row) and global [n, 19] float32 arrays."""
    lib = host_library()
    lib.kgn_featurize.restype = ctypes.c_int32
    lib.kgn_featurize.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_char_p, ctypes.c_int32]
    n = positions.n
    spatial = np.zeros((n, nn_y * nn_x * 22), np.float32)
    glob = np.zeros((n, 19), np.float32)
    err = _errbuf()
    rc = lib.kgn_featurize(ctypes.addressof(positions.array), n, nn_x, nn_y, int(use_nhwc), spatial.ctypes.data,
                           glob.ctypes.data, num_threads, err, len(err))
    if rc != 0:
        _raise(err)
    return spatial, glob
