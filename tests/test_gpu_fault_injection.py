"""Device error paths, forced from the host (kgh_debug_inject_fault).

The reference's error surface for a failed device call is CUDA_ERR
(cudaerrorcheck.h:10-12): a StringError naming the call, file and line. Here
a failed HIP call becomes KGH_ERR_HIP (KGH_ERR_OUT_OF_MEMORY for device
allocations) with that information, and the backend raises StringError. The
faults are synthetic: a checked call reports an error instead of running (a
launch check after its launch), so the GPU itself stays healthy and every
kernel exits normally. Each test checks that the error is reported at the
API it went through, that nothing leaks into later calls (the next call on
the same handle returns the same bits as before the fault), and that the
armed fault was consumed."""
import gc

import numpy as np
import pytest

from katago_amd import modelgen, nn

pytestmark = pytest.mark.gpu

KGH_ERR_HIP, KGH_ERR_OUT_OF_MEMORY = 2, 4


@pytest.fixture(autouse=True)
def disarm():
    """Disarms any fault, and checks that no HIP error is left pending on
    the thread before the test and after its objects are destroyed."""
    nn.inject_fault(nn.FAULT_ANY_CALL, 0)
    assert nn.peek_last_error() == 0
    yield
    nn.inject_fault(nn.FAULT_ANY_CALL, 0)
    gc.collect()
    assert nn.peek_last_error() == 0


def _device(model_dir, n=8, fp16=True):
    cfg = modelgen.configs()[1]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    dm = nn.DeviceModel(lm, use_fp16=fp16)
    sp, gl = modelgen.synthetic_inputs(9, n, board_sizes=(19, 9))
    bufs = [nn.DeviceBuffer.from_array(a) for a in (sp, gl, np.zeros(n, np.int32), np.zeros(n, np.float32))]
    return lm, dm, bufs, sp, gl


def _run(h, bufs, n, out):
    h.forward_device(n, *(b.ptr for b in bufs), out.ptr)
    h.synchronize()
    return out.to_array(np.float32, (n, h.row_floats))


def test_allocation_faults_in_handle_creation(model_dir):
    """The k-th allocation of a handle (device arena or pinned staging)
    fails: creation reports out of memory with the failing call, frees what
    it had allocated, and a handle created afterwards computes the same rows."""
    n = 8
    lm, dm, bufs, _, _ = _device(model_dir, n)
    ref_h = nn.DeviceHandle(dm, n)
    out = nn.DeviceBuffer(n * ref_h.row_floats * 4)
    ref = _run(ref_h, bufs, n, out)
    codes = set()
    for k in range(1, 80, 3):
        nn.inject_fault(nn.FAULT_ALLOCATION, k, nn.HIP_ERROR_OUT_OF_MEMORY)
        try:
            h = nn.DeviceHandle(dm, n)
        except nn.StringError as e:
            assert "out of memory" in str(e).lower(), str(e)
            assert e.code in (KGH_ERR_OUT_OF_MEMORY, KGH_ERR_HIP), e.code
            assert not nn.fault_pending()
            assert nn.peek_last_error() == 0, k
            codes.add(e.code)
            continue
        # Fewer allocations than k: the fault is still armed.
        assert nn.fault_pending()
        nn.inject_fault(nn.FAULT_ANY_CALL, 0)
        assert np.array_equal(_run(h, bufs, n, out), ref)
        break
    # Both kinds were hit: device buffers and pinned host staging.
    assert codes == {KGH_ERR_OUT_OF_MEMORY, KGH_ERR_HIP}, codes
    h = nn.DeviceHandle(dm, n)
    assert np.array_equal(_run(h, bufs, n, out), ref)


@pytest.mark.parametrize("fp16", [True, False], ids=["fp16", "fp32"])
def test_launch_faults_in_eager_forwards(model_dir, fp16):
    """A kernel launch reported as failed at the 1st, 5th, 17th and 24th
    launch of a forward: the forward raises naming the launch site; the
    launches already enqueued complete; the next forward on the same handle
    gives the same bits as before."""
    n = 8
    lm, dm, bufs, _, _ = _device(model_dir, n, fp16)
    h = nn.DeviceHandle(dm, n)
    h.set_graphs(False)
    out = nn.DeviceBuffer(n * h.row_floats * 4)
    ref = _run(h, bufs, n, out)
    for k in (1, 5, 17, 24):  # a C1 forward has ~27 launches
        nn.inject_fault(nn.FAULT_KERNEL_LAUNCH, k, nn.HIP_ERROR_LAUNCH_FAILURE)
        with pytest.raises(nn.StringError, match="kernel launch failed") as ei:
            h.forward_device(n, *(b.ptr for b in bufs), out.ptr)
        assert ei.value.code == KGH_ERR_HIP
        assert ".hip:" in str(ei.value)  # file and line of the check
        assert not nn.fault_pending()
        h.synchronize()
        assert nn.peek_last_error() == 0, k
        assert np.array_equal(_run(h, bufs, n, out), ref), k


def test_faults_during_graph_capture_and_replay(model_dir):
    """Repeated forwards run from a captured HIP graph: a launch fault while
    the graph is being captured abandons the capture (the stream leaves
    capture mode), and a failed graph launch is reported; in both cases the
    following forwards capture or replay normally."""
    n = 8
    lm, dm, bufs, _, _ = _device(model_dir, n)
    h = nn.DeviceHandle(dm, n)
    out = nn.DeviceBuffer(n * h.row_floats * 4)
    ref = _run(h, bufs, n, out)  # first call: eager
    nn.inject_fault(nn.FAULT_KERNEL_LAUNCH, 3)  # the repeat captures a graph
    with pytest.raises(nn.StringError, match="kernel launch failed"):
        h.forward_device(n, *(b.ptr for b in bufs), out.ptr)
    h.synchronize()
    for _ in range(3):  # capture again, then replays
        assert np.array_equal(_run(h, bufs, n, out), ref)
    nn.inject_fault(nn.FAULT_ANY_CALL, 2)  # a replay checks hipSetDevice, then the graph launch
    with pytest.raises(nn.StringError, match="hipGraphLaunch"):
        h.forward_device(n, *(b.ptr for b in bufs), out.ptr)
    h.synchronize()
    assert np.array_equal(_run(h, bufs, n, out), ref)


def test_faults_surface_through_get_output_and_the_evaluator(model_dir):
    """Through the backend (NeuralNet::getOutput, kgn_get_output) the fault
    is a StringError naming the failed call; through the NNEvaluator serve
    loop the client of the failed batch gets the error and later
    evaluations succeed (nneval.cpp's server thread keeps serving)."""
    n = 4
    cfg = modelgen.configs()[1]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    sp, gl = modelgen.synthetic_inputs(9, n)
    h = nn.ComputeHandle(nn.ComputeContext(lm, 19, 19, use_fp16=True), max_batch=n)
    ref = h.get_output(sp, gl)
    nn.inject_fault(nn.FAULT_KERNEL_LAUNCH, 2)
    with pytest.raises(nn.StringError, match="HIP backend: .*kernel launch failed"):
        h.get_output(sp, gl)
    assert not nn.fault_pending()
    again = h.get_output(sp, gl)
    for k in ref:
        assert np.array_equal(again[k], ref[k]), k

    ev = nn.Evaluator(lm, max_batch=4, use_fp16=True)
    one = ev.evaluate(sp[0], gl[0])
    nn.inject_fault(nn.FAULT_KERNEL_LAUNCH, 2)
    with pytest.raises(nn.StringError, match="kernel launch failed"):
        ev.evaluate(sp[0], gl[0])
    assert not nn.fault_pending()
    later = ev.evaluate(sp[0], gl[0])
    for k in one:
        assert np.array_equal(later[k], one[k]), k
    ev.close()


def test_handles_freed_after_their_model_or_context(model_dir):
    """A garbage collector may finalize a model before its handle (the
    objects of a reference cycle are finalized in no set order): freeing a
    handle after its model (kgh_handle_free), or a compute handle after its
    context (kgn_free_handle), frees cleanly and leaves no HIP error behind."""
    n = 4
    lm, dm, bufs, sp, gl = _device(model_dir, n)
    h = nn.DeviceHandle(dm, n)
    out = nn.DeviceBuffer(n * h.row_floats * 4)
    ref = _run(h, bufs, n, out)
    nn.hip_library().kgh_model_free(dm._ptr)  # straight through the C ABI: the handle is still live
    dm._ptr = nn.ctypes.c_void_p()
    h.close()
    assert nn.peek_last_error() == 0

    ctx = nn.ComputeContext(lm, 19, 19, use_fp16=True)
    ch = nn.ComputeHandle(ctx, max_batch=n)
    first = ch.get_output(sp, gl)
    nn.host_library().kgn_free_context(ctx._ptr)
    ctx._ptr = None
    ch.close()
    assert nn.peek_last_error() == 0

    # A fresh model and handle compute the same rows.
    dm2 = nn.DeviceModel(lm, use_fp16=True)
    h2 = nn.DeviceHandle(dm2, n)
    assert np.array_equal(_run(h2, bufs, n, out), ref)
    ctx2 = nn.ComputeContext(lm, 19, 19, use_fp16=True)
    again = nn.ComputeHandle(ctx2, max_batch=n).get_output(sp, gl)
    for k in first:
        assert np.array_equal(again[k], first[k]), k
