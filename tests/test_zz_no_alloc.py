"""kgh_forward_device_noalloc (the forward that allocates nothing, its
activations in the library's static device scratch) against
kgh_forward_device on a handle, through the C ABI: bitwise equal outputs on
two calls in a row, the second with a smaller batch and other inputs, so that
anything the first call left in the scratch would show."""
import numpy as np
import pytest

from katago_amd import modelgen, nn

pytestmark = pytest.mark.gpu


def _inputs(seed, n, nn_x, nn_y, boards):
    sp, gl = modelgen.synthetic_inputs(seed, n, nn_x=nn_x, nn_y=nn_y, board_sizes=boards)
    sym = (np.arange(n) * 3 % 8).astype(np.int32) if nn_x == nn_y else (np.arange(n) % 4).astype(np.int32)
    opt = ((np.arange(n) % 3) / 2.0).astype(np.float32)
    return [nn.DeviceBuffer.from_array(a) for a in (sp, gl, sym, opt)]


def _handle_forward(h, n, bufs, row_floats):
    out = nn.DeviceBuffer.from_array(np.full((n, row_floats), np.nan, np.float32))
    h.forward_device(n, *(b.ptr for b in bufs), out.ptr)
    h.synchronize()
    return out.to_array(np.float32, (n, row_floats))


def _noalloc_forward(dm, n, nn_x, nn_y, bufs, row_floats):
    out = nn.DeviceBuffer.from_array(np.full((n, row_floats), np.nan, np.float32))
    dm.forward_device_noalloc(n, nn_x, nn_y, *(b.ptr for b in bufs), out.ptr)
    # kgh_memcpy_dtoh is a blocking copy on the null stream, which the forward
    # above ran on: it returns after the forward.
    return out.to_array(np.float32, (n, row_floats))


@pytest.mark.parametrize("cfg_index,nn_x,nn_y,n1,n2", [
    (2, 19, 19, 16, 5),   # b18c384nbt fp16
    (0, 19, 19, 8, 3),    # b6c96 fp32
    (1, 10, 14, 12, 2),   # b10c128 fp16, rectangular context
], ids=["C2-fp16", "C0-fp32", "C1-10x14"])
def test_noalloc_forward_matches_handle_forward(model_dir, cfg_index, nn_x, nn_y, n1, n2):
    cfg = modelgen.configs()[cfg_index]
    lm = nn.LoadedModel(modelgen.ensure_model(model_dir, cfg))
    dm = nn.DeviceModel(lm, use_fp16=cfg.fp16)
    h = nn.DeviceHandle(dm, n1, nn_x, nn_y)
    h.set_graphs(False)
    rf = h.row_floats
    boards = (nn_x, 9) if nn_x == nn_y else ((nn_x, nn_y), (9, 13))
    first = _inputs(11, n1, nn_x, nn_y, boards)
    second = _inputs(12, n2, nn_x, nn_y, boards)
    ref1 = _handle_forward(h, n1, first, rf)
    ref2 = _handle_forward(h, n2, second, rf)
    got1 = _noalloc_forward(dm, n1, nn_x, nn_y, first, rf)
    got2 = _noalloc_forward(dm, n2, nn_x, nn_y, second, rf)
    for label, ref, got in (("first call", ref1, got1), ("second call", ref2, got2)):
        assert np.isfinite(ref).all(), label
        assert np.array_equal(ref, got), f"{label}: max-abs {np.nanmax(np.abs(ref - got))}"


def test_noalloc_rejects_batches_beyond_the_scratch_and_transformer_nets(model_dir):
    """Checked on the host before any launch: a batch whose activations do not
    fit the static scratch, and nets with transformer blocks (attention with
    rotary tables, or FFN blocks alone)."""
    cfg = modelgen.configs()[2]
    dm = nn.DeviceModel(nn.LoadedModel(modelgen.ensure_model(model_dir, cfg)), use_fp16=True)
    dummy = nn.DeviceBuffer(256)
    with pytest.raises(nn.StringError, match="need .* bytes of scratch"):
        dm.forward_device_noalloc(256, 19, 19, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr)
    cfg4 = modelgen.configs()[4]
    dm4 = nn.DeviceModel(nn.LoadedModel(modelgen.ensure_model(model_dir, cfg4)), use_fp16=True)
    with pytest.raises(nn.StringError, match="transformer"):
        dm4.forward_device_noalloc(1, 19, 19, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr)
    # A transformer net without rotary tables (FFN blocks only) is refused too.
    arch = modelgen.Arch("tiny-ffn-only", 17, 64, 64, 32, ["regular", "ffn", "ffn"], 16, 16, 32, 24, "ACTIVATION_SILU",
                         heads=2, kv_heads=2, q_head_dim=32, v_head_dim=32, ffn_c=96, trunk_rmsnorm=True,
                         transformer_std=0.08, residual_gain=0.5)
    path = modelgen.write_model(arch, 7, f"{model_dir}/{arch.name}.bin.gz")
    dm5 = nn.DeviceModel(nn.LoadedModel(path), use_fp16=True)
    with pytest.raises(nn.StringError, match="transformer"):
        dm5.forward_device_noalloc(1, 19, 19, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr)
