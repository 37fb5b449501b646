"""NNEvaluator's batching server loop (nneval.cpp:342-420, 549-750) over the
HIP backend: routing of rows to their own answers, batch-size bounds and
statistics (nneval.h:193-197), error paths; and on the GPU, rows served
through the evaluator equal a direct getOutput of the same rows.

CPU tests use debugSkipNeuralNet, whose server threads answer each row from
its own inputs: policy[p] = sum over channels of spatial[p], pass and win
logit = sum of the globals (computed in float32 here as a closed form).
"""
import threading

import numpy as np
import pytest

from katago_amd import modelgen, nn

HW = 361


def _rows(n, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, HW * 22)).astype(np.float32), rng.standard_normal((n, 19)).astype(np.float32))


def _expected_policy(spatial_row, global_row):
    p = spatial_row.reshape(HW, 22).sum(axis=1, dtype=np.float64)
    return np.concatenate([p, [global_row.sum(dtype=np.float64)]])


def test_rows_get_their_own_answers_under_concurrency():
    ev = nn.Evaluator(None, max_batch=8, num_server_threads=3, debug_skip_nn=True)
    sp, gl = _rows(64)
    results = [None] * 64
    errors = []

    def client(i):
        try:
            results[i] = ev.evaluate(sp[i], gl[i])
        except Exception as e:  # noqa: BLE001 - collected and asserted below
            errors.append(e)

    threads = [threading.Thread(target=client, args=(i,)) for i in range(64)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    for i in range(64):
        np.testing.assert_allclose(results[i]["policy"], _expected_policy(sp[i], gl[i]), rtol=1e-5, atol=1e-4)
        assert results[i]["value"][0] == pytest.approx(gl[i].sum(), rel=1e-5, abs=1e-5)
        np.testing.assert_allclose(results[i]["ownership"], 0.01 * results[i]["policy"][:HW], rtol=1e-6)
    rows, batches = ev.stats()
    assert rows == 64 and 8 <= batches <= 64  # at most max_batch rows per batch
    ev.close()


def test_native_clients_fill_batches_and_count_rows():
    ev = nn.Evaluator(None, max_batch=16, num_server_threads=2, debug_skip_nn=True)
    sp, gl = _rows(40, seed=1)
    secs, pol = ev.run_clients(sp, gl, num_clients=40, evals_per_client=25, want_policy=True)
    assert secs > 0
    for c in range(40):
        np.testing.assert_allclose(pol[c], _expected_policy(sp[c], gl[c]), rtol=1e-5, atol=1e-4)
    rows, batches = ev.stats()
    assert rows == 1000
    assert rows / batches <= 16
    assert batches >= 1000 // 16
    ev.clear_stats()
    assert ev.stats() == (0, 0)
    ev.close()


def test_single_server_thread_batch_of_one():
    ev = nn.Evaluator(None, max_batch=1, num_server_threads=1, debug_skip_nn=True)
    sp, gl = _rows(3, seed=2)
    secs, _ = ev.run_clients(sp, gl, num_clients=3, evals_per_client=4)
    assert ev.stats() == (12, 12)
    ev.close()


def test_board_larger_than_evaluator_is_rejected():
    ev = nn.Evaluator(None, nn_x=9, nn_y=9, max_batch=4, debug_skip_nn=True)
    with pytest.raises(nn.StringError, match="larger x or y size"):
        ev.evaluate(np.zeros(81 * 22, np.float32), np.zeros(19, np.float32), board_x=13, board_y=13)
    out = ev.evaluate(np.ones(81 * 22, np.float32), np.zeros(19, np.float32), board_x=9, board_y=9)
    assert out["policy"].shape == (82,) and out["policy"][0] == pytest.approx(22.0)
    ev.close()


def test_invalid_configuration_is_rejected():
    with pytest.raises(nn.StringError):
        nn.Evaluator(None, max_batch=0, debug_skip_nn=True)
    with pytest.raises(nn.StringError):
        nn.Evaluator(None, num_server_threads=0, debug_skip_nn=True)
    with pytest.raises(nn.StringError, match="needs a model"):
        nn.Evaluator(None, debug_skip_nn=False)


@pytest.mark.gpu
def test_evaluator_rows_equal_direct_get_output(model_dir):
    """Rows served through two server threads in batches of up to 16 equal the
    same rows in one direct getOutput call, bitwise (every reduction is per
    row and both batch sizes take the same kernels)."""
    cfg = modelgen.configs()[1]
    path = modelgen.ensure_model(model_dir, cfg)
    lm = nn.LoadedModel(path)
    n = 48
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, n)
    sp = np.ascontiguousarray(sp, dtype=np.float32).reshape(n, -1)
    gl = np.ascontiguousarray(gl, dtype=np.float32).reshape(n, -1)
    direct = nn.ComputeHandle(nn.ComputeContext(lm, 19, 19, use_fp16=True), max_batch=n).get_output(sp, gl)
    ev = nn.Evaluator(lm, max_batch=16, use_fp16=True, num_server_threads=2)
    secs, pol = ev.run_clients(sp, gl, num_clients=n, evals_per_client=3, want_policy=True)
    rows, batches = ev.stats()
    assert rows == 3 * n and rows / batches <= 16
    assert np.array_equal(pol, direct["policy"])
    one = ev.evaluate(sp[5], gl[5])
    for k in ("policy", "value", "score", "ownership"):
        assert np.array_equal(one[k], direct[k][5]), k
    ev.close()
