"""GPU parity of the sigmoid top-k selection (moonlight_route_sigmoid_topk,
moonlight_kernels.metal:469-512; moe_route_select + moe_route_finalize,
moe_route.h:47-99) against orc_route_sigmoid_topk, on logits built to
stress the order rules: many exact ties (equal scores must go to the lower
expert index first), NaN logits and -inf biases (never taken), rows with
fewer live experts than top_k (id -1, weight 0), and expert counts below 64
(lanes without an expert).  mlk_route_topk runs the decode path's routing
kernels: route_kernel for 1 row (route_single_64) and 2-8 rows,
route_select_kernel for more; more than 64 experts take the arg-max scan.
Ids must match exactly, weights to f32 rounding.
"""
import numpy as np
import pytest

import oracle_lib as O
from floyd_amd import native

pytestmark = pytest.mark.gpu


def tied_logits(rows, experts, seed):
    rng = np.random.default_rng(seed)
    # few distinct values: most selections are decided by the tie rule
    logits = (rng.integers(-3, 4, size=(rows, experts)) * 0.5).astype(np.float32)
    bias = (rng.integers(-2, 3, size=experts) * 0.25).astype(np.float32)
    logits[rows // 2] = 0.75  # one row of all-equal logits
    if experts > 8:
        logits[0, 3] = np.nan
        logits[-1, 5] = np.nan
        bias[7] = -np.inf
    return logits, bias


def run_device(logits, bias, top_k, normalize=1, scale=2.5):
    rows, experts = logits.shape
    d_l = native.DeviceBuffer.from_array(logits)
    d_b = native.DeviceBuffer.from_array(bias)
    d_i = native.DeviceBuffer(rows * top_k * 4)
    d_w = native.DeviceBuffer(rows * top_k * 4)
    native.route_topk(d_l, d_b, rows, experts, top_k, normalize, scale, d_i, d_w)
    ids = d_i.download(np.int32, rows * top_k).reshape(rows, top_k)
    w = d_w.download(np.float32, rows * top_k).reshape(rows, top_k)
    for b in (d_l, d_b, d_i, d_w):
        b.close()
    return ids, w


@pytest.mark.parametrize("rows,experts,top_k", [
    (1, 64, 6), (1, 40, 6), (5, 64, 6), (8, 64, 8), (64, 64, 6), (200, 33, 4), (9, 96, 6)])
def test_route_topk_ties(device, rows, experts, top_k):
    print(f"[gpu] route_topk rows={rows} experts={experts} top_k={top_k}", flush=True)
    logits, bias = tied_logits(rows, experts, 100 + rows + experts)
    ids, w = run_device(logits, bias, top_k)
    e_ids, e_w = O.route(logits, bias, top_k, 1, 2.5)
    assert np.array_equal(ids, e_ids)
    np.testing.assert_allclose(w, e_w, rtol=2e-7, atol=0)


def test_route_topk_too_few_live(device):
    # only 3 experts can be taken: the remaining slots hold -1 and weight 0
    print("[gpu] route_topk with 3 live experts of 64", flush=True)
    logits = np.zeros((2, 64), np.float32)
    bias = np.full(64, -np.inf, np.float32)
    bias[[9, 40, 2]] = [0.5, 0.5, 0.25]
    logits[1, 40] = np.nan
    ids, w = run_device(logits, bias, 6)
    e_ids, e_w = O.route(logits, bias, 6, 1, 2.5)
    assert e_ids[0].tolist() == [9, 40, 2, -1, -1, -1]
    assert np.array_equal(ids, e_ids)
    np.testing.assert_allclose(w, e_w, rtol=2e-7, atol=0)
