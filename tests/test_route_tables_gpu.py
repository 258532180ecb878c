"""GPU parity of the device route tables (prepare_route_tables,
moonlight_metal.m:525-559) against orc_route_tables (pinned by brute force in
test_oracle_math.py): the distinct experts in first-appearance order over
(row, slot), the count per expert, and each expert's (row, slot) entries in
order, bit for bit.  Every builder of the tables is covered:

  1 row     forward pass: routing inside the first expert launch
            (route_single_64)
  2 rows    forward pass: route_kernel (one workgroup, small_tables)
  4, 5, 8   forward pass on the MoE GEMM path: routing inside the GEMM prep
            launch (small_tables)
  64, 2048  forward pass: route_select_kernel + route_lists_kernel
  fixed     caller-given ids (moe_route_fixed semantics) through
            moonlight_test_moe at 4 and 64 rows
"""
import numpy as np
import pytest

import container_util as CU
import oracle_lib as O
from floyd_amd import session as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(tmp_path_factory, device):
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=8, dbits=8, seed=31337)
    path = CU.write_container(str(tmp_path_factory.mktemp("route_tables")), cfg, tensors)
    model = S.Model.open(path)
    yield cfg, tensors, model
    model.close()


def check_tables(sess, ids):
    rows, k = ids.shape
    t = sess.route_tables(rows)
    n, unique, counts, er, es = O.route_tables(ids, 64, rows)
    assert n > 0 and t["n_unique"] == n
    assert np.array_equal(t["unique"][:n], unique)
    assert np.array_equal(t["counts"], counts)
    # compact lists in first-appearance order, each expert's entries in
    # (row, slot) order as the reference's rows[e * max_batch + j]
    start = 0
    for e in unique:
        c = int(counts[e])
        assert t["offsets"][e] == start, e
        seg = slice(start, start + c)
        assert np.array_equal(t["list_rows"][seg], er[e * rows:e * rows + c]), e
        assert np.array_equal(t["list_slots"][seg], es[e * rows:e * rows + c]), e
        start += c
    assert start == rows * k
    q = np.arange(rows * k)
    pos = t["list_pos"]
    assert np.array_equal(t["list_rows"][pos], q // k)
    assert np.array_equal(t["list_slots"][pos], q % k)
    return n


@pytest.mark.parametrize("rows", [1, 2, 4, 5, 8, 64, 2048])
def test_forward_tables(tiny, rows):
    cfg, tensors, model = tiny
    print(f"[gpu] route tables of a {rows}-row forward", flush=True)
    ids = np.random.default_rng(rows).integers(0, cfg["vocab_size"], rows).astype(np.int32)
    sess = S.Session(model, max(rows, 64), rows)
    sess.prefill(ids)
    last = cfg["layer_count"] - 1
    routes = sess.test_copy_routes(last, rows)
    n = check_tables(sess, routes)
    print(f"[gpu] {n} distinct experts", flush=True)
    sess.close()


@pytest.mark.parametrize("rows", [4, 64])
def test_fixed_tables(tiny, rows):
    cfg, tensors, model = tiny
    rng = np.random.default_rng(100 + rows)
    # a few popular experts so that lists are long and interleaved
    ids = np.stack([rng.choice(12, 6, replace=False) * 5 % 64 for _ in range(rows)]).astype(
        np.int32)
    sess = S.Session(model, 64, 64)
    sess.fix_routes(ids)
    x = O.fill_normal(rows * 256, 900 + rows).reshape(rows, 256)
    got = sess.test_moe(2, x)
    assert got is not None and np.array_equal(got["ids"], ids)
    check_tables(sess, ids)
    sess.fix_routes(None)
    sess.close()
