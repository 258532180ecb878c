"""GPU parity of the prefill path: batches of >= 16 token rows (>= 5 in the
MoE layer) run every q8/q4 matmul on the int8-limb MFMA GEMM
(floyd_amd/csrc/qgemm.hip), in 32-row tiles where the tasks hold few rows and
128-row tiles otherwise, and route through the multi-workgroup routing kernels
when rows * top_k > 1024.

  test_tiny_moe_gemm         one MoE layer at 5, 40 and 200 rows, top-k routing,
                             three format mixes (tests/test_moonlight_metal_moe.c
                             semantics)
  test_tiny_prefill_gemm     a 40-token prefill through every GEMM path (q/kv_a,
                             o_proj, dense SwiGLU + down, experts) vs orc_forward
  test_tiny_prefill_expanded the attention on expanded per-head keys and
                             values (100 + 70 rows) vs orc_attention and
                             orc_forward
  test_moonlight_moe_fixed   the Moonlight MoE layer (config 3 shape) with Zipf
                             routes fixed per token (moe_route_fixed), q8 and q4,
                             T = 64 (32-row tiles), 512 and the full T = 2048

  test_gemm_outliers         dense projections (q_proj, kv_a, o_proj, the
                             11264-wide down projection) and the MoE layer at
                             Moonlight shape with outlier-heavy activations (a
                             few dims at 100-300x the row rms)
  test_moonlight_prefill_attention  prefill MLA at 16 heads / latent 512 over
                             511 and 512 rows (odd and even row pairs)
  test_moonlight_prefill_attention_chunks  the same in chunks of 200 + 80 + 2
                             rows (expanded heads at positions 0 and 200,
                             the absorbed form at 280)
  test_moonlight_dense_mlp   the 11264-wide dense SwiGLU block at T = 512

Tolerance: rel-L2 <= 1e-3 against the fp32 oracle
is the contract; the three-limb activation split (23 bits against each row's
max) keeps the measured error near fp32 rounding, so most gates are 1e-4.
"""
import numpy as np
import pytest

import container_util as CU
import oracle_lib as O
from conftest import rel_l2
from floyd_amd import session as S
from test_moonlight_scale_gpu import MOON, attention_names, moe_layer_names, oracle_with

pytestmark = pytest.mark.gpu

FORMATS = [(8, 8), (4, 4), (4, 8)]


@pytest.fixture(scope="module", params=FORMATS, ids=lambda p: f"e{p[0]}d{p[1]}")
def tiny(request, tmp_path_factory, device):
    ebits, dbits = request.param
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=ebits, dbits=dbits, seed=777 + ebits * 10 + dbits)
    path = CU.write_container(str(tmp_path_factory.mktemp(f"pf_e{ebits}d{dbits}")), cfg, tensors)
    model = S.Model.open(path)
    yield cfg, tensors, model
    model.close()


@pytest.mark.parametrize("rows", [5, 40, 200])
def test_tiny_moe_gemm(tiny, rows):
    cfg, tensors, model = tiny
    print(f"[gpu] tiny MoE GEMM rows={rows}", flush=True)
    x = O.fill_normal(rows * 256, 90 + rows).reshape(rows, 256)
    sess = S.Session(model, 256, 256)
    got = sess.test_moe(2, x)
    assert got is not None
    bias = tensors["model.layers.2.mlp.gate.e_score_correction_bias"]
    ids, w = O.route(got["logits"], bias, 6, 1, 2.446)
    assert np.array_equal(got["ids"], ids)
    assert np.array_equal(got["weights"].view(np.uint32), w.view(np.uint32))
    orc = CU.oracle_model(cfg, tensors, 8)
    e = {k: np.empty_like(x) for k in ("routed", "shared", "out")}
    e_ids = np.empty((rows, 6), np.int32)
    e_w = np.empty((rows, 6), np.float32)
    e_logits = np.empty((rows, 64), np.float32)
    assert O.lib().orc_moe_layer(orc.handle, 2, O.fptr(x), rows, O.iptr(e_ids), O.fptr(e_w),
                                 O.fptr(e_logits), O.fptr(e["routed"]), O.fptr(e["shared"]),
                                 O.fptr(e["out"]))
    assert np.array_equal(got["ids"], e_ids)
    errs = {k: rel_l2(got[k], e[k]) for k in e}
    print(f"[gpu] rel-L2 {errs}", flush=True)
    for k, v in errs.items():
        assert v < 1e-4, k
    sess.close()
    orc.close()


def test_tiny_prefill_gemm(tiny):
    cfg, tensors, model = tiny
    ids = np.random.default_rng(21).integers(0, cfg["vocab_size"], 40).astype(np.int32)
    print("[gpu] tiny 40-token prefill on the GEMM path", flush=True)
    orc = CU.oracle_model(cfg, tensors, 64)
    L = cfg["layer_count"]
    e_layers = np.empty((L, 40, 256), np.float32)
    e_trace = np.full((L, 40, 6), -1, np.int32)
    e_logits = np.empty(cfg["vocab_size"], np.float32)
    assert O.lib().orc_forward(orc.handle, O.iptr(ids), 40, 0, O.fptr(e_layers),
                               O.iptr(e_trace), O.fptr(e_logits))
    sess = S.Session(model, 64, 64)
    sess.trace_router(True)
    layers, logits = sess.prefill_layers(ids)
    # routes: in slot order, equal to the oracle's selection on the device's
    # router logits of the layer and to the oracle's own forward, with no
    # mismatched row (tests/test_moonlight_metal_runtime.c:205-213)
    for l in range(cfg["first_dense_layer_count"], L):
        routes = sess.test_copy_routes(l, 40)
        want, _ = O.route(sess.router_trace(l, 40),
                          tensors[f"model.layers.{l}.mlp.gate.e_score_correction_bias"], 6, 1,
                          2.446)
        assert np.array_equal(routes, want), l
        diff = [r for r in range(40) if list(routes[r]) != list(e_trace[l, r])]
        print(f"[gpu] layer {l} rows routed unlike the oracle's own top-k: {diff}", flush=True)
        assert not diff, (l, diff)
    for l in range(L):
        err = rel_l2(layers[l], e_layers[l])
        print(f"[gpu] layer {l} rel-L2 {err:.2e} max-abs "
              f"{np.max(np.abs(layers[l] - e_layers[l])):.2e}", flush=True)
        assert err < 1e-4 and np.max(np.abs(layers[l] - e_layers[l])) < 2e-3, l
    # the reference's logits gate (test_moonlight_metal_runtime.c:216)
    assert np.max(np.abs(logits - e_logits)) < 3e-4 and rel_l2(logits, e_logits) < 1e-4
    assert int(np.argmax(logits)) == int(np.argmax(e_logits))
    # decode after a GEMM prefill continues from the same caches
    greedy = int(np.argmax(e_logits))
    dec = sess.decode(greedy)
    e_dec = np.empty_like(e_logits)
    assert O.lib().orc_forward(orc.handle, O.iptr(np.array([greedy], np.int32)), 1, 40, None,
                               None, O.fptr(e_dec))
    assert rel_l2(dec, e_dec) < 1e-4 and np.max(np.abs(dec - e_dec)) < 3e-4
    sess.close()
    orc.close()


def test_tiny_prefill_expanded(tiny):
    """Prefill MLA on the expanded per-head keys and values (64 rows or more):
    a 100-row prefill and a 70-row append at position 100 (keys from both
    calls), the attention alone against orc_attention, then the whole
    forward against orc_forward with the reference's logits gate
    (tests/test_moonlight_metal_runtime.c:216).  The 40-row prefill above
    covers the absorbed form at the same shape."""
    cfg, tensors, model = tiny
    hidden = cfg["hidden_size"]
    print("[gpu] tiny expanded prefill: attention 100 + 70 rows, forward", flush=True)
    orc = CU.oracle_model(cfg, tensors, 256)
    sess = S.Session(model, 256, 128)
    rng = np.random.default_rng(31)
    pos = 0
    for rows in (100, 70):
        x = rng.standard_normal((rows, hidden)).astype(np.float32)
        got = sess.test_attention(1, x, pos)
        assert got is not None
        expect = np.empty_like(x)
        assert O.lib().orc_attention(orc.handle, 1, O.fptr(x), rows, pos, O.fptr(expect))
        err = rel_l2(got, expect)
        print(f"[gpu] attention rows {rows} at {pos}: rel-L2 {err:.2e}", flush=True)
        assert err < 1e-4
        pos += rows
    sess.close()
    orc.close()
    ids = rng.integers(0, cfg["vocab_size"], 170).astype(np.int32)
    orc = CU.oracle_model(cfg, tensors, 256)
    sess = S.Session(model, 256, 128)
    for lo, hi in ((0, 100), (100, 170)):
        e_logits = np.empty(cfg["vocab_size"], np.float32)
        assert O.lib().orc_forward(orc.handle, O.iptr(ids[lo:hi]), hi - lo, lo, None, None,
                                   O.fptr(e_logits))
        logits = sess.prefill(ids[lo:hi]) if lo == 0 else sess.append(ids[lo:hi])
        err = np.max(np.abs(logits - e_logits))
        print(f"[gpu] forward rows {lo}..{hi}: logits max-abs {err:.2e}", flush=True)
        assert err < 3e-4 and rel_l2(logits, e_logits) < 1e-4
        assert int(np.argmax(logits)) == int(np.argmax(e_logits))
    sess.close()
    orc.close()


@pytest.fixture(scope="module", params=[8, 4], ids=["q8", "q4"])
def moon(request, device):
    bits = request.param
    print(f"[gpu] building the synthetic Moonlight model, experts and dense at {bits} bits",
          flush=True)
    model = S.Model.synthetic(expert_bits=bits, dense_bits=bits)
    O.lib().orc_set_threads(16)
    yield model
    model.close()


@pytest.mark.parametrize("rows", [64, 512, 2048])
def test_moonlight_moe_fixed(moon, rows):
    print(f"[gpu] Moonlight MoE layer, Zipf routes, T={rows}", flush=True)
    ids = O.zipf_routes(rows, 64, 6, seed=1100 + rows)
    x = O.fill_normal(rows * 2048, 300 + rows).reshape(rows, 2048)
    sess = S.Session(moon, rows, rows)
    sess.fix_routes(ids)
    got = sess.test_moe(1, x)
    assert got is not None
    assert np.array_equal(got["ids"], ids)
    w = np.empty((rows, 6), np.float32)
    assert O.lib().orc_route_fixed(O.fptr(got["logits"]), rows, 64, 6, 1, 2.446, O.iptr(ids),
                                   O.fptr(w))
    assert np.array_equal(got["weights"].view(np.uint32), w.view(np.uint32))
    orc = oracle_with(moon, moe_layer_names(1), 8)
    expect = np.empty_like(x)
    e_w = np.empty((rows, 6), np.float32)
    assert O.lib().orc_moe_layer_fixed(orc.handle, 1, O.fptr(x), rows, O.iptr(ids),
                                       O.fptr(e_w), O.fptr(expect))
    err = rel_l2(got["out"], expect)
    print(f"[gpu] T={rows} out rel-L2 {err:.2e}", flush=True)
    assert err < 1e-4
    sess.fix_routes(None)
    sess.close()
    orc.close()


def outlier_rows(rows, width, seed, dims=4):
    """x ~ N(0, 1) with `dims` fixed feature columns set to +-100..300 in every
    row: a few dimensions at 100-300x the rms of the others, as the hidden
    states of DeepSeek-V3-family models carry (a single column cannot exceed
    sqrt(width) times the rms of its own row)."""
    x = O.fill_normal(rows * width, seed).reshape(rows, width)
    rng = np.random.default_rng(seed)
    cols = rng.choice(width, dims, replace=False)
    x[:, cols] = (rng.uniform(100, 300, (rows, dims)) *
                  rng.choice([-1.0, 1.0], (rows, dims))).astype(np.float32)
    return x


# (weight, input width, output width, rows): the dense prefill projections
# at Moonlight shape; the down projection's 11264-wide rows limit the batch
# to what the session's input buffer holds (rows * 11264 <= 512 * 2048)
DENSE = [("model.layers.3.self_attn.q_proj.weight", 2048, 3072, 512),
         ("model.layers.3.self_attn.kv_a_proj_with_mqa.weight", 2048, 576, 511),
         ("model.layers.3.self_attn.o_proj.weight", 2048, 2048, 512),
         ("model.layers.0.mlp.down_proj.weight", 11264, 2048, 90),
         # few rows: the weight-streaming tiles (16 and 32 token rows)
         ("model.layers.3.self_attn.q_proj.weight", 2048, 3072, 16),
         ("model.layers.3.self_attn.kv_a_proj_with_mqa.weight", 2048, 576, 27),
         ("model.layers.0.mlp.down_proj.weight", 11264, 2048, 31)]


@pytest.mark.parametrize("name,width,out,rows", DENSE,
                         ids=[f"{d[0].split('.')[-2]}-{d[3]}" for d in DENSE])
def test_gemm_outliers_dense(moon, name, width, out, rows):
    print(f"[gpu] dense GEMM {name} T={rows} with outlier columns", flush=True)
    sess = S.Session(moon, 512, 512)
    orc = oracle_with(moon, [name], 8)
    for kind, x in (("normal", O.fill_normal(rows * width, 500 + rows).reshape(rows, width)),
                    ("outliers", outlier_rows(rows, width, 600 + rows))):
        got = sess.test_matmul(name, x, out)
        assert got is not None
        expect = np.empty((rows, out), np.float32)
        assert O.lib().orc_named_matmul(orc.handle, name.encode(), O.fptr(x), rows, width, out,
                                        O.fptr(expect))
        err = rel_l2(got, expect)
        print(f"[gpu] {kind}: rel-L2 {err:.2e}", flush=True)
        assert err < 1e-4, kind
    sess.close()
    orc.close()


def test_gemm_outliers_moe(moon):
    rows = 512
    print(f"[gpu] Moonlight MoE layer T={rows} with outlier columns", flush=True)
    ids = O.zipf_routes(rows, 64, 6, seed=4100)
    x = outlier_rows(rows, 2048, 4200)
    sess = S.Session(moon, rows, rows)
    sess.fix_routes(ids)
    got = sess.test_moe(1, x)
    assert got is not None and np.array_equal(got["ids"], ids)
    orc = oracle_with(moon, moe_layer_names(1), 8)
    expect = np.empty_like(x)
    e_w = np.empty((rows, 6), np.float32)
    assert O.lib().orc_moe_layer_fixed(orc.handle, 1, O.fptr(x), rows, O.iptr(ids), O.fptr(e_w),
                                       O.fptr(expect))
    # the layer output includes no residual here: compare the routed + shared sum
    err = rel_l2(got["out"], expect)
    print(f"[gpu] out rel-L2 {err:.2e}", flush=True)
    assert err < 1e-4
    sess.fix_routes(None)
    sess.close()
    orc.close()


@pytest.mark.parametrize("rows", [511, 512])
def test_moonlight_prefill_attention(moon, rows):
    """Prefill MLA (flash form over 16-key tiles, two query rows per
    workgroup) at 16 heads / latent 512 / rope 64 against orc_attention
    (moonlight_kernels.metal:218-375 with key_count = pos + r + 1); then
    prefill(n - 1) + decode(1) equals prefill(n) on the last row
    (tests/test_moonlight_metal_mla.c:219-238)."""
    layer = 2
    print(f"[gpu] Moonlight prefill attention, {rows} rows", flush=True)
    x = O.fill_normal(rows * 2048, 700 + rows).reshape(rows, 2048)
    sess = S.Session(moon, 1024, 512)
    got = sess.test_attention(layer, x, 0)
    assert got is not None
    orc = oracle_with(moon, attention_names(layer), 1024)
    expect = np.empty_like(x)
    assert O.lib().orc_attention(orc.handle, layer, O.fptr(x), rows, 0, O.fptr(expect))
    err = rel_l2(got, expect)
    print(f"[gpu] rel-L2 {err:.2e} max-abs {np.max(np.abs(got - expect)):.2e}", flush=True)
    assert err < 1e-4
    lat, rope = sess.test_copy_kv(layer, rows)
    elat = np.empty((rows, 512), np.float32)
    erope = np.empty((rows, 64), np.float32)
    assert O.lib().orc_model_copy_kv(orc.handle, layer, O.fptr(elat), O.fptr(erope), rows)
    assert rel_l2(lat, elat) < 1e-5 and rel_l2(rope, erope) < 1e-5
    split = S.Session(moon, 1024, 512)
    assert split.test_attention(layer, x[:rows - 1], 0) is not None
    last = split.test_attention(layer, x[rows - 1:], rows - 1)
    assert last is not None
    assert np.max(np.abs(last[0] - got[rows - 1])) < 3e-4
    assert rel_l2(last[0], expect[rows - 1]) < 1e-4
    split.close()
    sess.close()
    orc.close()


def test_moonlight_prefill_attention_chunks(moon):
    """Prefill MLA in chunks at 16 heads / latent 512 / rope 64: 200 rows at
    position 0 and 80 rows at position 200 (both on the expanded heads, the
    second expanding the first chunk's keys too), then 2 rows at 280 (the
    absorbed form), each against orc_attention continuing the same cache
    (moonlight_kernels.metal:218-375 with key_count = pos + r + 1)."""
    layer = 1
    print("[gpu] Moonlight prefill attention in chunks 200 + 80 + 2", flush=True)
    x = O.fill_normal(282 * 2048, 909).reshape(282, 2048)
    sess = S.Session(moon, 512, 256)
    orc = oracle_with(moon, attention_names(layer), 512)
    pos = 0
    for rows in (200, 80, 2):
        xs = np.ascontiguousarray(x[pos:pos + rows])
        got = sess.test_attention(layer, xs, pos)
        assert got is not None
        expect = np.empty_like(xs)
        assert O.lib().orc_attention(orc.handle, layer, O.fptr(xs), rows, pos, O.fptr(expect))
        err = rel_l2(got, expect)
        print(f"[gpu] {rows} rows at {pos}: rel-L2 {err:.2e} "
              f"max-abs {np.max(np.abs(got - expect)):.2e}", flush=True)
        assert err < 1e-4
        pos += rows
    sess.close()
    orc.close()


def test_moonlight_dense_mlp(moon):
    rows = 512
    print(f"[gpu] Moonlight dense SwiGLU block T={rows}", flush=True)
    names = [f"model.layers.0.mlp.{m}_proj.weight" for m in ("gate", "up", "down")]
    x = O.fill_normal(rows * 2048, 800).reshape(rows, 2048)
    sess = S.Session(moon, 512, 512)
    got = sess.test_dense_mlp(0, x)
    assert got is not None
    orc = oracle_with(moon, names, 8)
    expect = np.empty_like(x)
    assert O.lib().orc_dense_mlp(orc.handle, 0, O.fptr(x), rows, O.fptr(expect))
    err = rel_l2(got, expect)
    print(f"[gpu] rel-L2 {err:.2e}", flush=True)
    assert err < 1e-4
    sess.close()
    orc.close()
