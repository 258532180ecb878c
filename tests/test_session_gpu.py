"""GPU parity of the session API (include/moonlight_hip.h) against the CPU
oracle, on containers in the exact convert_moonlight.py layout.

Each test restates one of the reference's Moonlight tests with the oracle in
place of the external fixtures they read (those fixtures are not in the
reference tree):
  test_primitives  tests/test_moonlight_metal_primitives.c:118-175
  test_mla         tests/test_moonlight_metal_mla.c:110-258
  test_moe         tests/test_moonlight_metal_moe.c:151-262
  test_runtime     tests/test_moonlight_metal_runtime.c:60-285
The reference's max-abs gates are kept, and rel-L2 <= 1e-3 (BASELINE.json
north_star) is checked as well.  Routing ids are compared bit-exactly with the
oracle's selection run on the device-produced router logits.
"""
import numpy as np
import pytest

import container_util as CU
import oracle_lib as O
from conftest import rel_l2
from floyd_amd import session as S

pytestmark = pytest.mark.gpu

FORMATS = [(8, 8), (4, 4), (4, 8)]


@pytest.fixture(scope="module", params=FORMATS, ids=lambda p: f"e{p[0]}d{p[1]}")
def tiny(request, tmp_path_factory, device):
    ebits, dbits = request.param
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=ebits, dbits=dbits, seed=1234 + ebits * 10 + dbits)
    path = CU.write_container(str(tmp_path_factory.mktemp(f"tiny_e{ebits}d{dbits}")), cfg,
                              tensors)
    print(f"[gpu] tiny container e{ebits} d{dbits}: {path}", flush=True)
    model = S.Model.open(path)
    yield cfg, tensors, model
    model.close()


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def test_model_info_and_lifecycle(tiny):
    cfg, tensors, model = tiny
    info = model.info()
    assert info["hidden_size"] == 256 and info["layer_count"] == 4
    assert info["vocab_size"] == 512 and info["expert_count"] == 64
    assert abs(info["routed_scale"] - 2.446) < 1e-6 and info["rope_theta"] == 50000.0
    assert info["resident_bytes"] == sum(a.nbytes for a in tensors.values())
    assert "gfx950" in model.device_name()
    sess = S.Session(model, 64, 32)
    before = sess.stats()
    assert before["buffer_allocations"] >= 5
    assert before["resident_bytes"] > info["resident_bytes"]
    assert before["cpu_fallbacks"] == 0 and sess.position() == 0
    sess.reset()
    after = sess.stats()
    assert after["buffer_allocations"] == before["buffer_allocations"]
    assert after["resident_bytes"] == before["resident_bytes"]
    sess.close()
    with pytest.raises(S.SessionError, match="invalid context or batch size"):
        S.Session(model, 16, 32)


PROFILE_LINE = (r"moonlight profile rows=(\d+) start=(\d+) layers=(\d+) graph=([01]) "
                r"encode=([0-9.]+) wait=([0-9.]+) gpu=([0-9.]+) ms")


def test_moonlight_profile_lines(tiny, capfd, monkeypatch):
    """MOONLIGHT_PROFILE (moonlight_metal.m:1899, 1932-1937, 1972-1979): with
    the variable set, every forward prints one timing line on stderr (a
    forward is one submission here); the first decode runs eagerly and the
    later ones replay the captured graph.  Without it nothing is printed."""
    import re
    cfg, tensors, model = tiny
    sess = S.Session(model, 64, 8)
    monkeypatch.setenv("MOONLIGHT_PROFILE", "1")
    capfd.readouterr()
    sess.prefill([1, 2, 3])
    for tok in (4, 5, 6):
        sess.decode(tok)
    lines = [l for l in capfd.readouterr().err.splitlines() if l.startswith("moonlight profile")]
    got = [re.fullmatch(PROFILE_LINE, l) for l in lines]
    assert len(got) == 4 and all(got), lines
    fields = [(int(m[1]), int(m[2]), int(m[3]), int(m[4])) for m in got]
    assert fields == [(3, 0, cfg["layer_count"], 0), (1, 3, cfg["layer_count"], 0),
                      (1, 4, cfg["layer_count"], 1), (1, 5, cfg["layer_count"], 1)]
    assert all(float(m[7]) > 0.0 for m in got)
    monkeypatch.delenv("MOONLIGHT_PROFILE")
    sess.decode(7)
    assert "moonlight profile" not in capfd.readouterr().err
    sess.close()


def test_primitives(tiny):
    cfg, tensors, model = tiny
    orc = CU.oracle_model(cfg, tensors, 64)
    sess = S.Session(model, 64, 32)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, cfg["vocab_size"], 9).astype(np.int32)
    emb = sess.test_embed(ids)
    assert np.array_equal(emb, tensors["model.embed_tokens.weight"][ids])
    x = rng.normal(0, 1, (9, 256)).astype(np.float32)
    norm = sess.test_rmsnorm(x, "model.norm.weight")
    expect = np.empty_like(x)
    O.lib().orc_rmsnorm(O.fptr(x), O.fptr(tensors["model.norm.weight"]), O.fptr(expect), 9, 256,
                        1e-5)
    assert max_abs(norm, expect) < 3e-5
    xq = rng.normal(0, 1, (9, 256)).astype(np.float32)
    q = sess.test_matmul("model.layers.0.self_attn.q_proj.weight", xq, 192)
    eq = np.empty((9, 192), np.float32)
    assert O.lib().orc_named_matmul(orc.handle, b"model.layers.0.self_attn.q_proj.weight",
                                    O.fptr(xq), 9, 256, 192, O.fptr(eq))
    assert max_abs(q, eq) < 3e-5 and rel_l2(q, eq) < 1e-5
    logits = sess.test_matmul("lm_head.weight", norm, 512)
    el = np.empty((9, 512), np.float32)
    assert O.lib().orc_named_matmul(orc.handle, b"lm_head.weight", O.fptr(norm), 9, 256, 512,
                                    O.fptr(el))
    assert max_abs(logits, el) < 3e-5
    st = sess.stats()
    assert st["command_buffers"] == 4 and st["cpu_fallbacks"] == 0
    # wrong shapes / names are refused like resolve_matrix refuses them
    assert sess.test_matmul("lm_head.weight", norm, 511) is None
    assert sess.test_matmul("no.such.weight", norm, 512) is None
    assert sess.test_rmsnorm(x[:, :255], "model.norm.weight") is None
    sess.close()
    orc.close()


def test_mla(tiny):
    cfg, tensors, model = tiny
    n = 12
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (n, 256)).astype(np.float32)
    orc = CU.oracle_model(cfg, tensors, 64)
    expect = np.empty_like(x)
    assert O.lib().orc_attention(orc.handle, 0, O.fptr(x), n, 0, O.fptr(expect))
    full = S.Session(model, 64, 32)
    got = full.test_attention(0, x, 0)
    assert got is not None
    assert max_abs(got, expect) < 3e-4 and rel_l2(got, expect) < 1e-4
    assert full.test_kv_length(0) == n and full.position() == n
    lat, rope = full.test_copy_kv(0, n)
    elat = np.empty((n, 64), np.float32)
    erope = np.empty((n, 16), np.float32)
    assert O.lib().orc_model_copy_kv(orc.handle, 0, O.fptr(elat), O.fptr(erope), n)
    assert max_abs(lat, elat) < 3e-5 and max_abs(rope, erope) < 3e-5
    # prefill(n-1) + decode(1) equals prefill(n) on the last row
    split = S.Session(model, 64, 32)
    assert split.test_attention(0, x[:n - 1], 0) is not None
    last = split.test_attention(0, x[n - 1:], n - 1)
    assert last is not None and max_abs(last[0], got[n - 1]) < 3e-4
    assert split.test_kv_length(0) == n
    assert split.test_attention(0, x[:1], n + 1) is None  # out-of-order position
    assert full.stats()["cpu_fallbacks"] == 0
    split.reset()
    assert split.test_kv_length(0) == 0 and split.position() == 0
    full.close()
    split.close()
    orc.close()


# rows = 1: routing inline in the gate/up launch; rows = 2: the routing
# launch and the grouped GEMV; rows = 4: the int8-MFMA grouped GEMM (from 3
# rows, when the shapes allow it; more rows in test_prefill_gpu.py)
@pytest.mark.parametrize("rows", [1, 2, 4])
def test_moe(tiny, rows):
    cfg, tensors, model = tiny
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (rows, 256)).astype(np.float32)
    sess = S.Session(model, 64, 32)
    got = sess.test_moe(1, x)
    assert got is not None
    # routing: bit-exact with the oracle's selection on the device logits
    bias = tensors["model.layers.1.mlp.gate.e_score_correction_bias"]
    ids_dev_logits, w_dev_logits = O.route(got["logits"], bias, 6, 1, 2.446)
    assert np.array_equal(got["ids"], ids_dev_logits)
    assert np.array_equal(got["weights"].view(np.uint32), w_dev_logits.view(np.uint32))
    # full layer against the oracle's own computation
    orc = CU.oracle_model(cfg, tensors, 64)
    e_ids = np.empty((rows, 6), np.int32)
    e_w = np.empty((rows, 6), np.float32)
    e_logits = np.empty((rows, 64), np.float32)
    e_routed, e_shared, e_out = (np.empty_like(x) for _ in range(3))
    assert O.lib().orc_moe_layer(orc.handle, 1, O.fptr(x), rows, O.iptr(e_ids), O.fptr(e_w),
                                 O.fptr(e_logits), O.fptr(e_routed), O.fptr(e_shared),
                                 O.fptr(e_out))
    assert max_abs(got["logits"], e_logits) < 3e-5
    for r in range(rows):
        assert set(got["ids"][r]) == set(e_ids[r])
        for k in range(6):
            j = list(e_ids[r]).index(got["ids"][r, k])
            assert abs(got["weights"][r, k] - e_w[r, j]) < 3e-6
    assert max_abs(got["routed"], e_routed) < 3e-4 and rel_l2(got["routed"], e_routed) < 1e-4
    assert max_abs(got["shared"], e_shared) < 3e-4 and rel_l2(got["shared"], e_shared) < 1e-4
    assert max_abs(got["out"], e_out) < 5e-4 and rel_l2(got["out"], e_out) < 1e-4
    assert sess.stats()["command_buffers"] == 2
    assert sess.test_moe(0, x) is None  # dense layer has no experts
    sess.close()
    orc.close()


def test_decode_nan_row_reports_route_error(tmp_path, device):
    """A token whose embedding row is NaN makes every router logit NaN, so no
    expert is taken in any MoE layer (NaN never compares greater, as in the
    reference's arg-max).  The one-row decode path (routing inside the first
    expert launch, down projections and combine in one launch) must report
    the route error (prepare_route_tables rejects such ids,
    moonlight_metal.m:545) without touching the empty expert slots' weights,
    and a reset session decodes normally afterwards."""
    print("[gpu] decode of a NaN embedding row (no expert taken)", flush=True)
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=8, dbits=8, seed=4321)
    tensors["model.embed_tokens.weight"][5] = np.nan
    model = S.Model.open(CU.write_container(str(tmp_path), cfg, tensors))
    sess = S.Session(model, 32, 4)
    sess.prefill([1, 2, 3])
    # the first MoE layer fails first (moonlight_metal.m:1944 names it)
    with pytest.raises(S.SessionError, match="route table failed at layer 1$"):
        sess.decode(5)
    sess.reset()
    sess.prefill([1, 2, 3])
    logits = sess.decode(4)
    assert np.all(np.isfinite(logits))
    sess.close()
    model.close()


def test_dense_mlp(tiny):
    cfg, tensors, model = tiny
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (7, 256)).astype(np.float32)
    sess = S.Session(model, 64, 32)
    got = sess.test_dense_mlp(0, x)
    orc = CU.oracle_model(cfg, tensors, 64)
    expect = np.empty_like(x)
    assert O.lib().orc_dense_mlp(orc.handle, 0, O.fptr(x), 7, O.fptr(expect))
    assert max_abs(got, expect) < 3e-4 and rel_l2(got, expect) < 1e-4
    assert sess.test_dense_mlp(1, x) is None
    sess.close()
    orc.close()


def oracle_forward(orc, cfg, ids, start):
    n = len(ids)
    layers = np.empty((cfg["layer_count"], n, cfg["hidden_size"]), np.float32)
    trace = np.full((cfg["layer_count"], n, cfg["experts_per_token"]), -1, np.int32)
    logits = np.empty(cfg["vocab_size"], np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    assert O.lib().orc_forward(orc.handle, O.iptr(ids), n, start, O.fptr(layers), O.iptr(trace),
                               O.fptr(logits))
    return layers, trace, logits


# n = 4: every matmul on the GEMV; n = 14: the MoE layers on the int8-limb
# MFMA GEMM (three limbs, 23 bits against each row's max).  Both hold the
# reference's gates (tests/test_moonlight_metal_runtime.c:205-213): last-row
# logits within max-abs 3e-4, no route mismatch; routes are compared in slot
# order, bit-exactly with the oracle's selection on the device's own router
# logits of every layer and with the oracle's own forward.
@pytest.mark.parametrize("n", [4, 14])
def test_runtime(tiny, n):
    cfg, tensors, model = tiny
    gate = 3e-4
    rng = np.random.default_rng(5)
    ids = rng.integers(0, cfg["vocab_size"], n).astype(np.int32)
    orc = CU.oracle_model(cfg, tensors, 64)
    e_layers, e_trace, e_logits = oracle_forward(orc, cfg, ids, 0)
    sess = S.Session(model, 64, 32)
    sess.trace_router(True)
    layers, logits = sess.prefill_layers(ids)
    for l in range(cfg["layer_count"]):
        print(f"[gpu] n={n} layer {l} max-abs {max_abs(layers[l], e_layers[l]):.2e} "
              f"rel-L2 {rel_l2(layers[l], e_layers[l]):.2e}", flush=True)
        assert max_abs(layers[l], e_layers[l]) < 2e-3, l
        assert rel_l2(layers[l], e_layers[l]) < 1e-3, l
    bias_name = "model.layers.{}.mlp.gate.e_score_correction_bias"
    for l in range(cfg["first_dense_layer_count"], cfg["layer_count"]):
        routes = sess.test_copy_routes(l, len(ids))
        dev_logits = sess.router_trace(l, len(ids))
        want, _ = O.route(dev_logits, tensors[bias_name.format(l)], 6, 1, 2.446)
        assert np.array_equal(routes, want), l
        assert np.array_equal(routes, e_trace[l]), l
    print(f"[gpu] n={n} logits max-abs {max_abs(logits, e_logits):.2e}", flush=True)
    assert max_abs(logits, e_logits) < gate and rel_l2(logits, e_logits) < 1e-3
    greedy = int(np.argmax(e_logits))
    assert int(np.argmax(logits)) == greedy
    assert sess.position() == len(ids)
    dec = sess.decode(greedy)
    _, _, e_dec = oracle_forward(orc, cfg, [greedy], len(ids))
    assert int(np.argmax(dec)) == int(np.argmax(e_dec))
    assert rel_l2(dec, e_dec) < 1e-3
    assert sess.position() == len(ids) + 1
    st = sess.stats()
    assert st["prefill_tokens"] == len(ids) and st["decode_tokens"] == 1
    assert st["cpu_fallbacks"] == 0
    # fast path from a reset session: one submission per forward
    sess.reset()
    logits2 = sess.prefill(ids)
    assert max_abs(logits2, e_logits) < gate
    dec2 = sess.decode(greedy)
    assert np.array_equal(np.argmax(dec2), np.argmax(e_dec))
    assert sess.stats()["command_buffers"] <= 2 * cfg["layer_count"] + 2
    # split prefill + append equals the full prefill
    sess.reset()
    half = len(ids) // 2
    sess.prefill(ids[:half])
    logits3 = sess.append(ids[half:])
    assert max_abs(logits3, e_logits) < gate and sess.position() == len(ids)
    # request validation (moonlight_metal.m:1988-2037)
    with pytest.raises(S.SessionError, match="requires an empty session"):
        sess.prefill(ids[:2])
    sess.reset()
    with pytest.raises(S.SessionError, match="invalid Moonlight append request"):
        sess.append(ids[:2])
    with pytest.raises(S.SessionError, match="invalid Moonlight prefill request"):
        sess.prefill(np.zeros(33, np.int32))
    sess.close()
    orc.close()


def test_decode_graph(tiny):
    """One-row decode steps replay a captured graph from the second decode on;
    its logits equal the stream-ordered launches bit for bit at every
    position, also after a reset, and match the oracle."""
    cfg, tensors, model = tiny
    rng = np.random.default_rng(11)
    ids = rng.integers(0, cfg["vocab_size"], 9).astype(np.int32)
    eager = S.Session(model, 64, 32)
    graph = S.Session(model, 64, 32)
    assert not eager.decode_graph(False)
    orc = CU.oracle_model(cfg, tensors, 64)
    for rnd in range(2):
        print(f"[gpu] decode graph vs eager, pass {rnd}", flush=True)
        eager.reset()
        graph.reset()
        prompt = ids[: 5 + 2 * rnd]
        eager.prefill(prompt)
        graph.prefill(prompt)
        token = int(ids[-1])
        seq = list(prompt)
        for step in range(6):
            a = eager.decode(token)
            b = graph.decode(token)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rnd, step)
            seq.append(token)
            token = int(np.argmax(a))
        assert graph.decode_graph() and not eager.decode_graph()
        assert graph.position() == len(seq)
        O.lib().orc_model_reset(orc.handle)
        _, _, e_last = oracle_forward(orc, cfg, seq, 0)
        assert rel_l2(b, e_last) < 1e-3
        assert int(np.argmax(b)) == int(np.argmax(e_last))
    st = graph.stats()
    assert st["cpu_fallbacks"] == 0 and st["decode_tokens"] == 6
    eager.close()
    graph.close()
    orc.close()


def test_sampler(tiny):
    """Device token choice (choose_token, moonlight_chat.c:96-131) against the
    oracle on the same logits: greedy always, sampled draws wherever the draw
    is not within 1e-6 of a cumulative boundary; the caller's xorshift state
    advances exactly as random_unit's; decode_sample equals decode followed by
    the host choice, across graph-replayed steps."""
    from sampler_util import nucleus_choice, xorshift_unit
    cfg, tensors, model = tiny
    rng = np.random.default_rng(21)
    ids = rng.integers(0, cfg["vocab_size"], 6).astype(np.int32)
    sess = S.Session(model, 64, 32)
    with pytest.raises(S.SessionError, match="invalid Moonlight sample request"):
        sess.sample()
    logits = sess.prefill(ids)
    tok, st = sess.sample(0.0, 0.9, 5)
    assert tok == int(np.argmax(logits)) and st == 5
    # sharpen the tiny model's flat logits so the nucleus varies with top_p
    compared = 0
    for temperature, top_p in ((1.0, 0.9), (0.05, 0.5), (0.02, 0.95), (0.01, 1.0)):
        state = 1000 + int(top_p * 100)
        for _ in range(12):
            u, nxt = xorshift_unit(state)
            want, margin, count = nucleus_choice(logits, temperature, top_p, u)
            e_tok, e_state = O.choose_token(logits, temperature, top_p, state)
            tok, state = sess.sample(temperature, top_p, state)
            assert state == e_state == nxt
            if margin > 1e-6:
                assert tok == e_tok == want, (temperature, top_p, u, count)
                compared += 1
    assert compared >= 40
    # decode_sample against decode + the oracle's choice, greedy and sampled
    other = S.Session(model, 64, 32)
    other.prefill(ids)
    t_a = t_b = int(ids[-1])
    s_a = s_b = 31337
    for step in range(5):
        temperature = 0.0 if step % 2 == 0 else 0.03
        lg = sess.decode(t_a)
        t_a, s_a = O.choose_token(lg, temperature, 0.9, s_a)
        t_b, s_b = other.decode_sample(t_b, temperature, 0.9, s_b)
        assert s_a == s_b
        u = xorshift_unit(s_a)[0]
        if temperature == 0.0 or nucleus_choice(lg, temperature, 0.9, u)[1] > 1e-6:
            assert t_a == t_b, step
        t_b = t_a
    assert other.position() == sess.position() == len(ids) + 5
    assert other.decode_graph()
    sess.close()
    other.close()


def test_decode_sample_commits_forward(tmp_path, device):
    """A decode whose token choice fails (non-finite logits under top-p)
    still commits the forward: the KV entry stays, the position advances, the
    step is counted, and the next decode continues from there (the reference's
    choose_token cannot fail after a decode, moonlight_chat.c:96-131)."""
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=8, dbits=8, seed=4242)
    tensors["lm_head.weight"][7, 3] = np.nan  # logit 7 is NaN for every token
    model = S.Model.open(CU.write_container(str(tmp_path / "nan_head"), cfg, tensors))
    sess = S.Session(model, 64, 8)
    ids = np.array([3, 14, 15, 92], np.int32)
    logits = sess.prefill(ids)
    assert np.isnan(logits[7]) and np.isfinite(np.delete(logits, 7)).all()
    with pytest.raises(S.SessionError, match="logits are not finite"):
        sess.decode_sample(5, 1.0, 0.9, 77)
    assert sess.position() == 5
    assert sess.stats()["decode_tokens"] == 1
    # greedy skips the NaN (NaN never wins the arg-max) and continues
    tok, state = sess.decode_sample(6, 0.0, 1.0, 77)
    assert state == 77 and sess.position() == 6
    nxt = sess.decode(tok)
    assert sess.position() == 7 and np.isnan(nxt[7])
    # the same three steps on a fresh session with plain decodes agree
    ref = S.Session(model, 64, 8)
    ref.prefill(ids)
    ref.decode(5)
    lg = ref.decode(6)
    assert int(np.nanargmax(np.where(np.isnan(lg), -np.inf, lg))) == tok
    assert np.array_equal(ref.decode(tok).view(np.uint32), nxt.view(np.uint32))
    assert sess.stats()["decode_tokens"] == 3
    ref.close()
    sess.close()
    model.close()


# o_proj widths (heads x value_dim) whose matrix-core kernel is not
# instantiated at hidden 256 (q8 512: 2 weight DMAs per wave; q4 1024: the
# same): the one-row decode must route through the separate router launch
# instead of asking o_proj for router partials it cannot write.
@pytest.mark.parametrize("bits,heads,vdim", [(8, 16, 32), (4, 16, 64)])
def test_decode_router_fallback_shapes(tmp_path, device, bits, heads, vdim):
    print(f"[gpu] one-row decode, q{bits} o_proj {256} x {heads * vdim}", flush=True)
    cfg = dict(CU.TINY, head_count=heads, value_dim=vdim)
    tensors = CU.build_tensors(cfg, ebits=bits, dbits=bits, seed=777 + bits)
    model = S.Model.open(CU.write_container(str(tmp_path / f"o{heads * vdim}"), cfg, tensors))
    orc = CU.oracle_model(cfg, tensors, 32)
    ids = np.array([11, 22, 33, 44], np.int32)
    sess = S.Session(model, 32, 8)
    sess.trace_router(True)
    sess.prefill(ids)
    _, _, _ = oracle_forward(orc, cfg, ids, 0)
    token = 55
    for step in range(3):  # eager, captured, replayed
        got = sess.decode(token)
        _, e_trace, e_logits = oracle_forward(orc, cfg, [token], len(ids) + step)
        bias_name = "model.layers.{}.mlp.gate.e_score_correction_bias"
        for l in range(cfg["first_dense_layer_count"], cfg["layer_count"]):
            routes = sess.test_copy_routes(l, 1)
            want, _ = O.route(sess.router_trace(l, 1), tensors[bias_name.format(l)], 6, 1, 2.446)
            assert np.array_equal(routes, want), (step, l)
            assert np.array_equal(routes, e_trace[l]), (step, l)
        assert max_abs(got, e_logits) < 3e-4 and rel_l2(got, e_logits) < 1e-3, step
        token = int(np.argmax(e_logits))
    sess.close()
    orc.close()
    model.close()


def test_batch_beyond_one_routing_call(tmp_path, device):
    """max_batch 3000 (moonlight_metal.m:965-967 allows any max_batch up to the
    context): one routing call covers 16384 (row, slot) positions, 2730 rows
    at top-6, so the MoE block runs in row chunks.  The MoE hook over 2800
    rows equals, bit for bit, the hook over its two chunks called alone; a
    2800-token prefill matches the oracle, with routes bit-exact against the
    selection on the device's own router logits in every row."""
    print("[gpu] 2800-row batch: MoE hook in chunks, prefill vs oracle", flush=True)
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=8, dbits=8, seed=2800)
    model = S.Model.open(CU.write_container(str(tmp_path / "big"), cfg, tensors))
    n, chunk = 2800, 16384 // 6
    sess = S.Session(model, 3072, 3000)
    x = O.fill_normal(n * 256, 2801).reshape(n, 256)
    whole = sess.test_moe(1, x)
    assert whole is not None
    for lo, hi in ((0, chunk), (chunk, n)):
        part = sess.test_moe(1, np.ascontiguousarray(x[lo:hi]))
        for k in ("ids", "weights", "logits", "routed", "out"):
            assert np.array_equal(whole[k][lo:hi].view(np.uint8), part[k].view(np.uint8)), (k, lo)
    rng = np.random.default_rng(2802)
    ids = rng.integers(0, cfg["vocab_size"], n).astype(np.int32)
    sess.reset()
    sess.trace_router(True)
    logits = sess.prefill(ids)
    orc = CU.oracle_model(cfg, tensors, 3072)
    _, e_trace, e_logits = oracle_forward(orc, cfg, ids, 0)
    err = rel_l2(logits, e_logits)
    bias_name = "model.layers.{}.mlp.gate.e_score_correction_bias"
    mismatched = 0
    for l in range(cfg["first_dense_layer_count"], cfg["layer_count"]):
        routes = sess.test_copy_routes(l, n)
        want, _ = O.route(sess.router_trace(l, n), tensors[bias_name.format(l)], 6, 1, 2.446)
        assert np.array_equal(routes, want), l
        mismatched += int((routes != e_trace[l]).any(axis=1).sum())
    print(f"[gpu] 2800-token prefill logits rel-L2 {err:.2e}, "
          f"{mismatched} route rows differ from the oracle's forward", flush=True)
    assert err < 1e-3 and int(np.argmax(logits)) == int(np.argmax(e_logits))
    # near-ties of the sigmoid scores may order a few rows differently after
    # fp32 rounding of the router inputs; none is expected at this size
    assert mismatched <= n * 3 // 200
    sess.close()
    orc.close()
    model.close()


@pytest.mark.parametrize("rows", [6, 80])
@pytest.mark.parametrize("factor", [2 ** 10, 2 ** 20])
def test_attention_operand_range(tmp_path, device, factor, rows):
    """The attention products take split-f16 operands (|v| < 65504).  With
    q_proj and the rope rows of kv_a scaled by 2^10 (row scales times an
    exact power of two) the queries, absorbed queries and rope keys reach the
    hundreds to thousands and attention still matches the oracle; at 2^20
    they leave the f16 range, and the attention hook and a prefill report
    it instead of returning inf / NaN.  6 rows take the absorbed form, 80
    the expanded heads (64 rows or more)."""
    print(f"[gpu] attention operands scaled by {factor}, {rows} rows", flush=True)
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=8, dbits=8, seed=31337)
    lora = cfg["kv_lora_rank"]
    for l in range(cfg["layer_count"]):
        p = f"model.layers.{l}.self_attn."
        tensors[p + "q_proj.weight.qs"] = tensors[p + "q_proj.weight.qs"] * np.float32(factor)
        kv = tensors[p + "kv_a_proj_with_mqa.weight.qs"].copy()
        kv[lora:] *= np.float32(factor)
        tensors[p + "kv_a_proj_with_mqa.weight.qs"] = kv
    model = S.Model.open(CU.write_container(str(tmp_path / f"range{factor}"), cfg, tensors))
    rng = np.random.default_rng(8)
    x = rng.normal(0, 1, (rows, 256)).astype(np.float32)
    sess = S.Session(model, 128, 96)
    got = sess.test_attention(0, x, 0)
    if factor == 2 ** 10:
        orc = CU.oracle_model(cfg, tensors, 128)
        expect = np.empty_like(x)
        assert O.lib().orc_attention(orc.handle, 0, O.fptr(x), rows, 0, O.fptr(expect))
        assert got is not None and np.isfinite(got).all()
        err = rel_l2(got, expect)
        print(f"[gpu] scaled attention rel-L2 {err:.2e}", flush=True)
        assert err < 1e-4
        orc.close()
    else:
        assert got is None
        sess.reset()
        ids = [1, 2, 3] if rows < 64 else (np.arange(rows) % cfg["vocab_size"]).tolist()
        with pytest.raises(S.SessionError, match="outside the f16 range"):
            sess.prefill(ids)
    sess.close()
    model.close()
