#!/usr/bin/env python3
"""Benchmark of the MI355X Moonlight hot path (one GPU).

Metric: q8/q4 dequant-GEMV GB/s (% of HBM peak); Moonlight q8
decode tok/s.  A "step" is one dequant-GEMV launch over one batch of synthetic
input.  The headline workload is benchmark config 1: the q4 [11264 x 2048]
Moonlight dense-FFN projection, W ~ N(0, 0.02) rounded to bf16 and packed
with the container's per-row-scale int4 scheme, x ~ N(0, 1), batch 1.

`value` = algorithmic bytes per launch / average launch time (HIP events on the
library stream around K back-to-back launches replayed from one hipGraph),
rotating over enough weight copies (> 370 MB) that the 256 MB last-level cache
cannot serve them.  The other configs are reported under "extra".

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "q8/q4 dequant-GEMV GB/s (% HBM peak); Moonlight q8 decode tok/s, 1 GPU"


def gemv_bytes(fmt, out_width, in_width, rows):
    """Algorithmic HBM bytes of one GEMV launch: weights + scales + x + y."""
    wbytes = out_width * (in_width * 4 if fmt == 0 else in_width if fmt == 1
                          else (in_width + 1) // 2)
    scale = 0 if fmt == 0 else out_width * 4
    return wbytes + scale + rows * in_width * 4 + rows * out_width * 4


class GemvCase:
    """Synthetic resident inputs for one GEMV shape, replicated in HBM."""

    def __init__(self, native, fmt, out_width, in_width, rows, seed, min_bytes=400e6):
        self.native = native
        self.fmt, self.O, self.I, self.rows = fmt, out_width, in_width, rows
        wf = native.DeviceBuffer(out_width * in_width * 4)
        native.fill_normal(wf, out_width * in_width, seed, 0.0, 0.02, bf16=True)
        self.wbytes = out_width * (in_width if fmt == 1 else (in_width + 1) // 2
                                   if fmt == 2 else in_width * 4)
        first_w = native.DeviceBuffer(self.wbytes)
        first_s = native.DeviceBuffer(out_width * 4) if fmt else None
        if fmt == 0:
            native.load().mlk_memcpy_d2d(first_w.ptr, wf.ptr, self.wbytes)
        else:
            native.quantize(8 if fmt == 1 else 4, wf, out_width, in_width, first_w, first_s)
        wf.close()
        # >= 16 distinct copies and > min_bytes in total, so the last-level
        # cache (256 MB) cannot hold the rotation
        copies = max(16 if self.wbytes < 64e6 else 2, math.ceil(min_bytes / self.wbytes))
        self.w = [first_w]
        self.s = [first_s] if fmt else []
        for _ in range(copies - 1):
            w = native.DeviceBuffer(self.wbytes)
            native.load().mlk_memcpy_d2d(w.ptr, first_w.ptr, self.wbytes)
            self.w.append(w)
            if fmt:
                s = native.DeviceBuffer(out_width * 4)
                native.load().mlk_memcpy_d2d(s.ptr, first_s.ptr, out_width * 4)
                self.s.append(s)
        self.x = native.DeviceBuffer(rows * in_width * 4)
        native.fill_normal(self.x, rows * in_width, seed + 1, 0.0, 1.0)
        self.y = native.DeviceBuffer(rows * out_width * 4)
        native.synchronize()
        self.bytes = gemv_bytes(fmt, out_width, in_width, rows)

    def time(self, warmup, iters, use_graph=True):
        us = self.native.time_gemv(self.fmt, self.w, self.s, self.x, self.y, self.O, self.I,
                                   self.rows, warmup, iters, use_graph)
        return us, self.bytes / (us * 1e-6) / 1e9

    def time_median(self, windows=11, per_window=100):
        """Median (and spread) of the per-launch average over `windows`
        graph replays of `per_window` launches each (BASELINE.md section 5's
        median over >= 100 launches)."""
        us = sorted(self.native.time_gemv(self.fmt, self.w, self.s, self.x, self.y, self.O,
                                          self.I, self.rows, 2, per_window, True)
                    for _ in range(windows))
        return {"median_us": round(us[len(us) // 2], 3), "min_us": round(us[0], 3),
                "max_us": round(us[-1], 3), "launches": windows * per_window}

    def read_ceiling(self, warmup=5, iters=100):
        """Same-run ceiling of a GEMV of this shape: the fastest plain
        read-only stream of the same weight bytes, rotating over the same
        copies, over a few grid sizes (launch ramp and tail included)."""
        best = None
        scratch = self.native.DeviceBuffer(4096 * 4 * 4)
        for blocks in (256, 512, 1024, 2048, 4096):
            us = self.native.time_read(self.w, self.wbytes, blocks, scratch, warmup, iters)
            if best is None or us < best[0]:
                best = (us, blocks)
        scratch.close()
        return best

    def host_inputs(self):
        import numpy as np
        q = self.w[0].download(np.uint8 if self.fmt else np.float32)
        s = self.s[0].download(np.float32) if self.fmt else None
        x = self.x.download(np.float32).reshape(self.rows, self.I)
        return q, s, x

    def close(self):
        for b in self.w + self.s + [self.x, self.y]:
            b.close()


def moe_layer_bytes(unique, rows):
    """Algorithmic bytes of one q8 MoE decode layer:
    U routed experts x (gate + up + down + scales) + fused shared expert +
    f32 router and bias + the token rows in and out."""
    expert = 3 * 1408 * 2048 + 2 * 1408 * 4 + 2048 * 4
    shared = 3 * 2816 * 2048 + 2 * 2816 * 4 + 2048 * 4
    router = 64 * 2048 * 4 + 64 * 4
    return unique * expert + shared + router + rows * 2048 * 4 * 2


def attn_block_bytes(ctx, rows=1):
    """Algorithmic bytes of one q8 decode attention block at `ctx` cached
    keys: [q | kv_a] (3648 x 2048), kv_b (4096 x 512) and o_proj (2048 x 2048)
    with their row scales, the two RMSNorm weights, the latent + rope cache
    (ctx x 576 f32) and the token rows in and out."""
    rows_w = 3072 + 576 + 4096 + 2048
    weights = (3072 + 576) * 2048 + 4096 * 512 + 2048 * 2048 + rows_w * 4 + (2048 + 512) * 4
    return weights + ctx * 576 * 4 + rows * 2048 * 4 * 2


# Algorithmic bytes of one full q8 decode step: attention 13.8 MB x 27 layers,
# dense FFN 69.3 MB, MoE 69.9 MB x 26, f32 lm_head 1.342 GB, KV cache reads.
DECODE_STEP_BYTES = {4096: 3856274688, 16384: 4620686592}


def prefill_moe_ops(ids, rows, experts=64):
    """(algorithmic FLOP, int8 MFMA ops executed) of one MoE prefill layer with
    the given routes: routed 2*(3*1408*2048) FLOP per (token, expert), shared
    2*(3*2816*2048) per token, router 2*64*2048 per token; the MFMA path runs
    128-row tiles with three int8 activation limbs."""
    import numpy as np
    counts = np.bincount(np.asarray(ids).ravel(), minlength=experts)
    flop = counts.sum() * 2 * 3 * 1408 * 2048 + rows * (2 * 3 * 2816 * 2048 + 2 * 64 * 2048)
    padded = sum(-(-int(c) // 128) * 128 for c in counts if c)
    shared_pad = -(-rows // 128) * 128
    ops = 3 * 2 * (padded * 3 * 1408 * 2048 + shared_pad * 3 * 2816 * 2048)
    return int(flop), int(ops)


def prefill_moe(model, bits, extra, rows=2048):
    """Config 3: one MoE layer over 2048 tokens whose experts follow Zipf(1.1)
    (fixed per token), on the int8-MFMA grouped GEMM."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    from floyd_amd import session as S
    ids = oracle_lib.zipf_routes(rows, 64, 6, seed=2048)
    sess = S.Session(model, rows, rows)
    sess.fix_routes(ids)
    us, uniq = sess.time_moe(1, rows, seed=3, warmup=3, iters=20)
    sess.close()
    flop, ops = prefill_moe_ops(ids, rows)
    tflops = flop / (us * 1e-6) / 1e12
    extra[f"cfg3_moe_prefill_q{bits}_T{rows}"] = {
        "us": round(us, 1), "unique_experts": uniq, "algorithmic_flop": flop,
        "TFLOP/s": round(tflops, 1), "frac_of_fp16_dense_peak": round(tflops / 2500.0, 4),
        "int8_mfma_ops": ops, "int8_mfma_util": round(ops / (us * 1e-6) / 5.0e15, 4)}
    print(f"[bench] MoE prefill q{bits} T={rows}: {us:.1f} us, {tflops:.1f} TFLOP/s "
          f"(int8 MFMA busy {ops / (us * 1e-6) / 5.0e15:.2%})", file=sys.stderr, flush=True)


def sampler_timing(sess, logits, reps=50):
    """Wall time of one device token choice on the session's last logits
    (163,840 entries) against the CPU restatement of choose_token
    (moonlight_chat.c:96-131, glibc qsort, one thread) on the same logits."""
    out = {}
    for name, temperature, top_p in (("greedy", 0.0, 1.0), ("t1_topp0.9", 1.0, 0.9)):
        state = 12345
        for _ in range(3):
            sess.sample(temperature, top_p, state)
        t = []
        for _ in range(reps):
            t1 = time.perf_counter()
            _, state = sess.sample(temperature, top_p, state)
            t.append(time.perf_counter() - t1)
        out[name + "_us_wall"] = round(sorted(t)[len(t) // 2] * 1e6, 1)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    state, t = 12345, []
    for _ in range(5):
        t1 = time.perf_counter()
        _, state = O.choose_token(logits, 1.0, 0.9, state)
        t.append(time.perf_counter() - t1)
    out["cpu_t1_topp0.9_us"] = round(sorted(t)[len(t) // 2] * 1e6, 1)
    out["cpu_threads"] = 1
    print(f"[bench] sampler: greedy {out['greedy_us_wall']} us, top-p {out['t1_topp0.9_us_wall']}"
          f" us wall on the GPU; CPU choose_token {out['cpu_t1_topp0.9_us']} us",
          file=sys.stderr, flush=True)
    return out


def moonlight_extras(native, extra, decode_tokens):
    """Benchmark configs 2 and 4 on a synthetic Moonlight-16B-A3B q8 model built
    in HBM: one MoE layer at T = 1, 8, 64 and a full decode step at ctx 4096
    and 16384."""
    from floyd_amd import session as S
    t0 = time.perf_counter()
    model = S.Model.synthetic()
    extra["moonlight_model_build_s"] = round(time.perf_counter() - t0, 2)
    print(f"[bench] synthetic Moonlight q8 model in {extra['moonlight_model_build_s']} s",
          file=sys.stderr, flush=True)
    sess = S.Session(model, 128, 64)
    for rows in (1, 8, 64):
        # cold: the passes cycle through the 26 MoE layers, a fresh input per
        # pass (26 x 70 MB and more: the weights stream from HBM); warm, for
        # contrast: layer 1 on one input, its experts served from the 256 MB
        # last-level cache at T = 1
        us, uniq = sess.time_moe(-1, rows, seed=rows, warmup=26, iters=104)
        warm_us, _ = sess.time_moe(1, rows, seed=rows, warmup=5, iters=50)
        nbytes = int(round(moe_layer_bytes(uniq, rows)))
        gbs = nbytes / (us * 1e-6) / 1e9
        extra[f"cfg2_moe_decode_q8_T{rows}"] = {
            "us": round(us, 2), "unique_experts_mean": round(uniq, 2), "bytes": nbytes,
            "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "layers": "26-layer rotation, fresh input per pass", "warm_us_layer1": round(warm_us, 2)}
        print(f"[bench] MoE layer T={rows}: {us:.1f} us cold (26-layer rotation), U={uniq:.1f}, "
              f"{gbs:.0f} GB/s; {warm_us:.1f} us warm (one layer)", file=sys.stderr, flush=True)
    sess.close()
    prefill_moe(model, 8, extra)
    for ctx in (4096, 16384):
        sess = S.Session(model, ctx + 2 * decode_tokens + 8, 1)
        sess.fill_kv(ctx, seed=ctx)
        # one attention block, cold: cycling through the 27 layers' weights
        # and caches, a fresh input per pass (the cache row at ctx is
        # rewritten; the decodes below rewrite it again)
        us = sess.time_attention(-1, 1, ctx, seed=ctx, warmup=27, iters=108)
        nbytes = attn_block_bytes(ctx)
        gbs = nbytes / (us * 1e-6) / 1e9
        extra[f"attn_block_ctx{ctx}"] = {
            "us": round(us, 2), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "layers": "27-layer rotation, fresh input per pass"}
        print(f"[bench] attention block ctx {ctx}: {us:.1f} us cold, {gbs:.0f} GB/s",
              file=sys.stderr, flush=True)
        token = 1
        import numpy as np
        logits = np.empty(163840, np.float32)  # reused output buffer
        for _ in range(3):
            sess.decode(token, logits)
            token = int(logits.argmax())
        dev, wall = [], []
        for _ in range(decode_tokens):
            t1 = time.perf_counter()
            sess.decode(token, logits)
            wall.append(time.perf_counter() - t1)
            dev.append(sess.device_time_ms())
            token = int(logits.argmax())
        dev_ms = sorted(dev)[len(dev) // 2]
        wall_ms = sorted(wall)[len(wall) // 2] * 1e3
        nbytes = DECODE_STEP_BYTES[ctx]
        extra[f"cfg4_decode_q8_ctx{ctx}"] = {
            "tok_per_s": round(1e3 / wall_ms, 2), "ms_per_token_wall": round(wall_ms, 3),
            "ms_per_token_device": round(dev_ms, 3), "bytes": nbytes,
            "GB/s_device": round(nbytes / (dev_ms * 1e-3) / 1e9, 1),
            "frac_device": round(nbytes / (dev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "tokens": decode_tokens, "graph": sess.decode_graph()}
        print(f"[bench] decode ctx {ctx}: {wall_ms:.3f} ms/token wall "
              f"({1e3 / wall_ms:.1f} tok/s), device {dev_ms:.3f} ms",
              file=sys.stderr, flush=True)
        # the same steps ending in the device arg-max (greedy next token on
        # the GPU; only the token id crosses PCIe)
        dev, wall = [], []
        for _ in range(decode_tokens):
            t1 = time.perf_counter()
            token, _ = sess.decode_sample(token)
            wall.append(time.perf_counter() - t1)
            dev.append(sess.device_time_ms())
        dev_ms = sorted(dev)[len(dev) // 2]
        wall_ms = sorted(wall)[len(wall) // 2] * 1e3
        extra[f"cfg4_decode_q8_ctx{ctx}"]["device_greedy"] = {
            "tok_per_s": round(1e3 / wall_ms, 2), "ms_per_token_wall": round(wall_ms, 3),
            "ms_per_token_device": round(dev_ms, 3)}
        print(f"[bench] decode ctx {ctx} + device greedy: {wall_ms:.3f} ms/token wall "
              f"({1e3 / wall_ms:.1f} tok/s), device {dev_ms:.3f} ms",
              file=sys.stderr, flush=True)
        if ctx == 4096:
            extra["sampler_vocab163840"] = sampler_timing(sess, logits)
        sess.close()
    full_prefill(model, extra)
    model.close()
    model = S.Model.synthetic(expert_bits=4, dense_bits=4)
    prefill_moe(model, 4, extra)
    model.close()


def full_prefill(model, extra, rows=2048):
    """Full-model prefill of `rows` tokens (27 layers + lm_head of the last
    row), device time of the middle of three runs."""
    from floyd_amd import session as S
    sess = S.Session(model, rows + 16, rows)
    ids = [(7919 * i + 17) % 163840 for i in range(rows)]
    dev = []
    for _ in range(3):
        sess.reset()
        t1 = time.perf_counter()
        sess.prefill(ids)
        wall = time.perf_counter() - t1
        dev.append(sess.device_time_ms())
    dev_ms = sorted(dev)[1]
    extra[f"prefill_q8_T{rows}"] = {"ms_device": round(dev_ms, 2),
                                     "tok_per_s": round(rows / (dev_ms * 1e-3), 1),
                                     "ms_wall_last": round(wall * 1e3, 2)}
    print(f"[bench] prefill T={rows}: {dev_ms:.2f} ms device ({rows / (dev_ms * 1e-3):.0f} tok/s)",
          file=sys.stderr, flush=True)
    sess.close()


def moe_only(sizes=None):
    """Config 2 only: the MoE layer at T = 1, 8, 64, or at the row counts in
    `sizes` (profiler runs)."""
    from floyd_amd import session as S
    model = S.Model.synthetic()
    rows_list = sizes or (1, 8, 64)
    sess = S.Session(model, max(128, max(rows_list)), max(64, max(rows_list)))
    out = {}
    for rows in rows_list:
        us, uniq = sess.time_moe(-1, rows, seed=rows, warmup=26, iters=52)
        out[f"T{rows}"] = {"us": round(us, 2), "unique_experts_mean": round(uniq, 2)}
        print(f"[bench] MoE layer T={rows}: {us:.1f} us (26-layer rotation), U={uniq:.1f}",
              file=sys.stderr, flush=True)
    sess.close()
    model.close()
    print(json.dumps(out), flush=True)


def attn_only(sizes=None):
    """One decode attention block ([q | kv_a] GEMV, MLA chain, o_proj) at
    ctx 4096 and 16384, or at the contexts in `sizes`, stream launches
    (profiler runs and quick checks)."""
    from floyd_amd import session as S
    model = S.Model.synthetic()
    out = {}
    for ctx in sizes or (4096, 16384):
        sess = S.Session(model, ctx + 8, 1)
        sess.fill_kv(ctx, seed=ctx)
        us = sess.time_attention(-1, 1, ctx, warmup=27, iters=54)
        out[f"ctx{ctx}"] = {"us": round(us, 2)}
        print(f"[bench] attention block ctx={ctx}: {us:.1f} us (27-layer rotation)",
              file=sys.stderr, flush=True)
        sess.close()
    model.close()
    print(json.dumps(out), flush=True)


def prefill_only():
    """Config 3 (MoE prefill layer, q8 and q4) and the 2048-token full-model
    prefill, one JSON line (profiler runs and quick checks)."""
    from floyd_amd import session as S
    extra = {}
    model = S.Model.synthetic()
    prefill_moe(model, 8, extra)
    full_prefill(model, extra)
    model.close()
    model = S.Model.synthetic(expert_bits=4, dense_bits=4)
    prefill_moe(model, 4, extra)
    model.close()
    print(json.dumps(extra), flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/headline_traffic.json,
    each counter scaled by what it reads for a copy of known size), or None
    when that record is for another kernel instantiation."""
    path = os.path.join(ROOT, "profiles", "headline_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("kernel") != kernel:
        return None
    return rec.get("bytes_per_launch")


def cpu_baseline(case, budget_s=10.0):
    """The oracle's GEMV (restatement of the reference arithmetic) timed on the
    host cores on the same inputs, with the same parity check."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    from conftest import rel_l2
    q, s, x = case.host_inputs()
    threads = len(os.sched_getaffinity(0))
    case.native.gemv(case.fmt, case.w[0], case.s[0] if case.fmt else None, case.x, case.y,
                     case.O, case.I, case.rows)
    got = case.y.download(np.float32).reshape(case.rows, case.O)
    expect = oracle_lib.matmul(case.fmt, q, s, x, case.O, case.I, threads=threads)
    err = rel_l2(got, expect)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle_lib.matmul(case.fmt, q, s, x, case.O, case.I, threads=threads)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s or reps >= 20000:
            break
    per = elapsed / reps
    # the reference tests' serial semantics: one thread
    reps1, t0 = 0, time.perf_counter()
    while True:
        oracle_lib.matmul(case.fmt, q, s, x, case.O, case.I, threads=1)
        reps1 += 1
        elapsed1 = time.perf_counter() - t0
        if elapsed1 >= budget_s / 4 or reps1 >= 2000:
            break
    per1 = elapsed1 / reps1
    return {"value": round(case.bytes / per / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{reps} oracle GEMVs of the same workload, {elapsed:.1f} s "
                      f"(OpenMP over output rows, gcc -O3 -march=x86-64-v3)",
            "ms_per_step": round(per * 1e3, 4), "parity_rel_l2": err,
            "one_thread": {"value": round(case.bytes / per1 / 1e9, 3), "unit": "GB/s",
                           "ms_per_step": round(per1 * 1e3, 3),
                           "sample": f"{reps1} GEMVs, {elapsed1:.1f} s"}}


def decode_only(ctx, tokens):
    """Greedy decode steps of the synthetic q8 model at context ctx, one line
    per token (wall and device time): the workload of a decode profile.  Even
    steps copy the logits back and take the arg-max on the host; odd steps
    take it on the device and add one top-p draw (the sampler kernels)."""
    from floyd_amd import session as S
    model = S.Model.synthetic()
    sess = S.Session(model, ctx + tokens + 8, 1)
    sess.fill_kv(ctx, seed=ctx)
    token, state = 1, 12345
    for i in range(tokens):
        t1 = time.perf_counter()
        if i % 2 == 0:  # logits back to the host, greedy there
            logits = sess.decode(token)
            wall = (time.perf_counter() - t1) * 1e3
            token = int(logits.argmax())
        else:  # greedy on the device, then one top-p draw on the same logits
            token, _ = sess.decode_sample(token)
            wall = (time.perf_counter() - t1) * 1e3
            _, state = sess.sample(1.0, 0.9, state)
        print(f"[bench] decode {i}: {wall:.3f} ms wall, {sess.device_time_ms():.3f} ms device",
              file=sys.stderr, flush=True)
    sess.close()
    model.close()


def load_only(layers):
    """Model open from a container: a Moonlight-shaped q8 container with
    `layers` layers (random bytes: the loader never looks at values) is written
    under $TMPDIR, then moonlight_model_open is timed (page-cache preads into
    pinned staging, H2D copies, plan building) with one reader thread and with
    the default pool, alternating."""
    import shutil
    import tempfile
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import container_util as CU
    from floyd_amd import session as S
    cfg = dict(hidden_size=2048, layer_count=layers, head_count=16, expert_count=64,
               experts_per_token=6, dense_intermediate_size=11264, moe_intermediate_size=1408,
               first_dense_layer_count=1, q_lora_rank=0, kv_lora_rank=512, qk_nope_dim=128,
               qk_rope_dim=64, value_dim=128, shared_expert_count=2, normalize_topk=1,
               vocab_size=163840, rms_norm_epsilon=1e-5, rope_theta=50000.0,
               routed_scale=2.446)
    rng = np.random.default_rng(1)
    tensors = {}
    for name, kind, rows, cols in CU.tensor_specs(cfg):
        if kind == "n":
            tensors[name] = np.ones(cols, np.float32)
        elif kind == "b":
            tensors[name] = np.linspace(-0.1, 0.1, cols).astype(np.float32)
        elif kind == "f":
            tensors[name] = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        else:
            tensors[name] = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
            tensors[name + ".qs"] = np.full(rows, 1e-3, np.float32)
    root = tempfile.mkdtemp(prefix="mlh_load_")
    try:
        t0 = time.perf_counter()
        path = CU.write_container(os.path.join(root, "m"), cfg, tensors, shards=4)
        nbytes = sum(os.path.getsize(os.path.join(path, f)) for f in os.listdir(path))
        print(f"[bench] container: {len(tensors)} tensors, {nbytes / 1e9:.2f} GB written in "
              f"{time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
        n_tensors = len(tensors)
        del tensors
        result = {}
        for rnd in range(2):
            for threads in ("1", ""):
                os.environ["MLH_LOAD_THREADS"] = threads
                t1 = time.perf_counter()
                model = S.Model.open(path)
                dt = time.perf_counter() - t1
                model.close()
                key = "1 thread" if threads else "default pool"
                result.setdefault(key, []).append(dt)
                print(f"[bench] load ({key}, pass {rnd}): {dt:.3f} s, "
                      f"{nbytes / dt / 1e9:.2f} GB/s", file=sys.stderr, flush=True)
        os.environ.pop("MLH_LOAD_THREADS", None)
        print(json.dumps({"container_bytes": nbytes, "tensors": n_tensors,
                          "open_s": {k: round(min(v), 3) for k, v in result.items()},
                          "GB/s": {k: round(nbytes / min(v) / 1e9, 2)
                                   for k, v in result.items()}}), flush=True)
    finally:
        shutil.rmtree(root, ignore_errors=True)


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--cpu-budget", type=float, default=10.0)
    parser.add_argument("--no-moonlight", action="store_true",
                        help="skip the synthetic Moonlight MoE / decode measurements")
    parser.add_argument("--decode-tokens", type=int, default=20)
    parser.add_argument("--only-headline", action="store_true",
                        help="headline GEMV and the copy yardstick only (profiler runs)")
    parser.add_argument("--load-only", type=int, default=0, metavar="LAYERS",
                        help="only time moonlight_model_open on a Moonlight-shaped q8 "
                             "container of LAYERS layers written under $TMPDIR")
    parser.add_argument("--moe-only", action="store_true",
                        help="only config 2 (MoE decode layer at T = 1, 8, 64)")
    parser.add_argument("--prefill-only", action="store_true",
                        help="only config 3 (MoE prefill q8 / q4) and the 2048-token prefill")
    parser.add_argument("--attn-only", action="store_true",
                        help="only the decode attention block at ctx 4096 and 16384")
    parser.add_argument("--sizes", type=str, default="",
                        help="comma-separated MoE row counts (--moe-only) or contexts "
                             "(--attn-only) in place of the defaults")
    parser.add_argument("--gemv-only", type=str, default="", metavar="FMT,O,I,B",
                        help="only one GEMV shape (fmt 0 f32, 1 q8, 2 q4), graph launches "
                             "over rotated weight copies (profiler runs)")
    parser.add_argument("--decode-only", type=int, default=0, metavar="CTX",
                        help="only greedy decode steps of the synthetic model at context "
                             "CTX, printed per token (profiler runs)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the hot path is single-device "
              "(multi-GPU sharding is a design note, not a measured path)",
              file=sys.stderr)
        sys.exit(2)

    from floyd_amd import native
    device = native.init()
    print(f"[bench] device {device}", file=sys.stderr, flush=True)
    if args.load_only:
        load_only(args.load_only)
        return
    if args.decode_only:
        decode_only(args.decode_only, args.decode_tokens)
        return
    if args.gemv_only:
        fmt, o, i, rows = (int(v) for v in args.gemv_only.split(","))
        case = GemvCase(native, fmt, o, i, rows, seed=1000)
        us, gbs = case.time(args.warmup, args.steps)
        print(f"[bench] gemv fmt={fmt} {o}x{i} B={rows}: {us:.2f} us {gbs:.0f} GB/s "
              f"({case.bytes} bytes, {native.gemv_kernel_name(fmt, o, i, rows)})",
              file=sys.stderr, flush=True)
        print(json.dumps({"fmt": fmt, "O": o, "I": i, "rows": rows, "us": round(us, 3),
                          "GB/s": round(gbs, 1), "bytes": case.bytes}), flush=True)
        case.close()
        return
    if args.prefill_only:
        prefill_only()
        return
    sizes = [int(v) for v in args.sizes.split(",") if v]
    if args.moe_only:
        moe_only(sizes)
        return
    if args.attn_only:
        attn_only(sizes)
        return

    # headline: benchmark config 1, q4 [11264 x 2048], batch 1
    head = GemvCase(native, 2, 11264, 2048, 1, seed=101)
    head_us, head_gbs = head.time(args.warmup, args.steps, use_graph=True)
    head_us_stream, head_gbs_stream = head.time(args.warmup, args.steps, use_graph=False)
    print(f"[bench] q4 11264x2048 B=1: {head_us:.2f} us {head_gbs:.0f} GB/s (graph), "
          f"{head_us_stream:.2f} us (stream launches)", file=sys.stderr, flush=True)

    extra = {}
    extra_cases = {} if args.only_headline else {
            "cfg0_q8_11264x2048_b1": (1, 11264, 2048, 1),
            "cfg0_q8_11264x2048_b4": (1, 11264, 2048, 4),
            "cfg1_q4_2048x11264_b1": (2, 2048, 11264, 1),
            "q8_2048x11264_b1": (1, 2048, 11264, 1),
            "f32_lmhead_163840x2048_b1": (0, 163840, 2048, 1)}
    def with_ceiling(case, us):
        """The GEMV time against the same-run read-only ceiling of its weights."""
        c_us, c_blocks = case.read_ceiling()
        return {"read_ceiling_us": round(c_us, 3), "read_ceiling_blocks": c_blocks,
                "read_ceiling_GB/s": round(case.wbytes / (c_us * 1e-6) / 1e9, 1),
                "gemv_over_ceiling": round(c_us / us, 4)}

    head_median = head.time_median()
    head_ceiling = with_ceiling(head, head_us)
    print(f"[bench] headline median {head_median['median_us']} us; read ceiling "
          f"{head_ceiling['read_ceiling_us']} us ({head_ceiling['gemv_over_ceiling']:.0%} of it)",
          file=sys.stderr, flush=True)
    for index, (name, (fmt, o, i, rows)) in enumerate(extra_cases.items()):
        case = GemvCase(native, fmt, o, i, rows, seed=1000 + index)
        us, gbs = case.time(args.warmup, max(50, args.steps // 2))
        extra[name] = {"us": round(us, 3), "GB/s": round(gbs, 1),
                       "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": case.bytes}
        extra[name].update(case.time_median())
        extra[name].update(with_ceiling(case, us))
        print(f"[bench] {name}: {us:.2f} us {gbs:.0f} GB/s (median "
              f"{extra[name]['median_us']} us, read ceiling {extra[name]['read_ceiling_us']} us)",
              file=sys.stderr, flush=True)
        case.close()

    # copy yardstick: 256 MiB per launch, two buffer pairs
    nbytes = 256 << 20
    src = [native.DeviceBuffer(nbytes) for _ in range(2)]
    dst = [native.DeviceBuffer(nbytes) for _ in range(2)]
    copy_us = native.time_copy(src, dst, nbytes, 3, 20)
    extra["copy_256MiB"] = {"us": round(copy_us, 2),
                            "GB/s": round(2 * nbytes / (copy_us * 1e-6) / 1e9, 1)}
    for b in src + dst:
        b.close()

    if not args.no_moonlight and not args.only_headline:
        moonlight_extras(native, extra, args.decode_tokens)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(head, args.cpu_budget)
        print(f"[bench] cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads, "
              f"parity rel-L2 {cpu['parity_rel_l2']:.2e}", file=sys.stderr, flush=True)

    head_kernel = native.gemv_kernel_name(2, 11264, 2048, 1)
    line = {
        "metric": METRIC,
        "value": round(head_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head_us / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4 weights (u8 nibbles) x f32 activations, f32 accumulate",
        "data": "synthetic: W~N(0,0.02) bf16 -> per-row int4; x~N(0,1)",
        "config": {"workload": "config 1: q4 dequant-GEMV [11264 x 2048] "
                               "(Moonlight dense-FFN projection), batch 1",
                   "weight_copies": len(head.w), "timing": "hipGraph of K launches"},
        "roofline": {"bound": "hbm", "achieved": round(head_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(head_kernel), "algorithmic_bytes": head.bytes,
                     "kernel": head_kernel},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    line["extra"]["headline_stream_launch_us"] = round(head_us_stream, 3)
    line["extra"]["headline_median"] = head_median
    line["extra"]["headline_read_ceiling"] = head_ceiling
    head.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
