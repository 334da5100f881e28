"""Benchmark of the MI355X W4A8 engine on the Llama-3.2-1B decode GEMV chain.

    python bench.py [--gpus 1] [--steps 400] [--warmup 20] [--no-cpu] [--no-gemv]
                    [--no-caller] [--chain-only]

One step = one token's 65 W4A8 GEMVs (16 x q|k|v 3072x2048, o 2048x2048,
gate|up 16384x2048, down 2048x8192, then the LM head 128256x2048), each
preceded by the Q8_0 quantization of a float32 activation, in order: matrix
j+1 starts after matrix j's output is complete, as in a decode. The step is
a chain plan (w4a8_chain_plan_*: the 65 launches of the fused quantize + GEMV
kernel as raw AQL dispatches on the library's own queue, no cache fences
between them), launched for all timed steps at once and waited for; the same
chain through w4a8_chain_gemv, captured into a HIP graph and replayed, is the
chain_graph line. Weights (695,107,584 bytes of
Q4_0) are resident in HBM; the chain alone is larger than the 256 MB Infinity
Cache, so every step streams from HBM.

The chain runs on configuration 3's seeded inputs (weights default_rng(1000 +
j), activations default_rng(2000 + j)). The outputs are poisoned after the
warm-up, and after the timed replays every byte of all 65 outputs is compared
(SHA-256) with the oracle's digests in tests/golden/configs.json; the line
says "verified": true only when they all match. The GEMM sweep (configuration
4) and the 24-token prefill are checked the same way.

Prints one JSON line. Besides the chain (value), it reports:
  roofline     the chain's kernel (the fused quantize + GEMV, 65 launches per
               step): average algorithmic bytes per launch / average launch
               duration, both over the timed region (the host clock around the
               plan's launch and wait, dispatch boundaries included); beside
               it, kernel_durations: the same bytes over the dispatches' own
               spans, stamped inside the kernels by a timed launch of the same
               plan in the same run (w4a8_chain_plan_launch_timed: first wave
               start to last wave end of each dispatch, on the device's
               constant-rate clock), per shape and summed per step
  chain_graph  the chain through w4a8_chain_gemv in a HIP graph (HIP events
               on the launch stream around the replays), verified the same way
  chain_one_launch  the chain as one cooperative launch per step
               (W4A8_CHAIN_ONE_LAUNCH), verified the same way
  batch        the same 65 GEMVs per step in one w4a8_gemv_batch launch (no
               order inside a step)
  gemv         microseconds per GEMV at every shape, weights rotated past the
               Infinity Cache, launched back to back from a HIP graph
  gemm         the M > 1 sweep (M = 1 .. 64) at gate|up and down
  lm_head_argmax  the LM head with its greedy pick fused, and the sampler's
               top-40 candidates of the same logits (w4a8_topk)
  producers    rmsnorm / silu*up fused into the GEMV (staging or epilogue)
               against the standalone producer then the GEMV, and the same
               GEMV with no producer
  chain_fused_producers  the chain with those producers and the argmax
  prefill      24- and 64-token prompts through the 65 matrices (M > 1 GEMM)
  caller       the reference's decode-side caller (engine_t of
               board/tp/tp_llama.cpp, rebuilt against the reference driver
               headers: llm-kv260_amd/caller/engine_caller) on both engines:
               host-visible ms per token and us per call, split into the
               host quantize, the clean / invalidate copies and start + wait
  calls        what one call costs (llm-kv260_amd/caller/call_costs), column
               for column against the reference's per-call table: the
               synchronous gemv_dev_run, the device-side time per call, the
               standalone Q8_0 quantize, the clean / invalidate copies
  cpu_baseline the NumPy restatement of the contract on one core, and the
               C restatement on all cores, over one decode step
All launches come from C through the library's ABI; Python only sets them up.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llm-kv260_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
ROTATE_BYTES = 600 << 20       # > 2 x the 256 MB Infinity Cache


PMC_SUMMARY = os.path.join("profiles", "gemv_pmc_traffic_llama1b_decode.txt")


def pmc_traffic():
    """HBM bytes per launch from the committed rocprofv3 PMC summary (FETCH_SIZE +
    WRITE_SIZE, scaled by a plain copy of known size), or None when absent."""
    try:
        with open(os.path.join(ROOT, PMC_SUMMARY)) as f:
            for line in f:
                if line.startswith("JSON "):
                    return json.loads(line[5:])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class CStep(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("k", ctypes.c_int)]


def device_weights(torch, kv, rows, k, seed):
    """Q4_0 blocks of an N(0, 0.02) fp32 matrix drawn with the device RNG and
    quantized by the engine's own Q4_0 kernel (timing-only shapes)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn((rows, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    blocks = kv.quantize_q4_0(w)
    del w
    return blocks


FIXTURES = os.path.join(ROOT, "tests", "golden", "configs.json")


def fixtures():
    with open(FIXTURES) as f:
        return json.load(f)


def sha(a) -> str:
    import hashlib
    import numpy as np
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def host_weights(cf, m):
    """fp32 weights of one configuration matrix, drawn on the host from its seed."""
    import numpy as np
    w = np.empty((m.rows, m.k), np.float32)
    for r0, part in cf.weight_chunks(m):
        w[r0:r0 + part.shape[0]] = part
    return w


def seeded_blocks(torch, kv, cf, matrices):
    """Q4_0 blocks of the configuration matrices' seeded weights, drawn on the
    host (numpy releases the GIL, so eight threads draw at once) and quantized
    on the GPU by the engine's Q4_0 kernel."""
    from concurrent.futures import ThreadPoolExecutor
    out = []
    with ThreadPoolExecutor(8) as pool:
        for i, w in enumerate(pool.map(lambda m: host_weights(cf, m), matrices)):
            out.append(kv.quantize_q4_0(torch.from_numpy(w).cuda()))
            del w
            if i % 16 == 15:
                log(f"seeded weights: {i + 1}/{len(matrices)} matrices")
    torch.cuda.synchronize()
    return out


def verify(pairs) -> dict:
    """pairs: (name, device tensor, expected sha256). Every byte of every output."""
    bad = [name for name, t, want in pairs if sha(t.cpu().numpy()) != want]
    return {"ok": not bad, "outputs": len(pairs), "mismatched": bad[:8]}


def build_chain(torch, kv, cf):
    """Config 3: the 65 matrices' seeded weights and activations, whose outputs
    tests/golden/configs.json holds the oracle's digests of."""
    chain = cf.decode_chain()
    recs = fixtures()["config3"]
    mats = seeded_blocks(torch, kv, cf, chain)
    weights_ok = all(sha(b.cpu().numpy()) == r["q4_0"] for b, r in zip(mats, recs))
    xs = [torch.from_numpy(cf.activation(m)).cuda() for m in chain]
    ys = [torch.empty(m.rows, dtype=torch.float32, device="cuda") for m in chain]
    steps = (CStep * len(chain))(*[CStep(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), m.rows, m.k)
                                   for i, m in enumerate(chain)])
    torch.cuda.synchronize()
    return chain, mats, xs, ys, steps, recs, weights_ok


def poison(ts):
    for t in ts:
        t.fill_(float("nan"))


def graph_of(torch, stream, calls):
    """Capture calls (each takes a hipStream_t) into a HIP graph on `stream`."""
    with torch.cuda.stream(stream):
        for c in calls:                       # eager once: kernel attributes are set outside capture
            c(stream.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        st = torch.cuda.current_stream().cuda_stream
        for c in calls:
            c(st)
    return g


def time_replays(torch, stream, g, n, warmup, before=None):
    """ms per replay over exactly n replays, synchronized on both sides.
    before(): run after the warm-up, outside the timed region (e.g. poison the
    outputs so that what is verified afterwards was written by the timed replays)."""
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
    torch.cuda.synchronize()
    if before is not None:
        before()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(n):
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n, time.perf_counter() - t0


def time_gemv(torch, kv, cf, m, stream):
    """us per GEMV (engine-layout x) at one shape: back-to-back launches from a HIP
    graph over rotating weight copies (>= 600 MB; 3 x 148 MB for the LM head)."""
    L = kv.lib()
    base = device_weights(torch, kv, m.rows, m.k, 7)
    copies = 3 if m.weight_bytes > (100 << 20) else max(3, -(-ROTATE_BYTES // m.weight_bytes))
    mats = [base] + [base.clone() for _ in range(copies - 1)]
    x = kv.quantize_q8_0_engine(torch.from_numpy(cf.activation(m)).cuda())
    y = torch.empty(m.rows, dtype=torch.float32, device="cuda")
    launches = max(copies, 30)
    calls = [(lambda w: (lambda s: kv.check("w4a8_gemv", L.w4a8_gemv(w.data_ptr(), x.data_ptr(), y.data_ptr(),
                                                                    m.rows, m.k, s))))(mats[i % copies])
             for i in range(launches)]
    g = graph_of(torch, stream, calls)
    ms, _ = time_replays(torch, stream, g, 10, 2)
    us = ms * 1e3 / launches
    del g, mats, base
    return {"shape": f"{m.rows}x{m.k}", "us": round(us, 3), "gbps": round(m.algorithmic_bytes / us / 1e3, 1),
            "weight_copies": copies, "rotated_mb": round(copies * m.weight_bytes / 2**20, 1)}


def time_lm_argmax(torch, kv, cf, stream):
    """us per LM-head GEMV with the greedy argmax fused (w4a8_gemv_f32_argmax),
    fp32 activation, three rotating weight copies as for the plain LM head."""
    L = kv.lib()
    m = cf.LM_HEAD
    base = device_weights(torch, kv, m.rows, m.k, 7)
    mats = [base] + [base.clone() for _ in range(2)]
    x = torch.from_numpy(cf.activation(m)).cuda()
    y = torch.empty(m.rows, dtype=torch.float32, device="cuda")
    best = torch.empty(1, dtype=torch.int32, device="cuda")
    ws = kv.argmax_workspace()
    nbytes = ws.numel()
    launches = 30
    calls = [(lambda w: (lambda s: kv.check("w4a8_gemv_f32_argmax", L.w4a8_gemv_f32_argmax(
        w.data_ptr(), x.data_ptr(), y.data_ptr(), m.rows, m.k, best.data_ptr(), ws.data_ptr(), nbytes, s))))(
        mats[i % 3]) for i in range(launches)]
    g = graph_of(torch, stream, calls)
    ms, _ = time_replays(torch, stream, g, 10, 2)
    us = ms * 1e3 / launches
    del g
    # The sampler's candidates over the same logits (w4a8_topk, two launches).
    k = 40
    vals = torch.empty(k, dtype=torch.float32, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    tws = torch.empty(L.w4a8_topk_workspace_bytes(m.rows), dtype=torch.uint8, device="cuda")
    g = graph_of(torch, stream, [lambda s: kv.check("w4a8_topk", L.w4a8_topk(
        y.data_ptr(), m.rows, k, vals.data_ptr(), idx.data_ptr(), tws.data_ptr(), tws.numel(), s))] * launches)
    ms_k, _ = time_replays(torch, stream, g, 10, 2)
    del g, mats, base
    return {"shape": f"{m.rows}x{m.k}", "us": round(us, 3), "gbps": round(m.algorithmic_bytes / us / 1e3, 1),
            "argmax": int(best.cpu()[0]), "weight_copies": 3,
            "topk": {"k": k, "us": round(ms_k * 1e3 / launches, 3), "first": int(idx.cpu()[0]),
                     "launches": 2}}


def time_producers(torch, kv, cf, stream):
    """us per GEMV with its producer fused (rmsnorm in the staging before q|k|v,
    gate|up and the LM head; silu(gate) * up in down's staging, or as gate|up's
    epilogue), next to the same work as two launches (standalone producer +
    engine-layout GEMV) where one gives the same output, and the same GEMV on
    an fp32 x with no producer; weights rotated as for the per-shape GEMVs."""
    L = kv.lib()
    out = {}
    ws = kv.argmax_workspace()
    best = torch.empty(1, dtype=torch.int32, device="cuda")
    cases = (("qkv_rmsnorm", cf.LAYER_SHAPES[0], "rms"), ("gate_up_rmsnorm", cf.LAYER_SHAPES[2], "rms"),
             ("gate_up_rmsnorm_silu_epilogue", cf.LAYER_SHAPES[2], "pair"),
             ("down_silu_mul", cf.LAYER_SHAPES[3], "silu"), ("lm_head_rmsnorm_argmax", cf.LM_HEAD, "rms_argmax"))
    for name, m, kind in cases:
        base = device_weights(torch, kv, m.rows, m.k, 9)
        copies = 3 if m.weight_bytes > (100 << 20) else max(3, -(-ROTATE_BYTES // m.weight_bytes))
        mats = [base] + [base.clone() for _ in range(copies - 1)]
        g = torch.Generator(device="cuda")
        g.manual_seed(5)
        xin = torch.randn(2 * m.k if kind == "silu" else m.k, generator=g, device="cuda")
        norm = torch.randn(m.k, generator=g, device="cuda")
        xe = torch.empty(m.k + m.k // 8, dtype=torch.uint8, device="cuda")
        y = torch.empty(m.rows, dtype=torch.float32, device="cuda")
        launches = max(copies, 30)

        def fused(w, s):
            if kind == "pair":
                return L.w4a8_gemv_gate_up_silu(w.data_ptr(), xin.data_ptr(), norm.data_ptr(), 1e-5, y.data_ptr(),
                                                m.rows, m.k, s)
            if kind == "silu":
                return L.w4a8_gemv_silu_mul(w.data_ptr(), xin.data_ptr(), y.data_ptr(), m.rows, m.k, s)
            if kind == "rms":
                return L.w4a8_gemv_rmsnorm(w.data_ptr(), xin.data_ptr(), norm.data_ptr(), 1e-5, y.data_ptr(),
                                           m.rows, m.k, s)
            return L.w4a8_gemv_rmsnorm_argmax(w.data_ptr(), xin.data_ptr(), norm.data_ptr(), 1e-5, y.data_ptr(),
                                              m.rows, m.k, best.data_ptr(), ws.data_ptr(), ws.numel(), s)

        def split(w, s):
            st = (L.w4a8_silu_mul_q8_0(xin.data_ptr(), xe.data_ptr(), m.k, 1, s) if kind == "silu" else
                  L.w4a8_rmsnorm_q8_0(xin.data_ptr(), norm.data_ptr(), 1e-5, xe.data_ptr(), m.k, 1, s))
            return st or L.w4a8_gemv(w.data_ptr(), xe.data_ptr(), y.data_ptr(), m.rows, m.k, s)

        def plain(w, s):
            # The same GEMV on an fp32 x with no producer (fused quantize only).
            return L.w4a8_gemv_f32(w.data_ptr(), xin.data_ptr(), y.data_ptr(), m.rows, m.k, s)

        r = {"shape": f"{m.rows}x{m.k}"}
        # gate|up with the silu epilogue has no two-launch form of the same output.
        forms = (("fused_us", fused), ("plain_f32_us", plain)) if kind == "pair" else \
            (("fused_us", fused), ("two_launches_us", split), ("plain_f32_us", plain))
        for label, fn in forms:
            calls = [(lambda w: (lambda st: kv.check(name, fn(w, st))))(mats[i % copies]) for i in range(launches)]
            gr = graph_of(torch, stream, calls)
            ms, _ = time_replays(torch, stream, gr, 10, 2)
            r[label] = round(ms * 1e3 / launches, 3)
            del gr
        out[name] = r
        del mats, base
        torch.cuda.empty_cache()
    return out


def time_fused_chain(torch, kv, cf, chain, mats, ys, stream, steps, warmup, act="q8", plan=True):
    """The decode step with its producers fused and its one in-step data
    dependency kept: per layer q|k|v = W rmsnorm(x), o = W x, gate|up =
    W rmsnorm(x), down = W (silu(gate) * up) of gate|up's own output; the LM
    head = W rmsnorm(x) with its greedy pick. The rmsnorm inputs (the residual
    stream) and o's input (the attention output) are seeded vectors: attention
    and the residual adds are not part of the engine. act: "q8", gate|up
    computes silu(gate) * up and quantizes it in its epilogue
    (w4a8_gemv_gate_up_silu_q8_0) and down reads that engine-layout x
    (w4a8_gemv); "f32", gate|up stores the fp32 act (w4a8_gemv_gate_up_silu)
    and down quantizes it (w4a8_gemv_f32); "down", down computes silu in its
    own staging (w4a8_gemv_silu_mul). plan: also as a chain plan, every output
    checked against the graph's."""
    L = kv.lib()
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    k = cf.LAYER_SHAPES[0].k
    resid = torch.randn(k, generator=g, device="cuda")
    attn = torch.randn(k, generator=g, device="cuda")
    norm = torch.randn(k, generator=g, device="cuda")
    ws = kv.argmax_workspace()
    best = torch.empty(1, dtype=torch.int32, device="cuda")
    role_of = lambda i: "lm" if i == len(chain) - 1 else ("qkv", "o", "gate_up", "down")[i % 4]
    # q8: each layer's act in the engine layout, written by gate|up, read by down
    acts = {i: torch.empty(kv.engine_x_bytes(m.rows // 2), dtype=torch.uint8, device="cuda")
            for i, m in enumerate(chain) if act == "q8" and role_of(i) == "gate_up"}
    calls = []
    for i, m in enumerate(chain):
        w, y, role = mats[i], ys[i], role_of(i)
        if role == "gate_up" and act == "q8":
            calls.append((lambda w, m, e: lambda s: L.w4a8_gemv_gate_up_silu_q8_0(
                w.data_ptr(), resid.data_ptr(), norm.data_ptr(), 1e-5, e.data_ptr(), m.rows, m.k, s))(w, m, acts[i]))
        elif role == "down" and act == "q8":
            calls.append((lambda w, y, m, e: lambda s: L.w4a8_gemv(w.data_ptr(), e.data_ptr(), y.data_ptr(),
                                                                   m.rows, m.k, s))(w, y, m, acts[i - 1]))
        elif role == "gate_up" and act == "f32":
            calls.append((lambda w, y, m: lambda s: L.w4a8_gemv_gate_up_silu(
                w.data_ptr(), resid.data_ptr(), norm.data_ptr(), 1e-5, y.data_ptr(), m.rows, m.k, s))(w, y, m))
        elif role == "down" and act == "f32":
            a = ys[i - 1]                                    # gate|up's act, its first half
            calls.append((lambda w, y, m, a: lambda s: L.w4a8_gemv_f32(w.data_ptr(), a.data_ptr(), y.data_ptr(),
                                                                       m.rows, m.k, s))(w, y, m, a))
        elif role in ("qkv", "gate_up"):
            calls.append((lambda w, y, m: lambda s: L.w4a8_gemv_rmsnorm(w.data_ptr(), resid.data_ptr(), norm.data_ptr(),
                                                                        1e-5, y.data_ptr(), m.rows, m.k, s))(w, y, m))
        elif role == "o":
            calls.append((lambda w, y, m: lambda s: L.w4a8_gemv_f32(w.data_ptr(), attn.data_ptr(), y.data_ptr(),
                                                                    m.rows, m.k, s))(w, y, m))
        elif role == "down":
            gu = ys[i - 1]
            calls.append((lambda w, y, m, gu: lambda s: L.w4a8_gemv_silu_mul(w.data_ptr(), gu.data_ptr(), y.data_ptr(),
                                                                             m.rows, m.k, s))(w, y, m, gu))
        else:
            calls.append((lambda w, y, m: lambda s: L.w4a8_gemv_rmsnorm_argmax(
                w.data_ptr(), resid.data_ptr(), norm.data_ptr(), 1e-5, y.data_ptr(), m.rows, m.k, best.data_ptr(),
                ws.data_ptr(), ws.numel(), s))(w, y, m))
    checked = [(lambda c: lambda s: kv.check("fused chain", c(s)))(c) for c in calls]
    gr = graph_of(torch, stream, checked)
    ms, _ = time_replays(torch, stream, gr, steps, warmup)
    del gr
    out = {"us_per_step": round(ms * 1e3, 2), "tokens_per_s": round(1e3 / ms, 1), "launches_per_step": len(calls),
           "gbps": round(cf.chain_algorithmic_bytes() / (ms * 1e-3) / 1e9, 1),
           "act": {"q8": "gate|up epilogue quantizes silu(gate) * up; down reads the engine layout",
                   "f32": "gate|up epilogue stores silu(gate) * up as fp32; down quantizes it",
                   "down": "down computes silu(gate) * up in its own staging"}[act],
           "issued_by": "the stream entry points from a HIP graph",
           "dependency": "matrix j+1 after matrix j; down reads gate|up's output"}
    if act == "down" or not plan:
        return out
    # The same steps as a chain plan (w4a8_chain_plan_create_steps), then its
    # outputs and pick against the graph's, byte for byte.
    torch.cuda.synchronize()
    # What each step writes: gate|up's act (its first rows / 2 floats, or the
    # engine buffer), every other y whole.
    written = []
    for i, (m, y) in enumerate(zip(chain, ys)):
        if role_of(i) == "gate_up":
            written.append(acts[i] if act == "q8" else y[:m.rows // 2])
        else:
            written.append(y)
    ref = [t.clone() for t in written] + [best.clone()]
    S, plan_steps = kv.PlanStep, []
    for i, m in enumerate(chain):
        w, y, role = mats[i], ys[i], role_of(i)
        if role == "gate_up":
            kind, dst = (kv.PLAN_GATE_UP_SILU_Q8, acts[i]) if act == "q8" else (kv.PLAN_GATE_UP_SILU, y)
            plan_steps.append(S(kind, w.data_ptr(), resid.data_ptr(), dst.data_ptr(), m.rows, m.k, norm.data_ptr(),
                                1e-5))
        elif role == "down":
            kind, src = (kv.PLAN_GEMV_ENGINE, acts[i - 1]) if act == "q8" else (kv.PLAN_GEMV, ys[i - 1])
            plan_steps.append(S(kind, w.data_ptr(), src.data_ptr(), y.data_ptr(), m.rows, m.k, None, 0.0))
        elif role == "qkv":
            plan_steps.append(S(kv.PLAN_GEMV, w.data_ptr(), resid.data_ptr(), y.data_ptr(), m.rows, m.k,
                                norm.data_ptr(), 1e-5))
        elif role == "o":
            plan_steps.append(S(kv.PLAN_GEMV, w.data_ptr(), attn.data_ptr(), y.data_ptr(), m.rows, m.k, None, 0.0))
        else:
            plan_steps.append(S(kv.PLAN_ARGMAX, w.data_ptr(), resid.data_ptr(), y.data_ptr(), m.rows, m.k,
                                norm.data_ptr(), 1e-5, best.data_ptr(), ws.data_ptr()))
    arr = (S * len(plan_steps))(*plan_steps)
    plan = ctypes.c_void_p()
    kv.check("w4a8_chain_plan_create_steps",
             L.w4a8_chain_plan_create_steps(ctypes.cast(arr, ctypes.c_void_p), len(plan_steps), ctypes.byref(plan)))
    try:
        kv.check("w4a8_chain_plan_launch", L.w4a8_chain_plan_launch(plan, max(warmup, 1)))
        kv.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 60000))
        poison(ys)
        for e in acts.values():
            e.fill_(0xAA)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        kv.check("w4a8_chain_plan_launch", L.w4a8_chain_plan_launch(plan, steps))
        kv.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 120000))
        dt = time.perf_counter() - t0
        torch.cuda.synchronize()
    finally:
        kv.check("w4a8_chain_plan_destroy", L.w4a8_chain_plan_destroy(plan))
    same = all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(written + [best], ref))
    out["plan"] = {"us_per_step": round(dt * 1e6 / steps, 2), "tokens_per_s": round(steps / dt, 1),
                   "issued_by": "w4a8_chain_plan_create_steps / _launch / _wait",
                   "verified": same, "verification": "every output and the picked row equal the graph's"}
    return out


def time_prefill(torch, kv, cf, chain, mats, stream, mrows, reps=5):
    """A prompt of mrows tokens through the step's 65 matrices at once: per matrix
    one Q8_0 quantize of the mrows float32 activation rows and one M > 1 GEMM
    (int8 MFMA), in order, from a HIP graph. The reference prefills one decode
    pass per token (docs/buildlog/0008-openai-api.md:73-74)."""
    L = kv.lib()
    calls, keep, ys = [], [], []
    for i, m in enumerate(chain):
        x = torch.from_numpy(cf.prefill_activation(i, mrows, m.k)).cuda()
        xe = torch.empty((mrows, m.k + m.k // 8), dtype=torch.uint8, device="cuda")
        y = torch.empty((mrows, m.rows), dtype=torch.float32, device="cuda")
        keep += [x, xe]
        ys.append(y)
        calls.append((lambda w, x, xe, y, m: lambda s: kv.check("prefill", L.w4a8_quantize_q8_0(
            x.data_ptr(), xe.data_ptr(), m.k, mrows, s) or L.w4a8_gemm(w.data_ptr(), xe.data_ptr(), y.data_ptr(),
                                                                      mrows, m.rows, m.k, s)))(mats[i], x, xe, y, m))
    gr = graph_of(torch, stream, calls)
    ms, _ = time_replays(torch, stream, gr, reps, 1, before=lambda: poison(ys))
    recs = fixtures().get(f"config3_prefill{mrows}")
    checked = verify([(r["name"], y, r["y"]) for y, r in zip(ys, recs)]) if recs else None
    del gr, keep, ys
    torch.cuda.empty_cache()
    return {"tokens": mrows, "ms_per_prompt": round(ms, 4), "tokens_per_s": round(mrows / (ms * 1e-3), 1),
            "launches": 2 * len(chain), "verified": checked["ok"] if checked else None,
            "verification": checked or "no digests for this prompt length (timing only)"}


def time_gemm(torch, kv, cf, m, mrows, stream, base, rec):
    """us per M > 1 GEMM (engine-layout activation rows) over rotating copies of
    config 4's seeded weights `base`; the output of the timed launches is
    checked against the oracle's digest `rec`."""
    L = kv.lib()
    copies = max(3, -(-ROTATE_BYTES // m.weight_bytes))
    mats = [base] + [base.clone() for _ in range(copies - 1)]
    xr = kv.quantize_q8_0_engine(torch.from_numpy(cf.gemm_activation(mrows, m.k)).cuda())
    y = torch.empty((mrows, m.rows), dtype=torch.float32, device="cuda")
    calls = [(lambda w: (lambda s: kv.check("w4a8_gemm", L.w4a8_gemm(w.data_ptr(), xr.data_ptr(), y.data_ptr(),
                                                                    mrows, m.rows, m.k, s))))(mats[i])
             for i in range(copies)]
    g = graph_of(torch, stream, calls)
    ms, _ = time_replays(torch, stream, g, 5, 1, before=lambda: poison([y]))
    ok = verify([(f"{m.name} M={mrows}", y, rec["y"])])["ok"]
    us = ms * 1e3 / copies
    nbytes = m.weight_bytes + mrows * (m.k + m.k // 8) + 4 * mrows * m.rows
    del g, mats
    return {"shape": f"{m.rows}x{m.k}", "m": mrows, "us": round(us, 3), "gbps": round(nbytes / us / 1e3, 1),
            "tops": round(2 * mrows * m.rows * m.k / us / 1e6, 2), "verified": ok}


CALLER = os.path.join(ROOT, "llm-kv260_amd", "caller", "engine_caller")


def run_caller(tokens=20):
    """The reference's caller through the reference ABI, in a process of its own
    (it opens its own device context and pools), on the gemv2 and v1 engines."""
    import subprocess
    out = {}
    for name, extra in (("gemv2", []), ("v1", ["--v1"])):
        env = dict(os.environ, KV260GEMV_UDMABUF_SIZES="udmabuf0=1G")
        p = subprocess.run([CALLER, "--tokens", str(tokens), *extra], capture_output=True, text=True, timeout=300,
                           env=env)
        if p.returncode != 0:
            raise RuntimeError(f"engine_caller {name} failed: {p.stderr[-500:]}")
        out[name] = json.loads(p.stdout.strip().splitlines()[-1])
    return out


CALL_COSTS = os.path.join(ROOT, "llm-kv260_amd", "caller", "call_costs")


def run_call_costs():
    """Per-call costs through the reference ABI (the reference's bench_calls
    and bench_gemv2 tables, docs/buildlog/evidence/0012-bench-calls.txt and
    0013-bench-gemv2.txt), in a process of its own."""
    import subprocess
    env = dict(os.environ, KV260GEMV_UDMABUF_SIZES="udmabuf0=1G")
    p = subprocess.run([CALL_COSTS, "--reps", "200"], capture_output=True, text=True, timeout=300, env=env)
    if p.returncode != 0:
        raise RuntimeError(f"call_costs failed: {p.stderr[-500:]}")
    out = json.loads(p.stdout.strip().splitlines()[-1])
    out["reference_board"] = {"source": "docs/buildlog/evidence/0012-bench-calls.txt and 0013-bench-gemv2.txt "
                                        "(KV260, one rank's shard of four)",
                              "raw_best_us": {"tiny": 2.8, "x2048": 4.6, "x8192": 10.4},
                              "q8_us": {"k256": {"ref": 3.8, "neon": 1.0}, "k2048": {"ref": 30.3, "neon": 8.3},
                                        "k8192": {"ref": 121.7, "neon": 33.5}},
                              "gemv2_cold_prefetched_us": {"qkv": [66.5, 30.9], "o": [53.9, 21.2],
                                                           "gate_up": [348.1, 196.9], "down": [176.2, 77.1],
                                                           "lm_head": [2816.8, 2658.1]},
                              "token_65_calls_mac_ms": {"gap_0us": 13.35, "gap_300us": 8.14}}
    return out




def dispatch_spans(st, grid, passes):
    """Per-workgroup stamps (uint64 [slots, 2]: start, end) of a timed launch ->
    per-dispatch [passes * n, 2]: the earliest start and the latest end of its
    workgroups (w4a8_chain_plan_launch_timed's layout: dispatch after dispatch,
    grid[j] workgroups for step j)."""
    import numpy as np
    counts = np.tile(np.asarray(grid, dtype=np.int64), passes)
    first = np.concatenate(([0], np.cumsum(counts)[:-1]))
    t = st.astype(np.int64)
    return np.stack([np.minimum.reduceat(t[:, 0], first), np.maximum.reduceat(t[:, 1], first)], axis=1)


def stamp_stats(t, hz, chain, ms_per_step, dt_timed):
    """The timed launch's dispatch spans: t is int64 [passes * n, 2] (first wave
    start, last wave end) in ticks of hz. Per shape: the mean, median, min and
    max span; per step: the spans' sum, and the gaps between one dispatch's last
    wave end and the next one's first wave start (the dispatch boundary)."""
    import numpy as np
    n = len(chain)
    us = (t[:, 1] - t[:, 0]).astype(np.float64) / hz * 1e6
    passes = len(us) // n
    spans = us.reshape(passes, n)
    gaps = (t[1:, 0] - t[:-1, 1]).astype(np.float64) / hz * 1e6
    shapes = {}
    for j, m in enumerate(chain):
        key = m.name.split(".")[-1]
        shapes.setdefault(key, {"rows": m.rows, "k": m.k, "bytes": m.algorithmic_bytes, "cols": []})["cols"].append(j)
    per_shape = {}
    for key, d in shapes.items():
        v = spans[:, d["cols"]].reshape(-1)
        per_shape[key] = {"shape": f"{d['rows']}x{d['k']}", "dispatches": int(v.size),
                          "mean_us": round(float(v.mean()), 3), "median_us": round(float(np.median(v)), 3),
                          "min_us": round(float(v.min()), 3), "max_us": round(float(v.max()), 3),
                          "gbps_at_mean": round(d["bytes"] / (float(v.mean()) * 1e-6) / 1e9, 1)}
    step_sum = spans.sum(axis=1)
    first_to_last = (t[n - 1::n, 1] - t[0::n, 0]).astype(np.float64) / hz * 1e6
    chain_bytes = sum(m.algorithmic_bytes for m in chain)
    ks = float(step_sum.mean())
    return {
        "source": "in-kernel stamps: w4a8_chain_plan_launch_timed, the same plan and kernels (their timed twins), "
                  f"{passes} passes in one launch, this run",
        "clock_hz": int(hz), "passes": passes,
        "sum_us_per_step": round(ks, 2), "median_sum_us_per_step": round(float(np.median(step_sum)), 2),
        "achieved": round(chain_bytes / (ks * 1e-6) / 1e9, 1),
        "frac": round(chain_bytes / (ks * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "gap_us_mean": round(float(gaps.mean()), 3), "gap_us_median": round(float(np.median(gaps)), 3),
        "first_start_to_last_end_us_per_step": round(float(first_to_last.mean()), 2),
        "timed_launch_us_per_step": round(dt_timed * 1e6 / passes, 2),
        "untimed_us_per_step": round(ms_per_step * 1e3, 2),
        "per_shape": per_shape,
        "note": "kernel time only: each dispatch from its first workgroup's start to its last workgroup's end "
                "(every wave done, its stores landed); the boundaries between dispatches are the gaps",
    }


def write_stamp_summary(path, kd, argv):
    """The timed launch's per-shape spans as a short text summary (profiles/)."""
    lines = ["# Chain plan dispatch spans, stamped inside the kernels (w4a8_chain_plan_launch_timed)",
             f"# command: python bench.py {' '.join(argv)}",
             f"# {kd['passes']} passes x 65 dispatches; clock {kd['clock_hz']} Hz (s_memrealtime)",
             "",
             f"{'shape':10s} {'rows x k':>12s} {'n':>6s} {'mean us':>9s} {'median':>9s} {'min':>8s} {'max':>8s} "
             f"{'GB/s@mean':>10s}"]
    for key, r in kd["per_shape"].items():
        lines.append(f"{key:10s} {r['shape']:>12s} {r['dispatches']:6d} {r['mean_us']:9.3f} {r['median_us']:9.3f} "
                     f"{r['min_us']:8.3f} {r['max_us']:8.3f} {r['gbps_at_mean']:10.1f}")
    lines += ["",
              f"sum of the 65 spans per step: {kd['sum_us_per_step']} us (median {kd['median_sum_us_per_step']}), "
              f"{kd['achieved']} GB/s, frac {kd['frac']}",
              f"boundary (last workgroup end -> next dispatch's first workgroup start): mean {kd['gap_us_mean']} us, "
              f"median {kd['gap_us_median']} us",
              f"first start -> last end per step: {kd['first_start_to_last_end_us_per_step']} us; "
              f"timed launch {kd['timed_launch_us_per_step']} us/step (host clock); "
              f"untimed launch {kd['untimed_us_per_step']} us/step",
              "JSON " + json.dumps({k: v for k, v in kd.items() if k != "note"})]
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def cpu_baseline(chain, mats, xs, budget_s=30.0):
    """Three decode steps through the NumPy restatement of q4_0.py (1 core; the
    median step is reported), and up to five through the scalar C restatement with
    OpenMP over rows (all cores)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import c_oracle
    import q4_0_oracle

    host_w = [t.cpu().numpy() for t in mats]
    host_x = [t.cpu().numpy() for t in xs]
    np_runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        for m, w, x in zip(chain, host_w, host_x):
            xq, xd = q4_0_oracle.quantize_q8_0(x)
            q4_0_oracle.gemv_q4_0(w, m.k, xq, xd)
        np_runs.append(time.perf_counter() - t0)
    numpy_step = float(np.median(np_runs))
    cores = len(os.sched_getaffinity(0))
    c_runs = []
    for _ in range(max(1, min(5, int(budget_s / max(numpy_step, 1e-3))))):
        t0 = time.perf_counter()
        for m, w, x in zip(chain, host_w, host_x):
            xq, xd = c_oracle.quantize_q8_0(x)
            c_oracle.gemv_q4_0(w, m.k, xq, xd, threads=cores)
        c_runs.append(time.perf_counter() - t0)
    c_step = float(np.median(c_runs))
    return {
        "value": round(1.0 / numpy_step, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
        "sample": "median of 3 decode steps (65 GEMVs incl. LM head, 695 MB of Q4_0 each) through the "
                  "NumPy restatement of src/llm_kv260/q4_0.py (quantize_q8_0 + gemv_q4_0 per matrix), "
                  f"{numpy_step:.2f} s per step, {sum(np_runs):.1f} s in all",
        "c_openmp": {"value": round(1.0 / c_step, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
                     "sample": f"median of {len(c_runs)} decode steps through the scalar C restatement, "
                               f"OpenMP over rows, {c_step * 1e3:.1f} ms/step"},
    }


def headline(args, cf, ms_per_step, chain_gbs, chain_check, one_launch, wall, kd, traffic, graph, overlapped=None):
    """The fields every bench line carries: the metric, the chain and its roofline."""
    plan = not args.no_plan
    n = len(cf.decode_chain())
    chain_bytes = cf.chain_algorithmic_bytes()
    kernel = kd or None
    return {
        "metric": "1B-shape decode GEMV-chain tokens/s (W4A8 Q4_0 x Q8_0, 65 GEMVs per token)",
        "value": round(1e3 / ms_per_step, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8->int32, fp32 epilogue",
        "data": "synthetic, seeded: config 3's Q4_0 weights (numpy default_rng(1000 + j) N(0, 0.02), quantized "
                "on the GPU) and fp32 N(0, 1) activations (default_rng(2000 + j)); the timed outputs are "
                "checked against the oracle's SHA-256 digests in tests/golden/configs.json",
        "config": {"workload": "llama-3.2-1b decode GEMV chain: 16 x (qkv 3072x2048, o 2048x2048, "
                               "gate_up 16384x2048, down 2048x8192) + lm_head 128256x2048, M=1, "
                               "activation re-quantized to Q8_0 before every matrix, matrices in order",
                   "matrices_per_step": n, "weight_bytes_per_step": cf.chain_weight_bytes(),
                   "algorithmic_bytes_per_step": chain_bytes},
        "verified": (chain_check["ok"] and chain_check["weights_ok"] and chain_check.get("timed_launch_ok", True) and
                     graph["verified"] and (overlapped is None or overlapped["verified"]) and
                     (one_launch is None or one_launch["verified"])),
        "roofline": {"bound": "hbm", "achieved": round(chain_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(chain_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("chain_traffic_bytes_per_launch"), "traffic_source": PMC_SUMMARY,
                     "kernel": ("w4a8_plan_gemv_f32 (gemv_m1_dev.h's fused Q8_0 quantize + GEMV), the chain "
                                "plan's 65 dispatches" if plan else
                                "gemv_m1_kernel<X_F32> (fused Q8_0 quantize + GEMV), w4a8_chain_gemv's 65 launches"),
                     "bytes_per_launch": round(chain_bytes / n), "us_per_launch": round(ms_per_step * 1e3 / n, 3),
                     "timing": ("host clock around the plan's timed launch and its wait, the device idle on both "
                                "sides: step time / 65, dispatch boundaries included" if plan else
                                "HIP events on the launch stream around the timed graph replays: step time / 65, "
                                "launch boundaries included"),
                     "kernel_durations": kernel},
        "chain": {"us_per_step": round(ms_per_step * 1e3, 2), "gbps": round(chain_gbs, 1),
                  "hbm_frac": round(chain_gbs / HBM_PEAK_GBS, 4), "launches_per_step": n,
                  "issued_by": ("w4a8_chain_plan_launch (raw AQL dispatches, no cache fences between steps)"
                                if plan else "w4a8_chain_gemv from a HIP graph"),
                  "verified": chain_check["ok"], "verification": chain_check,
                  "dependency": "matrix j+1 starts after matrix j's output is complete"},
        "chain_graph": graph,
        "chain_overlapped": overlapped,
        "chain_one_launch": one_launch,
        "wall_s_timed": round(wall, 3),
    }


def chain_only_line(args, cf, ms_per_step, chain_gbs, chain_check, one_launch, wall, kd, graph, overlapped):
    out = headline(args, cf, ms_per_step, chain_gbs, chain_check, one_launch, wall, kd, pmc_traffic() or {}, graph,
                   overlapped)
    out["mode"] = "chain only: " + ("HIP graph" if args.no_plan else "plan, HIP graph") + (
        "" if one_launch is None else ", one-launch chain")
    return out


def time_plan(torch, kv, L, ptr, n, steps, warmup, ys, check, stamp_passes, overlapped=False):
    """ms per step of the chain plan: `warmup` passes, then exactly `steps`
    passes in one launch, waited for; the device is idle (synchronized) on
    both sides of the timed region and the outputs are poisoned before it;
    check() verifies them. Then, outside the timed region, `stamp_passes`
    passes of the same plan as a timed launch (its outputs poisoned and
    verified the same way): the raw stamps, their clock and the launch's host
    time."""
    import numpy as np
    plan = ctypes.c_void_p()
    create = L.w4a8_chain_plan_create_overlapped if overlapped else L.w4a8_chain_plan_create
    kv.check("w4a8_chain_plan_create", create(ptr, n, ctypes.byref(plan)))
    stamps = None
    try:
        kv.check("w4a8_chain_plan_launch", L.w4a8_chain_plan_launch(plan, max(warmup, 1)))
        kv.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 60000))
        poison(ys)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        kv.check("w4a8_chain_plan_launch", L.w4a8_chain_plan_launch(plan, steps))
        kv.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 120000))
        dt = time.perf_counter() - t0
        torch.cuda.synchronize()
        result = check()
        if stamp_passes:
            grid = [L.w4a8_chain_plan_workgroups(plan, j) for j in range(n)]
            buf = torch.zeros(2 * stamp_passes * sum(grid), dtype=torch.int64, device="cuda")
            poison(ys)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            kv.check("w4a8_chain_plan_launch_timed", L.w4a8_chain_plan_launch_timed(plan, stamp_passes,
                                                                                   buf.data_ptr()))
            kv.check("w4a8_chain_plan_wait", L.w4a8_chain_plan_wait(plan, 120000))
            dt_timed = time.perf_counter() - t1
            torch.cuda.synchronize()
            timed_check = check()
            hz = ctypes.c_int64()
            kv.check("w4a8_wall_clock_hz", L.w4a8_wall_clock_hz(ctypes.byref(hz)))
            per_wg = buf.cpu().numpy().view(np.uint64).reshape(-1, 2)
            if (per_wg == 0).any():
                raise RuntimeError("a workgroup of the timed launch left its stamp slot unwritten")
            stamps = (dispatch_spans(per_wg, grid, stamp_passes), hz.value, dt_timed, timed_check)
    finally:
        kv.check("w4a8_chain_plan_destroy", L.w4a8_chain_plan_destroy(plan))
    return dt * 1e3 / steps, dt, result, stamps


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-gemv", action="store_true", help="skip the per-shape GEMV and GEMM timings")
    ap.add_argument("--no-caller", action="store_true",
                    help="skip the reference-ABI caller and the per-call costs (child processes)")
    ap.add_argument("--chain-only", action="store_true",
                    help="time the chain (per-step, then one launch per step) and stop: the run the "
                         "chain's kernel-trace profile is taken from")
    ap.add_argument("--no-one-launch", action="store_true",
                    help="skip the one-launch (cooperative) chain")
    ap.add_argument("--no-plan", action="store_true",
                    help="time the chain through w4a8_chain_gemv only (the headline then comes from the HIP "
                         "graph)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="time the M > 1 sweep (configuration 4) and stop: the run the GEMM's counter summaries "
                         "are taken from")
    ap.add_argument("--stamp-passes", type=int, default=100,
                    help="passes of the plan's timed launch (in-kernel dispatch spans; 0 = none)")
    ap.add_argument("--stamp-summary", default=None, metavar="PATH",
                    help="write the timed launch's per-shape dispatch spans to PATH as a text summary")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="first copy MB of device memory once: a plain copy of known size whose "
                         "FETCH_SIZE / WRITE_SIZE counters scale the kernels' HBM traffic")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this engine runs every matrix unsplit on one GPU; --gpus {args.gpus} is not "
              "supported (the multi-GPU layout is a design note, not a build)", file=sys.stderr)
        return 2

    import torch
    import kv260gemv as kv
    from kv260gemv import configs as cf

    kv.require_device(0)
    torch.cuda.set_device(0)
    L = kv.lib()
    stream = torch.cuda.Stream()
    if args.copy_calibration:
        src = torch.empty(args.copy_calibration << 18, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.copy_calibration} MB")
        del src, dst
    if args.gemm_only:
        g4 = {(r["name"], r["m"]): r for r in fixtures()["config4"]}
        gemm = []
        for m, base in zip(cf.GEMM_SHAPES, seeded_blocks(torch, kv, cf, cf.GEMM_SHAPES)):
            for mrows in cf.GEMM_M:
                r = time_gemm(torch, kv, cf, m, mrows, stream, base, g4[(m.name, mrows)])
                gemm.append(dict(name=m.name, **r))
                log(f"gemm {m.name} M={mrows}: {r['us']} us, verified {r['verified']}")
            del base
            torch.cuda.empty_cache()
        ok = all(r["verified"] for r in gemm)
        print(json.dumps({"mode": "gemm only", "gemm": gemm, "verified": ok}), flush=True)
        return 0 if ok else 1
    log("building the 65-matrix decode chain (config 3's seeded weights) on the device")
    chain, mats, xs, ys, steps, recs, weights_ok = build_chain(torch, kv, cf)
    n = len(chain)
    chain_bytes = cf.chain_algorithmic_bytes()
    ptr = ctypes.cast(steps, ctypes.c_void_p)
    chain_digests = [(r["name"], y, r["y"]) for y, r in zip(ys, recs)]

    kd = {}
    if not args.no_plan:
        log(f"timing {args.steps} steps after {args.warmup} warm-up steps (chain plan)")
        ms_per_step, wall, chain_check, stamps = time_plan(torch, kv, L, ptr, n, args.steps, args.warmup, ys,
                                                           lambda: verify(chain_digests), args.stamp_passes)
        chain_check["weights_ok"] = weights_ok
        log(f"chain (plan): {ms_per_step * 1e3:.1f} us/step, {1e3 / ms_per_step:.0f} tokens/s, "
            f"outputs {'match' if chain_check['ok'] else 'DIFFER FROM'} the oracle's digests")
        if stamps is not None:
            st, hz, dt_timed, timed_check = stamps
            kd = stamp_stats(st, hz, chain, ms_per_step, dt_timed)
            kd["verified"] = timed_check["ok"]
            chain_check["timed_launch_ok"] = timed_check["ok"]
            log(f"chain (plan, timed launch): dispatch spans sum to {kd['sum_us_per_step']} us/step "
                f"(frac {kd['frac']}), boundary median {kd['gap_us_median']} us, verified {timed_check['ok']}")
            if args.stamp_summary:
                write_stamp_summary(args.stamp_summary, kd, sys.argv[1:])

    overlapped = None
    if not args.no_plan:
        log(f"timing {args.steps} steps after {args.warmup} warm-up steps (overlapped chain plan)")
        ms_ov, _, ov_check, _ = time_plan(torch, kv, L, ptr, n, args.steps, args.warmup, ys,
                                          lambda: verify(chain_digests), 0, overlapped=True)
        overlapped = {"us_per_step": round(ms_ov * 1e3, 2), "tokens_per_s": round(1e3 / ms_ov, 1),
                      "gbps": round(chain_bytes / (ms_ov * 1e-3) / 1e9, 1),
                      "hbm_frac": round(chain_bytes / (ms_ov * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                      "issued_by": "w4a8_chain_plan_create_overlapped: step j + 1 dispatched without the barrier bit, "
                                   "its weight loads issued at once, x read after an in-kernel wait for step j",
                      "verified": ov_check["ok"], "verification": ov_check}
        log(f"chain (overlapped plan): {overlapped['us_per_step']} us/step, verified {overlapped['verified']}")

    log(f"timing {args.steps} steps after {args.warmup} warm-up steps (HIP graph replay of w4a8_chain_gemv)")
    g_chain = graph_of(torch, stream, [lambda s: kv.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ptr, n, s))])
    ms_graph, wall_graph = time_replays(torch, stream, g_chain, args.steps, args.warmup, before=lambda: poison(ys))
    graph_check = verify(chain_digests)
    if args.no_plan:
        ms_per_step, wall, chain_check = ms_graph, wall_graph, dict(graph_check, weights_ok=weights_ok)
    tok_s = 1e3 / ms_per_step
    chain_gbs = chain_bytes / (ms_per_step * 1e-3) / 1e9
    graph = {"us_per_step": round(ms_graph * 1e3, 2), "tokens_per_s": round(1e3 / ms_graph, 1),
             "gbps": round(chain_bytes / (ms_graph * 1e-3) / 1e9, 1),
             "hbm_frac": round(chain_bytes / (ms_graph * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "launches_per_step": n,
             "kernel": "gemv_m1_kernel<X_F32>, 65 HIP launches per step from a graph",
             "timing": "HIP events on the launch stream around the timed graph replays",
             "verified": graph_check["ok"], "verification": graph_check}
    log(f"chain (HIP graph): {graph['us_per_step']} us/step, {graph['tokens_per_s']} tokens/s, "
        f"verified {graph['verified']}")
    del g_chain

    # The same chain as one cooperative launch per step (opt-in mode).
    one_launch = None
    if not args.no_one_launch:
        assert L.w4a8_chain_set_mode(kv.CHAIN_ONE_LAUNCH) == 0
        try:
            timeouts0 = L.w4a8_chain_timeouts()
            g_one = graph_of(torch, stream, [lambda s: kv.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ptr, n, s))])
            ms_one, _ = time_replays(torch, stream, g_one, args.steps, args.warmup, before=lambda: poison(ys))
            one_check = verify(chain_digests)
            one_check["waits_given_up"] = L.w4a8_chain_timeouts() - timeouts0
            del g_one
        finally:
            L.w4a8_chain_set_mode(kv.CHAIN_PER_STEP)
        one_launch = {"us_per_step": round(ms_one * 1e3, 2), "tokens_per_s": round(1e3 / ms_one, 1),
                      "gbps": round(chain_bytes / (ms_one * 1e-3) / 1e9, 1), "launches_per_step": 1,
                      "kernel": "chain_kernel (cooperative, grid barrier between matrices)",
                      "verified": one_check["ok"] and one_check["waits_given_up"] == 0, "verification": one_check}
        log(f"one-launch chain: {one_launch['us_per_step']} us/step, verified {one_launch['verified']}")

    if not args.chain_only:
        g_batch = graph_of(torch, stream, [lambda s: kv.check("w4a8_gemv_batch", L.w4a8_gemv_batch(ptr, n, s))])
        ms_batch, _ = time_replays(torch, stream, g_batch, args.steps, args.warmup, before=lambda: poison(ys))
        batch_check = verify(chain_digests)
        batch_gbs = chain_bytes / (ms_batch * 1e-3) / 1e9
        log(f"batch: {ms_batch * 1e3:.1f} us/step, {batch_gbs:.0f} GB/s (one launch, no order inside a step), "
            f"verified {batch_check['ok']}")
        del g_batch
        prefill = [time_prefill(torch, kv, cf, chain, mats, stream, mr) for mr in (cf.PREFILL_M, 64)]
        for r in prefill:
            log(f"prefill {r['tokens']} tokens: {r['ms_per_prompt']} ms, {r['tokens_per_s']} tokens/s "
                f"(vs {r['tokens'] * ms_per_step:.3f} ms as one decode step per token), verified {r['verified']}")
    if args.chain_only:
        out = chain_only_line(args, cf, ms_per_step, chain_gbs, chain_check, one_launch, wall, kd, graph, overlapped)
        print(json.dumps(out), flush=True)
        return 0 if out["verified"] else 1

    fused_chain = time_fused_chain(torch, kv, cf, chain, mats, ys, stream, args.steps, args.warmup, act="q8",
                                   plan=not args.no_plan)
    fused_f32 = time_fused_chain(torch, kv, cf, chain, mats, ys, stream, args.steps, args.warmup, act="f32",
                                 plan=not args.no_plan)
    staged = time_fused_chain(torch, kv, cf, chain, mats, ys, stream, args.steps, args.warmup, act="down")
    fused_chain["fp32_act"] = {"us_per_step": fused_f32["us_per_step"], "act": fused_f32["act"]}
    if "plan" in fused_f32:
        fused_chain["fp32_act"]["plan"] = fused_f32["plan"]
    fused_chain["silu_in_down_staging_us_per_step"] = staged["us_per_step"]
    plan_txt = lambda r: "" if "plan" not in r else (f", as a chain plan {r['plan']['us_per_step']} us/step "
                                                     f"(verified {r['plan']['verified']})")
    log(f"fused chain (rmsnorm fused, silu in gate|up's epilogue, LM head with argmax): act quantized in the "
        f"epilogue {fused_chain['us_per_step']} us/step{plan_txt(fused_chain)}; fp32 act "
        f"{fused_f32['us_per_step']} us/step{plan_txt(fused_f32)}; silu in down's staging "
        f"{staged['us_per_step']} us/step")

    gemv, gemm = {}, []
    shapes = (cf.LM_HEAD,) if args.no_gemv else (cf.LM_HEAD, cf.O_PROJ) + cf.LAYER_SHAPES
    for m in shapes:
        r = time_gemv(torch, kv, cf, m, stream)
        gemv[m.name if m is not cf.O_PROJ else "o_proj_config0"] = r
        log(f"gemv {m.name} {r['shape']}: {r['us']} us, {r['gbps']} GB/s")
        torch.cuda.empty_cache()
    if not args.no_gemv:
        g4 = {(r["name"], r["m"]): r for r in fixtures()["config4"]}
        for m, base in zip(cf.GEMM_SHAPES, seeded_blocks(torch, kv, cf, cf.GEMM_SHAPES)):
            for mrows in cf.GEMM_M:
                r = time_gemm(torch, kv, cf, m, mrows, stream, base, g4[(m.name, mrows)])
                gemm.append(dict(name=m.name, **r))
                log(f"gemm {m.name} M={mrows}: {r['us']} us, {r['gbps']} GB/s, {r['tops']} TOP/s, "
                    f"verified {r['verified']}")
            del base
            torch.cuda.empty_cache()
    producers = {} if args.no_gemv else time_producers(torch, kv, cf, stream)
    for name, r in producers.items():
        log(f"producer {name} {r['shape']}: fused {r['fused_us']} us, two launches {r.get('two_launches_us')} us, "
            f"no producer {r['plain_f32_us']} us")
    lm_argmax = time_lm_argmax(torch, kv, cf, stream)
    log(f"gemv lm_head + argmax: {lm_argmax['us']} us, {lm_argmax['gbps']} GB/s")
    log(f"top-{lm_argmax['topk']['k']} candidates of the logits: {lm_argmax['topk']['us']} us "
        f"(first {lm_argmax['topk']['first']}, argmax {lm_argmax['argmax']})")
    lm = gemv["lm_head"]
    lm_gbs = cf.LM_HEAD.algorithmic_bytes / lm["us"] / 1e3

    traffic = pmc_traffic() or {}
    caller = calls = None
    if not args.no_caller:
        log("the reference's caller through the reference ABI (host-visible)")
        caller = run_caller()
        log("per-call costs through the reference ABI")
        calls = run_call_costs()
    for name, r in (caller or {}).items():
        log(f"caller {name}: {r['ms_per_token']:.3f} ms/token, {r['us_per_call']['total']:.1f} us/call host-visible")
    cpu = None
    if not args.no_cpu:
        log("CPU baseline (bounded sample)")
        cpu = cpu_baseline(chain, mats, xs)
    verified = (chain_check["ok"] and weights_ok and chain_check.get("timed_launch_ok", True) and
                batch_check["ok"] and graph["verified"] and (overlapped is None or overlapped["verified"]) and
                fused_chain.get("plan", {}).get("verified", True) and
                fused_chain["fp32_act"].get("plan", {}).get("verified", True) and
                (one_launch is None or one_launch["verified"]) and
                all(r["verified"] for r in gemm) and prefill[0]["verified"] is True)

    out = headline(args, cf, ms_per_step, chain_gbs, chain_check, one_launch, wall, kd, traffic, graph, overlapped)
    out["verified"] = verified
    out["verification"] = {"chain": chain_check, "chain_graph": graph_check, "batch": batch_check,
                           "fused_chain_plan": fused_chain.get("plan", {}).get("verified"),
                           "fused_chain_fp32_act_plan": fused_chain["fp32_act"].get("plan", {}).get("verified"),
                           "one_launch": one_launch["verified"] if one_launch else None,
                           "gemm": {f"{r['name']} M={r['m']}": r["verified"] for r in gemm},
                           "prefill24": prefill[0]["verification"],
                           "digests": "tests/golden/configs.json (config3, config3_prefill24, config4)"}
    out.update({
        "roofline_batch": {"achieved": round(batch_gbs, 1), "frac": round(batch_gbs / HBM_PEAK_GBS, 4),
                           "unit": "GB/s", "kernel": "gemv_batch_kernel, one step's 65 GEMVs per launch",
                           "traffic": traffic.get("batch_traffic_bytes_per_launch"),
                           "bytes_per_launch": chain_bytes, "us_per_launch": round(ms_batch * 1e3, 3)},
        "roofline_lm_head": {"achieved": round(lm_gbs, 1), "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "unit": "GB/s",
                             "kernel": "gemv_m1_kernel<X_ENGINE>, LM head 128256x2048, 3 rotating weight copies",
                             "traffic": traffic.get("lm_head_traffic_bytes_per_launch"),
                             "bytes_per_launch": cf.LM_HEAD.algorithmic_bytes, "us_per_launch": lm["us"]},
        "batch": {"us_per_step": round(ms_batch * 1e3, 2), "gbps": round(batch_gbs, 1),
                  "hbm_frac": round(batch_gbs / HBM_PEAK_GBS, 4), "launches_per_step": 1,
                  "tokens_per_s": round(1e3 / ms_batch, 1), "verified": batch_check["ok"],
                  "dependency": "none inside a step (w4a8_gemv_batch); steps in order"},
        "gemv": gemv,
        "gemm": gemm,
        "lm_head_argmax": lm_argmax,
        "producers": producers,
        "chain_fused_producers": fused_chain,
        "prefill": prefill,
        "caller": caller,
        "calls": calls,
        "cpu_baseline": cpu,
    })
    print(json.dumps(out), flush=True)
    if not verified:
        log("a timed output differs from the oracle's digest (see \"verification\")")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
