"""Benchmark of the MI355X W4A8 engine on the Llama-3.2-1B decode GEMV chain.

    python bench.py [--gpus 1] [--steps 400] [--warmup 20] [--no-cpu] [--no-gemv]

One step = one token's 65 W4A8 GEMVs (16 x q|k|v 3072x2048, o 2048x2048,
gate|up 16384x2048, down 2048x8192, then the LM head 128256x2048), each
preceded by the Q8_0 quantization of a float32 activation, in order: matrix
j+1 starts after matrix j's output is complete, as in a decode. The step is
issued by w4a8_chain_gemv (65 launches of the fused quantize + GEMV kernel),
captured once into a HIP graph and replayed. Weights (695,107,584 bytes of
Q4_0) are resident in HBM; the chain alone is larger than the 256 MB Infinity
Cache, so every step streams from HBM.

Prints one JSON line. Besides the chain (value), it reports:
  roofline     the chain's kernel (the fused quantize + GEMV, 65 launches per
               step): average algorithmic bytes per launch / average launch
               duration, both over the timed region (HIP events on the launch
               stream around the graph replays)
  batch        the same 65 GEMVs per step in one w4a8_gemv_batch launch (no
               order inside a step)
  gemv         microseconds per GEMV at every shape, weights rotated past the
               Infinity Cache, launched back to back from a HIP graph
  gemm         the M > 1 sweep (M = 1 .. 64) at gate|up and down
  lm_head_argmax  the LM head with its greedy pick fused, and the sampler's
               top-40 candidates of the same logits (w4a8_topk)
  producers    rmsnorm / silu*up fused into the GEMV's staging against the
               standalone producer then the GEMV
  chain_fused_producers  the chain with those producers and the argmax
  prefill      24- and 64-token prompts through the 65 matrices (M > 1 GEMM)
  caller       the reference's decode-side caller (engine_t of
               board/tp/tp_llama.cpp, rebuilt against the reference driver
               headers: llm-kv260_amd/caller/engine_caller) on both engines:
               host-visible ms per token and us per call, split into the
               host quantize, the clean / invalidate copies and start + wait
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
    quantized by the engine's own Q4_0 kernel."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn((rows, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    blocks = kv.quantize_q4_0(w)
    del w
    return blocks


def build_chain(torch, kv, cf):
    chain = cf.decode_chain()
    mats, xs, ys = [], [], []
    for i, m in enumerate(chain):
        mats.append(device_weights(torch, kv, m.rows, m.k, m.w_seed))
        xs.append(torch.from_numpy(cf.activation(m)).cuda())
        ys.append(torch.empty(m.rows, dtype=torch.float32, device="cuda"))
        if i % 16 == 15:
            log(f"chain weights: {i + 1}/{len(chain)} matrices")
    steps = (CStep * len(chain))(*[CStep(mats[i].data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(), m.rows, m.k)
                                   for i, m in enumerate(chain)])
    torch.cuda.synchronize()
    return chain, mats, xs, ys, steps


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


def time_replays(torch, stream, g, n, warmup):
    """ms per replay over exactly n replays, synchronized on both sides."""
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
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
    """us per GEMV with its producer fused into the activation staging (rmsnorm
    before q|k|v, gate|up and the LM head; silu(gate) * up before down), next to
    the same work as two launches (standalone producer + engine-layout GEMV)
    and the plain fp32 GEMV; weights rotated as for the per-shape GEMVs."""
    L = kv.lib()
    out = {}
    ws = kv.argmax_workspace()
    best = torch.empty(1, dtype=torch.int32, device="cuda")
    cases = (("qkv_rmsnorm", cf.LAYER_SHAPES[0], "rms"), ("gate_up_rmsnorm", cf.LAYER_SHAPES[2], "rms"),
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

        r = {"shape": f"{m.rows}x{m.k}"}
        for label, fn in (("fused_us", fused), ("two_launches_us", split)):
            calls = [(lambda w: (lambda st: kv.check(name, fn(w, st))))(mats[i % copies]) for i in range(launches)]
            gr = graph_of(torch, stream, calls)
            ms, _ = time_replays(torch, stream, gr, 10, 2)
            r[label] = round(ms * 1e3 / launches, 3)
            del gr
        out[name] = r
        del mats, base
        torch.cuda.empty_cache()
    return out


def time_fused_chain(torch, kv, cf, chain, mats, ys, stream, steps, warmup, silu_epilogue=True):
    """The decode step with its producers fused and its one in-step data
    dependency kept: per layer q|k|v = W rmsnorm(x), o = W x, gate|up =
    W rmsnorm(x), down = W (silu(gate) * up) of gate|up's own output; the LM
    head = W rmsnorm(x) with its greedy pick. The rmsnorm inputs (the residual
    stream) and o's input (the attention output) are seeded vectors: attention
    and the residual adds are not part of the engine. silu_epilogue: gate|up
    computes silu(gate) * up as its epilogue (w4a8_gemv_gate_up_silu) and down
    quantizes that; otherwise down computes silu in its own staging
    (w4a8_gemv_silu_mul)."""
    L = kv.lib()
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    k = cf.LAYER_SHAPES[0].k
    resid = torch.randn(k, generator=g, device="cuda")
    attn = torch.randn(k, generator=g, device="cuda")
    norm = torch.randn(k, generator=g, device="cuda")
    ws = kv.argmax_workspace()
    best = torch.empty(1, dtype=torch.int32, device="cuda")
    calls = []
    for i, m in enumerate(chain):
        w, y = mats[i], ys[i]
        role = "lm" if i == len(chain) - 1 else ("qkv", "o", "gate_up", "down")[i % 4]
        if role == "gate_up" and silu_epilogue:
            calls.append((lambda w, y, m: lambda s: L.w4a8_gemv_gate_up_silu(
                w.data_ptr(), resid.data_ptr(), norm.data_ptr(), 1e-5, y.data_ptr(), m.rows, m.k, s))(w, y, m))
        elif role == "down" and silu_epilogue:
            act = ys[i - 1]                                  # gate|up's act, its first half
            calls.append((lambda w, y, m, act: lambda s: L.w4a8_gemv_f32(w.data_ptr(), act.data_ptr(), y.data_ptr(),
                                                                         m.rows, m.k, s))(w, y, m, act))
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
    return {"us_per_step": round(ms * 1e3, 2), "tokens_per_s": round(1e3 / ms, 1), "launches_per_step": len(calls),
            "gbps": round(cf.chain_algorithmic_bytes() / (ms * 1e-3) / 1e9, 1),
            "silu": "gate|up epilogue" if silu_epilogue else "down's staging",
            "dependency": "matrix j+1 after matrix j; down reads gate|up's output through silu(gate) * up"}


def time_prefill(torch, kv, cf, chain, mats, stream, mrows, reps=5):
    """A prompt of mrows tokens through the step's 65 matrices at once: per matrix
    one Q8_0 quantize of the mrows float32 activation rows and one M > 1 GEMM
    (int8 MFMA), in order, from a HIP graph. The reference prefills one decode
    pass per token (docs/buildlog/0008-openai-api.md:73-74)."""
    L = kv.lib()
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    calls, keep = [], []
    for i, m in enumerate(chain):
        x = torch.randn((mrows, m.k), generator=g, device="cuda")
        xe = torch.empty((mrows, m.k + m.k // 8), dtype=torch.uint8, device="cuda")
        y = torch.empty((mrows, m.rows), dtype=torch.float32, device="cuda")
        keep += [x, xe, y]
        calls.append((lambda w, x, xe, y, m: lambda s: kv.check("prefill", L.w4a8_quantize_q8_0(
            x.data_ptr(), xe.data_ptr(), m.k, mrows, s) or L.w4a8_gemm(w.data_ptr(), xe.data_ptr(), y.data_ptr(),
                                                                      mrows, m.rows, m.k, s)))(mats[i], x, xe, y, m))
    gr = graph_of(torch, stream, calls)
    ms, _ = time_replays(torch, stream, gr, reps, 1)
    del gr, keep
    torch.cuda.empty_cache()
    return {"tokens": mrows, "ms_per_prompt": round(ms, 4), "tokens_per_s": round(mrows / (ms * 1e-3), 1),
            "launches": 2 * len(chain)}


def time_gemm(torch, kv, cf, m, mrows, stream):
    """us per M > 1 GEMM (engine-layout activation rows), rotating weight copies."""
    L = kv.lib()
    base = device_weights(torch, kv, m.rows, m.k, 8)
    copies = max(3, -(-ROTATE_BYTES // m.weight_bytes))
    mats = [base] + [base.clone() for _ in range(copies - 1)]
    xr = kv.quantize_q8_0_engine(torch.from_numpy(cf.gemm_activation(mrows, m.k)).cuda())
    y = torch.empty((mrows, m.rows), dtype=torch.float32, device="cuda")
    calls = [(lambda w: (lambda s: kv.check("w4a8_gemm", L.w4a8_gemm(w.data_ptr(), xr.data_ptr(), y.data_ptr(),
                                                                    mrows, m.rows, m.k, s))))(mats[i])
             for i in range(copies)]
    g = graph_of(torch, stream, calls)
    ms, _ = time_replays(torch, stream, g, 5, 1)
    us = ms * 1e3 / copies
    nbytes = m.weight_bytes + mrows * (m.k + m.k // 8) + 4 * mrows * m.rows
    del g, mats, base
    return {"shape": f"{m.rows}x{m.k}", "m": mrows, "us": round(us, 3), "gbps": round(nbytes / us / 1e3, 1),
            "tops": round(2 * mrows * m.rows * m.k / us / 1e6, 2)}


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-gemv", action="store_true", help="skip the per-shape GEMV and GEMM timings")
    ap.add_argument("--no-caller", action="store_true", help="skip the reference-ABI caller (a child process)")
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
    log("building the 65-matrix decode chain on the device")
    chain, mats, xs, ys, steps = build_chain(torch, kv, cf)
    n = len(chain)
    chain_bytes = cf.chain_algorithmic_bytes()
    ptr = ctypes.cast(steps, ctypes.c_void_p)

    log(f"timing {args.steps} steps after {args.warmup} warm-up steps (HIP graph replay)")
    g_chain = graph_of(torch, stream, [lambda s: kv.check("w4a8_chain_gemv", L.w4a8_chain_gemv(ptr, n, s))])
    ms_per_step, wall = time_replays(torch, stream, g_chain, args.steps, args.warmup)
    tok_s = 1e3 / ms_per_step
    chain_gbs = chain_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"chain: {ms_per_step * 1e3:.1f} us/step, {tok_s:.0f} tokens/s, {chain_gbs:.0f} GB/s")

    g_batch = graph_of(torch, stream, [lambda s: kv.check("w4a8_gemv_batch", L.w4a8_gemv_batch(ptr, n, s))])
    ms_batch, _ = time_replays(torch, stream, g_batch, args.steps, args.warmup)
    batch_gbs = chain_bytes / (ms_batch * 1e-3) / 1e9
    log(f"batch: {ms_batch * 1e3:.1f} us/step, {batch_gbs:.0f} GB/s (one launch, no order inside a step)")
    del g_chain, g_batch
    prefill = [time_prefill(torch, kv, cf, chain, mats, stream, mr) for mr in (24, 64)]
    for r in prefill:
        log(f"prefill {r['tokens']} tokens: {r['ms_per_prompt']} ms, {r['tokens_per_s']} tokens/s "
            f"(vs {r['tokens'] * ms_per_step:.3f} ms as one decode step per token)")
    fused_chain = time_fused_chain(torch, kv, cf, chain, mats, ys, stream, args.steps, args.warmup)
    staged = time_fused_chain(torch, kv, cf, chain, mats, ys, stream, args.steps, args.warmup, silu_epilogue=False)
    fused_chain["silu_in_down_staging_us_per_step"] = staged["us_per_step"]
    log(f"fused chain: {fused_chain['us_per_step']} us/step, {fused_chain['tokens_per_s']} tokens/s "
        f"(rmsnorm fused, silu in gate|up's epilogue, LM head with argmax); {staged['us_per_step']} us/step "
        "with silu in down's staging")

    gemv, gemm = {}, []
    shapes = (cf.LM_HEAD,) if args.no_gemv else (cf.LM_HEAD, cf.O_PROJ) + cf.LAYER_SHAPES
    for m in shapes:
        r = time_gemv(torch, kv, cf, m, stream)
        gemv[m.name if m is not cf.O_PROJ else "o_proj_config0"] = r
        log(f"gemv {m.name} {r['shape']}: {r['us']} us, {r['gbps']} GB/s")
        torch.cuda.empty_cache()
    if not args.no_gemv:
        for m in cf.GEMM_SHAPES:
            for mrows in cf.GEMM_M:
                r = time_gemm(torch, kv, cf, m, mrows, stream)
                gemm.append(dict(name=m.name, **r))
                log(f"gemm {m.name} M={mrows}: {r['us']} us, {r['gbps']} GB/s, {r['tops']} TOP/s")
            torch.cuda.empty_cache()
    producers = {} if args.no_gemv else time_producers(torch, kv, cf, stream)
    for name, r in producers.items():
        log(f"producer {name} {r['shape']}: fused {r['fused_us']} us, two launches {r['two_launches_us']} us")
    lm_argmax = time_lm_argmax(torch, kv, cf, stream)
    log(f"gemv lm_head + argmax: {lm_argmax['us']} us, {lm_argmax['gbps']} GB/s")
    log(f"top-{lm_argmax['topk']['k']} candidates of the logits: {lm_argmax['topk']['us']} us "
        f"(first {lm_argmax['topk']['first']}, argmax {lm_argmax['argmax']})")
    lm = gemv["lm_head"]
    lm_gbs = cf.LM_HEAD.algorithmic_bytes / lm["us"] / 1e3

    traffic = pmc_traffic() or {}
    caller = None
    if not args.no_caller:
        log("the reference's caller through the reference ABI (host-visible)")
        caller = run_caller()
    for name, r in (caller or {}).items():
        log(f"caller {name}: {r['ms_per_token']:.3f} ms/token, {r['us_per_call']['total']:.1f} us/call host-visible")
    cpu = None
    if not args.no_cpu:
        log("CPU baseline (bounded sample)")
        cpu = cpu_baseline(chain, mats, xs)

    out = {
        "metric": "1B-shape decode GEMV-chain tokens/s (W4A8 Q4_0 x Q8_0, 65 GEMVs per token)",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8->int32, fp32 epilogue",
        "data": "synthetic: Q4_0 weights from N(0,0.02) drawn with the device RNG per matrix and quantized by "
                "the engine; fp32 N(0,1) activations, numpy-seeded per matrix",
        "config": {"workload": "llama-3.2-1b decode GEMV chain: 16 x (qkv 3072x2048, o 2048x2048, "
                               "gate_up 16384x2048, down 2048x8192) + lm_head 128256x2048, M=1, "
                               "activation re-quantized to Q8_0 before every matrix, matrices in order",
                   "matrices_per_step": n, "weight_bytes_per_step": cf.chain_weight_bytes(),
                   "algorithmic_bytes_per_step": chain_bytes},
        "roofline": {"bound": "hbm", "achieved": round(chain_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(chain_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("chain_traffic_bytes_per_launch"), "traffic_source": PMC_SUMMARY,
                     "kernel": "gemv_m1_kernel<X_F32> (fused Q8_0 quantize + GEMV), the chain's 65 launches",
                     "bytes_per_launch": round(chain_bytes / n), "us_per_launch": round(ms_per_step * 1e3 / n, 3)},
        "roofline_batch": {"achieved": round(batch_gbs, 1), "frac": round(batch_gbs / HBM_PEAK_GBS, 4),
                           "unit": "GB/s", "kernel": "gemv_batch_kernel, one step's 65 GEMVs per launch",
                           "traffic": traffic.get("batch_traffic_bytes_per_launch"),
                           "bytes_per_launch": chain_bytes, "us_per_launch": round(ms_batch * 1e3, 3)},
        "roofline_lm_head": {"achieved": round(lm_gbs, 1), "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "unit": "GB/s",
                             "kernel": "gemv_m1_kernel<X_ENGINE>, LM head 128256x2048, 3 rotating weight copies",
                             "traffic": traffic.get("lm_head_traffic_bytes_per_launch"),
                             "bytes_per_launch": cf.LM_HEAD.algorithmic_bytes, "us_per_launch": lm["us"]},
        "chain": {"us_per_step": round(ms_per_step * 1e3, 2), "gbps": round(chain_gbs, 1),
                  "hbm_frac": round(chain_gbs / HBM_PEAK_GBS, 4), "launches_per_step": n,
                  "dependency": "matrix j+1 starts after matrix j's output is complete"},
        "batch": {"us_per_step": round(ms_batch * 1e3, 2), "gbps": round(batch_gbs, 1),
                  "hbm_frac": round(batch_gbs / HBM_PEAK_GBS, 4), "launches_per_step": 1,
                  "tokens_per_s": round(1e3 / ms_batch, 1),
                  "dependency": "none inside a step (w4a8_gemv_batch); steps in order"},
        "gemv": gemv,
        "gemm": gemm,
        "lm_head_argmax": lm_argmax,
        "producers": producers,
        "chain_fused_producers": fused_chain,
        "prefill": prefill,
        "caller": caller,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
