#!/usr/bin/env python3
"""Measures the W8A8 decoder datapath on one MI355X (BASELINE.json metric: decode & prefill tok/s at
batch 1; W8A8 GEMV % of HBM peak) and prints ONE JSON line.

Workload: the Llama-3.2-1B-shaped config (the one the metric's GEMV and
MFMA roofline fractions are quoted on): synthetic N(0, 0.02) weights quantised to int8, the
seeded 512-token prompt prefilled, then greedy decode at batch 1. A step is one decode token;
`value` is decode tokens/s over exactly --steps steps with everything resident in HBM.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--config c4-llama3.2-1b]

Extra fields: prefill tok/s (the 512-row prompt in one t2r_prefill), per-kernel-class HIP-event
durations from the timed region, the roofline of the dominant kernel (the fused SwiGLU GEMV:
RMSNorm + quant + W1/W3 + SiLU gate), and the CPU baseline (the bit-exact NumPy restatement in
oracle/, timed on a bounded sample on this host).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA, published


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(cfg):
    """Algorithmic bytes of one launch of each decode kernel class (weights int8 + fp32 row scales
    + fp32 inputs / outputs / gains): what the launch must move, once."""
    d, q, kv, F, V = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden, cfg.vocab
    return {
        "qkv": (q + 2 * kv) * d + 4 * (q + 2 * kv) + 4 * d + 4 * d + 4 * (q + 2 * kv),
        "wo": d * q + 4 * d + 4 * q + 4 * d + 4 * d,
        "ffn_up": 2 * F * d + 2 * 4 * F + 4 * d + 4 * d + 4 * F,
        "ffn_down": d * F + 4 * d + 4 * F + 4 * d + 4 * d,
        "cls": V * d + 4 * V + 4 * d + 4 * d + 4 * V,
    }


MFMA_INT8_PEAK_TOPS = 5000.0            # MI355X dense int8 matrix peak (5.0 POP/s)


def gemm_weights(cfg):
    """Weights (N x K) of each prefill GEMM class per layer: ops per launch are 2 * rows * this. (An
    MoE model's expert FFN runs as row GEMVs over the selected experts, not as a GEMM class.)"""
    d, q, kv, F = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
    w = {"qkv": (q + 2 * kv) * d, "wo": d * q}
    if not cfg.n_experts:
        w.update({"ffn_up": 2 * F * d, "ffn_down": d * F})
    return w


def measured_traffic(kind, cfg_name):
    """HBM bytes per launch of the dominant kernel, as measured by the rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE passes summarised in profiles/ (scaled by a known-size copy); None when not recorded
    for this configuration. The counters need the profiler, so the bench reads the recorded figure."""
    path = os.path.join(ROOT, "profiles", "gemv_swiglu_c4_decode_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            _, k, c, v = line.split()
            if k == kind and c == cfg_name:
                return int(v)
    return None


def profiled_avg_us(kind, cfg_name):
    """The dominant kernel's average duration in the committed rocprofv3 --kernel-trace --stats summary of
    this bench (profiles/gemv_swiglu_c4_decode.md, line `rocprof_avg_us: <class> <config> <us>`), so that the
    line's roofline fraction follows from profiles/; None when not recorded for this configuration."""
    path = os.path.join(ROOT, "profiles", "gemv_swiglu_c4_decode.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("rocprof_avg_us:"):
            _, k, c, v = line.split()
            if k == kind and c == cfg_name:
                return float(v)
    return None


def host_cpu():
    """This host's CPU model, logical cores, and the BLAS threads the oracle's matrix products use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        from threadpoolctl import threadpool_info
        blas = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        blas = 1
    return model, os.cpu_count() or 1, int(blas)


def oracle_on_gpu_cache(qm, rm, P):
    """The oracle holding the KV rows 0..P-1 that the GPU prefill wrote (bit-identical to the oracle's own
    prefill of the prompt, which its tests check), so the CPU is timed at the GPU run's positions."""
    from oracle import OracleModel
    om = OracleModel(qm)
    om.kc[:, :P] = rm.kc[:, :P].cpu().numpy()
    om.vc[:, :P] = rm.vc[:, :P].cpu().numpy()
    return om


def cpu_decode(om, tok, P, seconds, max_steps=64):
    """Greedy decode steps of the oracle at positions P, P + 1, ... for about `seconds` (the first step
    untimed: it converts the weights to the matrix-product layout). Returns (tok/s, steps, logits)."""
    import numpy as np
    snap = (om.kc[:, P].copy(), om.vc[:, P].copy())
    om.forward(tok, P)
    om.kc[:, P], om.vc[:, P] = snap
    n, logits, t0 = 0, [], time.perf_counter()
    while time.perf_counter() - t0 < seconds and n < max_steps and P + n < om.cfg.seq_len:
        lg = om.forward(tok, P + n)
        logits.append(lg)
        tok = int(np.argmax(lg))
        n += 1
    dt = time.perf_counter() - t0
    return n / dt, n, dt, logits


def cpu_prefill(om, prompt, P, rows):
    """The oracle's prefill of the prompt's last `rows` rows (positions P - rows .. P - 1, attending to the
    cache rows before them): rows/s at the prompt's longest contexts."""
    rows = min(rows, P)
    t0 = time.perf_counter()
    om.prefill(prompt[P - rows:P], start=P - rows)
    dt = time.perf_counter() - t0
    return rows / dt, rows, dt


def prefill_gemm_rates(rm, cfg, prompt):
    """The prompt prefilled once more with HIP events around each GEMM launch (the per-class scopes of a
    multi-row linear cover the GEMM alone): per class and overall int8 TOPS at M = len(prompt) rows."""
    P = len(prompt)
    rm.reset()
    rm.profile(kinds=("qkv", "wo", "ffn_up", "ffn_down"), max_launches=4 * cfg.layers + 8)
    rm.prefill(prompt)
    pprof = rm.profile_read()
    rm.profile(kinds=())
    gemm_ops = {k: 2 * P * v for k, v in gemm_weights(cfg).items()}
    g_ops = sum(gemm_ops[k] * len(v) for k, v in pprof.items() if k in gemm_ops)
    g_ms = sum(sum(v) for k, v in pprof.items() if k in gemm_ops)
    rates = {k: {"launches": len(v), "avg_us": round(sum(v) / len(v) * 1e3, 3),
                 "TOPS": round(gemm_ops[k] / (sum(v) / len(v) * 1e-3) * 1e-12, 1)}
             for k, v in pprof.items() if k in gemm_ops and v}
    g_tops = g_ops / (g_ms * 1e-3) * 1e-12 if g_ms > 0 else None
    if g_tops:
        rates["all"] = {"rows": P, "TOPS": round(g_tops, 1), "frac": round(g_tops / MFMA_INT8_PEAK_TOPS, 4),
                        "peak_TOPS": MFMA_INT8_PEAK_TOPS, "total_us": round(g_ms * 1e3, 1)}
    return rates, g_ms, g_tops


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="c4-llama3.2-1b")
    ap.add_argument("--prefill-reps", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="time eager decode steps instead of a HIP graph")
    ap.add_argument("--batch", default="4,8,16",
                    help="batched-decode sizes to time (t2r_decode_batch; '' to skip)")
    ap.add_argument("--batch-steps", type=int, default=32)
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5",
                    help="configs whose GPU and CPU decode / prefill rates go into the line's `configs` ('' to skip)")
    ap.add_argument("--config-cpu-seconds", type=float, default=4.0)
    ap.add_argument("--copy-calib-mb", type=int, default=0,
                    help="first copy this many MiB device to device (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the datapath runs on a single "
              f"MI355X; no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cfg = C.get(args.config)
    if args.copy_calib_mb > 0:
        n = args.copy_calib_mb << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {n} bytes read, {n} bytes written")
        del src, dst
    t0 = time.time()
    qm = W.QuantModel(cfg)
    log(f"{cfg.name}: weights generated and quantised in {time.time() - t0:.1f} s")
    prompt = cfg.prompt()
    P = len(prompt)
    rm = ResidentModel(qm, device="cuda:0", max_rows=P)
    sync = torch.cuda.synchronize

    # ---- prefill tok/s: the whole prompt in one call
    times = []
    for r in range(args.prefill_reps + 1):
        rm.reset()
        sync()
        t = time.perf_counter()
        rm.prefill(prompt)
        sync()
        times.append(time.perf_counter() - t)
    prefill_s = float(np.median(times[1:])) if len(times) > 1 else times[0]
    log(f"prefill {P} rows: {prefill_s * 1e3:.2f} ms ({P / prefill_s:.0f} tok/s)")
    # the same prefill replayed from a HIP graph (no host launch work)
    prefill_graph_s = None
    if not args.no_graph and P <= rm.max_rows:
        gp = rm.capture_prefill(prompt)
        gts = []
        for r in range(args.prefill_reps + 1):
            rm.reset()
            sync()
            t = time.perf_counter()
            gp.replay()
            sync()
            gts.append(time.perf_counter() - t)
        prefill_graph_s = float(np.median(gts[1:])) if len(gts) > 1 else gts[0]
        del gp
        log(f"prefill {P} rows from a HIP graph: {prefill_graph_s * 1e3:.2f} ms")
    # the prefill GEMMs' int8 MFMA rate: one more prefill with HIP events around each GEMM launch
    prefill_gemm, g_ms, g_tops = prefill_gemm_rates(rm, cfg, prompt)
    if g_tops:
        log(f"prefill GEMMs: {g_ms * 1e3:.0f} us, {g_tops:.0f} int8 TOPS ({g_tops / MFMA_INT8_PEAK_TOPS:.3f} of peak)")
    after_prompt = rm.next.clone()

    # ---- decode: greedy on the device, batch 1, positions P .. P + steps.
    steps = min(args.steps, cfg.seq_len - P)
    warm = min(args.warmup, steps)

    def rewind():
        rm.tok.copy_(after_prompt)
        rm.pos.fill_(P)

    # (1) eager steps with HIP events around every kernel class: the per-class breakdown
    rewind()
    for _ in range(warm):
        rm.step(logits=False, advance=True)
    rewind()
    rm.profile(max_launches=steps * (cfg.layers * 6 + 4))
    sync()
    t = time.perf_counter()
    for _ in range(steps):
        rm.step(logits=False, advance=True)
    sync()
    eager_dt = time.perf_counter() - t
    prof = rm.profile_read()
    rm.profile(kinds=())
    log(f"decode eager: {eager_dt / steps * 1e3:.3f} ms/token ({steps / eager_dt:.1f} tok/s)")

    # (2) the timed region of `value`: one HIP graph of all `steps` decode steps (launch-free)
    dom_ms = None
    graph = None
    if not args.no_graph:
        try:
            rewind()
            graph = rm.capture_decode(steps)
            graph.replay()                                  # warm-up replay
            sync()
        except Exception as e:                              # capture not available: eager timing only
            log(f"HIP graph capture failed ({e}); timing eager steps")
            graph = None
    if graph is not None:
        rewind()
        sync()
        t = time.perf_counter()
        graph.replay()
        sync()
        dt = time.perf_counter() - t
        mode = "hip-graph"
    else:
        dt, mode = eager_dt, "eager"
    tok_s = steps / dt
    log(f"decode {mode}: {steps} steps, {dt / steps * 1e3:.3f} ms/token ({tok_s:.1f} tok/s)")
    rm.check_status("decode")                               # a replay's device status (RuntimeError if set)

    # (3) batched decode: B sequences per step, each continuing the prompt from its own copy of the
    # prompt's KV rows; greedy tokens and positions stay on the device
    batch = {}
    from t2r_amd import abi
    for B in [int(b) for b in args.batch.split(",") if b.strip()]:
        K = min(args.batch_steps, cfg.seq_len - P - 2)
        if B > rm.max_rows or K < 1:
            continue
        kc, vc = rm.batch_caches(B)
        kc[:] = rm.kc
        vc[:] = rm.vc
        lg = torch.empty((B, cfg.vocab), dtype=torch.float32, device=rm.device)
        toks, poss = rm.rows_tok[:B], rm.rows_pos[:B]

        def bstep():
            abi.check("t2r_decode_batch", rm.lib.t2r_decode_batch(
                rm.handle, abi.ptr(toks), abi.ptr(poss), B, abi.ptr(kc), abi.ptr(vc), kc[0].numel(), abi.ptr(lg),
                abi.ptr(toks), abi.stream_ptr()))
            poss.add_(1)
        tok0 = (after_prompt.to(torch.int64) + torch.arange(B, device=rm.device)) % cfg.vocab

        def rewind_b():
            toks.copy_(tok0)
            poss.fill_(P)
        rewind_b()
        bstep()
        bstep()
        rewind_b()
        sync()
        t = time.perf_counter()
        for _ in range(K):
            bstep()
        sync()
        edt = time.perf_counter() - t
        # the same K steps replayed from one HIP graph (the step's launches without host work)
        bdt, bmode = edt, "eager"
        if not args.no_graph:
            try:
                side = torch.cuda.Stream(device=rm.device)
                side.wait_stream(torch.cuda.current_stream(rm.device))
                rewind_b()
                with torch.cuda.stream(side):
                    bstep()
                torch.cuda.current_stream(rm.device).wait_stream(side)
                sync()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=side):
                    for _ in range(K):
                        bstep()
                rewind_b()
                g.replay()
                rewind_b()
                sync()
                t = time.perf_counter()
                g.replay()
                sync()
                bdt, bmode = time.perf_counter() - t, "hip-graph"
                del g
            except Exception as e:                          # capture not available: eager timing only
                log(f"batched HIP graph capture failed ({e}); eager timing")
        rm.check_status(f"batched decode B={B}")
        batch[str(B)] = {"tok_s": round(B * K / bdt, 1), "ms_per_step": round(bdt / K * 1e3, 4), "steps": K,
                         "mode": bmode, "eager_tok_s": round(B * K / edt, 1)}
        log(f"batched decode B={B} ({bmode}): {bdt / K * 1e3:.3f} ms/step ({B * K / bdt:.0f} tok/s aggregate); "
            f"eager {edt / K * 1e3:.3f} ms/step")
        del kc, vc, lg

    nbytes = gemv_bytes(cfg)
    classes = {}
    gemv_b = gemv_t = 0.0
    for k, ts in prof.items():
        avg = sum(ts) / len(ts)
        rec = {"launches": len(ts), "avg_us": round(avg * 1e3, 3), "total_ms": round(sum(ts), 3)}
        if k in nbytes and not cfg.moe:
            rec["bytes_per_launch"] = nbytes[k]
            rec["GBps"] = round(nbytes[k] / (avg * 1e-3) / 1e9, 1)
            gemv_b += nbytes[k] * len(ts)
            gemv_t += sum(ts) * 1e-3
        classes[k] = rec
    dom = classes.get("ffn_up", {})
    if dom_ms:                                              # from the timed region itself
        dom = {"launches": len(dom_ms), "avg_us": round(sum(dom_ms) / len(dom_ms) * 1e3, 3),
               "GBps": round(nbytes["ffn_up"] / (sum(dom_ms) / len(dom_ms) * 1e-3) / 1e9, 1)}
    achieved_event = dom.get("GBps")
    # the line's fraction from the committed rocprofv3 summary's average (reproducible from profiles/); the
    # live HIP-event timing of the same kernel beside it
    prof_us = profiled_avg_us("ffn_up", cfg.name)
    if prof_us:
        achieved, avg_us, src = round(nbytes["ffn_up"] / (prof_us * 1e-6) / 1e9, 1), prof_us, \
            "rocprofv3 --kernel-trace --stats average, profiles/gemv_swiglu_c4_decode.md"
    else:
        achieved, avg_us, src = achieved_event, dom.get("avg_us"), "HIP events in this run"
    out = {
        "metric": "decode & prefill tok/s at batch 1; W8A8 GEMV % of HBM peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(dt / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (N(0, 0.02) random weights, per-row int8; seeded uniform prompt ids)",
        "config": {"workload": f"{cfg.name}: decode at batch 1 after a {P}-token prefill", "model": cfg.name,
                   "global_batch": 1, "seq_len": cfg.seq_len, "prompt": P, "decode_steps": steps,
                   "parallelism": "none (1 GPU)"},
        "prefill_tok_s": round(P / prefill_s, 1),
        "prefill_ms": round(prefill_s * 1e3, 3),
        "prefill_graph_ms": round(prefill_graph_s * 1e3, 3) if prefill_graph_s else None,
        "kernels": classes,
        "gemv_all_GBps": round(gemv_b / gemv_t / 1e9, 1) if gemv_t else None,
        "gemv_all_frac": round(gemv_b / gemv_t / 1e9 / HBM_PEAK_GBS, 4) if gemv_t else None,
        "decode_mode": mode,
        "batch_decode": batch,
        "prefill_gemm": prefill_gemm,
        "eager_tok_s": round(steps / eager_dt, 2),
        "roofline": {"kernel": "k_gemv_pw<EPI_SWIGLU> (fused RMSNorm + SwiGLU decode GEMV, prologue wave)", "bound": "hbm",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
                     "bytes_per_launch": nbytes["ffn_up"], "avg_us": avg_us, "duration_source": src,
                     "traffic": measured_traffic("ffn_up", cfg.name),
                     "avg_us_event": dom.get("avg_us"), "achieved_event": achieved_event,
                     "frac_event": round(achieved_event / HBM_PEAK_GBS, 4) if achieved_event else None,
                     "launches_event": dom.get("launches")},
    }

    # ---- CPU baseline at the GPU run's positions (+ a bit-exactness spot check of those positions)
    if not args.no_cpu_baseline:
        cpu_model, ncpu, blas = host_cpu()
        rm.reset()
        rm.prefill(prompt)
        tok0 = int(rm.next.item())
        om = oracle_on_gpu_cache(qm, rm, P)
        rate, n, cdt, cpu_logits = cpu_decode(om, tok0, P, args.cpu_seconds)
        out["cpu_baseline"] = {"value": round(rate, 3), "unit": "tok/s", "cores": blas, "kind": "port",
                               "sample": f"{n} greedy decode steps of the NumPy restatement at positions {P}.."
                                         f"{P + n - 1} after the {P}-token prompt ({cdt:.1f} s)",
                               "cpu": cpu_model, "host_logical_cores": ncpu}
        tok, same = tok0, True
        for i, lg in enumerate(cpu_logits[:4]):
            g = rm.decode(tok, P + i).cpu().numpy()
            same &= bool(np.array_equal(g.view(np.uint32), lg.view(np.uint32)))
            tok = int(np.argmax(lg))
        out["parity_spot_check"] = {"positions": f"{P}..{P + min(4, len(cpu_logits)) - 1}", "bit_exact": same}
        log(f"cpu baseline: {rate:.2f} tok/s on {blas} BLAS threads ({cpu_model}); GPU == CPU logits: {same}")
    rm.close()
    del rm

    # ---- every config: GPU decode (HIP graph) and prefill, CPU decode and prefill samples
    if args.configs:
        out["configs"] = per_config(args, out if not args.no_cpu_baseline else None)
    print(json.dumps(out), flush=True)


def per_config(args, c4_out):
    """Decode and prefill tok/s of each BASELINE.json config on the GPU and of the CPU restatement on this
    host (BLAS threads stated), at the config's own prompt length; bounded samples. The headline config
    reuses the numbers measured above."""
    import numpy as np
    import torch
    import t2r_amd.config as C
    from t2r_amd import weights as W
    from t2r_amd.model import ResidentModel
    cpu_model, ncpu, blas = host_cpu()
    table = {"cpu": cpu_model, "host_logical_cores": ncpu, "blas_threads": blas}
    for key in [k.strip() for k in args.configs.split(",") if k.strip()]:
        cfg = C.get(key)
        if c4_out is not None and cfg.name == args.config:
            table[cfg.name] = {"gpu_decode_tok_s": c4_out["value"], "gpu_prefill_tok_s": c4_out["prefill_tok_s"],
                               "gpu_prefill_ms": c4_out["prefill_ms"], "gpu_prefill_graph_ms": c4_out["prefill_graph_ms"],
                               "prefill_gemm_TOPS": c4_out["prefill_gemm"].get("all", {}).get("TOPS"),
                               "prefill_gemm_frac": c4_out["prefill_gemm"].get("all", {}).get("frac"),
                               "cpu_decode_tok_s": c4_out["cpu_baseline"]["value"],
                               "decode_positions": f"{cfg.prompt_len}..", "prompt": cfg.prompt_len}
            continue
        t0 = time.time()
        qm = W.QuantModel(cfg)
        prompt = cfg.prompt()
        P = len(prompt)
        rm = ResidentModel(qm, device="cuda:0", max_rows=min(P, 2048))
        # GPU prefill: the whole prompt in one call (median of 3)
        ts = []
        for _ in range(4):
            rm.reset()
            torch.cuda.synchronize()
            t = time.perf_counter()
            rm.prefill(prompt)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t)
        pre = float(np.median(ts[1:]))
        tok0 = int(rm.next.item())
        # the same prefill replayed from a HIP graph (prompts of at most 512 rows: one t2r_prefill_at call)
        pre_g = None
        if P <= 512:
            gp = rm.capture_prefill(prompt)
            gts = []
            for _ in range(4):
                rm.reset()
                torch.cuda.synchronize()
                t = time.perf_counter()
                gp.replay()
                torch.cuda.synchronize()
                gts.append(time.perf_counter() - t)
            pre_g = float(np.median(gts[1:]))
            assert int(rm.next.item()) == tok0, "the prefill graph's greedy token differs from the eager prefill's"
            del gp
        gemm, _, g_tops = prefill_gemm_rates(rm, cfg, prompt)
        # GPU decode: a HIP graph of the config's decode steps (at most 64) from the prompt's end
        K = max(1, min(cfg.decode_steps, 64, cfg.seq_len - P))
        rm.tok.fill_(tok0)
        rm.pos.fill_(P)
        g = rm.capture_decode(K)
        rm.tok.fill_(tok0)
        rm.pos.fill_(P)
        g.replay()
        rm.tok.fill_(tok0)
        rm.pos.fill_(P)
        torch.cuda.synchronize()
        t = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        gdt = time.perf_counter() - t
        del g
        rm.check_status(f"{cfg.name} decode")
        rec = {"prompt": P, "gpu_prefill_tok_s": round(P / pre, 1), "gpu_prefill_ms": round(pre * 1e3, 3),
               "gpu_prefill_graph_ms": round(pre_g * 1e3, 3) if pre_g else None,
               "gpu_prefill_graph_tok_s": round(P / pre_g, 1) if pre_g else None,
               "gpu_decode_tok_s": round(K / gdt, 1),
               "gpu_decode_steps": K, "decode_positions": f"{P}..{P + K - 1}",
               "prefill_gemm_TOPS": gemm.get("all", {}).get("TOPS"), "prefill_gemm_frac": gemm.get("all", {}).get("frac")}
        if c4_out is not None:
            rm.reset()
            rm.prefill(prompt)
            om = oracle_on_gpu_cache(qm, rm, P)
            rate, n, cdt, _ = cpu_decode(om, tok0, P, args.config_cpu_seconds, max_steps=32)
            prate, rows, pdt = cpu_prefill(om, prompt, P, 16 if P <= 512 else 4)
            rec.update({"cpu_decode_tok_s": round(rate, 3), "cpu_decode_steps": n,
                        "cpu_prefill_tok_s": round(prate, 3),
                        "cpu_prefill_sample": f"rows {P - rows}..{P - 1} ({pdt:.1f} s)"})
        rm.close()
        del rm, qm
        table[cfg.name] = rec
        log(f"{cfg.name}: {rec} ({time.time() - t0:.0f} s)")
    return table


if __name__ == "__main__":
    main()
