"""Benchmark of the MoE block hot path on one MI355X.

Workload C2: Qwen3-Next-style MoE layer, batch-1 decode —
H=2048, 512 routed experts, top-10 softmax routing renormalised, expert
intermediate 512, one sigmoid-gated shared expert (intermediate 512), 4-bit
affine weights with group 64 and f16 scale/bias, seeded synthetic data.

A step is one MoE layer for one token (pbmoe_moe_layer): router logits,
top-k/softmax/renorm, gate/up + SiLU, down, weighted combine and the shared
expert.  The timed steps replay a hipGraph of the per-layer launches, the way
a decode loop runs in production; the plain-stream time is reported beside
it.  Steps cycle through --layers distinct
resident layer copies (default 48, ~44 GB) so successive steps read
different weights and the 256 MB Infinity Cache cannot serve them; inputs
are resident in HBM before the timed region.

Prints ONE JSON line.  value = microseconds per token per MoE layer (lower is
better); roofline = algorithmic HBM bytes per layer over the measured layer
time against the 8 TB/s HBM peak; cpu_baseline = the oracle (a C
restatement of the reference's sequential CPU path) timed on this host on a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "MoE layer µs/token + achieved HBM GB/s (% of peak), batch-1 decode"
HBM_PEAK_GBPS = 8000.0
SEED = 20261201


class HipEvents:
    """hipEvent timing on an explicit stream (the library's own stream)."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self):
        e = C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, ev, stream):
        assert self.hip.hipEventRecord(ev, C.c_void_p(stream)) == 0

    def capture(self, stream, fn):
        """Record fn's launches on `stream` into an instantiated hipGraph."""
        self.hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p,
                                                 C.c_size_t]
        self.hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        assert self.hip.hipStreamBeginCapture(C.c_void_p(stream), 0) == 0
        fn()
        g = C.c_void_p()
        assert self.hip.hipStreamEndCapture(C.c_void_p(stream), C.byref(g)) == 0
        ge = C.c_void_p()
        assert self.hip.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
        return ge

    def launch_graph(self, ge, stream):
        assert self.hip.hipGraphLaunch(ge, C.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.hip.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return float(ms.value)


def build_layers(ctx, cfg, n_layers: int, tokens: int, centred: bool = False):
    from pb_amd import abi, synth
    from pb_amd.flashmoe import MoeLayer

    lay = abi.q4_layout_fixed(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype)
    layers = []
    for l in range(n_layers):
        slots = ctx.array(cfg.experts * lay.expert_bytes, np.uint8)
        abi.check(abi.lib().pbmoe_synth_fill_q4(ctx.handle, slots.ptr, C.byref(lay), cfg.hidden, cfg.intermediate,
                                                SEED, synth.T_EXPERT, l, 0, cfg.experts))
        if centred:
            abi.check(abi.lib().pbmoe_synth_center_q4(ctx.handle, slots.ptr, C.byref(lay), cfg.hidden,
                                                      cfg.intermediate, cfg.experts))
        host = synth.make_layer(cfg, SEED, l, abi.q4_layout_fixed, with_slots=False)
        router = ctx.to_device(host.router_f16)
        bias = ctx.to_device(host.selection_bias) if host.selection_bias is not None else None
        shared = ctx.to_device(host.shared_slot) if cfg.shared_intermediate else None
        gate = ctx.to_device(host.shared_gate_f16) if host.shared_gate_f16 is not None else None
        m = MoeLayer(ctx, l, cfg, lay).bind_device(slots, router, bias, host.shared_layout, shared, gate)
        layers.append((m, host))
    ctx.sync()
    return lay, layers


def cpu_baseline(cfg, host_layers, tokens: int, budget_s: float, threads: int):
    """Time the oracle (sequential reference restatement) on a bounded sample:
    route + expert phase for single tokens of the same workload."""
    from oracle import oracle as orc
    from pb_amd import abi, synth

    lay = abi.q4_layout_fixed(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype)
    olay = orc.make_layout(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype, lay.offsets, int(lay.expert_bytes))
    samples = []
    # pre-generate inputs and the host slots each sampled token needs (untimed)
    for i in range(64):
        host = host_layers[i % len(host_layers)]
        route_kw = dict(kind=cfg.routing, order=orc.ORDER_CANONICAL if cfg.routing >= 2 else orc.ORDER_REFERENCE_SLOT,
                        bias=host.selection_bias, n_group=cfg.n_group, topk_group=cfg.topk_group,
                        policy=cfg.normalization, routed_scale=cfg.routed_scale)
        xh, rh = synth.activations(SEED + 17, i, tokens, cfg.hidden)
        logits = np.stack([orc.router_logits(host.router_f16, xh[t]) for t in range(tokens)])
        ids, w = orc.route_rows(logits, cfg.k, **route_kw)
        uniq = sorted(set(int(e) for e in ids.ravel()))
        slots = np.concatenate([synth.q4_experts(SEED, synth.T_EXPERT, host.layer, e, 1, cfg.hidden, cfg.intermediate,
                                                 cfg.group, cfg.sb_dtype, lay.offsets, int(lay.expert_bytes))
                                for e in uniq])
        remap = {e: j for j, e in enumerate(uniq)}
        sl = None
        if host.shared_layout is not None:
            sl = orc.make_layout(cfg.hidden, cfg.shared_intermediate, cfg.group, cfg.sb_dtype,
                                 host.shared_layout.offsets, int(host.shared_layout.expert_bytes))
        samples.append((host, xh, rh, np.vectorize(remap.get)(ids).astype(np.int32), len(uniq), slots, sl, route_kw))
    done, t_total = 0, 0.0
    while t_total < budget_s and done < 4096:
        host, xh, rh, rid, nu, slots, sl, route_kw = samples[done % len(samples)]
        t0 = time.perf_counter()
        logits = np.stack([orc.router_logits_mt(host.router_f16, xh[t], orc.DT_F16, threads) for t in range(tokens)])
        _, w = orc.route_rows(logits, cfg.k, **route_kw)
        orc.moe_block(olay, slots, nu, xh, rh, rid, w, shared_layout=sl, shared_slot=host.shared_slot,
                      shared_gate_w=host.shared_gate_f16, threads=threads)
        t_total += time.perf_counter() - t0
        done += 1
    us = t_total / done / tokens * 1e6
    how = "one thread (the reference's sequential loop)" if threads == 1 else \
        f"{threads} OpenMP threads over router rows and (token, expert) jobs"
    return {"value": round(us, 3), "unit": "us/token/layer", "cores": threads, "kind": "port",
            "sample": f"{done} single-call layers x {tokens} token(s) of the same config "
                      f"({t_total:.1f} s, oracle router+routing+experts+combine, {how})"}


def host_cores() -> int:
    """Threads of the all-cores baseline: OMP_NUM_THREADS where set (the GPU
    box sets it to the CPU share one GPU's job may use), else every CPU this
    process may run on."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = int(env)
    return max(1, n)


def cpu_baselines(cfg, host_layers, tokens: int, budget_s: float) -> dict:
    """The oracle on all the job's cores (the reported baseline) and on one
    core (the reference's own sequential path), each on about `budget_s` of
    work; the record names the host's CPU count beside the threads used."""
    cores = host_cores()
    one = cpu_baseline(cfg, host_layers, tokens, budget_s, 1)
    host = {"nproc": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "threads_rule": "OMP_NUM_THREADS where set (the CPU share of one GPU's job on the GPU box), "
                            "else every CPU of the process's affinity mask"}
    if cores == 1:
        one["host"] = host
        return one
    rec = cpu_baseline(cfg, host_layers, tokens, budget_s, cores)
    rec["single_core"] = one
    rec["host"] = host
    return rec


KERNEL_NAMES = {"stage": "router_stage_kernel", "gateup": "route_gateup_kernel", "down": "down_rows_kernel"}


def load_traffic(phase: str, workload: str):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC
    summary (written by --pmc-summary ... --traffic-out), or None when no
    summary covers this kernel/workload."""
    path = os.path.join(ROOT, "profiles", "decode_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        ent = rec[workload][KERNEL_NAMES[phase]]
        return int(ent["traffic_bytes"]), "profiles/decode_traffic.json"
    except (OSError, KeyError, ValueError, TypeError):
        return None, None


def copy_calibration(ctx, mb: int, reps: int) -> None:
    """A plain device-to-device copy of known size on the library stream
    (the runtime's copy kernel): the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters of a PMC run to bytes."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    n = mb << 20
    src, dst = ctx.array(n, np.uint8), ctx.array(n, np.uint8)
    for _ in range(reps):
        assert hip.hipMemcpyAsync(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), n, 3, C.c_void_p(ctx.stream())) == 0
    ctx.sync()
    print(f"[bench] copy calibration: {reps} x {n} bytes device-to-device", file=sys.stderr, flush=True)


def read_calibration(ctx, mb: int, reps: int) -> None:
    """pbmoe_stream_read over a device buffer of known size (16-byte lane
    loads, the access shape of the decode weight reads): the reference
    point for the read-traffic counters of a PMC run."""
    from pb_amd import abi
    n = mb << 20
    src, out = ctx.array(n, np.uint8), ctx.array(1, np.uint32)
    for _ in range(reps):
        abi.check(abi.lib().pbmoe_stream_read(ctx.handle, src.ptr, n, out.ptr))
    ctx.sync()
    print(f"[bench] read calibration: {reps} x {n} bytes", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# rocprofv3 PMC summaries (--pmc-summary): per-kernel means of the counters
# of one or more rocprofv3 output directories (rocpd SQLite databases)
# ---------------------------------------------------------------------------
SIMD_NUM = 1024  # MI355X: 256 CUs x 4 SIMDs
XCD_NUM = 8      # rocpd stores GRBM_GUI_ACTIVE summed over the 8 XCDs of a dispatch
CALIB_READ_KERNEL, CALIB_COPY_KERNEL = "stream_read_kernel", "__amd_rocclr_copyBuffer"


def _short_kernel(name: str) -> str:
    base = name.split("(")[0].replace("void ", "").strip()
    return base.split("::")[-1] if "::" in base else base


def pmc_collect(dirs) -> dict:
    """{kernel (template arguments kept): {"dispatches": n, "duration_us": mean,
    counter: mean value per dispatch, ...}} over every *_results.db under dirs."""
    import glob
    import sqlite3
    vals: dict = {}
    for d in dirs:
        for db in sorted(glob.glob(os.path.join(d, "**", "*_results.db"), recursive=True)):
            con = sqlite3.connect(db)
            for kname, cname, v, dur, did in con.execute(
                    "select kernel_name, counter_name, value, duration, dispatch_id from counters_collection"):
                k = vals.setdefault(_short_kernel(kname), {"_disp": {}, "_ctr": {}})
                k["_disp"][(db, did)] = dur
                k["_ctr"].setdefault(cname, {}).setdefault((db, did), 0.0)
                k["_ctr"][cname][(db, did)] += v  # instances of one dispatch are summed
            con.close()
    out = {}
    for kname, k in vals.items():
        rec = {"dispatches": len(k["_disp"]), "duration_us": float(np.mean(list(k["_disp"].values()))) / 1e3,
               "max": {}}
        for cname, per in k["_ctr"].items():
            rec[cname] = float(np.mean(list(per.values())))
            rec["max"][cname] = float(np.max(list(per.values())))
        out[kname] = rec
    return out


def _read_bytes(r: dict):
    """FETCH_SIZE's request terms: 128-byte (TCC_BUBBLE), 32-byte and the
    remaining 64-byte requests of TCC_EA0_RDREQ."""
    b, r32, rall = r.get("TCC_BUBBLE_sum"), r.get("TCC_EA0_RDREQ_32B_sum"), r.get("TCC_EA0_RDREQ_sum")
    if b is None or r32 is None or rall is None:
        return None
    return 128.0 * b + 64.0 * (rall - b - r32) + 32.0 * r32


def _write_bytes(r: dict):
    w, w64 = r.get("TCC_EA0_WRREQ_sum"), r.get("TCC_EA0_WRREQ_64B_sum")
    if w is None or w64 is None:
        return None
    return 64.0 * w64 + 32.0 * (w - w64)


def _find(summary: dict, needle: str):
    return next((v for k, v in summary.items() if needle in k), None)


def pmc_derive(summary: dict, read_cal_bytes: int = 0, copy_cal_bytes: int = 0) -> dict:
    """Derived per-kernel figures: MFMA busy (% of SIMD cycles), shader clock,
    VALU instructions per MFMA, and read/write bytes from the raw TCC request
    terms, scaled by the read-stream and copy calibration launches when
    present (known bytes over the bytes the same terms report for them)."""
    # the calibration launches are the largest dispatches of their kernels
    # (the runtime's copy kernel also serves the small uploads)
    cal = {}
    rk = _find(summary, CALIB_READ_KERNEL)
    if rk and read_cal_bytes and _read_bytes(rk["max"]):
        cal["read_scale"] = read_cal_bytes / _read_bytes(rk["max"])
    ck = _find(summary, CALIB_COPY_KERNEL)
    if ck and copy_cal_bytes and _write_bytes(ck["max"]):
        cal["write_scale"] = copy_cal_bytes / _write_bytes(ck["max"])
        if _read_bytes(ck["max"]):
            cal["copy_read_scale"] = copy_cal_bytes / _read_bytes(ck["max"])
    out = {"calibration": cal, "kernels": {}}
    for k, r in summary.items():
        d = {"dispatches": r["dispatches"], "duration_us": round(r["duration_us"], 3)}
        gui = r.get("GRBM_GUI_ACTIVE")
        if gui:
            gui /= XCD_NUM  # cycles of one XCD
            d["clock_ghz"] = round(gui / (r["duration_us"] * 1e3), 3)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in r:
                d["mfma_busy_pct"] = round(100.0 * r["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * SIMD_NUM), 2)
        if r.get("SQ_INSTS_MFMA"):
            if "SQ_INSTS_VALU" in r:
                d["valu_per_mfma"] = round((r["SQ_INSTS_VALU"] - r["SQ_INSTS_MFMA"]) / r["SQ_INSTS_MFMA"], 2)
            if "SQ_INSTS_LDS" in r:
                d["lds_per_mfma"] = round(r["SQ_INSTS_LDS"] / r["SQ_INSTS_MFMA"], 3)
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in r:
            d["mfma_f16_tflops"] = round(r["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512 / (r["duration_us"] * 1e-6) / 1e12, 1)
        rb, wb = _read_bytes(r), _write_bytes(r)
        if rb is not None:
            d["read_bytes_counted"] = int(rb)
            if "read_scale" in cal:
                d["read_bytes"] = int(rb * cal["read_scale"])
        if wb is not None:
            d["write_bytes_counted"] = int(wb)
            if "write_scale" in cal:
                d["write_bytes"] = int(wb * cal["write_scale"])
        for c in r:
            if c not in ("dispatches", "duration_us", "max"):
                d[c] = round(r[c], 1)
        out["kernels"][k] = d
    return out


def write_traffic(rec: dict, config: str, tokens: int, path: str) -> None:
    """Per decode kernel of `config`: calibrated read + write bytes per launch
    beside the algorithmic bytes (configs.decode_phase_bytes)."""
    from pb_amd.configs import CONFIGS, decode_phase_bytes
    cfg = CONFIGS[config]
    alg = decode_phase_bytes(cfg, cfg.k, tokens)
    cal = rec["calibration"]
    if "read_scale" not in cal or "write_scale" not in cal:
        raise SystemExit("traffic needs both calibration launches (--read-calibration-mb, --copy-calibration-mb)")
    ent = {}
    for phase, kname in KERNEL_NAMES.items():
        k = next((v for n, v in rec["kernels"].items() if n.startswith(kname)), None)
        if k is None or "read_bytes" not in k or "write_bytes" not in k:
            continue
        t = k["read_bytes"] + k["write_bytes"]
        ent[kname] = {"read_bytes": k["read_bytes"], "write_bytes": k["write_bytes"], "traffic_bytes": t,
                      "algorithmic_bytes": alg[phase], "traffic_over_algorithmic": round(t / alg[phase], 3),
                      "dispatches": k["dispatches"]}
    out = {config: ent, "calibration": {
        "method": "TCC_EA0_RDREQ / RDREQ_32B / TCC_BUBBLE and TCC_EA0_WRREQ / WRREQ_64B per dispatch, as bytes "
                  "by FETCH_SIZE's and WRITE_SIZE's request sizes, each scaled by known-size reference launches "
                  "(pbmoe_stream_read: reads; runtime copy: writes)",
        "read_scale": round(cal["read_scale"], 4), "write_scale": round(cal["write_scale"], 4),
        "copy_read_scale": round(cal.get("copy_read_scale", float("nan")), 4)}, "sources": rec["sources"]}
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"[bench] traffic written to {path}", file=sys.stderr)


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16


def prefill_flops(cfg, tokens: int, routes: int) -> dict:
    """Algorithmic flops of the grouped prefill GEMMs (2 per multiply-add):
    gate/up 2 x 2*H*I per routed row (+ shared rows), down 2*H*I per row."""
    H, I, Is = cfg.hidden, cfg.intermediate, cfg.shared_intermediate
    rows_sh = tokens if Is else 0
    gateup = 2 * 2 * H * (routes * I + rows_sh * Is)
    down = 2 * H * (routes * I + rows_sh * Is)
    return {"gateup": gateup, "down": down}


def bench_prefill(args, cfg, ctx, ev) -> dict:
    """Layer-major prefill of T tokens through one MoE layer per step
    (pbmoe_moe_prefill: dispatch plan, grouped gate/up GEMM + SwiGLU,
    grouped down GEMM, combine).  C3 routes come from Zipf(1.1)-drawn router
    logits; other configs route x through the bound router."""
    from pb_amd import abi, synth
    T = args.tokens if args.tokens > 1 else cfg.tokens
    stream = ctx.stream()
    L = max(1, min(args.layers, 4))
    lay, layers = build_layers(ctx, cfg, L, T)
    xh, rh = synth.activations(SEED, 303, T, cfg.hidden)
    x, res = ctx.to_device(xh), ctx.to_device(rh)
    ids = ctx.array((T, cfg.k), np.uint32)
    w = ctx.array((T, cfg.k), np.float32)
    out = ctx.array((T, cfg.hidden), np.float32)
    if cfg.name.startswith("c3"):
        logits_h, _ = synth.drawn_logits_zipf(SEED, 0, T, cfg.experts, cfg.k, 1.1)
        layers[0][0].route_logits(ctx.to_device(logits_h), ids, w)
    else:
        layers[0][0].route(x, ids, w)
    ctx.sync()

    def step(i):
        layers[i % L][0].qwen_layer_major_experts(x, res, ids, w, out)

    for i in range(args.warmup):
        step(i)
    ctx.sync()
    K = max(20, args.steps)
    marks = [ev.create() for _ in range(K + 1)]
    ev.record(marks[0], stream)
    for i in range(K):
        step(i)
        ev.record(marks[i + 1], stream)
    ctx.sync()
    per_step = np.asarray([ev.elapsed_ms(marks[i], marks[i + 1]) * 1e3 for i in range(K)])
    us_step = float(np.median(per_step))
    spread = {"median_us": round(us_step, 3), "min_us": round(float(per_step.min()), 3),
              "max_us": round(float(per_step.max()), 3), "steps": K}
    n_ph = min(K, 64)
    evs = [[ev.create() for _ in range(6)] for _ in range(n_ph)]
    for i in range(n_ph):
        arr = (C.c_void_p * 6)(*[e.value for e in evs[i]])
        abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, arr, 6))
        step(i)
    abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, None, 0))
    ctx.sync()
    names = ("gateup", "down", "combine")
    phase_us = {nm: float(np.mean([ev.elapsed_ms(e[2 * j], e[2 * j + 1]) * 1e3 for e in evs]))
                for j, nm in enumerate(names)}
    fl = prefill_flops(cfg, T, T * cfg.k)
    kernels = {nm: {"us": round(phase_us[nm], 3)} for nm in names}
    # the GEMMs issue the activation hi and lo products; the gate/up GEMM skips
    # the lo products of tiles whose activations are all f16 values (lo == 0)
    x_f16 = bool(np.array_equal(xh.astype(np.float16).astype(np.float32), xh))
    issue = {"gateup": 1 if x_f16 else 2, "down": 2}
    for nm in ("gateup", "down"):
        tf = fl[nm] / (phase_us[nm] * 1e-6) / 1e12
        kernels[nm].update({"flops": fl[nm], "TFLOPs": round(tf, 1), "mfma_issued_TFLOPs": round(issue[nm] * tf, 1)})
    total_tf = (fl["gateup"] + fl["down"]) / (us_step * 1e-6) / 1e12
    print(f"[bench] prefill {cfg.name} T={T}: {us_step:.1f} us/layer, {total_tf:.1f} TFLOP/s; kernels (us): "
          + ", ".join(f"{k} {v:.1f}" for k, v in phase_us.items()), file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_prefill_baseline(cfg, layers[0][1], xh, rh, ids.download().astype(np.int32), w.download(),
                                   args.cpu_seconds)
    g = kernels["gateup"]
    return {
        "metric": "MoE layer prefill µs/token + MFMA utilisation",
        "value": round(us_step / T, 4),
        "unit": "us/token/layer",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "spread": spread,
        "timing": "median over the steps, each bracketed by hipEvents (back to back on the library stream)",
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (exact 4-bit codes x f16 hi+lo activations; lo products skipped where the "
                 "activations are f16 values), f32 accumulate",
        "data": "synthetic",
        "config": {"workload": cfg.name, "tokens": T, "hidden": cfg.hidden, "experts": cfg.experts, "k": cfg.k,
                   "intermediate": cfg.intermediate, "shared_intermediate": cfg.shared_intermediate,
                   "quant": f"q4 affine g{cfg.group}", "layers_cycled": L},
        "tokens_per_s": round(T / (us_step * 1e-6), 1),
        "expert_TFLOPs": round(total_tf, 1),
        "roofline": {"bound": "mfma", "achieved": g["TFLOPs"], "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(g["TFLOPs"] / MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "q4_gemm_t128_kernel (gate/up)", "flops_per_launch": g["flops"],
                     "launch_us": g["us"], "mfma_issued_frac": round(g["mfma_issued_TFLOPs"] / MFMA_PEAK_TFLOPS, 4),
                     "activations_f16_valued": x_f16},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }


def cpu_prefill_baseline(cfg, host, xh, rh, ids_h, w_h, budget_s: float):
    """The oracle's expert phase for a bounded sample of the same routed
    tokens (one thread), per token."""
    from oracle import oracle as orc
    from pb_amd import abi, synth
    lay = abi.q4_layout_fixed(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype)
    olay = orc.make_layout(cfg.hidden, cfg.intermediate, cfg.group, cfg.sb_dtype, lay.offsets, int(lay.expert_bytes))
    slots = synth.q4_experts(SEED, synth.T_EXPERT, host.layer, 0, cfg.experts, cfg.hidden, cfg.intermediate, cfg.group,
                             cfg.sb_dtype, lay.offsets, int(lay.expert_bytes))
    sl = None
    if host.shared_layout is not None:
        sl = orc.make_layout(cfg.hidden, cfg.shared_intermediate, cfg.group, cfg.sb_dtype,
                             host.shared_layout.offsets, int(host.shared_layout.expert_bytes))
    done, t_total, chunk = 0, 0.0, 8
    while t_total < budget_s and done + chunk <= xh.shape[0]:
        r = slice(done, done + chunk)
        t0 = time.perf_counter()
        orc.moe_block(olay, slots, cfg.experts, xh[r], rh[r], ids_h[r], w_h[r], shared_layout=sl,
                      shared_slot=host.shared_slot, shared_gate_w=host.shared_gate_f16, threads=1)
        t_total += time.perf_counter() - t0
        done += chunk
    return {"value": round(t_total / done * 1e6, 1), "unit": "us/token/layer", "cores": 1, "kind": "port",
            "sample": f"{done} tokens of the same routed chunk through the oracle expert phase ({t_total:.1f} s)"}


def stack_bytes_per_token(acfg, mcfg, layers: int, position: int) -> dict:
    """Algorithmic HBM bytes of one token through the C4 stack: per layer the
    four attention projections, the KV rows 0..position (f16 keys and
    values), and the MoE layer (router, the K selected experts)."""
    from pb_amd.configs import algorithmic_bytes, q4_proj_bytes
    H, g = acfg.hidden, acfg.group
    attn = (q4_proj_bytes(acfg.q_width, H, g) + 2 * q4_proj_bytes(acfg.kv_width, H, g)
            + q4_proj_bytes(H, acfg.q_width, g) + (position + 1) * acfg.kv_width * 2 * 2 + 6 * H * 4)
    moe = algorithmic_bytes(mcfg, mcfg.k, 1, fused_norm=True)
    return {"attention": attn * layers, "moe": moe * layers, "total": (attn + moe) * layers}


STACK_KERNELS = ("qkv_rows", "attn_chunk", "attn_merge", "o_rows", "router_stage", "route_gateup", "down")


def stack_kernel_times(ctx, ev, token, layers: int, tokens: int = 4) -> dict:
    """Mean duration of each kernel of a stack layer over `tokens` eager
    tokens: 14 hipEvents per layer call attached to the dispatch packets
    (pbmoe_set_phase_events; the first 6 time the MoE layer's three kernels,
    the other 8 the four attention kernels)."""
    from pb_amd import abi
    sets = [[ev.create() for _ in range(14)] for _ in range(tokens * layers)]
    it = iter(sets)

    def arm():
        arr = (C.c_void_p * 14)(*[e.value for e in next(it)])
        abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, arr, 14))

    for _ in range(tokens):
        token(arm=arm)
    abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, None, 0))
    ctx.sync()
    order = (6, 8, 10, 12, 0, 2, 4)  # start event of each kernel in STACK_KERNELS order
    return {nm: float(np.mean([ev.elapsed_ms(e[i], e[i + 1]) * 1e3 for e in sets]))
            for nm, i in zip(STACK_KERNELS, order)}


def bench_stack(args, ctx, ev) -> dict:
    """Workload C4: one token through the 48-layer decode stack —
    per layer the GQA attention block (pbmoe_attention_decode: input RMSNorm
    inside the q/k/v projection, q/k norm + RoPE, f16 KV cache at context
    4096, o_proj + residual) and the C1 MoE layer (pbmoe_moe_layer_norm: the
    post-attention RMSNorm inside the router stage).  --stack-norms split
    runs the two norms as separate passes instead (post_normed output of the
    attention call, next-layer norm fused into the MoE combine), for
    comparison.  KV rows 0..4094 hold synthetic f16 values, the timed token
    is position 4095; expert and attention weights are seeded zero-mean 4-bit
    (the stack's activations stay bounded across 48 layers).  The timed steps
    replay a hipGraph of one token's launches."""
    from pb_amd import abi, synth
    from pb_amd.configs import C1, C4_ATTN, C4_LAYERS
    from pb_amd.flashmoe import AttentionLayer

    acfg, mcfg, L = C4_ATTN, C1, C4_LAYERS
    H, pos = acfg.hidden, acfg.max_context - 1
    stream = ctx.stream()
    t_setup = time.perf_counter()
    _, moes = build_layers(ctx, mcfg, L, 1, centred=True)
    atts = [AttentionLayer(ctx, l, acfg).bind_synth(SEED, l) for l in range(L)]
    rng = np.random.default_rng(SEED)
    keys = rng.standard_normal((pos, acfg.kv_width)).astype(np.float16)
    vals = rng.standard_normal((pos, acfg.kv_width)).astype(np.float16)
    for a in atts:
        kp, vp = a.kv_cache()
        abi.check(abi.lib().pbmoe_upload(ctx.handle, kp, keys.ctypes.data, keys.nbytes))
        abi.check(abi.lib().pbmoe_upload(ctx.handle, vp, vals.ctypes.data, vals.nbytes))
    h0, _ = synth.activations(SEED, 4000, 1, H)
    w0 = atts[0].input_norm_h
    x0 = (h0 / np.sqrt(np.mean(h0 * h0) + acfg.eps) * w0).astype(np.float32)
    x_a, h_a = ctx.to_device(x0), ctx.to_device(h0)
    x_b, h_b = ctx.array((1, H), np.float32), ctx.array((1, H), np.float32)
    mid, post = ctx.array((1, H), np.float32), ctx.array((1, H), np.float32)
    ids = ctx.array((1, mcfg.k), np.uint32)
    wts = ctx.array((1, mcfg.k), np.float32)
    ctx.sync()
    print(f"[bench] stack setup {time.perf_counter() - t_setup:.1f} s: {L} layers, context {pos + 1}",
          file=sys.stderr, flush=True)

    fused = args.stack_norms == "fused"

    def token(parts=("attn", "moe"), arm=None):
        bufs = ((x_a, h_a), (x_b, h_b))
        for l in range(L):
            (x, h), (xn, hn) = bufs[l % 2], bufs[(l + 1) % 2]
            if arm is not None:
                arm()
            if fused:
                if "attn" in parts:
                    atts[l].decode(h, h, pos, mid, input_norm=atts[l].input_norm)
                if "moe" in parts:
                    moes[l][0].forward_norm(mid, atts[l].post_norm, hn, ids, wts)
                continue
            if "attn" in parts:
                atts[l].decode(x, h, pos, mid, post_norm=atts[l].post_norm, post_normed=post)
            if "moe" in parts:
                moes[l][0].forward(post, mid, hn, ids, wts, next_norm=atts[(l + 1) % L].input_norm, next_normed=xn)

    for _ in range(args.warmup):
        token()
    ctx.sync()
    res = {}
    K = max(20, args.steps)
    spread = {}
    for name, parts in (("token", ("attn", "moe")), ("attention", ("attn",)), ("moe", ("moe",))):
        graph = ev.capture(stream, lambda: token(parts))
        ev.launch_graph(graph, stream)
        ctx.sync()
        marks = [ev.create() for _ in range(K + 1)]
        ev.record(marks[0], stream)
        for i in range(K):
            ev.launch_graph(graph, stream)
            ev.record(marks[i + 1], stream)
        ctx.sync()
        per = np.asarray([ev.elapsed_ms(marks[i], marks[i + 1]) for i in range(K)])
        res[name] = float(np.median(per))
        spread[name] = {"median_ms": round(res[name], 4), "min_ms": round(float(per.min()), 4),
                        "max_ms": round(float(per.max()), 4)}
    ms = res["token"]
    nbytes = stack_bytes_per_token(acfg, mcfg, L, pos)
    gbps = nbytes["total"] / (ms * 1e-3) / 1e9
    print(f"[bench] stack: {ms:.3f} ms/token ({1e3 / ms:.1f} tokens/s); attention-only {res['attention']:.3f} ms, "
          f"MoE-only {res['moe']:.3f} ms; {gbps:.0f} GB/s", file=sys.stderr, flush=True)
    kernels_us = stack_kernel_times(ctx, ev, token, L)
    print("[bench] stack kernels (us, eager, per layer): "
          + ", ".join(f"{k} {v:.2f}" for k, v in kernels_us.items()), file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_stack_baseline(acfg, mcfg, [h for _, h in moes[:2]], pos, keys, vals, args.cpu_seconds)
    return {
        "metric": "decode stack tokens/s (48 layers: GQA attention + MoE), batch 1",
        "value": round(1e3 / ms, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "spread": spread,
        "timing": f"median over {K} back-to-back replays of one token's hipGraph, each bracketed by hipEvents",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (f16 KV cache, 4-bit weights)",
        "data": "synthetic",
        "config": {"workload": "c4_stack_decode", "layers": L, "context": pos + 1, "hidden": H,
                   "norms": args.stack_norms,
                   "q_heads": acfg.q_heads, "kv_heads": acfg.kv_heads, "head_dim": acfg.head_dim,
                   "experts": mcfg.experts, "k": mcfg.k, "intermediate": mcfg.intermediate,
                   "quant": "q4 affine g64 f16 scale/bias (zero-mean)"},
        "tokens_per_s": round(1e3 / ms, 2),
        "phase_ms": {"attention_only": round(res["attention"], 4), "moe_only": round(res["moe"], 4)},
        "kernels_us": {k: round(v, 3) for k, v in kernels_us.items()},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "whole token (all kernels of the 48 layers)", "bytes_per_token": nbytes["total"],
                     "bytes_attention": nbytes["attention"], "bytes_moe": nbytes["moe"]},
        "cpu_baseline": cpu,
    }


def cpu_stack_baseline(acfg, mcfg, host_layers, pos: int, keys, vals, budget_s: float):
    """The oracle on a bounded sample of the stack: attention layers at the
    same context (or_attention_decode) and MoE layers (router + routing +
    experts + combine), each timed for about half the budget; the per-token
    figure is 48 x (attention layer + MoE layer)."""
    from oracle import oracle as orc
    from pb_amd import abi, synth
    from pb_amd.configs import C4_LAYERS

    mats = synth.attn_host_mats(acfg, SEED, 0, abi.q4_layout_fixed)
    qn, kn, _, _ = synth.attn_norms(acfg, SEED, 0)
    att = orc.AttnOracle(mats, qn, kn, acfg.hidden, acfg.q_heads, acfg.kv_heads, acfg.head_dim, acfg.rope_theta,
                         acfg.group, acfg.sb_dtype, acfg.max_context)
    att.cache_k[:pos] = keys.astype(np.float32)
    att.cache_v[:pos] = vals.astype(np.float32)
    x = synth.activations(SEED, 4001, 1, acfg.hidden)[0].ravel()
    n_att, t_att = 0, 0.0
    while t_att < budget_s / 2 and n_att < 64:
        t0 = time.perf_counter()
        att.decode(x, pos)
        t_att += time.perf_counter() - t0
        n_att += 1
    moe = cpu_baseline(mcfg, host_layers, 1, budget_s / 2, 1)
    per_layer_us = t_att / n_att * 1e6 + moe["value"]
    tok_s = 1e6 / (per_layer_us * C4_LAYERS)
    return {"value": round(tok_s, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{n_att} attention layers at context {pos + 1} ({t_att:.1f} s) + MoE: {moe['sample']}; "
                      f"per token = {C4_LAYERS} x {per_layer_us:.0f} us"}


NORM_SEED_TENSOR = 9001  # seeded input-RMSNorm weight of the chained decode bench


def decode_leg(ctx, ev, cfg, layers, T: int, K: int, R: int, warmup: int, phases: bool) -> dict:
    """Chained decode steps: step i runs the MoE layer on copy i mod L from
    the un-normalised hidden state h_i (pbmoe_moe_layer_norm: the input
    RMSNorm inside the router stage, h_i also the residual) and writes
    h_{i+1}, which step i + 1 reads, so every step waits for the one before
    it as a decode loop does.  Timed: a hipGraph of K chained steps replayed
    R times back to back (median replay); also the same K steps as one ABI
    call each, and (phases) the mean per-kernel durations from hipEvents on
    the dispatch packets over min(K, 512) eager steps."""
    from pb_amd import abi, synth
    H, L = cfg.hidden, len(layers)
    stream = ctx.stream()
    _, h0 = synth.activations(SEED, 999, T, H)
    nw = synth.uniform_f32(SEED, NORM_SEED_TENSOR, 0, 0, 0, H, 0.5, 1.0)
    hb = [ctx.to_device(h0), ctx.array((T, H), np.float32)]
    norm_w = ctx.to_device(nw)
    ids = ctx.array((T, cfg.k), np.uint32)
    w = ctx.array((T, cfg.k), np.float32)
    state = {"i": 0}  # global step index: buffer parity and layer copy

    def step():
        i = state["i"]
        layers[i % L][0].forward_norm(hb[i % 2], norm_w, hb[(i + 1) % 2], ids, w)
        state["i"] = i + 1

    for _ in range(warmup):
        step()
    ctx.sync()
    a, b = ev.create(), ev.create()
    ev.record(a, stream)
    for _ in range(K):
        step()
    ev.record(b, stream)
    us_stream = ev.elapsed_ms(a, b) * 1e3 / K
    ctx.sync()
    # one graph per (layer copy, buffer parity) a replay starts from; the
    # replays continue the chain where the previous one stopped
    i0 = state["i"]
    starts = [(i0 + r * K) for r in range(R)]
    graphs = {}
    for st in starts:
        key = (st % L, st % 2)
        if key not in graphs:
            state["i"] = st
            graphs[key] = ev.capture(stream, lambda: [step() for _ in range(K)])
    state["i"] = i0
    marks = [ev.create() for _ in range(R + 1)]
    ev.record(marks[0], stream)
    for r in range(R):
        ev.launch_graph(graphs[(starts[r] % L, starts[r] % 2)], stream)
        ev.record(marks[r + 1], stream)
    ctx.sync()
    state["i"] = i0 + R * K
    per_step = np.asarray([ev.elapsed_ms(marks[r], marks[r + 1]) * 1e3 / K for r in range(R)])
    us = float(np.median(per_step))
    spread = {"median_us": round(us, 3), "min_us": round(float(per_step.min()), 3),
              "max_us": round(float(per_step.max()), 3), "replays": R, "steps_per_replay": K}
    out = {"us": us, "us_stream": us_stream, "spread": spread,
           "timing": f"median over {R} back-to-back hipGraph replays of {K} chained layer steps each (step i on "
                     f"layer copy i mod {L}, its input the hidden state step i - 1 wrote; pbmoe_moe_layer_norm, "
                     "the input RMSNorm fused); stream_us_per_layer: the same chained steps as one ABI call each"}
    # per-kernel durations (events attached to the dispatch packets) and
    # the distinct experts the chained steps select
    n_ph = max(min(K, 512), 48) if phases else 16
    evs = [[ev.create() for _ in range(6)] for _ in range(n_ph)]
    uniq = []
    for j in range(n_ph):
        if phases:
            arr = (C.c_void_p * 6)(*[e.value for e in evs[j]])
            abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, arr, 6))
        step()
        if j < 16:
            ctx.sync()
            uniq.append(len(set(ids.download().ravel().tolist())))
    abi.check(abi.lib().pbmoe_set_phase_events(ctx.handle, None, 0))
    ctx.sync()
    out["unique"] = float(np.mean(uniq))
    out["phase_steps"] = n_ph
    if phases:
        out["phase_us"] = {name: float(np.mean([ev.elapsed_ms(e[2 * j], e[2 * j + 1]) * 1e3 for e in evs]))
                           for j, name in enumerate(("stage", "gateup", "down"))}
    print(f"[bench] {cfg.name} T={T}: {us:.2f} us/layer (graph, median of {R} replays of {K} chained steps; "
          f"min {per_step.min():.2f}, max {per_step.max():.2f}), {us_stream:.2f} us/layer (stream); "
          f"unique experts {out['unique']:.1f}"
          + ("; kernels (us): " + ", ".join(f"{k} {v:.2f}" for k, v in out["phase_us"].items()) if phases else ""),
          file=sys.stderr, flush=True)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480,
                    help="steps timed per replay (decode: MoE layers; c4_stack: tokens; prefill: layer calls)")
    ap.add_argument("--replays", type=int, default=20, help="timed replays of the --steps steps (at least 20)")
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="c2_qwen3next_decode")
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stack-norms", choices=("fused", "split"), default="fused",
                    help="c4_stack: RMSNorms inside the projection/router kernels, or as separate passes")
    ap.add_argument("--prefill", action="store_true",
                    help="layer-major prefill of --tokens (default: the config's) instead of decode")
    ap.add_argument("--headline-only", action="store_true",
                    help="decode: time the headline shape only (no C2 4/8-token and C3 prefill legs)")
    ap.add_argument("--expert-phase", action="store_true",
                    help="also time pbmoe_moe_decode alone (routes fixed)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run a plain device copy of this size (PMC calibration runs)")
    ap.add_argument("--read-calibration-mb", type=int, default=0,
                    help="also run pbmoe_stream_read over a buffer of this size (PMC calibration runs)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 PMC output directories instead of benchmarking (no GPU)")
    ap.add_argument("--pmc-out", help="with --pmc-summary: also write the JSON summary to this file")
    ap.add_argument("--traffic-out", help="with --pmc-summary over a decode run of --config: write the per-kernel "
                                          "HBM traffic file that the roofline's traffic field reads")
    args = ap.parse_args()

    if args.pmc_summary:
        rec = pmc_derive(pmc_collect(args.pmc_summary), args.read_calibration_mb << 20,
                         args.copy_calibration_mb << 20)
        rec["sources"] = args.pmc_summary
        txt = json.dumps(rec, indent=1, sort_keys=True)
        if args.pmc_out:
            with open(args.pmc_out, "w") as f:
                f.write(txt + "\n")
        print(txt)
        if args.traffic_out:
            write_traffic(rec, args.config, args.tokens, args.traffic_out)
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X only: the MoE block is single-GPU in this build "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        return 2

    from pb_amd import abi, synth
    from pb_amd.configs import CONFIGS, algorithmic_bytes, decode_phase_bytes, down_prefetch_bytes

    if args.config in ("c4_stack", "c4_stack_decode"):
        ctx = abi.Context(0)
        rec = bench_stack(args, ctx, HipEvents())
        print(json.dumps(rec))
        ctx.close()
        return 0
    cfg = CONFIGS[args.config]
    T = args.tokens
    ctx = abi.Context(0)
    ev = HipEvents()
    if args.prefill or cfg.name.startswith("c3"):
        rec = bench_prefill(args, cfg, ctx, ev)
        print(json.dumps(rec))
        ctx.close()
        return 0
    t_setup = time.perf_counter()
    lay, layers = build_layers(ctx, cfg, args.layers, T)
    print(f"[bench] setup {time.perf_counter() - t_setup:.1f} s, {args.layers} layers bound", file=sys.stderr,
          flush=True)
    K, R = args.steps, max(20, args.replays)
    head = decode_leg(ctx, ev, cfg, layers, T, K, R, args.warmup, phases=True)
    us_step = head["us"]
    bytes_layer = algorithmic_bytes(cfg, int(round(head["unique"])), T, fused_norm=True)
    gbps = bytes_layer / (us_step * 1e-6) / 1e9
    ph_bytes = decode_phase_bytes(cfg, int(round(head["unique"])), T, fused_norm=True)
    phase_us = head["phase_us"]
    kernels = {k: {"us": round(phase_us[k], 3), "bytes": ph_bytes[k],
                   "GBps": round(ph_bytes[k] / (phase_us[k] * 1e-6) / 1e9, 1)} for k in phase_us}
    dominant = max(phase_us, key=phase_us.get)
    dom_gbps = kernels[dominant]["GBps"]
    traffic, traffic_src = load_traffic(dominant, cfg.name)
    # route_gateup_kernel also touches the down weights of the selected
    # experts (prefetch for the down kernel); its traffic includes them
    pf_bytes = down_prefetch_bytes(cfg, int(round(head["unique"])), T) if dominant == "gateup" else 0

    us_expert = None
    if args.expert_phase:
        # expert phase alone (routes fixed, pbmoe_moe_decode)
        xh, rh = synth.activations(SEED, 999, T, cfg.hidden)
        x, res = ctx.to_device(xh), ctx.to_device(rh)
        ids = ctx.array((T, cfg.k), np.uint32)
        w = ctx.array((T, cfg.k), np.float32)
        out = ctx.array((T, cfg.hidden), np.float32)
        L = len(layers)
        for i in range(L):
            layers[i][0].route(x, ids, w)
        ctx.sync()
        a, b = ev.create(), ev.create()
        ev.record(a, ctx.stream())
        for i in range(args.steps):
            layers[i % L][0].submit_scheduled_expert_command(x, res, ids, w, out)
        ev.record(b, ctx.stream())
        us_expert = round(ev.elapsed_ms(a, b) * 1e3 / args.steps, 3)
        ctx.sync()

    # the other BASELINE shapes in the same run: C2 with 4 and 8 tokens on the
    # same resident layer copies, and the C3 prefill of 2048 tokens
    extra = {}
    if not args.headline_only and T == 1 and cfg.name == "c2_qwen3next_decode":
        for t_extra in (4, 8):
            leg = decode_leg(ctx, ev, cfg, layers, t_extra, K, R, args.warmup, phases=True)
            u = leg["unique"]
            nb = algorithmic_bytes(cfg, int(round(u)), t_extra, fused_norm=True)
            extra[f"c2_t{t_extra}"] = {
                "tokens": t_extra, "us_per_layer": round(leg["us"], 3),
                "us_per_token_layer": round(leg["us"] / t_extra, 3),
                "tokens_per_s": round(t_extra / (leg["us"] * 1e-6), 1),
                "unique_experts_mean": round(u, 2), "algorithmic_bytes": nb,
                "achieved_GBps": round(nb / (leg["us"] * 1e-6) / 1e9, 1),
                "hbm_frac": round(nb / (leg["us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                "kernels_us": {k: round(v, 3) for k, v in leg["phase_us"].items()},
                "spread": leg["spread"], "timing": leg["timing"]}
        pargs = argparse.Namespace(**vars(args))
        pargs.tokens, pargs.steps, pargs.warmup = 1, 40, 20
        pargs.cpu_seconds = min(args.cpu_seconds, 4.0)
        from pb_amd.configs import C3
        prec = bench_prefill(pargs, C3, ctx, ev)
        extra["c3_prefill"] = {
            "tokens": prec["config"]["tokens"], "us_per_layer": round(prec["ms_per_step"] * 1e3, 2),
            "us_per_token_layer": prec["value"], "tokens_per_s": prec["tokens_per_s"],
            "layer_TFLOPs": prec["expert_TFLOPs"],
            "layer_mfma_frac": round(prec["expert_TFLOPs"] / MFMA_PEAK_TFLOPS, 4),
            "gateup": prec["kernels"]["gateup"], "down": prec["kernels"]["down"],
            "combine": prec["kernels"]["combine"], "roofline": prec["roofline"],
            "spread": prec["spread"], "cpu_baseline": prec["cpu_baseline"], "timing": prec["timing"]}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baselines(cfg, [h for _, h in layers[:4]], T, args.cpu_seconds)

    rec = {
        "metric": METRIC,
        "value": round(us_step / T, 3),
        "unit": "us/token/layer",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg.name, "tokens": T, "hidden": cfg.hidden, "experts": cfg.experts, "k": cfg.k,
                   "intermediate": cfg.intermediate, "shared_intermediate": cfg.shared_intermediate,
                   "quant": "q4 affine g64 f16 scale/bias", "layers_cycled": len(layers)},
        "tokens_per_s": round(T / (us_step * 1e-6), 1),
        "achieved_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "expert_phase_us": us_expert,
        "stream_us_per_layer": round(head["us_stream"], 3),
        "timing": head["timing"],
        "spread": head["spread"],
        "roofline": {"bound": "hbm", "achieved": dom_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(dom_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": KERNEL_NAMES[dominant], "bytes_per_launch": ph_bytes[dominant],
                     "launch_us": kernels[dominant]["us"], "traffic_source": traffic_src,
                     "launch_us_source": "mean of hipEvents attached to this kernel's dispatch packets "
                                         f"(pbmoe_set_phase_events) over {head['phase_steps']} chained eager steps "
                                         "on the library stream",
                     "prefetch_bytes": pf_bytes},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    rec.update(extra)
    if args.copy_calibration_mb:
        copy_calibration(ctx, args.copy_calibration_mb, 3)
    if args.read_calibration_mb:
        read_calibration(ctx, args.read_calibration_mb, 3)
    print(json.dumps(rec))
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
