"""Throughput of the fused layer-op path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]

Headline workload: the T3 prefill op chain -- gather of 512 token rows from
an [8194,1024] f32 table plus learned position rows 0..511 (one fused
kernel), LayerNorm+affine over [512,1024], tanh-GELU over [512,4096].  One
step = one pass of that chain.  Inputs are synthetic (seeded), resident in
HBM before the timed region; each step uses the next of several buffer sets
whose combined footprint exceeds twice the 256 MB Infinity Cache, so the
bytes come from HBM.  Steps are replayed from HIP graphs (captured once),
timed with events on the launch stream.

Prints ONE JSON line on stdout.  value = algorithmic bytes per step /
time per step (GB/s).  roofline = the dominant kernel (GELU), timed per
launch with HIP events.  cpu_baseline = the oracle (a C restatement of
ggml-cpu's arithmetic) running the same chain on the host.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
MALL_DEFEAT_BYTES = 512 * 1024 * 1024


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--quick", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the launches used by the FETCH_SIZE/WRITE_SIZE counter runs")
    return ap.parse_args()


# --------------------------------------------------------------------------- #
# prebuilt calls: descriptors are built once, launches are plain ctypes calls
# --------------------------------------------------------------------------- #

class PrefillSet:
    """Device buffers + descriptors of one T3-prefill step."""

    def __init__(self, C, W, torch, inp, f16_table=False):
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
        tab = inp["table"].astype(np.float16) if f16_table else inp["table"]
        self.t = {
            "table": d(tab), "ids": d(inp["ids"]), "pos_table": d(inp["pos_table"]), "pos_ids": d(inp["pos_ids"]),
            "ln_w": d(inp["ln_w"]), "ln_b": d(inp["ln_b"]), "ffn": d(inp["ffn"]),
        }
        self.t["h"] = torch.empty((W.N_PREFILL, W.D_MODEL), dtype=torch.float32, device="cuda")
        self.t["ln"] = torch.empty_like(self.t["h"])
        self.t["g"] = torch.empty_like(self.t["ffn"])
        self.d = {k: C.desc(v) for k, v in self.t.items()}
        self.r = {k: C.ctypes.byref(v) for k, v in self.d.items()}
        self.L = C.load()
        self.C = C

    def gather(self, s):
        r = self.r
        return self.L.cbx_get_rows_add(r["table"], r["ids"], r["pos_table"], r["pos_ids"], r["h"], s)

    def layer_norm(self, s):
        r = self.r
        return self.L.cbx_layer_norm(r["h"], r["ln_w"], r["ln_b"], 1e-5, -1, r["ln"], s)

    def embed_layer_norm(self, s):
        r = self.r
        return self.L.cbx_get_rows_add_layer_norm(r["table"], r["ids"], r["pos_table"], r["pos_ids"], r["ln_w"],
                                                  r["ln_b"], 1e-5, r["h"], r["ln"], s)

    def gelu(self, s):
        return self.L.cbx_gelu(self.r["ffn"], self.r["g"], s)

    def step(self, s):
        """Fused chain: token+position gather with LayerNorm, then GELU."""
        rc = self.embed_layer_norm(s) | self.gelu(s)
        if rc:
            raise self.C.CbxError(rc, self.C.last_error())

    def step_unfused(self, s):
        rc = self.gather(s) | self.layer_norm(s) | self.gelu(s)
        if rc:
            raise self.C.CbxError(rc, self.C.last_error())


def cur_stream(torch):
    import ctypes

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def capture(torch, fn):
    """HIP graph of fn(stream) captured through torch."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn(cur_stream(torch))
    return g


def time_graph_steps(torch, graphs_all, graphs_one, n_sets, steps):
    """Replay exactly `steps` steps: whole rotations, then single-set graphs."""
    full, rem = divmod(steps, n_sets)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(full):
        graphs_all.replay()
    for i in range(rem):
        graphs_one[i].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def per_launch_ms(torch, fns, reps):
    """Average duration of one launch of a kernel in a back-to-back stream of
    its launches: one HIP graph holds a launch per buffer set (rotating
    inputs); it is replayed until `reps` launches have run, with events on
    the launch stream around the whole batch.  (An event pair around a
    single launch adds several microseconds of its own.)"""
    g = capture(torch, lambda s: [fn(s) for fn in fns])
    n_rep = max(1, reps // len(fns))
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n_rep):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (n_rep * len(fns))
    del g
    return ms


# --------------------------------------------------------------------------- #
# workloads
# --------------------------------------------------------------------------- #

def bench_prefill(C, W, torch, steps, warmup, f16_table=False, fused=True):
    inp = W.prefill_inputs(f16_table=False)
    nbytes = W.prefill_bytes(f16_table, fused)
    per_step = sum(nbytes.values())
    n_sets = max(2, math.ceil(MALL_DEFEAT_BYTES / per_step))
    log(f"prefill{' f16' if f16_table else ''}{'' if fused else ' unfused'}: {per_step} B/step, {n_sets} buffer sets")
    sets = [PrefillSet(C, W, torch, inp, f16_table) for _ in range(n_sets)]
    step = (lambda st: st.step) if fused else (lambda st: st.step_unfused)

    # eager pass + parity of set 0 against the oracle (the product path is the HIP library)
    from oracle import oracle as O

    for st in sets:
        step(st)(cur_stream(torch))
    torch.cuda.synchronize()
    tab = inp["table"].astype(np.float16) if f16_table else inp["table"]
    h_ref = O.get_rows_add(tab, inp["ids"], inp["pos_table"], inp["pos_ids"], nth=8)
    ln_ref = O.layer_norm(h_ref, inp["ln_w"], inp["ln_b"], 1e-5, nth=8)
    g_ref = O.unary(O.GELU, inp["ffn"], nth=8)
    for name, ref in (("h", h_ref), ("ln", ln_ref), ("g", g_ref)):
        got = sets[-1].t[name].cpu().numpy()
        if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
            raise SystemExit(f"bench: {name} differs from the oracle")

    g_all = capture(torch, lambda s: [step(st)(s) for st in sets])
    g_one = [capture(torch, step(st)) for st in sets]
    time_graph_steps(torch, g_all, g_one, n_sets, warmup)
    ms = time_graph_steps(torch, g_all, g_one, n_sets, steps)
    # replays must reproduce the eager result
    torch.cuda.synchronize()
    if not np.array_equal(sets[0].t["g"].cpu().numpy().view(np.uint32), g_ref.view(np.uint32)):
        raise SystemExit("bench: graph replay result differs")

    reps = 400
    if fused:
        k_ms = {"embed_layer_norm": per_launch_ms(torch, [st.embed_layer_norm for st in sets], reps),
                "gelu": per_launch_ms(torch, [st.gelu for st in sets], reps)}
    else:
        k_ms = {"gather_pos": per_launch_ms(torch, [st.gather for st in sets], reps),
                "layer_norm": per_launch_ms(torch, [st.layer_norm for st in sets], reps),
                "gelu": per_launch_ms(torch, [st.gelu for st in sets], reps)}
    del g_all, g_one, sets
    return {"ms_per_step": ms / steps, "bytes_per_step": per_step, "n_sets": n_sets,
            "kernel_ms": k_ms, "kernel_bytes": nbytes}


def bench_decode(C, W, torch, reps=200):
    """T3 decode step: RMSNorm+gamma [1,1024], RoPE q,k [1,16,64] at positions
    0..29, SiLU(gate)*up [1,4096]; 30 steps captured as one graph."""
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    L = C.load()
    cache = C.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    steps = []
    for s in range(30):
        t = {"x": d(W.normal(W.seed_of(1, 0) + s, (1, 1024))), "g": d(W.normal(W.seed_of(1, 1), (1024,), 1.0, 0.02)),
             "q": d(W.normal(W.seed_of(1, 2) + 97 * s, (1, 16, 64))),
             "k": d(W.normal(W.seed_of(1, 3) + 97 * s, (1, 16, 64))),
             "pos": d(np.array([s], dtype=np.int32)),
             "gate": d(W.normal(W.seed_of(1, 5) + s, (1, 4096))), "up": d(W.normal(W.seed_of(1, 6) + s, (1, 4096)))}
        t["y"] = torch.empty_like(t["x"])
        t["qo"], t["ko"], t["h"] = torch.empty_like(t["q"]), torch.empty_like(t["k"]), torch.empty_like(t["gate"])
        r = {k: C.ctypes.byref(C.desc(v)) for k, v in t.items()}
        steps.append((t, r))

    def run(s):
        for _, r in steps:
            rc = (L.cbx_rms_norm_mul(r["x"], r["g"], 1e-5, r["y"], s) |
                  L.cbx_rope_ext(r["q"], r["pos"], cache.handle, r["qo"], s) |
                  L.cbx_rope_ext(r["k"], r["pos"], cache.handle, r["ko"], s) |
                  L.cbx_swiglu(r["gate"], r["up"], r["h"], s))
            if rc:
                raise C.CbxError(rc, C.last_error())

    run(cur_stream(torch))
    g = capture(torch, run)
    for _ in range(10):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / (reps * 30)
    cache.close()
    return {"us_per_step_chain": us, "bytes_per_step": 77824 + 4}


def bench_snake(C, W, torch):
    """HiFT Snake on [16,64,120000] (ggml (C=64, T) channel innermost): 983 MB."""
    x = torch.empty((16, 120000, 64), dtype=torch.float32, device="cuda").normal_()
    y = torch.empty_like(x)
    a = torch.empty(64, device="cuda").uniform_(0.5, 1.5)
    ai = 1.0 / (a + 1e-9)
    L = C.load()
    r = [C.ctypes.byref(C.desc(v)) for v in (x, a, ai, y)]
    fn = lambda s: L.cbx_snake(r[0], r[1], r[2], r[3], s)  # noqa: E731
    fn(cur_stream(torch))
    ms = per_launch_ms(torch, [fn], 20)
    nbytes = 2 * x.numel() * 4 + 2 * 64 * 4
    return {"ms": ms, "bytes": nbytes, "GBps": nbytes / ms / 1e6}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gelu_512x4096_and_embed_ln_traffic.md")


def recorded_traffic(key):
    """HBM bytes per launch of a kernel as last measured with rocprofv3 --pmc
    FETCH_SIZE and WRITE_SIZE (copy-calibrated), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith(f"traffic_bytes_per_launch {key}:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def traffic_probe(C, W, torch):
    """A few launches for counter runs (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE):
    a plain f32 copy of 64 MiB (the calibration kernel of known size), then
    GELU [512,4096] and the fused embedding + LayerNorm on rotating buffer
    sets.  Prints the expected bytes of each."""
    x = torch.empty(16 << 20, dtype=torch.float32, device="cuda").uniform_()
    ys = [torch.empty_like(x) for _ in range(4)]
    L = C.load()
    s = cur_stream(torch)
    dx = C.ctypes.byref(C.desc(x))
    for y in ys:
        rc = L.cbx_cpy(dx, C.ctypes.byref(C.desc(y)), s)
        if rc:
            raise C.CbxError(rc, C.last_error())
    torch.cuda.synchronize()
    inp = W.prefill_inputs()
    sets = [PrefillSet(C, W, torch, inp) for _ in range(8)]
    for st in sets:
        st.gelu(s)
    torch.cuda.synchronize()
    for st in sets:
        st.embed_layer_norm(s)
    torch.cuda.synchronize()
    nb = W.prefill_bytes()
    print(json.dumps({"copy_bytes_read": x.numel() * 4, "copy_bytes_written": x.numel() * 4,
                      "gelu_bytes_read": nb["gelu"] // 2, "gelu_bytes_written": nb["gelu"] // 2,
                      "embed_layer_norm_bytes": nb["embed_layer_norm"]}), flush=True)


def cpu_baseline(W, seconds):
    """The oracle runs the same prefill chain on the host cores."""
    from oracle import oracle as O

    inp = W.prefill_inputs()
    per_step = sum(W.prefill_bytes(False).values())
    nth = max(1, min(16, os.cpu_count() or 1))
    reps = 0
    t0 = time.perf_counter()
    while True:
        h = O.get_rows_add(inp["table"], inp["ids"], inp["pos_table"], inp["pos_ids"], nth=nth)
        O.layer_norm(h, inp["ln_w"], inp["ln_b"], 1e-5, nth=nth)
        O.unary(O.GELU, inp["ffn"], nth=nth)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 100000:
            break
    return {"value": per_step * reps / el / 1e9, "unit": "GB/s", "cores": nth, "kind": "port",
            "sample": f"{reps} steps of the T3 prefill op chain (gather+pos f32, LayerNorm, GELU), "
                      f"{el:.1f} s, OpenMP row split as ggml-cpu"}


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this op path has no cross-GPU exchange and runs on one "
              "device; --gpus above 1 is not supported.", file=sys.stderr)
        return 2
    import torch

    from chatterbox_amdvulkan_amd import cbxops as C
    from chatterbox_amdvulkan_amd import workloads as W

    torch.cuda.set_device(0)
    C.init(0)
    if a.traffic_probe:
        traffic_probe(C, W, torch)
        return 0
    res = bench_prefill(C, W, torch, a.steps, a.warmup)
    details = {"prefill_f32_fused": {k: v for k, v in res.items()}}
    if not a.quick:
        def gbps(r):
            return r["bytes_per_step"] / (r["ms_per_step"] * 1e-3) / 1e9

        ru = bench_prefill(C, W, torch, max(200, a.steps // 4), 20, fused=False)
        details["prefill_f32_unfused"] = dict(ru, GBps=gbps(ru))
        r16 = bench_prefill(C, W, torch, max(200, a.steps // 4), 20, f16_table=True)
        details["prefill_f16_table_fused"] = dict(r16, GBps=gbps(r16))
        details["t3_decode"] = bench_decode(C, W, torch)
        details["hift_snake_16x64x120000"] = bench_snake(C, W, torch)
    k_ms = res["kernel_ms"]["gelu"]
    k_bytes = res["kernel_bytes"]["gelu"]
    achieved = k_bytes / (k_ms * 1e-3) / 1e9
    value = res["bytes_per_step"] / (res["ms_per_step"] * 1e-3) / 1e9
    out = {
        "metric": "fused-op HBM GB/s (% of peak) + T3 per-token norm/rope/act µs, 1 GPU",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "t3_prefill_op_chain",
                   "embed_layer_norm": "512 ids of [8194,1024] f32 + pos rows 0..511, then LayerNorm eps 1e-5 "
                                       "affine, one kernel writing h and LN(h)",
                   "gelu": "[512,4096] tanh (fp16-table semantics)",
                   "hbm_pct_of_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
                   "buffer_sets": res["n_sets"]},
        "roofline": {"bound": "hbm", "kernel": "gelu [512,4096] f32", "achieved": round(achieved, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": recorded_traffic("gelu_512x4096"),
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT),
                     "launch_ms": k_ms, "algorithmic_bytes": k_bytes},
    }
    if "t3_decode" in details:
        out["t3_decode_us_per_step_chain"] = round(details["t3_decode"]["us_per_step_chain"], 3)
    out["details"] = details
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(W, a.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
