#!/usr/bin/env python3
"""MoE-layer forward benchmark on one MI355X.

Workload (default): the full-size FP4 MoE layer at decode -- hidden 4096,
256 routed experts, top-8, expert intermediate 2048, one bf16 shared expert
of 2048, FP4 e2m1/E8M0 routed weights quantised from N(0, 0.02), sigmoid gate
with route scale 2.5, B = 1 token of bf16 N(0, 1).  All weights are resident
in HBM before timing.  A step is one layer forward; steps rotate over
``--layers`` independently drawn layers and ``--inputs`` token batches, so
that consecutive steps read different experts (more than the 256 MB
Infinity Cache per cycle).

Prints ONE JSON line: tokens/s of the layer (the metric), the roofline of
the dominant kernel (the routed + shared gate/up kernel: algorithmic bytes
per launch over its HIP-event-timed average duration), and a CPU baseline
(the oracle, timed on a bounded sample on this host's cores).

    python bench.py [--steps K] [--warmup W] [--tokens T] [--no-sweep] [--no-cpu]
    python bench.py --mode copy --bytes N      # plain copy kernel of known size
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "deepseeker-v4.1_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import dsk_moe  # noqa: E402
from dsk_moe import _lib  # noqa: E402
from dsk_moe import synth as gsynth  # noqa: E402
from dsk_moe.ops import make_desc, ptr, stream_of, workspace  # noqa: E402

METRIC = "MoE-layer tokens/s at B=1/64/4096; % of HBM GB/s (decode) / MFMA peak (prefill)"
PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes/s
PEAK_BF16 = 2.5e15         # MI355X dense bf16 MFMA, FLOP/s
H, E, K_TOP, I, IS = 4096, 256, 8, 2048, 2048
SPIN_CYCLES = 50_000_000   # head-start kernel before the event-timed launches (~20 ms)


# ------------------------------------------------------------------ HIP events
class HipEvents:
    """Raw hipEvent_t objects (the library records them on the layer's stream)."""

    def __init__(self, n: int):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.ev = []
        for _ in range(n):
            h = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(h)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.ev.append(h)

    def array(self, start: int, n: int):
        return (ctypes.c_void_p * n)(*[e.value for e in self.ev[start:start + n]])

    def record(self, i: int, stream: ctypes.c_void_p) -> None:
        if self.hip.hipEventRecord(self.ev[i], stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def ms(self, a: int, b: int) -> float:
        out = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(out), self.ev[a], self.ev[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return float(out.value)


# ------------------------------------------------------------------ byte/flop models
def fp4_role_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * k // 32


def q3_role_bytes(n: int, k: int) -> int:
    return n * k * 3 // 8 + 2 * (n * k // 64) * 2                 # codes + fp16 scale + fp16 bias


def expert_bytes(quant: str = "fp4") -> int:
    if quant == "q3":
        return 2 * q3_role_bytes(I, H) + q3_role_bytes(H, I)    # 11,010,048 at the full shape
    return 2 * fp4_role_bytes(I, H) + fp4_role_bytes(H, I)      # 13,369,344 at the full shape


def up_kernel_bytes(u: int, t: int, quant: str = "fp4") -> int:
    """Algorithmic HBM bytes of one routed gate/up launch (the decode path's
    k_up_stream): routed w1+w3 of the u active experts, x, and the h planes
    written (bf16 hi and lo)."""
    role = q3_role_bytes(I, H) if quant == "q3" else fp4_role_bytes(I, H)
    return u * 2 * role + t * H * 2 + t * K_TOP * I * 4


def layer_bytes(u: int, t: int, quant: str = "fp4") -> int:
    return u * expert_bytes(quant) + 3 * IS * H * 2 + E * H * 4 + 2 * t * H * 2


PREFILL_MIN_TOKENS = 128     # batches from this size run the expert products as MFMA GEMM tiles


def layer_flops(t: int) -> int:
    return 2 * t * K_TOP * 3 * H * I + 2 * t * 3 * H * IS + 2 * t * H * E


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    measurement (FETCH_SIZE / WRITE_SIZE scaled by a copy of known size), or
    None when no measurement for this kernel on this workload exists."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(kernel)
    if not entry or entry.get("workload") != workload:
        return None
    return int(entry["bytes_per_launch"])


# ------------------------------------------------------------------ timed forward
def forward_timed(layer, x, out, idx, w, ev: HipEvents, slot: int, repeat: int):
    dev = x.device
    desc = make_desc(tokens=x.shape[0], hidden=H, n_experts=E, top_k=K_TOP, inter=I,
                     inter_shared=IS, score_func=layer.score_func, quant=layer.bank.quant,
                     x_dtype=x.dtype, gate_dtype=layer.gate_w.dtype,
                     route_scale=layer.route_scale, limit=layer.limit)
    ws = workspace(desc, dev)
    s = layer.shared
    _lib.call("dsk_moe_forward_timed", ctypes.byref(desc), ptr(x), ptr(layer.gate_w),
              ptr(layer.gate_b), ptr(layer.bank.table), ptr(s.w1), ptr(s.w3), ptr(s.w2),
              ptr(None), ptr(out), ptr(idx), ptr(w), ptr(ws), ws.numel(), stream_of(dev),
              ev.array(slot * _lib.STAGE_EVENTS, _lib.STAGE_EVENTS), repeat)


def run_workload(layers, t: int, steps: int, warmup: int, n_inputs: int, seed: int = 123):
    """Time `steps` layer forwards at batch t; returns a dict of measurements."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + t)
    xs = [torch.randn((t, H), generator=g, device=dev).to(torch.bfloat16) for _ in range(n_inputs)]
    out = torch.empty((t, H), dtype=torch.bfloat16, device=dev)
    idxs = [torch.empty((t, K_TOP), dtype=torch.int32, device=dev) for _ in range(steps)]
    ws_ = torch.empty((t, K_TOP), dtype=torch.float32, device=dev)
    nl = len(layers)
    for s in range(warmup):
        layers[s % nl](xs[s % n_inputs], out=out)
    torch.cuda.synchronize()
    # 1) throughput: back-to-back layers, no events inside the timed region
    t0 = time.perf_counter()
    for s in range(steps):
        layers[s % nl](xs[s % n_inputs], out=out, idx=idxs[s])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # 2) stage timing: one launch per stage, events between the stages, same
    # rotation as above (cold weights).  A spin kernel first gives the GPU a
    # head start so that the host has queued every launch and event before the
    # GPU reaches it: the events then time GPU work only, not submission.
    # Each recorded event also costs GPU time (a marker packet): an empty pair
    # of events after every step measures it, and it is subtracted from the
    # stage times.
    n_t = min(steps, 40)
    ne = _lib.STAGE_EVENTS
    ev = HipEvents(n_t * ne)
    mk = HipEvents(2 * n_t)
    stream = stream_of(dev)
    torch.cuda._sleep(SPIN_CYCLES)
    for s in range(n_t):
        forward_timed(layers[s % nl], xs[s % n_inputs], out, idxs[s], ws_, ev, s, 1)
        mk.record(2 * s, stream)
        mk.record(2 * s + 1, stream)
    torch.cuda.synchronize()
    st = np.array([[ev.ms(s * ne + i, s * ne + i + 1) for i in range(5)] for s in range(n_t)])
    marker = np.array([mk.ms(2 * s, 2 * s + 1) for s in range(n_t)])
    uniq = [len(torch.unique(ix).tolist()) for ix in idxs[:n_t]]
    return {"wall_s": wall, "stage_ms": st, "marker_ms": marker, "unique": uniq}


# ------------------------------------------------------------------ layer stack
def run_stack(n_layers: int, batches, steps: int, warmup: int = 3, n_inputs: int = 8) -> dict:
    """The resident stack: layers [0, n/2) FP4, [n/2, n) q3, each of the full
    layer shape, on an RMSNorm residual stream (eps 1e-6, unit gamma), run as
    one captured HIP graph per batch size.  A step copies the next input into
    the graph's static buffer and replays the whole stack."""
    from dsk_moe.stack import MoEStack

    layers = [gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                                quant="fp4" if l < n_layers // 2 else "q3", seed=4000 + l, device="cuda:0")
              for l in range(n_layers)]
    stack = MoEStack(layers, eps=1e-6)
    resident = sum(t.numel() * t.element_size() for lay in layers
                   for t in [p for parts in lay.bank.roles.values() for p in parts]
                   + [lay.shared.w1, lay.shared.w3, lay.shared.w2, lay.gate_w])
    out = {}
    for b in batches:
        g = torch.Generator(device="cuda:0").manual_seed(31 + b)
        xs = [torch.randn((b, H), generator=g, device="cuda:0").to(torch.bfloat16) for _ in range(n_inputs)]
        rec = []
        stack(xs[0], record=rec)
        quants = ["fp4" if l < n_layers // 2 else "q3" for l in range(n_layers)]
        step_bytes = sum(layer_bytes(len(torch.unique(r[2]).tolist()), b, q) for r, q in zip(rec, quants))
        del rec
        stack.capture(b)
        for i in range(warmup):
            stack.replay(xs[i % n_inputs])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            stack.replay(xs[i % n_inputs])
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        # the same steps launched eagerly (per-kernel launches from the host)
        bufs = stack._buffers(xs[0])
        eo = torch.empty_like(xs[0])
        for i in range(warmup):
            stack(xs[i % n_inputs], out=eo, bufs=bufs)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for i in range(steps):
            stack(xs[i % n_inputs], out=eo, bufs=bufs)
        torch.cuda.synchronize()
        wall_e = time.perf_counter() - t1
        out[f"stack{n_layers}_B{b}"] = {
            "tokens_per_s": round(b * steps / wall, 1), "ms_per_step": round(wall / steps * 1e3, 4),
            "us_per_layer": round(wall / steps / n_layers * 1e6, 2),
            "eager_ms_per_step": round(wall_e / steps * 1e3, 4),
            "hbm_frac_wall": round(step_bytes / (wall / steps) / PEAK_HBM, 4),
            "resident_GB": round(resident / 1e9, 1),
            "layers": f"{n_layers // 2} FP4 + {n_layers - n_layers // 2} q3, RMSNorm residual, HIP graph replay"}
        print(f"# stack{n_layers} B={b}: {out[f'stack{n_layers}_B{b}']}", file=sys.stderr, flush=True)
    del stack, layers
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------ CPU baseline
def cpu_baseline(layer, n_tokens: int = 3):
    """The oracle (torch fp32 + numpy, the reference's algorithm restated) on
    this host, one token per layer call, experts dequantised lazily."""
    from oracle import formats as F
    from oracle import layer as L

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    spec = L.LayerSpec(H=H, E=E, k=K_TOP, I=I, I_shared=IS)
    gate_w, gate_b = layer.gate_w.cpu(), layer.gate_b.cpu()
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
    g = torch.Generator().manual_seed(7)
    xs = [torch.randn((1, H), generator=g).to(torch.bfloat16) for _ in range(n_tokens + 1)]
    raw = {}
    idx_all = set()
    for x in xs:                                    # fetch the raw bytes the oracle will read
        from oracle import router as R
        idx, *_ = R.route(x.float().numpy(), gate_w.numpy(), gate_b.numpy(), K_TOP)
        idx_all.update(int(v) for v in idx.ravel())
    for e in idx_all:
        raw[e] = {r: [t[e].cpu().numpy() for t in layer.bank.roles[r]] for r in ("w1", "w3", "w2")}

    class HostBank:
        quant = "fp4"

        def __init__(self):
            self.cache = {}

        def dequant(self, e, role):
            if (e, role) not in self.cache:
                self.cache[(e, role)] = F.fp4_dequant(*raw[e][role])
            return self.cache[(e, role)]

    L.moe_forward(xs[0], gate_w, gate_b, HostBank(), shared, spec)      # warm-up
    times = []
    for x in xs[1:]:
        t0 = time.perf_counter()
        L.moe_forward(x, gate_w, gate_b, HostBank(), shared, spec)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": 1.0 / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n_tokens} single-token layer calls (B=1) of the oracle after 1 warm-up, "
                      f"median {med:.3f} s; experts dequantised per call; {platform.processor() or platform.machine()}, "
                      f"torch {torch.__version__}"}


# ------------------------------------------------------------------ copy calibration
def copy_mode(nbytes: int, steps: int) -> None:
    dev = torch.device("cuda:0")
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_()
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        b.copy_(a)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"mode": "copy", "bytes_read": nbytes, "bytes_written": nbytes,
                      "ms": dt * 1e3, "GBps_rw": 2 * nbytes / dt / 1e9}), flush=True)


# ------------------------------------------------------------------ main
def main() -> int:
    ap = argparse.ArgumentParser(description="MoE-layer forward benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--inputs", type=int, default=16)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quant", choices=("fp4", "q3"), default="fp4", help="routed expert format")
    ap.add_argument("--zipf", type=float, default=None,
                    help="gate bias = log Zipf(s) popularity (skewed routing, as in the prefill sweep)")
    ap.add_argument("--mode", choices=("layer", "copy"), default="layer")
    ap.add_argument("--bytes", type=int, default=1 << 30)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the MoE-layer path is built and timed on a single "
              "MI355X (--gpus 1); multi-GPU sharding is a design note only.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    dsk_moe.load_library()
    if args.mode == "copy":
        copy_mode(args.bytes, args.steps)
        return 0

    t_gen = time.perf_counter()
    layers = [gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                                quant=args.quant, seed=1000 + i, device="cuda:0", zipf_s=args.zipf)
              for i in range(args.layers)]
    torch.cuda.synchronize()
    print(f"# generated {args.layers} resident layers in {time.perf_counter() - t_gen:.1f} s", file=sys.stderr, flush=True)

    T = args.tokens
    r = run_workload(layers, T, args.steps, args.warmup, args.inputs)
    ms_step = r["wall_s"] / args.steps * 1e3
    value = T * args.steps / r["wall_s"]
    st = r["stage_ms"]
    marker_ms = float(np.median(r["marker_ms"]))
    u = np.array(r["unique"])
    up_ms = np.maximum(st[:, 2] - marker_ms, 1e-6)
    up_bytes = np.array([up_kernel_bytes(int(x), T, args.quant) for x in u])
    achieved = float(up_bytes.sum() / (up_ms.sum() * 1e-3))
    prefill = T >= PREFILL_MIN_TOKENS
    workload = (f"full-size {args.quant.upper()} MoE layer {'prefill' if prefill else 'decode'}, B={T}"
                + (f", Zipf({args.zipf}) gate bias" if args.zipf else ""))
    if prefill:
        # gate/up GEMM of the prefill path: routed (T*k rows) and shared (T rows) w1, w3
        up_flops = 2 * T * K_TOP * 2 * H * I + 2 * T * 2 * H * IS
        achieved_f = up_flops / (float(up_ms.mean()) * 1e-3)
        roofline = {"bound": "mfma", "achieved": round(achieved_f / 1e12, 1), "peak": PEAK_BF16 / 1e12,
                    "unit": "TFLOP/s", "frac": round(achieved_f / PEAK_BF16, 4),
                    "traffic": measured_traffic("k_pf_up", workload),
                    "kernel": f"k_pf_up (routed {args.quant.upper()} + shared bf16 w1/w3 GEMM tiles, SwiGLU epilogue)",
                    "flops_per_launch": int(up_flops),
                    "avg_launch_us": round(float(up_ms.mean()) * 1e3, 2),
                    "timing": "HIP events around one launch per step, minus the GPU time of an "
                              "empty event pair"}
    else:
        roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4),
                    "traffic": measured_traffic("k_up_stream", workload),
                    "kernel": f"k_up_stream (routed {args.quant.upper()} w1/w3, SwiGLU and route weight epilogue)",
                    "bytes_per_launch": int(up_bytes.mean()),
                    "avg_launch_us": round(float(up_ms.mean()) * 1e3, 2),
                    "timing": "HIP events around one launch per step (cold weights), minus the "
                              "GPU time of an empty event pair"}
    layer_b = np.array([layer_bytes(int(x), T, args.quant) for x in u])
    stage_names = ["route", "dispatch", "gate_up", "down", "combine"]
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "hidden": H,
                   "n_experts": E, "top_k": K_TOP, "inter": I, "shared_inter": IS,
                   "routed_format": ("q3-affine-g64 (fp16 scale/bias)" if args.quant == "q3"
                                     else "fp4-e2m1/e8m0-g32"), "shared_format": "bf16",
                   "gate": "sigmoid, route_scale 2.5", "tokens": T,
                   "layers_rotated": args.layers, "inputs_rotated": args.inputs},
        "roofline": roofline,
        "stage_us": {n: round(max(float(st[:, i].mean()) - marker_ms, 0.0) * 1e3, 2)
                     for i, n in enumerate(stage_names)},
        "event_marker_us": round(marker_ms * 1e3, 2),
        "layer_hbm_frac_wall": round(float(layer_b.mean() / (ms_step * 1e-3)) / PEAK_HBM, 4),
        "unique_experts_mean": float(u.mean()),
    }
    if not args.no_sweep:
        sweep = {}
        for tb in (8, 64):
            rs = run_workload(layers, tb, 40, 5, args.inputs, seed=77)
            us = np.array(rs["unique"])
            lb = np.array([layer_bytes(int(x), tb) for x in us])
            sweep[f"B{tb}"] = {"tokens_per_s": round(tb * 40 / rs["wall_s"], 1),
                               "ms_per_step": round(rs["wall_s"] / 40 * 1e3, 4),
                               "unique_experts_mean": float(us.mean()),
                               "layer_hbm_frac": round(float(lb.mean() / (rs["wall_s"] / 40)) / PEAK_HBM, 4)}
        zl = gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                               seed=3000, device="cuda:0", zipf_s=1.1)
        rs = run_workload([zl], 4096, 5, 1, 2, seed=99)
        step_s = rs["wall_s"] / 5
        sweep["T4096_prefill_zipf"] = {"tokens_per_s": round(4096 / step_s, 1),
                                       "ms_per_step": round(step_s * 1e3, 3),
                                       "mfma_frac": round(layer_flops(4096) / step_s / PEAK_BF16, 4),
                                       "stage_us": {n: round(float(rs["stage_ms"][:, i].mean()) * 1e3, 1)
                                                    for i, n in enumerate(stage_names)}}
        # routed experts in 3-bit affine (group 64, fp16 scale / bias), B = 1, 16, 64
        q3_layers = [gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                                       quant="q3", seed=2000 + i, device="cuda:0") for i in range(2)]
        for tb in (1, 16, 64):
            n_steps = 100 if tb == 1 else 40
            rs = run_workload(q3_layers, tb, n_steps, 5, args.inputs, seed=55)
            us = np.array(rs["unique"])
            lb = np.array([layer_bytes(int(x), tb, "q3") for x in us])
            sweep[f"q3_B{tb}"] = {"tokens_per_s": round(tb * n_steps / rs["wall_s"], 1),
                                  "ms_per_step": round(rs["wall_s"] / n_steps * 1e3, 4),
                                  "unique_experts_mean": float(us.mean()),
                                  "layer_hbm_frac": round(float(lb.mean() / (rs["wall_s"] / n_steps)) / PEAK_HBM, 4)}
        del q3_layers
        sweep.update(run_stack(40, (1, 2), steps=30))
        line["sweep"] = sweep
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(layers[0])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
