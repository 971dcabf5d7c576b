#!/usr/bin/env python3
"""MoE-layer forward benchmark on one MI355X.

Workload (default): the full-size FP4 MoE layer at decode -- hidden 4096,
256 routed experts, top-8, expert intermediate 2048, one bf16 shared expert
of 2048, FP4 e2m1/E8M0 routed weights quantised from N(0, 0.02), sigmoid gate
with route scale 2.5, B = 1 token of bf16 N(0, 1).  All weights are resident
in HBM before timing.  A step is one layer forward; steps rotate over
``--layers`` independently drawn layers and ``--inputs`` token batches, so
consecutive steps read different experts (each cycle moves more than the
256 MB Infinity Cache).

``value`` is tokens/s over exactly ``--steps`` timed steps (wall clock,
synchronised on both sides).  Kernel times come from a separate run of
``--timed-steps`` steps of the same rotation through
``dsk_moe_forward_timed``: every stage's kernels carry HIP events as their
own begin / end timestamps (hipExtLaunchKernel), the durations a profiler
reports; medians, p10 and p90 over those steps are printed.

Prints ONE JSON line: the metric, the roofline of the routed-expert stage
(routed gate/up + down kernels: routed-expert bytes / their time, the
primary decode fraction), each kernel's algorithmic bytes and fraction, the
whole layer's fraction, the measured copy / GEMM peaks of this box, a sweep
of the other batch sizes, and CPU baselines (the oracle on a bounded sample
of each workload, on this host's cores).

    python bench.py [--steps K] [--warmup W] [--tokens T] [--quant fp4|q3] [--zipf S]
                    [--no-sweep] [--no-cpu]
    python bench.py --mode copy  --bytes N    # device copy of known size (bandwidth, counter scale)
    python bench.py --mode read  --bytes N    # streaming read (sum) of N bytes
    python bench.py --mode mfma               # bf16 GEMM 8192^3, random and constant operands
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import ctypes
import json
import os
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
PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes/s (published)
PEAK_BF16 = 2.5e15         # MI355X dense bf16 MFMA, FLOP/s (published)
H, E, K_TOP, I, IS = 4096, 256, 8, 2048, 2048
SPIN_CYCLES = 50_000_000   # head-start kernel before each chunk of timed steps (~20 ms)
STAGES = ("gate", "route", "gate_up", "down", "combine")
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


# ------------------------------------------------------------------ HIP events
class HipEvents:
    """Raw hipEvent_t objects handed to dsk_moe_forward_timed."""

    def __init__(self, n: int):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = []
        for _ in range(n):
            h = ctypes.c_void_p()
            if self.hip.hipEventCreateWithFlags(ctypes.byref(h), HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            self.ev.append(h)

    def array(self, start: int, n: int):
        return (ctypes.c_void_p * n)(*[e.value for e in self.ev[start:start + n]])

    def ms(self, a: int, b: int) -> float:
        """Elapsed ms from event a to event b; NaN when either was never recorded
        (a stage that launched no kernel)."""
        out = ctypes.c_float()
        rc = self.hip.hipEventElapsedTime(ctypes.byref(out), self.ev[a], self.ev[b])
        if rc != 0:
            self.hip.hipGetLastError()        # the failed query must not surface in a later HIP call
            return float("nan")
        return float(out.value)

    def close(self) -> None:
        for e in self.ev:
            self.hip.hipEventDestroy(e)
        self.ev = []


# ------------------------------------------------------------------ byte / flop models
def fp4_role_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * k // 32


def q3_role_bytes(n: int, k: int) -> int:
    return n * k * 3 // 8 + 2 * (n * k // 64) * 2                 # codes + fp16 scale + fp16 bias


def role_bytes(n: int, k: int, quant: str) -> int:
    return q3_role_bytes(n, k) if quant == "q3" else fp4_role_bytes(n, k)


def expert_bytes(quant: str = "fp4") -> int:
    """13,369,344 (FP4) / 11,010,048 (q3) at the full shape."""
    return 2 * role_bytes(I, H, quant) + role_bytes(H, I, quant)


def mx_decode(t: int, quant: str) -> bool:
    """FP4 experts and one or two bf16 tokens at the full shape run the MX decode kernels."""
    return quant == "fp4" and t <= 2


def stage_bytes(u: int, t: int, quant: str) -> dict:
    """Algorithmic HBM bytes of each decode-pipeline stage for u active experts, t tokens.
    MX kernels: gate (fp32 gate + shared w1/w3 + x + scores + h_s planes), route (shared
    w2 + scores + h_s planes + shared output), gate/up (routed w1/w3 + x + h planes), down
    (routed w2 + h planes + shared output + out).  Otherwise: gate (fp32 gate + x +
    scores), route (shared w1/w3 + scores + h_s planes), gate/up (as above), down (routed
    w2 + shared w2 + h / h_s planes + out)."""
    up = u * 2 * role_bytes(I, H, quant) + t * H * 2 + t * K_TOP * I * 4
    if mx_decode(t, quant):
        return {"gate": E * H * 4 + 2 * IS * H * 2 + t * H * 2 + t * E * 4 + t * IS * 4,
                "route": H * IS * 2 + t * E * 4 + t * IS * 4 + t * H * 2,
                "gate_up": up,
                "down": u * role_bytes(H, I, quant) + t * K_TOP * I * 4 + 2 * t * H * 2,
                "combine": 0}
    return {"gate": E * H * 4 + t * H * 2 + t * E * 4,
            "route": 2 * IS * H * 2 + t * E * 4 + t * IS * 4,
            "gate_up": up,
            "down": u * role_bytes(H, I, quant) + H * IS * 2 + t * K_TOP * I * 4 + t * IS * 4 + t * H * 2,
            "combine": 0}


def layer_bytes(u: int, t: int, quant: str = "fp4") -> int:
    return u * expert_bytes(quant) + 3 * IS * H * 2 + E * H * 4 + 2 * t * H * 2


def layer_flops(t: int) -> int:
    return 2 * t * K_TOP * 3 * H * I + 2 * t * 3 * H * IS + 2 * t * H * E


def up_flops(t: int) -> int:
    """gate/up GEMM of the prefill path: routed (t*k rows) and shared (t rows) w1, w3."""
    return 2 * t * K_TOP * 2 * H * I + 2 * t * 2 * H * IS


PREFILL_MIN_TOKENS = 128     # batches from this size run the expert products as MFMA GEMM tiles


TRAFFIC_SOURCE = ("read from profiles/traffic.json, not measured by this run: rocprofv3 --pmc FETCH_SIZE "
                  "and WRITE_SIZE passes of the same workload, scaled by what they read for a 256 MiB copy")


def measured_traffic(kernels: list[str], workload: str):
    """HBM bytes per launch of `kernels` (summed) from the committed rocprofv3 --pmc
    measurement (FETCH_SIZE / WRITE_SIZE scaled by a copy of known size), or None
    when one of them has no measurement on this workload."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    table = json.loads(path.read_text())
    total = 0
    for k in kernels:
        entry = table.get(k)
        if not entry or entry.get("workload") != workload:
            return None
        total += int(entry["bytes_per_launch"])
    return total


def pf_up_kernels(quant: str) -> list[str]:
    """The prefill gate/up stage's kernels: FP4 layers of the full shape run the
    routed MX tiles and the shared expert's bf16 tiles (x's FP8 planes are
    written by the top-k kernel of the route stage)."""
    return ["k_pf_mx_up", "k_pf_up"] if quant == "fp4" else ["k_pf_up"]


def traffic_fields(kernels: list[str], workload: str) -> dict:
    """roofline["traffic"] and where it comes from."""
    t = measured_traffic(kernels, workload)
    return {"traffic": t, "traffic_source": TRAFFIC_SOURCE if t is not None else
            "no committed FETCH_SIZE / WRITE_SIZE measurement for this kernel and workload"}


def pct(a: np.ndarray) -> dict | None:
    """median / p10 / p90 (None for a stage that launched no kernel)."""
    a = np.asarray(a, dtype=np.float64)
    if np.isnan(a).all():
        return None
    return {"median": round(float(np.nanmedian(a)), 2), "p10": round(float(np.nanpercentile(a, 10)), 2),
            "p90": round(float(np.nanpercentile(a, 90)), 2)}


# ------------------------------------------------------------------ timed forward
def forward_timed(layer, x, out, idx, w, ev: HipEvents, slot: int):
    dev = x.device
    desc = make_desc(tokens=x.shape[0], hidden=layer.gate_w.shape[1], n_experts=layer.bank.n_experts,
                     top_k=layer.top_k, inter=layer.bank.inter, inter_shared=layer.shared.inter,
                     score_func=layer.score_func, quant=layer.bank.quant, x_dtype=x.dtype,
                     gate_dtype=layer.gate_w.dtype, route_scale=layer.route_scale, limit=layer.limit)
    ws = workspace(desc, dev)
    s = layer.shared
    _lib.call("dsk_moe_forward_timed", ctypes.byref(desc), ptr(x), ptr(layer.gate_w),
              ptr(layer.gate_b), ptr(layer.bank.table), ptr(s.w1), ptr(s.w3), ptr(s.w2),
              ptr(None), ptr(out), ptr(idx), ptr(w), ptr(ws), ws.numel(), stream_of(dev),
              ev.array(slot * _lib.STAGE_EVENTS, _lib.STAGE_EVENTS), 1)


def run_workload(layers, t: int, steps: int, warmup: int, n_inputs: int, timed_steps: int,
                 seed: int = 123) -> dict:
    """`steps` back-to-back layer forwards at batch t (wall clock), then `timed_steps`
    forwards of the same rotation with kernel-timestamp events per stage."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + t)
    xs = [torch.randn((t, H), generator=g, device=dev).to(torch.bfloat16) for _ in range(n_inputs)]
    out = torch.empty((t, H), dtype=torch.bfloat16, device=dev)
    k = layers[0].top_k
    idx = torch.empty((t, k), dtype=torch.int32, device=dev)
    wts = torch.empty((t, k), dtype=torch.float32, device=dev)
    nl = len(layers)
    for s in range(warmup):
        layers[s % nl](xs[s % n_inputs], out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        layers[s % nl](xs[s % n_inputs], out=out)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # kernel timing: chunks of 40 steps, each after a spin kernel that gives the host a
    # head start, so every launch is queued before the GPU reaches it
    ne = _lib.STAGE_EVENTS
    stage_ms, layer_ms, uniq = [], [], []
    chunk = 40
    for c0 in range(0, timed_steps, chunk):
        n = min(chunk, timed_steps - c0)
        ev = HipEvents(n * ne)
        idxs = [torch.empty((t, k), dtype=torch.int32, device=dev) for _ in range(n)]
        torch.cuda._sleep(SPIN_CYCLES)
        for i in range(n):
            s = c0 + i
            forward_timed(layers[s % nl], xs[s % n_inputs], out, idxs[i], wts, ev, i)
        torch.cuda.synchronize()
        for i in range(n):
            row = [ev.ms(i * ne + 2 * j, i * ne + 2 * j + 1) for j in range(len(STAGES))]
            stage_ms.append(row)
            # the layer's kernel time: the stages' kernels back to back (launching with
            # timestamp events spaces the kernels out, so the span between the first
            # begin and the last end is not the layer's time in an untimed run)
            layer_ms.append(float(np.nansum(row)))
            uniq.append(len(torch.unique(idxs[i]).tolist()))
        ev.close()
    return {"wall_s": wall, "stage_us": np.array(stage_ms) * 1e3, "layer_us": np.array(layer_ms) * 1e3,
            "unique": np.array(uniq)}


def decode_summary(r: dict, t: int, quant: str, steps: int) -> dict:
    """Per-stage kernel times and fractions of the decode / grouped path."""
    st, u = r["stage_us"], r["unique"]
    sb = [stage_bytes(int(x), t, quant) for x in u]
    kern = {}
    for j, name in enumerate(STAGES):
        b = np.array([s[name] for s in sb], dtype=np.float64)
        us = st[:, j]
        e = {"us": pct(us)}
        if b.sum() > 0 and not np.isnan(us).any():
            e["bytes_mean"] = int(b.mean())
            e["hbm_frac"] = round(float(b.sum() / (us.sum() * 1e-6)) / PEAK_HBM, 4)
        kern[name] = e
    routed = u.astype(np.float64) * expert_bytes(quant)
    routed_us = st[:, 2] + st[:, 3]
    lb = np.array([layer_bytes(int(x), t, quant) for x in u], dtype=np.float64)
    wall_step = r["wall_s"] / steps
    return {"stages": kern,
            "routed_stage": {"bytes_mean": int(routed.mean()), "us": pct(routed_us),
                             "hbm_frac": round(float(routed.sum() / (routed_us.sum() * 1e-6)) / PEAK_HBM, 4)},
            "layer": {"bytes_mean": int(lb.mean()), "kernels_us": pct(r["layer_us"]),
                      "hbm_frac": round(float(lb.sum() / (r["layer_us"].sum() * 1e-6)) / PEAK_HBM, 4),
                      "hbm_frac_wall": round(float(lb.mean() / wall_step) / PEAK_HBM, 4)},
            "unique_experts_mean": float(u.mean())}


def prefill_summary(r: dict, t: int, steps: int) -> dict:
    st = r["stage_us"]
    up = st[:, 2]
    return {"stages": {n: {"us": pct(st[:, j])} for j, n in enumerate(STAGES)},
            "gate_up_mfma_frac": round(up_flops(t) / (float(np.median(up)) * 1e-6) / PEAK_BF16, 4),
            "layer": {"flops": layer_flops(t), "kernels_us": pct(r["layer_us"]),
                      "mfma_frac": round(layer_flops(t) / (float(np.median(r["layer_us"])) * 1e-6) / PEAK_BF16, 4),
                      "mfma_frac_wall": round(layer_flops(t) / (r["wall_s"] / steps) / PEAK_BF16, 4)},
            "unique_experts_mean": float(r["unique"].mean())}


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
def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


class HostBank:
    """Routed experts of a resident layer copied to host memory as raw bytes (before
    timing); ``dequant`` decodes with the oracle's format code.  ``prefetch`` decodes
    the roles the oracle layer will ask for on a thread pool, in its order."""

    def __init__(self, layer, experts, pool: cf.ThreadPoolExecutor):
        from oracle import formats as F
        self.F, self.quant, self.pool = F, layer.bank.quant, pool
        ex = torch.tensor(sorted(set(int(e) for e in experts)), dtype=torch.long, device="cuda:0")
        self.pos = {int(e): i for i, e in enumerate(ex.tolist())}
        self.raw = {r: [t.index_select(0, ex).cpu().numpy() for t in layer.bank.roles[r]]
                    for r in ("w1", "w3", "w2")}
        self.ready: dict = {}

    def _decode(self, e: int, role: str):
        parts = [a[self.pos[e]] for a in self.raw[role]]
        return self.F.fp4_dequant(*parts) if self.quant == "fp4" else self.F.q3_dequant(*parts)

    def prefetch(self, experts) -> None:
        self.ready = {(int(e), r): self.pool.submit(self._decode, int(e), r)
                      for e in sorted(set(int(v) for v in experts)) for r in ("w1", "w3", "w2")}

    def dequant(self, e, role):
        f = self.ready.pop((int(e), role), None)
        return f.result() if f is not None else self._decode(int(e), role)


def oracle_call(layer, x: torch.Tensor, bank: HostBank, shared, spec, gate) -> float:
    """Seconds for one oracle layer forward (router, lazy dequant of the selected
    experts on the thread pool, expert math, combine)."""
    from oracle import layer as L
    from oracle import router as R
    t0 = time.perf_counter()
    routing = R.route(x.float().numpy(), gate[0], gate[1], spec.k, spec.score_func, spec.route_scale)
    bank.prefetch(routing[0].ravel())
    L.moe_forward(x, None, None, bank, shared, spec, routing=routing)
    return time.perf_counter() - t0


def cpu_baseline(layer, zipf_layer=None) -> dict:
    """The oracle (torch fp32 + numpy: the reference's algorithm restated) on this
    host's cores, on bounded samples: B=1 (median of 5 calls after 1 warm-up), B=64
    (one call), and 1024 of the 4096 tokens of the Zipf prefill workload (one call)."""
    from oracle import layer as L
    from oracle import router as R

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    spec = L.LayerSpec(H=H, E=E, k=K_TOP, I=I, I_shared=IS)
    g = torch.Generator().manual_seed(7)
    out = {}
    with cf.ThreadPoolExecutor(max_workers=cores) as pool:
        for name, lay, t, calls in (("B1", layer, 1, 6), ("B64", layer, 64, 1),
                                    ("T4096_zipf_sample1024", zipf_layer, 1024, 1)):
            if lay is None:
                continue
            gate = (lay.gate_w.cpu().float().numpy(), lay.gate_b.cpu().numpy())
            shared = tuple(s.cpu() for s in (lay.shared.w1, lay.shared.w3, lay.shared.w2))
            xs = [torch.randn((t, H), generator=g).to(torch.bfloat16) for _ in range(calls)]
            needed = set()
            for x in xs:
                needed.update(int(v) for v in R.route(x.float().numpy(), gate[0], gate[1], K_TOP)[0].ravel())
            bank = HostBank(lay, needed, pool)
            times = [oracle_call(lay, x, bank, shared, spec, gate) for x in xs]
            if calls > 1:
                times = times[1:]                       # first call is the warm-up
            med = float(np.median(times))
            out[name] = {"tokens_per_s": round(t / med, 3), "s_per_call": round(med, 3),
                         "calls_timed": len(times), "tokens_per_call": t}
            print(f"# cpu baseline {name}: {out[name]}", file=sys.stderr, flush=True)
    b1 = out["B1"]
    return {"value": b1["tokens_per_s"], "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": (f"B=1: median of {b1['calls_timed']} single-token layer calls of the oracle after "
                       f"1 warm-up (router, lazy per-expert dequant on {cores} threads, torch fp32 "
                       f"expert math); {cpu_model()}; torch {torch.__version__}"),
            "configs": out}


# ------------------------------------------------------------------ machine peaks
def copy_rate(nbytes: int, steps: int) -> dict:
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
    return {"mode": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "ms": round(dt * 1e3, 4),
            "GBps_read_plus_write": round(2 * nbytes / dt / 1e9, 1)}


def read_rate(nbytes: int, steps: int) -> dict:
    dev = torch.device("cuda:0")
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_()
    for _ in range(3):
        a.sum()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        a.sum()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"mode": "read", "bytes_read": nbytes, "ms": round(dt * 1e3, 4), "GBps": round(nbytes / dt / 1e9, 1)}


def gemv_rate(rows: int = 65536, cols: int = 8192, steps: int = 20) -> dict:
    """bf16 matrix-vector product through torch (rows x cols, 1 GiB): the rate at
    which this box streams a weight matrix row by row into a GEMV."""
    dev = torch.device("cuda:0")
    w = torch.randn((rows, cols), device=dev, dtype=torch.bfloat16)
    x = torch.randn((cols,), device=dev, dtype=torch.bfloat16)
    y = torch.empty((rows,), device=dev, dtype=torch.bfloat16)
    for _ in range(3):
        torch.mv(w, x, out=y)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        torch.mv(w, x, out=y)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    nbytes = rows * cols * 2
    del w
    return {"mode": "gemv", "bytes_read": nbytes, "ms": round(dt * 1e3, 4), "GBps": round(nbytes / dt / 1e9, 1)}


def mfma_rate(n: int = 8192, steps: int = 20) -> dict:
    """bf16 GEMM n x n x n through torch (hipBLASLt, A times B transposed: both
    operands K-contiguous, as the weight rows and token rows of the prefill GEMM)
    with random N(0,1) operands and with constant operands: the dense bf16 matrix
    rate this box sustains."""
    dev = torch.device("cuda:0")
    res = {"mode": "mfma", "gemm": f"bf16 {n}x{n}x{n}, A @ B^T", "flop_per_call": 2 * n ** 3}
    for kind in ("random", "constant"):
        if kind == "random":
            a = torch.randn((n, n), device=dev, dtype=torch.bfloat16)
            b = torch.randn((n, n), device=dev, dtype=torch.bfloat16)
        else:
            a = torch.full((n, n), 0.5, device=dev, dtype=torch.bfloat16)
            b = torch.full((n, n), 0.25, device=dev, dtype=torch.bfloat16)
        c = torch.empty((n, n), device=dev, dtype=torch.bfloat16)
        for _ in range(3):
            torch.matmul(a, b.t(), out=c)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            torch.matmul(a, b.t(), out=c)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        res[f"TFLOPs_{kind}"] = round(2 * n ** 3 / dt / 1e12, 1)
        res[f"frac_of_peak_{kind}"] = round(2 * n ** 3 / dt / PEAK_BF16, 4)
    return res


# ------------------------------------------------------------------ main
def main() -> int:
    ap = argparse.ArgumentParser(description="MoE-layer forward benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--timed-steps", type=int, default=120, help="steps timed per kernel (median/p10/p90)")
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--inputs", type=int, default=16)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="leave the 40-layer stack out of the sweep")
    ap.add_argument("--quant", choices=("fp4", "q3"), default="fp4", help="routed expert format")
    ap.add_argument("--zipf", type=float, default=None,
                    help="gate bias = log Zipf(s) popularity (skewed routing, as in the prefill sweep)")
    ap.add_argument("--mode", choices=("layer", "copy", "read", "mfma", "stack"), default="layer",
                    help="layer: the headline line; copy / read / mfma: the box's peaks; stack: only the "
                         "40-layer stack at 1 and 2 tokens (--steps replays each)")
    ap.add_argument("--bytes", type=int, default=1 << 30)
    ap.add_argument("--stack-batch", type=int, default=0, help="--mode stack: this batch size only")
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
        print(json.dumps(copy_rate(args.bytes, args.steps)), flush=True)
        return 0
    if args.mode == "read":
        print(json.dumps(read_rate(args.bytes, args.steps)), flush=True)
        return 0
    if args.mode == "mfma":
        print(json.dumps(mfma_rate()), flush=True)
        return 0
    if args.mode == "stack":
        batches = (args.stack_batch,) if args.stack_batch else (1, 2)
        print(json.dumps(run_stack(40, batches, steps=args.steps)), flush=True)
        return 0

    t_gen = time.perf_counter()
    layers = [gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                                quant=args.quant, seed=1000 + i, device="cuda:0", zipf_s=args.zipf)
              for i in range(args.layers)]
    torch.cuda.synchronize()
    print(f"# generated {args.layers} resident layers in {time.perf_counter() - t_gen:.1f} s",
          file=sys.stderr, flush=True)

    T = args.tokens
    r = run_workload(layers, T, args.steps, args.warmup, args.inputs, args.timed_steps)
    ms_step = r["wall_s"] / args.steps * 1e3
    value = T * args.steps / r["wall_s"]
    prefill = T >= PREFILL_MIN_TOKENS
    workload = (f"full-size {args.quant.upper()} MoE layer {'prefill' if prefill else 'decode'}, B={T}"
                + (f", Zipf({args.zipf}) gate bias" if args.zipf else ""))
    timing = (f"kernel begin/end timestamps (HIP events carried by the launches), "
              f"{'median' if T >= PREFILL_MIN_TOKENS else 'mean'} over {args.timed_steps} steps of the "
              f"same cold-weight rotation")
    if prefill:
        summ = prefill_summary(r, T, args.steps)
        up_us = summ["stages"]["gate_up"]["us"]["median"]
        achieved = up_flops(T) / (up_us * 1e-6)
        roofline = {"bound": "mfma", "achieved": round(achieved / 1e12, 1), "peak": PEAK_BF16 / 1e12,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4),
                    **traffic_fields(pf_up_kernels(args.quant), workload),
                    "kernel": ("gate/up stage: k_pf_mx_up (routed FP4 w1/w3 on scaled FP4 x FP8 MFMAs, x as "
                               "FP8 planes from the top-k kernel) + k_pf_up (shared bf16 w1/w3), SwiGLU epilogues"
                               if args.quant == "fp4" else
                               f"k_pf_up (routed {args.quant.upper()} + shared bf16 w1/w3 GEMM tiles, SwiGLU epilogue)"),
                    "flops_per_launch": int(up_flops(T)), "avg_launch_us": up_us, "timing": timing}
    else:
        summ = decode_summary(r, T, args.quant, args.steps)
        rs = summ["routed_stage"]
        routed_us = float(np.mean(r["stage_us"][:, 2] + r["stage_us"][:, 3]))
        achieved = rs["bytes_mean"] / (routed_us * 1e-6)
        mx = mx_decode(T, args.quant)
        up_k = ("k_up_grouped" if T >= 8 else "k_up_q3" if args.quant == "q3" else
                "k_up_mx" if mx else "k_up_stream")
        dn_k = ("k_down_q3" if args.quant == "q3" and T <= 4 else "k_down_mx" if mx else
                "k_down_decode_staged" if T <= 2 else "k_down_grouped + k_combine")
        roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4),
                    **traffic_fields([up_k, dn_k], workload),
                    "kernel": f"routed-expert stage: {up_k} (routed w1/w3, SwiGLU x route weight) + "
                              f"{dn_k} " + ("(routed w2, add of the shared output)" if mx else
                                             "(routed and shared w2, combine)"),
                    "bytes_per_launch": rs["bytes_mean"],
                    "bytes_note": "routed-expert bytes only (U experts x 3 roles); the kernels also "
                                  "move activations (stages[*].bytes_mean)",
                    "avg_launch_us": round(routed_us, 2), "timing": timing}
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
        "detail": summ,
    }
    peaks = {"hbm_GBps_published": PEAK_HBM / 1e9, "bf16_TFLOPs_published": PEAK_BF16 / 1e12}
    cp = copy_rate(1 << 30, 20)
    rd = read_rate(1 << 31, 20)
    gv = gemv_rate()
    peaks.update({"copy_GBps_measured": cp["GBps_read_plus_write"], "read_GBps_measured": rd["GBps"],
                  "gemv_read_GBps_measured": gv["GBps"]})
    mf = mfma_rate(8192, 10)
    peaks.update({"bf16_gemm_TFLOPs_measured_random": mf["TFLOPs_random"],
                  "bf16_gemm_TFLOPs_measured_constant": mf["TFLOPs_constant"]})
    line["peaks"] = peaks
    zl = None
    if not args.no_sweep:
        sweep = {}
        for tb in (8, 64):
            rs_ = run_workload(layers, tb, 40, 5, args.inputs, 100, seed=77)
            s_ = decode_summary(rs_, tb, "fp4", 40)
            sweep[f"B{tb}"] = {"tokens_per_s": round(tb * 40 / rs_["wall_s"], 1),
                               "ms_per_step": round(rs_["wall_s"] / 40 * 1e3, 4), **s_}
        zl = gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                               seed=3000, device="cuda:0", zipf_s=1.1)
        rs_ = run_workload([zl], 4096, 10, 2, 2, 20, seed=99)
        sweep["T4096_prefill_zipf"] = {"tokens_per_s": round(4096 * 10 / rs_["wall_s"], 1),
                                       "ms_per_step": round(rs_["wall_s"] / 10 * 1e3, 3),
                                       **prefill_summary(rs_, 4096, 10)}
        # routed experts in 3-bit affine (group 64, fp16 scale / bias), B = 1, 16, 64;
        # 4 layers rotated (each cycle moves more than the Infinity Cache)
        q3_layers = [gsynth.make_layer(hidden=H, n_experts=E, top_k=K_TOP, inter=I, inter_shared=IS,
                                       quant="q3", seed=2000 + i, device="cuda:0") for i in range(4)]
        for tb in (1, 16, 64):
            n_steps = 100 if tb == 1 else 40
            rs_ = run_workload(q3_layers, tb, n_steps, 5, args.inputs, 100, seed=55)
            s_ = decode_summary(rs_, tb, "q3", n_steps)
            sweep[f"q3_B{tb}"] = {"tokens_per_s": round(tb * n_steps / rs_["wall_s"], 1),
                                  "ms_per_step": round(rs_["wall_s"] / n_steps * 1e3, 4), **s_}
        del q3_layers
        torch.cuda.empty_cache()
        if not args.no_stack:
            sweep.update(run_stack(40, (1, 2), steps=30))
        line["sweep"] = sweep
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(layers[0], zl)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
