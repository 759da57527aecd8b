#!/usr/bin/env python3
"""Causal multi-head attention fwd+bwd throughput on one MI355X (gfx950).

One step is one pass of the hot path over one batch, every kernel launched through the
C ABI (include/attn_capi.h) on torch's current stream.  fp32 default (--path x3): fp32
attention on the bf16 matrix cores, every fp32 operand carried as three bf16 planes (24
significant bits) and every product as six plane products accumulated in fp32 (the
*_f32x3 entry points; within the 1e-5 gate of torch fp32 on every head of config 2 for seeds
42, 1 and 2, worst 6.7e-6, tests/test_gpu_f32x3_seeds.py; its fp64 distance is within 3x the
fp32 MFMA path's in max-abs and 4x in rms, tests/test_gpu_f32x3.py):
    attn_fwd_x3       planes of q, k, v; qkv -> O (B,H,T,d), m, l  reference model.cu:305-311
    bwd_prep_x3       D = rowsum(dO*O), planes of dO                reference model.cu:609
    bwd_dkdv_ds_x3    dK, dV -> dqkv[:, :, k and v blocks]; dS      reference model.cu:609, 653
    bwd_dq_ds_x3      dQ = dS K -> dqkv[:, :, q block]              reference model.cu:609, 653
bf16 default and --path packed (fp32 on the fp32 MFMA): the split-transposes are fused into
the attention kernels' tile copies and stores, so qkv (B,T,3C) is read and dqkv (B,T,3C)
written directly:
    attn_fwd_packed   qkv -> O (B,H,T,d), m, l                    reference model.cu:305-311
    bwd_dq_packed     D = rowsum(dO*O), dQ -> dqkv[:, :, q block]  reference model.cu:609, 653
    bwd_dkdv_packed   dK, dV -> dqkv[:, :, k and v blocks]         reference model.cu:609, 653
fp32 on the fp32 MFMA takes the backward's dS-first order instead (attn_packed_causal_
backward_ds_f32's stages: dK/dV write dS, dQ is computed from it):
    bwd_prep_packed     D = rowsum(dO*O)                           reference model.cu:609
    bwd_dkdv_ds_packed  dK, dV -> dqkv[:, :, k and v blocks]; dS     reference model.cu:609, 653
    bwd_dq_ds_packed    dQ = dS K -> dqkv[:, :, q block]             reference model.cu:609, 653
--path split runs the reference's launcher sequence with separate split-transpose kernels:
    qkv (B,T,3C) --split-transpose--> q,k,v (B,H,T,d)             reference model.cu:305
    tiled forward          -> O, m, l                             reference model.cu:311
    backward stage 1       -> D = rowsum(dO*O), dQ                 reference model.cu:609
    backward stage 2       -> dK, dV                               reference model.cu:609
    dq,dk,dv --split-transpose backward--> dqkv (B,T,3C)          reference model.cu:653
packed and split produce bitwise the same O, m, l and dqkv (tests/test_gpu_packed.py).  Inputs (qkv,
dO) are synthetic N(0,1) from a fixed seed and resident in HBM before the timed region
starts.

value = algorithmic FLOPs of causal attention fwd+bwd, 7*B*H*T^2*d (FlashAttention-2
convention: fwd 2*B*H*T^2*d, bwd 5*B*H*T^2*d), divided by the wall-clock time of the K
timed steps.  Before the W warmup steps, untimed steps run for --ramp-s seconds (ramp_s in
the line, default 0.5) so that the GPU's clocks have left their idle state: a few
milliseconds of warmup alone leave the timed steps partly at ramp-up clocks (config 2:
~10% below the steady rate).  The roofline object describes the dominant kernel (the launch
with the most algorithmic work, the dK/dV stage on every path; its average duration is
measured with HIP events recorded on the launch stream around it in every timed step)
against its algorithmic FLOPs:
    forward 2 units, backward dK/dV 4 units (S recompute, dP, dV, dK), backward dQ 1 unit
    (dQ; its S and dP recomputes, where it makes them, duplicate work already counted), unit =
    B*H*T^2*d.  bwd_prep_x3 is HBM-bound: it reads O and dO (fp32) and writes the three bf16
    planes of dO and D, 14*B*H*T*d + 4*B*H*T bytes.
The other kernels' durations (the line's "kernels" table) come from a separate pass after the
timed steps, with an event after every launch: each event record takes about 2.5 us of GPU
time, so events around all five launches of the config-2 step would add about 16 us to a
343 us step.
For the x3 path the roofline is the bf16 MFMA's: achieved = 6 x the algorithmic FLOPs (six
bf16 plane products per fp32 product) per second against the bf16 peak, with the fp32
algorithmic rate (TFLOP/s, not a fraction of any peak) beside it.
The split-transpose kernels are HBM-bound: 6*B*T*C*elem_bytes algorithmic bytes each.
roofline.traffic is the dominant kernel's measured HBM bytes per dispatch, read from
profiles/hbm_traffic.md (rocprofv3 FETCH_SIZE and WRITE_SIZE of this same bench command,
scaled by a device-copy calibration); null when that file has no row for the workload.

secondary: the same workload through the other paths (fp32: the fp32 MFMA path, packed and
the reference's split sequence), the step in bf16 at config 2's shape and at configs 3 and 4
(each with its roofline object, a CPU baseline on a bounded sample of its heads and the
bf16 parity gate), and the reference's materialised mode (fp32, config 2: its six products
on the causal GEMM, which skips the blocks the mask leaves unused, and the fused softmax
kernels) as a timed fwd+bwd with a per-launch table and its own roofline object.

parity_gate: the north star's gate applied to the cpu_baseline comparison (fp32: max-abs
<= 1e-5; bf16: rel-L2 <= 2e-2; O, dQ, dK, dV), on the headline and on each secondary
configuration that has a cpu_baseline.  When any fails the line is still printed and the
exit status is 3: the throughput of a result that fails parity is not valid.

training_step: BASELINE config 5, the reference's GPT-2-small training step (L12 C768 H12
T1024 B8 V50257, fp32, forward + backward + fused clip/AdamW) through the harness of
libtcamd_gpt, once per attention mode (fused_x3 / fused: this build's path on the bf16 MFMA
with three-plane fp32 operands / on the fp32 MFMA; tiled_split: the reference's tiled
launcher sequence; materialized: the reference's default): tokens/s and the share of the
step in the attention launches.

cpu_baseline: the torch-CPU fp32 restatement of the reference attention
(pytorch_src/model.py:43-52, forward + autograd backward) timed on this host on the same
inputs, which also gives a max-abs parity figure for the GPU result.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 5] [--ramp-s 0.5] [--config c2]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))

# MI355X published dense peaks (TFLOP/s) and HBM bandwidth (GB/s).
PEAK_TFLOPS = {"f32": 157.3, "bf16": 2516.6}
PEAK_HBM_GBS = 8000.0

# (B, H, T, d, dtype, qk_scale)
CONFIGS = {
    "c2": (8, 12, 1024, 64, "f32", 1.0),
    "c3": (16, 16, 2048, 64, "bf16", 1.0),
    "c4": (2, 16, 8192, 128, "bf16", 0.5),
}
CONFIG_NAMES = {
    "c2": "causal attention fwd+bwd, GPT-2-small shape (BASELINE config 2)",
    "c3": "causal attention fwd+bwd, bf16 (BASELINE config 3)",
    "c4": "long-context causal attention fwd+bwd, bf16 (BASELINE config 4)",
}
METRIC = "causal attn fwd+bwd TFLOP/s & % MFMA peak, B8 H12 T1024 d64 fp32/bf16"

# kernel -> algorithmic FLOP units (unit = B*H*T^2*d) or HBM bytes factor
FLOP_UNITS = {"attn_fwd": 2, "bwd_dq": 1, "bwd_dkdv": 4,
              "attn_fwd_packed": 2, "bwd_dq_packed": 1, "bwd_dkdv_packed": 4,
              "attn_fwd_x3": 2, "bwd_dq_x3": 1, "bwd_dkdv_x3": 4,
              "bwd_dkdv_ds_x3": 4, "bwd_dq_ds_x3": 1,
              "bwd_dkdv_ds_packed": 4, "bwd_dq_ds_packed": 1}
X3_PRODUCTS = 6  # bf16 plane products per fp32 product on the x3 path


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ramp-s", type=float, default=0.5,
                    help="seconds of untimed steps before the warmup steps (GPU clocks out of "
                         "their idle state; 0 disables)")
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    ap.add_argument("--dtype", choices=["f32", "bf16"], default=None,
                    help="override the config's dtype")
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--path", choices=["x3", "packed", "split"], default=None,
                    help="x3 (fp32 default): fp32 on the bf16 MFMA as three bf16 planes; "
                         "packed (bf16 default; fp32 on the fp32 MFMA): attention reads qkv and "
                         "writes dqkv directly (split-transposes fused into its tile copies); "
                         "split: the reference's launcher sequence with separate "
                         "split-transpose kernels")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--secondary-cpu-seconds", type=float, default=6.0,
                    help="target CPU time of the cpu_baseline sample of each bf16 secondary "
                         "configuration (c3, c4)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the bf16 secondary measurements")
    ap.add_argument("--secondary-steps", type=int, default=20)
    ap.add_argument("--gpt-steps", type=int, default=5,
                    help="timed steps of the config-5 training-step harness per attention "
                         "mode (0 skips it)")
    ap.add_argument("--gpt-modes", default="fused_x3,fused,tiled_split,materialized",
                    help="attention modes of the training-step measurement (comma separated)")
    ap.add_argument("--materialized-only", action="store_true",
                    help="instead of the bench: only the materialised mode's timed launches "
                         "(config 2, fp32; the secondary line's measurement), one JSON line")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the bench: run 10 plain device copies of MIB MiB (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def copy_calibration(mib):
    """10 launches of torch's device copy of `mib` MiB: FETCH_SIZE and WRITE_SIZE of this
    kernel should each read mib*1024 KiB per dispatch; the ratio calibrates the counters."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda:0", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 10}), flush=True)
    return 0


def load_lib():
    sys.path.insert(0, REPO)
    import __graft_entry__
    return __graft_entry__.load_package()


class PathRunner:
    """Device buffers of one workload and the launches of one step."""

    def __init__(self, lib, B, H, T, d, dtype, seed, qk_scale, path="packed"):
        import torch
        self.lib, self.torch = lib, torch
        self.path = path
        self.B, self.H, self.T, self.d = B, H, T, d
        self.C = H * d
        self.dtype = dtype
        self.tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
        self.scale = 1.0 / math.sqrt(d)
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev).manual_seed(seed)
        qkv = torch.randn((B, T, 3, H, d), generator=g, device=dev, dtype=torch.float32)
        qkv[:, :, :2] *= qk_scale
        self.qkv = qkv.reshape(B, T, 3 * self.C).to(self.tdt).contiguous()
        self.do = torch.randn((B, H, T, d), generator=g, device=dev,
                              dtype=torch.float32).to(self.tdt).contiguous()
        e = lambda: torch.empty((B, H, T, d), device=dev, dtype=self.tdt)
        self.q, self.k, self.v, self.o = e(), e(), e(), e()
        self.dq, self.dk, self.dv = e(), e(), e()
        st = lambda: torch.empty((B, H, T), device=dev, dtype=torch.float32)
        self.m, self.l, self.ws = st(), st(), st()
        self.dqkv = torch.empty_like(self.qkv)
        if path == "x3":
            if dtype != "f32":
                raise ValueError("the x3 path computes fp32 attention")
            self.planes = torch.empty(lib.f32x3_workspace_bytes(B, H, T, d), device=dev,
                                      dtype=torch.uint8)
        if path == "packed" and dtype == "f32":  # the dS-first backward's dS
            self.ds = torch.empty(lib.f32_ds_workspace_bytes(B, H, T, d) // 4, device=dev,
                                  dtype=torch.float32)

    def launches(self):
        L, a = self.lib, (self.B, self.H, self.T, self.d)
        B, H, T, d = a
        if self.path == "x3":
            # the forward splits k, v (and writes the planes of q); the backward's three
            # stages (packed_causal_attention_backward_f32x3 in one call)
            return (
                ("attn_fwd_x3", lambda: L.packed_causal_attention_forward_f32x3(
                    self.qkv, self.o, B, H, T, d, self.scale, self.planes, self.m, self.l)),
                ("bwd_prep_x3", lambda: L.packed_causal_attention_backward_prep_f32x3(
                    self.qkv, self.o, self.do, self.ws, B, H, T, d, self.planes, True)),
                ("bwd_dkdv_ds_x3", lambda: L.causal_attention_backward_dkdv_ds_f32x3(
                    self.qkv, self.m, self.l, self.ws, self.dqkv, B, H, T, d, self.scale,
                    self.planes)),
                ("bwd_dq_ds_x3", lambda: L.causal_attention_backward_dq_ds_f32x3(
                    self.dqkv, B, H, T, d, self.scale, self.planes)),
            )
        if self.path == "packed" and self.dtype == "f32":
            # the split-transposes happen inside the attention kernels' tile copies/stores;
            # the backward in the dS-first order
            return (
                ("attn_fwd_packed", lambda: L.packed_causal_attention_forward(
                    self.qkv, self.o, B, H, T, d, self.scale, self.m, self.l)),
                ("bwd_prep_packed", lambda: L.packed_causal_attention_backward_prep(
                    self.o, self.do, self.ws, B, H, T, d)),
                ("bwd_dkdv_ds_packed", lambda: L.packed_causal_attention_backward_dkdv_ds(
                    self.qkv, self.do, self.m, self.l, self.ws, self.dqkv, self.ds, B, H, T, d,
                    self.scale)),
                ("bwd_dq_ds_packed", lambda: L.causal_attention_backward_dq_ds(
                    self.qkv, self.dqkv, self.ds, B, H, T, d, self.scale)),
            )
        if self.path == "packed":
            # the split-transposes happen inside the attention kernels' tile copies/stores
            return (
                ("attn_fwd_packed", lambda: L.packed_causal_attention_forward(
                    self.qkv, self.o, B, H, T, d, self.scale, self.m, self.l)),
                ("bwd_dq_packed", lambda: L.packed_causal_attention_backward_dq(
                    self.qkv, self.o, self.do, self.m, self.l, self.dqkv, self.ws, B, H, T, d,
                    self.scale)),
                ("bwd_dkdv_packed", lambda: L.packed_causal_attention_backward_dkdv(
                    self.qkv, self.do, self.m, self.l, self.ws, self.dqkv, B, H, T, d,
                    self.scale)),
            )
        return (
            ("split_fwd", lambda: L.qkv_split_transpose_forward(
                self.qkv, self.q, self.k, self.v, B, T, H, d)),
            ("attn_fwd", lambda: L.tiled_causal_attention_forward(
                self.q, self.k, self.v, self.o, B, H, T, d, self.scale, self.m, self.l)),
            ("bwd_dq", lambda: L.tiled_causal_attention_backward_dq(
                self.q, self.k, self.v, self.o, self.do, self.m, self.l, self.dq, self.ws,
                B, H, T, d, self.scale)),
            ("bwd_dkdv", lambda: L.tiled_causal_attention_backward_dkdv(
                self.q, self.k, self.v, self.do, self.m, self.l, self.ws, self.dk, self.dv,
                B, H, T, d, self.scale)),
            ("split_bwd", lambda: L.qkv_split_transpose_backward(
                self.dq, self.dk, self.dv, self.dqkv, B, T, H, d)),
        )

    def step(self):
        for _, fn in self.launches():
            fn()

    def flops_total(self):
        return 7.0 * self.B * self.H * self.T * self.T * self.d

    def kernel_work(self, name):
        """(algorithmic amount per launch, unit) of one kernel."""
        unit = float(self.B * self.H * self.T * self.T * self.d)
        if name in FLOP_UNITS:
            return FLOP_UNITS[name] * unit, "flop"
        if name == "bwd_prep_x3":
            n = float(self.B * self.H * self.T * self.d)
            return 14.0 * n + 4.0 * self.B * self.H * self.T, "byte"
        if name == "bwd_prep_packed":  # O and dO read in fp32, D written
            n = float(self.B * self.H * self.T * self.d)
            return 8.0 * n + 4.0 * self.B * self.H * self.T, "byte"
        elem = 2 if self.dtype == "bf16" else 4
        return 6.0 * self.B * self.T * self.C * elem, "byte"

    def dominant(self):
        """Name of the launch with the most algorithmic FLOPs (the dK/dV stage)."""
        flop = [(self.kernel_work(n)[0], n) for n, _ in self.launches()
                if self.kernel_work(n)[1] == "flop"]
        return max(flop)[1]

    def timed(self, steps, warmup, ramp_s=0.0, breakdown_steps=20, event_every=None):
        """Time `steps` steps after `ramp_s` seconds of untimed steps and `warmup` more, with
        events on the launch stream around the dominant launch of every `event_every`-th
        timed step only (default steps // 20: about 20 sampled steps spread over the run, every
        step below 40; an event record costs GPU time between launches); then the other
        launches' durations from `breakdown_steps` more steps (not timed) with an event after
        every launch."""
        torch = self.torch
        t_end = time.perf_counter() + ramp_s
        while time.perf_counter() < t_end:
            for _ in range(10):
                self.step()
            torch.cuda.synchronize()
        for _ in range(warmup):
            self.step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        launches = self.launches()
        dom = self.dominant()
        every = event_every if event_every else max(1, steps // 20)
        sampled = range(0, steps, every)
        evs = {i: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for i in sampled}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            ev = evs.get(i)
            for name, fn in launches:
                if ev is not None and name == dom:
                    ev[0].record(stream)
                    fn()
                    ev[1].record(stream)
                else:
                    fn()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        dom_ms = sum(a.elapsed_time(b) for a, b in evs.values()) / len(evs)
        n = max(1, breakdown_steps)
        evb = [[torch.cuda.Event(enable_timing=True) for _ in range(len(launches) + 1)]
               for _ in range(n)]
        for i in range(n):
            evb[i][0].record(stream)
            for j, (_, fn) in enumerate(launches):
                fn()
                evb[i][j + 1].record(stream)
        torch.cuda.synchronize()
        per_kernel = {}
        for j, (name, _) in enumerate(launches):
            ms = [evb[i][j].elapsed_time(evb[i][j + 1]) for i in range(n)]
            per_kernel[name] = sum(ms) / len(ms)
        per_kernel[dom] = dom_ms  # the timed steps' own measurement
        return wall, per_kernel

    def outputs_finite(self):
        torch = self.torch
        outs = (self.o, self.dqkv) if self.path in ("packed", "x3") else (
            self.o, self.dq, self.dk, self.dv, self.dqkv)
        return all(bool(torch.isfinite(t.float()).all()) for t in outs)

    def head_major_inputs(self):
        """(q, k, v) as (B, H, T, d) views of qkv (the split-transpose's outputs)."""
        B, H, T, d = self.B, self.H, self.T, self.d
        x = self.qkv.view(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
        return x[0], x[1], x[2]

    def head_major_grads(self):
        """(dq, dk, dv) as (B, H, T, d) tensors, whichever path produced them."""
        if self.path == "split":
            return self.dq, self.dk, self.dv
        B, H, T, d = self.B, self.H, self.T, self.d
        g = self.dqkv.view(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
        return g[0], g[1], g[2]


def measured_traffic(config, dtype, kernel):
    """HBM bytes per dispatch of `kernel` from profiles/hbm_traffic.md (rocprofv3
    FETCH_SIZE + WRITE_SIZE of this bench command, scaled by the copy calibration that file
    states), or None when the file has no row for this (config, dtype, kernel)."""
    path = os.path.join(REPO, "profiles", "hbm_traffic.md")
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None
    for ln in lines:
        # | config | dtype | path | kernel | FETCH KiB | WRITE KiB | traffic_bytes | ...
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 7 and cells[:2] == [config, dtype] and cells[3] == kernel:
            try:
                return int(cells[6])
            except ValueError:
                return None
    return None


def roofline_of(runner, per_kernel, config):
    name = runner.dominant()
    amount, kind = runner.kernel_work(name)
    sec = per_kernel[name] * 1e-3
    extra = {}
    if kind == "flop" and runner.path == "x3":
        alg = amount / sec / 1e12
        achieved = X3_PRODUCTS * alg
        peak = PEAK_TFLOPS["bf16"]
        bound, unit = "mfma", "TFLOP/s"
        extra = {"mfma_type": "bf16 (fp32 operands as three bf16 planes, six products each)",
                 "fp32_algorithmic_tflops": round(alg, 3)}
    elif kind == "flop":
        achieved = amount / sec / 1e12
        peak = PEAK_TFLOPS[runner.dtype]
        bound, unit = "mfma", "TFLOP/s"
    else:
        achieved = amount / sec / 1e9
        peak = PEAK_HBM_GBS
        bound, unit = "hbm", "GB/s"
    return name, dict({"bound": bound, "achieved": round(achieved, 3), "peak": peak,
                       "unit": unit, "frac": round(achieved / peak, 4),
                       "traffic": measured_traffic(config, runner.dtype, name)}, **extra)


def kernel_table(runner, per_kernel):
    out = {}
    for name, ms in per_kernel.items():
        amount, kind = runner.kernel_work(name)
        if kind == "flop":
            rate = amount / (ms * 1e-3) / 1e12
            out[name] = {"ms": round(ms, 4), "tflops": round(rate, 2)}
            if runner.path == "x3":  # runs on the bf16 MFMA: its fraction of that peak
                out[name]["frac_bf16_mfma_executed"] = round(
                    X3_PRODUCTS * rate / PEAK_TFLOPS["bf16"], 4)
            else:
                out[name]["frac_mfma"] = round(rate / PEAK_TFLOPS[runner.dtype], 4)
        else:
            rate = amount / (ms * 1e-3) / 1e9
            out[name] = {"ms": round(ms, 4), "gbs": round(rate, 1),
                         "frac_hbm": round(rate / PEAK_HBM_GBS, 4)}
    return out


def cpu_baseline(runner, target_s):
    """Time the torch-CPU fp32 restatement on this host (bounded sample) and compare its
    result with the GPU's last step on the same inputs."""
    import numpy as np
    import torch
    from oracle import attention_ref as ref

    torch.set_num_threads(os.cpu_count() or 1)
    cores = torch.get_num_threads()
    B, H, T, d = runner.B, runner.H, runner.T, runner.d
    f = lambda t: t.float().cpu()
    q, k, v = (f(t).contiguous() for t in runner.head_major_inputs())
    do = f(runner.do)
    # sample: whole (b, h) heads in groups of up to 8 slices of one batch row, cycling over
    # the workload's heads until about target_s of CPU time has been spent (the first pass
    # over each head also gives the GPU-vs-CPU difference)
    heads = [(b, h) for b in range(B) for h in range(H)]
    groups = []
    per = max(1, min(8, int(8 * (1024 / T) ** 2)))  # T x T matrices of a group: ~8 at T = 1024
    for i in range(0, len(heads), per):
        grp = heads[i:i + per]
        for b in sorted({b for b, _ in grp}):
            hs = [h for bb, h in grp if bb == b]
            groups.append((b, hs[0], hs[-1] + 1))
    ref.attention_fwd_bwd(q[:1, :1], k[:1, :1], v[:1, :1], do[:1, :1], runner.scale)  # warm-up
    errs = {n: 0.0 for n in ("o", "dq", "dk", "dv")}
    sq_diff = {n: 0.0 for n in errs}
    sq_ref = {n: 0.0 for n in errs}
    dq_, dk_, dv_ = runner.head_major_grads()
    got = {"o": f(runner.o), "dq": f(dq_), "dk": f(dk_), "dv": f(dv_)}
    n_eval, t_cpu, gi = 0, 0.0, 0
    while t_cpu < target_s and gi < 1000 * len(groups):
        b, h0, h1 = groups[gi % len(groups)]
        t0 = time.perf_counter()
        r = ref.attention_fwd_bwd(q[b:b + 1, h0:h1], k[b:b + 1, h0:h1], v[b:b + 1, h0:h1],
                                  do[b:b + 1, h0:h1], runner.scale)
        t_cpu += time.perf_counter() - t0
        if gi < len(groups):
            for n in errs:
                want = getattr(r, n).double()
                diff = got[n][b:b + 1, h0:h1].double() - want
                errs[n] = max(errs[n], diff.abs().max().item())
                sq_diff[n] += float((diff * diff).sum())
                sq_ref[n] += float((want * want).sum())
        n_eval += h1 - h0
        gi += 1
    compared = sum(h1 - h0 for _, h0, h1 in groups[:min(gi, len(groups))])
    flops = runner.flops_total() * n_eval / len(heads)
    # rel-L2 as scripts/compare_parity.py:17 defines it, over the compared heads
    rel = {n: math.sqrt(sq_diff[n]) / (math.sqrt(sq_ref[n]) + 1e-12) for n in errs}
    return {
        "value": round(flops / t_cpu / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{n_eval} (b,h)-head evaluations ({n_eval / len(heads):.2f} passes over "
                   f"the {len(heads)} heads of the same workload and inputs, T={T}, d={d}), "
                   f"torch {torch.__version__} CPU fp32 restatement of "
                   f"pytorch_src/model.py:43-52 fwd + autograd bwd, {t_cpu:.1f} s"
                   + (" on the bf16-rounded inputs widened to fp32" if runner.dtype == "bf16"
                      else "")
                   + f"; {os.cpu_count()} host CPUs; value = the sample's FLOPs (7*T^2*d per "
                   f"head) / its CPU time, i.e. extrapolated to the whole workload at the "
                   f"sampled per-head rate; GPU difference over {compared} heads"),
        "seconds": round(t_cpu, 2),
        "gpu_vs_cpu_max_abs": {n: float(f"{e:.3e}") for n, e in errs.items()},
        "gpu_vs_cpu_rel_l2": {n: float(f"{e:.3e}") for n, e in rel.items()},
        "heads_compared": compared,
    }


def parity_gate(dtype, cpu):
    """The north star's gate on the GPU-vs-CPU comparison of the cpu_baseline leg: fp32
    max-abs <= 1e-5 (scripts/compare_parity.py:108-109's tolerance), bf16 rel-L2 <= 2e-2,
    for O, dQ, dK, dV."""
    if cpu is None:
        return {"checked": False, "pass": None}
    if dtype == "bf16":
        vals, tol, kind = cpu["gpu_vs_cpu_rel_l2"], 2e-2, "rel_l2"
    else:
        vals, tol, kind = cpu["gpu_vs_cpu_max_abs"], 1e-5, "max_abs"
    return {"checked": True, "kind": kind, "tolerance": tol, "heads": cpu["heads_compared"],
            "pass": all(v <= tol for v in vals.values())}


def secondary(lib, cfg, dtype, steps, seed, path="packed", ramp_s=0.0, cpu_s=0.0):
    B, H, T, d, _, qk = CONFIGS[cfg]
    r = PathRunner(lib, B, H, T, d, dtype, seed, qk, path)
    wall, per_kernel = r.timed(steps, 3, ramp_s)
    ms = wall / steps * 1e3
    tf = r.flops_total() / (ms * 1e-3) / 1e12
    attn_ms = sum(ms_ for n, ms_ in per_kernel.items() if n in FLOP_UNITS)
    dom, roof = roofline_of(r, per_kernel, cfg)
    peak_key = "fp32_equivalent_frac" if path == "x3" else "frac_mfma_peak"
    out = {"config": cfg, "path": path, "shape": f"B{B} H{H} T{T} d{d}", "dtype": dtype,
           "ms_per_step": round(ms, 4), "tflops": round(tf, 2),
           peak_key: round(tf / PEAK_TFLOPS[dtype], 4),
           "attn_only_tflops": round(r.flops_total() / (attn_ms * 1e-3) / 1e12, 2),
           "roofline": dict(roof, kernel=dom),
           "kernels": kernel_table(r, per_kernel), "finite": r.outputs_finite()}
    if cpu_s > 0:
        out["cpu_baseline"] = cpu_baseline(r, cpu_s)
        out["parity_gate"] = parity_gate(dtype, out["cpu_baseline"])
    del r
    return out


# The materialised entry points run the softmax with zero_block 128: the products read a
# probability row only up to the end of its 128-column diagonal block.
MAT_ZERO_BLOCK = 128


def materialized(lib, steps, seed):
    """The reference's materialised mode (src/model.cu:313-332 forward, 617-650 backward) at
    config 2 fp32, launch by launch as attn_materialized_causal_{forward,backward}_f32 run it:
    QK^T, the causal softmax, PV; dO V^T, P^T dO, the softmax backward, dS K, dS^T Q.  The six
    products run on the causal GEMM (attn_matmul_batched_strided_causal_f32), which skips the
    blocks the mask makes unused; each launch is timed with HIP events.  roofline: the launch
    with the longest average, a GEMM, against the fp32 MFMA peak with its algorithmic work
    (one unit B*H*T^2*d: the causal half of the full product); the softmax kernels' rates
    are HBM rates of the bytes they must move (forward: the causal half of S read, P written
    where the products read it, up to the end of each row's 128-column diagonal block;
    backward: the causal halves of dP and P read, dS written likewise)."""
    import torch
    B, H, T, d, _, _ = CONFIGS["c2"]
    g = torch.Generator(device="cpu").manual_seed(seed)
    q, k, v, do = (torch.randn((B, H, T, d), generator=g).to("cuda:0") for _ in range(4))
    sq = lambda: torch.empty((B * H * T, T), device="cuda:0")
    scores, probs, dprobs, dscores = sq(), sq(), sq(), sq()
    out, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
    scale = 1.0 / math.sqrt(d)
    BH, sh, ss = B * H, T * d, T * T
    L = lib
    gemm = lambda A, Bm, C, M, N, K, sA, sB, sC, ta, tb, tri: (
        lambda: L.matmul_batched_strided_causal(A, Bm, C, M, N, K, sA, sB, sC, BH, ta, tb, tri))
    launches = [
        ("gemm_qk", gemm(q, k, scores, T, T, d, sh, sh, ss, False, True, L.GEMM_LOWER_OUT)),
        ("softmax_fwd", lambda: L.causal_softmax_forward(scores, probs, B, H, T, scale,
                                                         zero_block=MAT_ZERO_BLOCK)),
        ("gemm_pv", gemm(probs, v, out, T, d, T, ss, sh, sh, False, False, L.GEMM_LOWER_A)),
        ("gemm_dp", gemm(do, v, dprobs, T, T, d, sh, sh, ss, False, True, L.GEMM_LOWER_OUT)),
        ("gemm_dv", gemm(probs, do, dv, T, d, T, ss, sh, sh, True, False, L.GEMM_UPPER_A)),
        ("softmax_bwd", lambda: L.causal_softmax_backward(dprobs, probs, dscores, B, H, T,
                                                          scale, zero_block=MAT_ZERO_BLOCK)),
        ("gemm_dq", gemm(dscores, k, dq, T, d, T, ss, sh, sh, False, False, L.GEMM_LOWER_A)),
        ("gemm_dk", gemm(dscores, q, dk, T, d, T, ss, sh, sh, True, False, L.GEMM_UPPER_A)),
    ]
    for _ in range(3):
        for _, fn in launches:
            fn()
    torch.cuda.synchronize()
    # the whole mode through its two entry points (what a caller runs), then launch by launch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        L.materialized_causal_attention_forward(q, k, v, scores, probs, out, B, H, T, d, scale)
        L.materialized_causal_attention_backward(q, k, v, probs, do, dprobs, dscores, dq, dk,
                                                 dv, B, H, T, d, scale)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(launches) + 1)]
          for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        for j, (_, fn) in enumerate(launches):
            fn()
            ev[i][j + 1].record()
    torch.cuda.synchronize()
    unit = float(B * H * T * T * d)
    half = B * H * T * (T + 1) / 2.0 * 4  # bytes of the causal half of one T x T matrix set
    zb = MAT_ZERO_BLOCK  # bytes written: row i up to min(T, (i // zb + 1) * zb)
    blk = B * H * 4.0 * sum(min(T, (i // zb + 1) * zb) for i in range(T))
    alg = {"softmax_fwd": (half + blk, "byte"), "softmax_bwd": (2 * half + blk, "byte")}
    kernels = {}
    for j, (name, _) in enumerate(launches):
        t = sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(steps)) / steps
        amount, kind = alg.get(name, (unit, "flop"))
        if kind == "flop":
            kernels[name] = {"ms": round(t, 4), "tflops": round(amount / (t * 1e-3) / 1e12, 2),
                             "frac_mfma": round(amount / (t * 1e-3) / 1e12 / PEAK_TFLOPS["f32"], 4)}
        else:
            kernels[name] = {"ms": round(t, 4), "gbs": round(amount / (t * 1e-3) / 1e9, 1),
                             "frac_hbm": round(amount / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    dom = max((n for n in kernels if n.startswith("gemm")), key=lambda n: kernels[n]["ms"])
    achieved = unit / (kernels[dom]["ms"] * 1e-3) / 1e12
    out_d = {"config": "c2", "mode": "materialised (causal GEMMs + fused softmax)",
             "dtype": "f32", "ms_per_step": round(ms, 4),
             "tflops_algorithmic": round(7 * unit / (ms * 1e-3) / 1e12, 2),
             "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                          "peak": PEAK_TFLOPS["f32"], "unit": "TFLOP/s",
                          "frac": round(achieved / PEAK_TFLOPS["f32"], 4),
                          "traffic": measured_traffic("c2", "f32", f"materialized_{dom}"),
                          "kernel": dom},
             "kernels": kernels,
             "finite": bool(torch.isfinite(dq).all() and torch.isfinite(out).all())}
    del scores, probs, dprobs, dscores
    return out_d


# the reference's GPT-2-small training step (fp32, AdamW).
GPT_C5 = dict(V=50257, T=1024, C=768, L=12, H=12, d_ff=3072, B=8)


def gpt_training_step(mode, steps, warmup, seed):
    """Config 5 through the GPT training-step harness (libtcamd_gpt: the reference's
    TransformerModel forward/backward + fused clip/AdamW, rocBLAS GEMMs) with the attention
    of every block in `mode`: tokens/s of the whole step (forward, backward, optimizer) and
    the share of the step spent in the attention launches (HIP events around them)."""
    import numpy as np
    import torch
    import __graft_entry__
    gpt = __graft_entry__.load_gpt()
    c = GPT_C5
    cfg = gpt.default_config(c["V"], c["T"], c["C"], c["L"], c["H"], c["d_ff"], c["B"], mode)
    model = gpt.GPT(cfg)
    rng = np.random.default_rng(seed)
    flat = (rng.standard_normal(model.n_params, dtype=np.float32) * 0.02).astype(np.float32)
    off = 0  # LayerNorm gamma 1, beta and biases 0 (src/model.cu:219-241)
    for name, shape in gpt.param_layout(c["V"], c["T"], c["C"], c["L"], c["d_ff"]):
        n = int(np.prod(shape))
        leaf = name.split(".")[-1]
        if leaf.endswith("_g"):
            flat[off:off + n] = 1.0
        elif leaf.endswith("_b"):
            flat[off:off + n] = 0.0
        off += n
    model.set_parameters(flat)
    del flat
    g = torch.Generator(device="cpu").manual_seed(seed)
    tokens = torch.randint(0, c["V"], (c["B"], c["T"]), generator=g, dtype=torch.int32).cuda()
    targets = torch.randint(0, c["V"], (c["B"], c["T"]), generator=g, dtype=torch.int32).cuda()
    loss = torch.zeros(1, device="cuda:0")
    for _ in range(warmup):
        model.forward_backward(tokens, targets, loss)
        model.optimizer_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.forward_backward(tokens, targets, loss)
        model.optimizer_step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    model.set_attention_timing(True)
    model.forward_backward(tokens, targets, loss)
    model.optimizer_step()
    attn_ms = model.last_attention_ms()
    torch.cuda.synchronize()
    out = {"config": "c5", "workload": "GPT-2-small training step (BASELINE config 5)",
           "attention": mode, "dtype": "f32", "ms_per_step": round(ms, 3),
           "tokens_per_s": round(c["B"] * c["T"] / (ms * 1e-3), 1),
           "attention_ms": round(attn_ms, 3),
           "attention_share": round(attn_ms / ms, 4),
           "loss": round(float(loss.item()), 5), "finite": bool(math.isfinite(loss.item())),
           "params": model.n_params}
    model.close()
    torch.cuda.empty_cache()
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(attention is independent per (batch, head): it shards by batch or head with no "
              "exchange inside the path, and each GPU runs this same single-GPU kernel set)", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    lib = load_lib()
    if args.materialized_only:
        print(json.dumps(materialized(lib, args.steps, args.seed)), flush=True)
        return 0
    B, H, T, d, cdt, qk = CONFIGS[args.config]
    dtype = args.dtype or cdt
    path = args.path or ("x3" if dtype == "f32" and d <= 64 else "packed")
    runner = PathRunner(lib, B, H, T, d, dtype, args.seed, qk, path)
    wall, per_kernel = runner.timed(args.steps, args.warmup, args.ramp_s)
    ms = wall / args.steps * 1e3
    value = runner.flops_total() / (ms * 1e-3) / 1e12
    dom, roof = roofline_of(runner, per_kernel, args.config)
    attn_ms = sum(ms_ for n, ms_ in per_kernel.items() if n in FLOP_UNITS)
    props = torch.cuda.get_device_properties(0)
    if path == "x3":
        line_x3 = {"frac_bf16_mfma_executed": round(X3_PRODUCTS * value / PEAK_TFLOPS["bf16"],
                                                    4)}
    else:
        line_x3 = {}
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ramp_s": args.ramp_s,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "path": path,
        "data": "synthetic N(0,1) qkv and dO from a fixed seed, resident in HBM",
        "config": {"workload": CONFIG_NAMES[args.config], "B": B, "H": H, "T": T,
                   "d_head": d, "causal": True,
                   "step": " + ".join(n for n, _ in runner.launches()),
                   "flops_per_step": runner.flops_total()},
        ("fp32_equivalent_frac" if path == "x3" else "frac_mfma_peak"):
            round(value / PEAK_TFLOPS[dtype], 4),
        "attn_only_tflops": round(runner.flops_total() / (attn_ms * 1e-3) / 1e12, 3),
        "arithmetic": (("fp32 operands as three bf16 planes (24 significant bits) on the bf16 "
                        "MFMA, six plane products per fp32 product, fp32 accumulation; "
                        "fp32_equivalent_frac is the fp32 algorithmic rate over the fp32 MFMA "
                        "peak (a comparison, not a fraction of a peak this path runs on), "
                        "frac_bf16_mfma_executed the executed bf16 work over the bf16 peak")
                       if path == "x3" else f"{dtype} MFMA, fp32 accumulation"),
        **line_x3,
        "roofline": dict(roof, kernel=dom),
        "kernels": kernel_table(runner, per_kernel),
        "finite": runner.outputs_finite(),
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "torch": torch.__version__},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(runner, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    line["parity_gate"] = parity_gate(dtype, line["cpu_baseline"])
    del runner
    torch.cuda.empty_cache()
    if not args.no_secondary:
        others = {"x3": ["packed", "split"], "packed": ["split"], "split": ["packed"]}[path]
        sec = [secondary(lib, args.config, dtype, args.secondary_steps, args.seed, o,
                         args.ramp_s) for o in others]
        if dtype != "bf16":
            sec.append(secondary(lib, args.config, "bf16", args.secondary_steps, args.seed,
                                 ramp_s=args.ramp_s))
        # the bf16 configurations, each with a CPU baseline on a bounded sample of its heads
        cpu_s = 0.0 if args.no_cpu_baseline else args.secondary_cpu_seconds
        for c in ("c3", "c4"):
            if c != args.config:
                sec.append(secondary(lib, c, "bf16", args.secondary_steps, args.seed,
                                     ramp_s=args.ramp_s, cpu_s=cpu_s))
        sec.append(materialized(lib, max(3, args.secondary_steps // 4), args.seed))
        line["secondary"] = sec
    if args.gpt_steps > 0:
        line["training_step"] = [gpt_training_step(m, args.gpt_steps, 2, args.seed)
                                 for m in args.gpt_modes.split(",")]
    print(json.dumps(line), flush=True)
    failed = [("headline", line["parity_gate"])] if line["parity_gate"]["pass"] is False else []
    failed += [(f"{s_.get('config')} {s_.get('path', s_.get('mode'))}", s_["parity_gate"])
               for s_ in line.get("secondary", [])
               if s_.get("parity_gate", {}).get("pass") is False]
    if failed:
        print("bench.py: results fail the parity gate against the CPU restatement "
              f"({failed}); the throughput figures of the line above are not valid",
              file=sys.stderr)
        return 3
    return 0


if __name__ == "__main__":
    sys.exit(main())
