#!/usr/bin/env python3
"""Benchmark of the SF37 MoE FFN layer on one MI355X.

Workload: one MoE layer decode step of 8 tokens,
E=288 experts, K=4096, F=1280, top-8, Q3GU gate/up + Q2D down experts and a
Q8_0 shared expert, router logits injected i.i.d. N(0,1) (uniform routing).
A step is the whole layer on device-resident inputs: router GEMV over the 8
tokens (computed although the injected logits drive the selection), top-8
selection, shared expert, routed experts, shared + routed.  With the fused
decode path that is six kernel launches (route, select, up, mid, down,
combine); for one token the select work runs inside the up launch.

Steps rotate over --layers independently seeded layers (each with its own
input tokens), so consecutive steps never reuse weights and the 256 MB
last-level cache cannot serve them.  value = algorithmic HBM bytes per step
(distinct selected experts x 6,225,920 + shared 16,711,680 + router
4,718,592 + x/out activations) / measured step time.

roofline: the kernel with the largest share of the step time, its
algorithmic bytes per launch over its average launch time from HIP events
on the launch stream in a second, identical pass with stage events enabled.
cpu_baseline: the reference CPU MoE path (sf37_ops.c/sf37_quant.c built with
the reference `make cpu` flags) on one step's tokens, single core.

Also on the line: config0 (the one-token decode step,
same layers) with its own roofline; parity of the HIP layer against the
reference CPU layer on the same weights and x (router logits from x):
indices equal and max |gpu - cpu| / max(|cpu|, 1), for the decode configs
and 8 sampled tokens of each prefill chunk; prefill (configs 3 and 2) with
its matrix-core figures and a CPU baseline timed on the leading tokens of
the config 3 chunk; stack.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0     # MI355X dense fp16/bf16 matrix peak
EXPERT_BYTES = 6_225_920
GATE_UP_EXPERT_BYTES = 2 * 2_252_800
DOWN_EXPERT_BYTES = 1_720_320
Q8K_BLOCK = 268


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8, help="distinct layers rotated per step")
    ap.add_argument("--decode-tokens", type=int, default=8,
                    help="tokens per decode step (8 = BASELINE configs[1]; 1..16 take the fused decode path)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run 10 device-to-device copies of MIB MiB (calibrates the HBM counters)")
    ap.add_argument("--prefill-steps", type=int, default=5, help="timed layers per prefill config (0 = skip)")
    ap.add_argument("--prefill-only", action="store_true", help="only the prefill configs (2 and 3)")
    ap.add_argument("--stack-layers", type=int, default=45, help="layers of the config 4 stack (0 = skip)")
    ap.add_argument("--stack-steps", type=int, default=20, help="timed decode tokens through the stack")
    ap.add_argument("--stack-prefill-steps", type=int, default=2, help="timed 2048-token chunks through the stack")
    ap.add_argument("--stack-only", action="store_true", help="only the config 4 stack")
    ap.add_argument("--opt", action="append", default=[], metavar="NAME=VALUE",
                    help="library option (sf37_hip_set_option) set before measuring; repeatable")
    return ap.parse_args()


def copy_calibration(mib):
    """10 device-to-device copies of mib MiB each (the runtime's copy kernel):
    FETCH_SIZE / WRITE_SIZE per dispatch of this run against the known size
    give the scale that turns those counters into HBM bytes."""
    from sf37_amd import hip
    hip.init()
    n = mib << 20
    a, b = hip.Tensor.alloc(n), hip.Tensor.alloc(n)
    L = hip.lib()
    for _ in range(10):
        hip.check(L.sf37_hip_tensor_copy(b, 0, a, 0, n), "copy")
    hip.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_dispatch": n, "dispatches": 10}), flush=True)


class Hip:
    """hipEvent timing on the null stream (the library's launch stream)."""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        self.L.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.L.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.L.hipEventSynchronize.argtypes = [C.c_void_p]
        self.L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.L.hipDeviceSynchronize.argtypes = []

    def event(self):
        e = C.c_void_p()
        assert self.L.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream=None):
        assert self.L.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.L.hipEventSynchronize(b) == 0
        t = C.c_float()
        assert self.L.hipEventElapsedTime(C.byref(t), a, b) == 0
        return t.value

    def sync(self):
        assert self.L.hipDeviceSynchronize() == 0


def main():
    args = parse()
    if args.copy_calib:
        copy_calibration(args.copy_calib)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(expert parallelism across GPUs is a design, not built)", file=sys.stderr)
        sys.exit(2)

    from sf37_amd import configs, hip, moe

    hip.init()
    H = Hip()
    n_tok, E, K, F, TOPK = args.decode_tokens, moe.EXPERTS, moe.EMBD, moe.EXPERT_FF, moe.EXPERT_USED
    if not 1 <= n_tok <= 16:
        print(f"bench.py: --decode-tokens {n_tok}: the decode step takes 1..16 tokens", file=sys.stderr)
        sys.exit(2)
    # the router GEMV/GEMM runs inside the layer although injected logits select
    hip.set_option("router_with_logits", 1)
    for kv in args.opt:
        name, _, val = kv.partition("=")
        hip.set_option(name, int(val))        # raises on an unknown name
    if args.prefill_only:
        lay = moe.SynthLayer(seed=moe.layer_seed(args.seed, 0))
        print(json.dumps({"prefill": [prefill_bench(args, H, lay, c) for c in (3, 2)]}), flush=True)
        return
    if args.stack_only:
        print(json.dumps({"stack": stack_bench(args, H)}), flush=True)
        return

    dec = decode_bench(args, H, n_tok)
    dec1 = decode_bench(args, H, 1, layers=dec["layers"], summary=True) if n_tok != 1 else None
    q3q2 = {f"decode_{t}tok": shared_q3q2_bench(args, H, dec["layers"], t) for t in sorted({n_tok, 1}, reverse=True)}
    prefill = [prefill_bench(args, H, dec["layers"][0], c) for c in (3, 2)] if args.prefill_steps > 0 else None

    cpu, parity = None, None
    if not args.no_cpu:
        lay0 = dec["layers"][0]
        cpu = cpu_baseline(lay0, dec["xs"][0], dec["sels"][0], dec["step_bytes"][0], n_tok, args.cpu_seconds)
        parity = {f"config{1 if n_tok == 8 else 'x'}_decode_{n_tok}tok":
                  parity_vs_cpu(lay0, dec["xs"][0].read(np.float32).reshape(n_tok, K))}
        if dec1 is not None:
            parity["config0_decode_1tok"] = parity_vs_cpu(lay0, dec["xs"][0].read(np.float32).reshape(n_tok, K)[:1])
        if prefill:
            for pf in prefill:
                c = pf["config"]
                xs_c = configs.x_device(c, args.seed + 1000 * c, pf["tokens"])
                parity[f"config{c}_prefill_{pf['tokens']}tok_sample8"] = parity_vs_cpu(
                    lay0, xs_c.read(np.float32).reshape(pf["tokens"], K), n_check=8)
                if c == 3 and cpu is not None:
                    pf["cpu_baseline"] = cpu_prefill_baseline(lay0, xs_c.read(np.float32).reshape(pf["tokens"], K),
                                                              args.cpu_seconds)
                xs_c.free()
            for pf in prefill:
                if pf["config"] != 3 and cpu is not None:
                    pf["cpu_baseline"] = dict(prefill[0].get("cpu_baseline") or {}, note=
                                              "the CPU path is per token (sf37.c:7786-7797); the config 3 sample "
                                              "time applies to any chunk")
    for lay in dec["layers"]:
        lay.free()
    stack = stack_bench(args, H) if args.stack_layers > 0 else None

    value, ms_per_step, mean_bytes = dec["value"], dec["ms_per_step"], dec["mean_bytes"]
    line = {
        "metric": "MoE layer decode HBM GB/s (% of peak); prefill tokens/s/layer, MFMA util",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized by the reference quantizer; x ~ N(0,1); "
                "injected N(0,1) router logits)",
        "config": {"workload": ("BASELINE configs[1]: " if n_tok == 8 else "")
                               + f"one MoE layer decode step, {n_tok} tokens, uniform routing",
                   "experts": E, "hidden": K, "expert_ff": F, "top_k": TOPK,
                   "formats": "Q3GU gate/up, Q2D down, Q8_0 shared, fp32 router",
                   "layers_rotated": args.layers, "hbm_bytes_per_step": int(mean_bytes),
                   "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2)},
        "roofline": dec["roofline"],
        "cpu_baseline": cpu,
        "stages": dec["stages"],
        "stage_timing": STAGE_TIMING_NOTE,
        "config0": dec1,
        "shared_q3q2": q3q2,
        "parity": parity,
        "prefill": prefill,
        "stack": stack,
    }
    print(json.dumps(line), flush=True)


STAGE_TIMING_NOTE = ("stage and roofline kernel times are HIP events recorded around each launch on the launch "
                     "stream in a second identical pass: they include the dispatch, so short kernels read longer "
                     "than rocprofv3's kernel durations (profiles/ holds the rocprofv3 traces of the same command)")


def decode_bench(args, H, n_tok, layers=None, summary=False):
    """Timed decode steps of n_tok tokens over --layers rotated layers (made
    here unless given); the dominant kernel's roofline from a second pass
    with stage events.  With summary, only the figures are returned (the
    inputs made here are freed)."""
    from sf37_amd import configs, hip, moe
    E, K, F, TOPK = moe.EXPERTS, moe.EMBD, moe.EXPERT_FF, moe.EXPERT_USED
    own = layers is None
    layers = [] if own else layers
    xs, lgs, sels = [], [], []
    for l in range(args.layers):
        seed = moe.layer_seed(args.seed, l)
        if own:
            layers.append(moe.SynthLayer(seed=seed))
        xs.append(configs.x_device(1, seed, n_tok))
        lg = configs.logits_for(1, seed, n_tok)
        lgs.append(hip.Tensor.from_array(lg))
    out = hip.Tensor.alloc(n_tok * K * 4)
    sel = hip.Tensor.alloc(n_tok * TOPK * 4)
    wts = hip.Tensor.alloc(n_tok * TOPK * 4)
    L = hip.lib()
    structs = [lay.weights_struct() for lay in layers]

    def step(i):
        l = i % args.layers
        hip.check(L.sf37_hip_moe_layer(out, sel, wts, structs[l], lgs[l], xs[l], n_tok), "moe layer")

    # distinct experts per layer's routing -> algorithmic bytes per step and
    # per kernel of the fused path
    P = n_tok * TOPK
    step_bytes, kern_bytes = [], []
    for l in range(args.layers):
        step(l)
        s = sel.read(np.int32).reshape(n_tok, TOPK)
        sels.append(s)
        distinct = len(np.unique(s))
        lay = layers[l]
        act = n_tok * K * 4 * 2
        step_bytes.append(distinct * EXPERT_BYTES + lay.shared_bytes() + lay.router_bytes() + act)
        sh_gu = lay.sh_gate.nbytes + lay.sh_up.nbytes
        nb, nbf = K // 256, F // 256
        kern_bytes.append({
            # router weights + x in; logits, selection candidates (12 B), x activation
            # blocks (288 B) and Q8_0 of x out
            "dec_route": lay.router_bytes() + n_tok * K * 4 + n_tok * E * (4 + 12) + n_tok * nb * 288
                         + n_tok * K + n_tok * (K // 32) * 4,
            # candidates in, selections out; shared gate/up weights + Q8_0 x in, gate/up rows
            # out (a launch of its own above one token, else part of dec_up)
            "dec_select": n_tok * E * 12 + P * 8 + sh_gu + n_tok * K + n_tok * (K // 32) * 4
                          + 2 * n_tok * F * 4,
            # routed gate/up weights of the distinct experts + x blocks in, gate/up rows out
            "dec_up": distinct * GATE_UP_EXPERT_BYTES + n_tok * nb * 288 + 2 * P * F * 4,
            # gate/up rows in, mid and its activation blocks out; shared gate/up rows in,
            # Q8_0 shared mid out
            "dec_mid": 2 * P * F * 4 + P * F * 4 + P * nbf * 288 + 2 * n_tok * F * 4 + n_tok * F
                       + n_tok * (F // 32) * 4,
            # routed down weights + mid blocks in, per-pair rows out; shared down weights +
            # Q8_0 shared mid in, shared rows out
            "dec_down": distinct * DOWN_EXPERT_BYTES + P * nbf * 288 + P * K * 4
                        + lay.sh_down.nbytes + n_tok * F + n_tok * (F // 32) * 4 + n_tok * K * 4,
            # per-pair rows and shared rows in, out
            "dec_combine": P * K * 4 + n_tok * K * 4 + n_tok * K * 4,
        })
    hip.synchronize()

    for i in range(args.warmup):
        step(i)
    H.sync()
    a, b = H.event(), H.event()
    H.record(a)
    for i in range(args.steps):
        step(i)
    H.record(b)
    ms = H.elapsed_ms(a, b)
    H.sync()
    ms_per_step = ms / args.steps
    mean_bytes = float(np.mean([step_bytes[i % args.layers] for i in range(args.steps)]))
    value = mean_bytes / (ms_per_step * 1e-3) / 1e9

    # second identical pass with stage events: per-kernel launch times
    L.sf37_hip_profile_enable(1)
    hip.profile_read()
    for i in range(args.steps):
        step(i)
    prof = hip.profile_read()
    L.sf37_hip_profile_enable(0)
    kern = max(("dec_route", "dec_select", "dec_up", "dec_mid", "dec_down", "dec_combine"), key=lambda k: prof[k][0])
    k_ms, k_n = prof[kern]
    if k_n == 0:
        raise SystemExit("bench.py: the fused decode kernels did not run")
    if prof["dec_select"][1] == 0:      # the select work ran inside dec_up
        for kb in kern_bytes:
            kb["dec_up"] += kb.pop("dec_select")
    k_avg_ms = k_ms / k_n
    k_mean_bytes = float(np.mean([kern_bytes[i % args.layers][kern] for i in range(args.steps)]))
    achieved = k_mean_bytes / (k_avg_ms * 1e-3) / 1e9
    traffic = measured_traffic(kern, n_tok)
    stages = {k: {"ms_per_launch": round(v[0] / max(v[1], 1), 5), "launches": v[1]} for k, v in prof.items() if v[1]}
    roof = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": kern, "bytes_per_launch": int(k_mean_bytes), "ms_per_launch": round(k_avg_ms, 5)}
    for t in [out, sel, wts] + lgs:
        t.free()
    res = {"value": value, "ms_per_step": ms_per_step, "mean_bytes": mean_bytes, "roofline": roof,
           "stages": stages}
    if summary:
        if own:
            for lay in layers:
                lay.free()
        for x in xs:
            x.free()
        return {"workload": ("BASELINE configs[0]: " if n_tok == 1 else "")
                            + f"one MoE layer decode step, {n_tok} token(s), uniform routing",
                "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms_per_step, 5),
                "hbm_bytes_per_step": int(mean_bytes), "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
                "roofline": roof, "stages": stages}
    res.update(layers=layers, xs=xs, sels=sels, step_bytes=step_bytes)
    return res


def shared_q3q2_bench(args, H, layers, n_tok):
    """The decode step with the shared expert in Q3GU gate/up and Q2D down
    (the BASELINE configurations' "same formats" option, 6,225,920 bytes),
    on the same routed experts, inputs and injected routing as the headline,
    whose shared expert is the reference engine's own Q8_0 (sf37.c:1780-1782).
    The library runs that shared expert as one more expert of weight 1 with
    the shared clamp through the Q8_K decode launches, then the routed
    launches add it."""
    from sf37_amd import configs, hip, moe
    K, F, TOPK = moe.EMBD, moe.EXPERT_FF, moe.EXPERT_USED
    L = hip.lib()
    shared, structs, xs, lgs, step_bytes = [], [], [], [], []
    for l, lay in enumerate(layers):
        seed = moe.layer_seed(args.seed, l)
        sg = hip.synth_quant("q3", F, K, seed, moe.STREAM["sh_gate"])
        su = hip.synth_quant("q3", F, K, seed, moe.STREAM["sh_up"])
        sd = hip.synth_quant("q2", K, F, seed, moe.STREAM["sh_down"])
        shared.append((sg, su, sd))
        structs.append(hip.LayerWeights(lay.router.h, lay.router_bias.h, lay.gate.h, lay.up.h, lay.down.h, sg.h,
                                        su.h, sd.h, lay.n_expert, lay.topk, lay.in_dim, lay.mid_dim, 3.0,
                                        lay.clamp_routed, lay.clamp_shared, hip.TYPE_F32, hip.TYPE_Q3GU))
        xs.append(configs.x_device(1, seed, n_tok))
        lgs.append(hip.Tensor.from_array(configs.logits_for(1, seed, n_tok)))
    out = hip.Tensor.alloc(n_tok * K * 4)
    sel = hip.Tensor.alloc(n_tok * TOPK * 4)
    wts = hip.Tensor.alloc(n_tok * TOPK * 4)
    n = len(layers)

    def step(i):
        hip.check(L.sf37_hip_moe_layer(out, sel, wts, structs[i % n], lgs[i % n], xs[i % n], n_tok),
                  "moe layer (q3q2 shared)")

    for l in range(n):
        step(l)
        distinct = len(np.unique(sel.read(np.int32)))
        sh = sum(t.nbytes for t in shared[l])
        step_bytes.append(distinct * EXPERT_BYTES + sh + layers[l].router_bytes() + n_tok * K * 4 * 2)
    for i in range(args.warmup):
        step(i)
    H.sync()
    a, b = H.event(), H.event()
    H.record(a)
    for i in range(args.steps):
        step(i)
    H.record(b)
    ms = H.elapsed_ms(a, b) / args.steps
    H.sync()
    mean_bytes = float(np.mean([step_bytes[i % n] for i in range(args.steps)]))
    value = mean_bytes / (ms * 1e-3) / 1e9
    for t in [out, sel, wts] + xs + lgs + [x for sh in shared for x in sh]:
        t.free()
    return {"workload": (f"BASELINE configs[{1 if n_tok == 8 else 0}] with " if n_tok in (1, 8) else "")
                        + f"the shared expert in Q3GU/Q2D, {n_tok} token(s)",
            "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5),
            "hbm_bytes_per_step": int(mean_bytes), "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2)}


def parity_vs_cpu(layer, x, n_check=None):
    """The HIP layer (router logits from x) against the reference CPU layer
    (oracle/_ref/libsf37cpu_ref.so: the reference's sf37_ops.c / sf37_quant.c
    composed as layer_moe_ffn, sf37.c:2127-2194) on the first n_check rows of
    x: whether both select the same experts per token, and
    max |gpu - cpu| / max(|cpu|, 1) over the outputs."""
    import oracle
    from sf37_amd import hip
    lib = oracle.cpu_baseline_lib("reference")
    kind = "reference"
    if lib is None:
        lib, kind = oracle.cpu_baseline_lib("port"), "port"
    if lib is None:
        return None
    n_tok, K = x.shape
    E, F, TOPK = layer.n_expert, layer.mid_dim, layer.topk
    xd = hip.Tensor.from_array(np.ascontiguousarray(x, np.float32))
    out, sel, wts = hip.Tensor.alloc(n_tok * K * 4), hip.Tensor.alloc(n_tok * TOPK * 4), \
        hip.Tensor.alloc(n_tok * TOPK * 4)
    hip.check(hip.lib().sf37_hip_moe_layer(out, sel, wts, layer.weights_struct(), None, xd, n_tok), "moe layer (parity)")
    n = n_tok if n_check is None else min(n_check, n_tok)
    got = out.read(np.float32).reshape(n_tok, K)[:n]
    gsel = sel.read(np.int32).reshape(n_tok, TOPK)[:n]
    for t in (xd, out, sel, wts):
        t.free()
    dense = layer.host_dense()
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    bp = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint8))

    def cpu_rows(experts):
        want = np.zeros((n, K), np.float32)
        csel = np.zeros((n, TOPK), np.int32)
        for t in range(n):
            lib.sf37cpu_moe_ffn_token(fp(want[t]), csel[t].ctypes.data_as(C.POINTER(C.c_int32)),
                                      fp(dense["router"]), fp(dense["router_bias"]), bp(experts["gate"]),
                                      bp(experts["up"]), bp(experts["down"]), bp(dense["sh_gate"]),
                                      bp(dense["sh_up"]), bp(dense["sh_down"]), E, TOPK, K, F,
                                      layer.clamp_routed, layer.clamp_shared, fp(np.ascontiguousarray(x[t], np.float32)))
        return want, csel

    want, csel = cpu_rows(layer.host_experts(np.unique(gsel)))
    same = bool(np.array_equal(np.sort(gsel, axis=1), np.sort(csel, axis=1)))
    if not same:                       # the CPU chose other experts: run it with those present
        want, csel = cpu_rows(layer.host_experts(np.unique(np.concatenate([gsel.ravel(), csel.ravel()]))))
    diff = np.abs(got.astype(np.float64) - want)
    scale = np.maximum(np.abs(want.astype(np.float64)), 1.0)
    err = diff / scale
    ok = bool(np.all((diff <= 5e-2) | (diff <= 1e-1 * scale)))
    return {"reference": f"CPU MoE layer from the reference sources ({kind}), same weights and x, router from x",
            "tokens_compared": int(n), "indices_equal": same, "max_abs_rel": float(f"{err.max():.4e}"),
            "max_abs": float(f"{diff.max():.4e}"), "within_reference_tolerance": ok,
            "tolerance": "an element fails when |diff| > 5e-2 and |diff| > 1e-1 * max(1, |cpu|) (the reference's "
                         "own Q8_K-GPU-vs-CPU MoE check, tests/test_sf37_cuda_ops.cu:20-30,814); the GPU path "
                         "quantises activations to Q8_K as the reference CUDA path does, the CPU path keeps fp32"}


def cpu_prefill_baseline(layer, x, budget_s):
    """The reference CPU MoE path over the leading tokens of a prefill chunk
    (the CPU engine runs a chunk token by token, sf37.c:7786-7797), for about
    budget_s seconds; tokens/s/layer of that sample."""
    import oracle
    lib = oracle.cpu_baseline_lib("reference")
    kind = "reference"
    if lib is None:
        lib, kind = oracle.cpu_baseline_lib("port"), "port"
    if lib is None:
        return None
    K, F, E, TOPK = layer.in_dim, layer.mid_dim, layer.n_expert, layer.topk
    dense = layer.host_dense()
    experts = layer.host_experts(np.arange(E))
    out = np.zeros(K, np.float32)
    csel = np.zeros(TOPK, np.int32)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    bp = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint8))
    n, t0 = 0, time.perf_counter()
    while n < x.shape[0]:
        lib.sf37cpu_moe_ffn_token(fp(out), csel.ctypes.data_as(C.POINTER(C.c_int32)), fp(dense["router"]),
                                  fp(dense["router_bias"]), bp(experts["gate"]), bp(experts["up"]),
                                  bp(experts["down"]), bp(dense["sh_gate"]), bp(dense["sh_up"]),
                                  bp(dense["sh_down"]), E, TOPK, K, F, 0.0, 0.0, fp(np.ascontiguousarray(x[n])))
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 2), "unit": "tokens/s/layer", "cores": 1, "kind": kind,
            "sample": f"the first {n} tokens of the config 3 chunk (its x rows, routing from x) through the "
                      f"reference CPU MoE path, one token at a time as the CPU engine runs a chunk, {dt:.1f} s"}


def prefill_bench(args, H, layer, config):
    """One MoE layer over a prefill chunk (512 tokens,
    Zipf-skewed routing; configs[3]: 4096 tokens, uniform): router GEMM,
    top-8, shared expert, routed experts on the matrix cores, add.  Reports
    tokens/s/layer and, for the two matrix-core kernels, achieved fp16 MFMA
    TFLOP/s (algorithmic 2*M*N*K per pair) from HIP-event stage times."""
    from sf37_amd import configs, hip
    n_tok = configs.CONFIG_TOKENS[config]
    K, F, E, TOPK = layer.in_dim, layer.mid_dim, layer.n_expert, layer.topk
    seed = args.seed + 1000 * config
    x = configs.x_device(config, seed, n_tok)
    lg = hip.Tensor.from_array(configs.logits_for(config, seed, n_tok))
    out, sel, wts = hip.Tensor.alloc(n_tok * K * 4), hip.Tensor.alloc(n_tok * TOPK * 4), \
        hip.Tensor.alloc(n_tok * TOPK * 4)
    L = hip.lib()
    st = layer.weights_struct()

    def step():
        hip.check(L.sf37_hip_moe_layer(out, sel, wts, st, lg, x, n_tok), "moe layer (prefill)")

    step()
    H.sync()
    a, b = H.event(), H.event()
    H.record(a)
    for _ in range(args.prefill_steps):
        step()
    H.record(b)
    ms = H.elapsed_ms(a, b) / args.prefill_steps
    L.sf37_hip_profile_enable(1)
    hip.profile_read()
    for _ in range(args.prefill_steps):
        step()
    prof = hip.profile_read()
    L.sf37_hip_profile_enable(0)
    P = n_tok * TOPK
    flops = {"pf_gate_up": 2.0 * P * (2 * F) * K, "pf_down": 2.0 * P * F * K}
    mfma = {}
    for k, f in flops.items():
        k_ms, k_n = prof[k]
        if k_n == 0:
            raise SystemExit(f"bench.py: {k} did not run for config {config}")
        t = f / (k_ms / k_n * 1e-3) / 1e12
        mfma[k] = {"achieved": round(t, 1), "ms_per_launch": round(k_ms / k_n, 4),
                   "frac": round(t / MFMA_F16_PEAK_TFLOPS, 4), "timing": "HIP events"}
    routed_ms = sum(prof[k][0] / prof[k][1] for k in flops)
    routed_t = sum(flops.values()) / (routed_ms * 1e-3) / 1e12
    counts = np.bincount(sel.read(np.int32).ravel(), minlength=E)
    # VALU issue the exact arithmetic needs at least (the matrix-core kernels'
    # bound): per padded pair, output and 256-block the canonical epilogue's 5
    # operations; per tile the weights' dequantisation (1.5 operations per Q3
    # code, 1 per Q2 code); at 16 lanes per cycle per SIMD, 1024 SIMDs, 2.4 GHz
    tiles = [min(64, c - 64 * i) for c in counts for i in range((int(c) + 63) // 64)]
    padded = sum(32 * ((t + 31) // 32) for t in tiles)
    nbk, nbf = K // 256, F // 256
    valu = {"pf_gate_up": padded * 2 * F * nbk * 5 + len(tiles) * 2 * F * K * 1.5,
            "pf_down": padded * K * nbf * 5 + len(tiles) * K * F * 1.0}
    lane_ops_per_s = 1024 * 16 * 2.4e9
    for k, v in valu.items():
        ceil_ms = v / lane_ops_per_s * 1e3
        mfma[k]["valu_ceiling_ms"] = round(ceil_ms, 4)
        mfma[k]["frac_of_valu_ceiling"] = round(ceil_ms / mfma[k]["ms_per_launch"], 4)
    mfma["executed_over_algorithmic_flops"] = round(padded / P, 4)
    stages = {k: round(v[0] / v[1], 4) for k, v in prof.items() if v[1]}
    return {"config": config, "tokens": n_tok, "ms_per_layer": round(ms, 4),
            "tokens_per_s_per_layer": round(n_tok / (ms * 1e-3), 1),
            "routed_mfma": {"bound": "mfma", "achieved": round(routed_t, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(routed_t / MFMA_F16_PEAK_TFLOPS, 4),
                            "dtype": "f16 operands holding exact small integers, fp32 accumulate",
                            "timing": "HIP events around each launch on its stream (include the dispatch; "
                                      "profiles/prefill_layer_kernel_trace.md has rocprofv3 kernel durations)"},
            "kernels": mfma, "max_pairs_per_expert": int(counts.max()), "idle_experts": int((counts == 0).sum()),
            "stage_ms": stages}


def stack_bench(args, H):
    """--stack-layers independently seeded layers resident
    in HBM, h <- h + MoE_l(RMSNorm_l(h)) through all of them, Zipf-skewed
    injected router logits (the router still runs).  Decode: one token through
    the stack per step; prefill: one 2048-token chunk per step.  Each step
    starts from its own input rows (a device copy into h, inside the step) and
    steps rotate over two logits sets per layer.  HBM bytes per step = over
    the layers, distinct selected experts x 6,225,920 + shared + router + norm
    weights + the fp32 activation rows the norm, layer and add read and write
    (7 x tokens x 16 KiB)."""
    from sf37_amd import configs, hip, moe
    t0 = time.time()
    S = moe.SynthStack(master=moe.layer_seed(args.seed, 4000), n_layers=args.stack_layers)
    hip.synchronize()
    gen_s = time.time() - t0
    print(f"stack: {S.n_layers} layers generated in {gen_s:.1f} s", file=sys.stderr, flush=True)
    Lh = hip.lib()
    K, TOPK, NL = S.in_dim, moe.EXPERT_USED, S.n_layers
    lay0 = S.layers[0]
    fixed = lay0.shared_bytes() + lay0.router_bytes() + K * 2
    resident = NL * (lay0.n_expert * EXPERT_BYTES + fixed)
    res = {"workload": "BASELINE configs[4]: MoE stack, RMSNorm(w+1) + residual between layers, Zipf routing",
           "layers": NL, "resident_weight_bytes": int(resident), "generate_s": round(gen_s, 1)}
    for mode, n_tok, steps in (("decode", 1, args.stack_steps), ("prefill", 2048, args.stack_prefill_steps)):
        if steps <= 0:
            continue
        n_sets = 2
        xs = [configs.x_device(4, 4000 + 10 * s + n_tok, n_tok) for s in range(n_sets)]
        lgs = [[hip.Tensor.from_array(configs.logits_for(4, moe.layer_seed(4000 + 10 * s + n_tok, l), n_tok))
                for l in range(NL)] for s in range(n_sets)]
        sels = [hip.Tensor.alloc(n_tok * TOPK * 4) for _ in range(NL)]
        h, xn, y = (hip.Tensor.alloc(n_tok * K * 4) for _ in range(3))
        wts = hip.Tensor.alloc(n_tok * TOPK * 4)

        def step(i):
            s = i % n_sets
            hip.check(Lh.sf37_hip_tensor_copy(h, 0, xs[s], 0, n_tok * K * 4), "stack input copy")
            S.forward(h, n_tok, xn, y, sels, wts, lgs[s])

        step_bytes = []
        for s in range(n_sets):
            step(s)
            b = 0
            for l in range(NL):
                distinct = len(np.unique(sels[l].read(np.int32)))
                b += distinct * EXPERT_BYTES + fixed + 7 * n_tok * K * 4
            step_bytes.append(b)
        H.sync()
        a, b = H.event(), H.event()
        H.record(a)
        for i in range(steps):
            step(i)
        H.record(b)
        ms = H.elapsed_ms(a, b) / steps
        H.sync()
        Lh.sf37_hip_profile_enable(1)
        hip.profile_read()
        for i in range(steps):
            step(i)
        prof = hip.profile_read()
        Lh.sf37_hip_profile_enable(0)
        mean_bytes = float(np.mean([step_bytes[i % n_sets] for i in range(steps)]))
        gbs = mean_bytes / (ms * 1e-3) / 1e9
        kern_ms = sum(v[0] for v in prof.values()) / steps
        res[mode] = {"tokens": n_tok, "steps": steps, "ms_per_step": round(ms, 4),
                     "tokens_per_s": round(n_tok / (ms * 1e-3), 1), "hbm_bytes_per_step": int(mean_bytes),
                     "hbm_gbs": round(gbs, 1), "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
                     "ms_per_layer": round(ms / NL, 4), "kernel_ms_per_step": round(kern_ms, 4),
                     "stage_ms_per_step": {k: round(v[0] / steps, 4) for k, v in prof.items() if v[1]}}
        print(f"stack {mode}: {res[mode]['tokens_per_s']} tokens/s, {res[mode]['hbm_gbs']} GB/s",
              file=sys.stderr, flush=True)
        for t in xs + [x for ls in lgs for x in ls] + sels + [h, xn, y, wts]:
            t.free()
    S.free()
    return res


def measured_traffic(kern, n_tok):
    """HBM bytes per launch of kern at n_tok tokens from the counter summary
    in profiles/ (rocprofv3 FETCH_SIZE / WRITE_SIZE scaled by a copy
    calibration, table rows "| kernel | tokens | fetch | write | hbm bytes |"),
    or None."""
    path = os.path.join(ROOT, "profiles", "decode_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == kern and cells[1] == str(n_tok) and cells[4].isdigit():
            return int(cells[4])
    return None


def cpu_baseline(layer, x_dev, sel, step_bytes, n_tok, budget_s):
    """Reference CPU MoE path on this step's tokens (1 core)."""
    import oracle
    kind = "reference"
    lib = oracle.cpu_baseline_lib("reference")
    if lib is None:
        kind = "port"
        lib = oracle.cpu_baseline_lib("port")
    if lib is None:
        return None
    K, F, E = layer.in_dim, layer.mid_dim, layer.n_expert
    dense = layer.host_dense()
    experts = layer.host_experts(np.unique(sel))
    x = x_dev.read(np.float32).reshape(n_tok, K)
    out = np.zeros(K, np.float32)
    got_sel = np.zeros(8, np.int32)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    bp = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint8))
    reps, t0 = 0, time.perf_counter()
    # router logits on the CPU come from x (the CPU path has no injected
    # logits), so it may pick other experts; the timing covers the same work
    # (router + shared + 8 routed experts per token)
    while True:
        for t in range(n_tok):
            lib.sf37cpu_moe_ffn_token(fp(out), got_sel.ctypes.data_as(C.POINTER(C.c_int32)), fp(dense["router"]),
                                      fp(dense["router_bias"]), bp(experts["gate"]), bp(experts["up"]),
                                      bp(experts["down"]), bp(dense["sh_gate"]), bp(dense["sh_up"]),
                                      bp(dense["sh_down"]), E, 8, K, F, 0.0, 0.0, fp(np.ascontiguousarray(x[t])))
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 20:
            break
    dt = (time.perf_counter() - t0) / reps
    cpu_model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(step_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "ms_per_token": round(dt * 1e3 / n_tok, 3),
            "sample": f"{reps} x one {n_tok}-token decode step of layer 0 through the reference CPU MoE path "
                      f"(layer_moe_ffn composition, sf37.c:2127-2194), {dt * 1e3:.1f} ms/step on {cpu_model}"}


if __name__ == "__main__":
    main()
