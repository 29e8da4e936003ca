#!/usr/bin/env python3
"""MSDA benchmark on one MI355X: the reference's headline workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--preset decoder]

One step = one forward + one backward (all three gradients, grad_value
zero-fill included) of multi-scale deformable attention over one batch of the
preset's synthetic inputs, already resident in HBM.  Steps are launched
through the C ABI (libmsda_hip.so) and replayed from a HIP graph, so the
timed region measures the device, not the Python launcher (the reference's
published numbers are device times too: benchmarks/modal_benchmark.py:101-124).

Prints ONE JSON line:
  value        algorithmic GB/s of the fwd+bwd step (bytes by the reference's
               accounting, labs/03_the_machine.py:232-251)
  ms_per_step  fwd+bwd wall time per step over the K timed steps
  fwd_us / bwd_us / fwd_gbps ...  per-call device times from HIP events around
               graph replays of R calls (bwd = every kernel of one msda_backward
               call: owner + gradient kernels, or zero-fill + atomic kernel);
               *_cold_us with L2 and Infinity Cache flushed before each call;
               bwd_deterministic_us the bitwise-reproducible backward
  roofline     backward pass (the dominant cost) vs 8 TB/s HBM
  roofline_fwd forward kernel vs 8 TB/s HBM (the operator's stated target)
  other_presets fwd / bwd / fwd+bwd device times and GB/s of the other
               benchmark presets (encoder, high-contention, Mask2Former, tiny)
  fused_front_end  decoder shapes: the fused MSDeformAttn front-end (softmax,
               reference point + offset in the kernels) vs the same front-end
               composed from PyTorch ops around the operator
  projections  the attention layer's projections either side of the operator
               (value / offset+logit / output) on the library's MFMA kernels vs
               torch's linear (+ masked_fill) and its backward
  cpu_baseline the CPU oracle (grid_sample restatement) on the host cores
  rel_err      the timed steps' output and three gradients against that
               oracle run (norm-relative; max-abs in cpu_baseline)
  peak_mb      peak device memory of one fwd+bwd through the public operator
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "msda-triton_amd"))

HBM_PEAK_GBPS = 8000.0

# msda_backward_plan codes -> the kernels one msda_backward call runs.
BACKWARD_KERNELS = {
    0: "msda_backward call (zero-fill + direct atomic bwd_kernel)",
    1: "msda_backward call (zero-fill + row-dedup atomic bwd_priv_kernel)",
    2: "msda_backward call (one owner_kernel launch: band workgroups for grad_value, then "
       "scatter-free gradient workgroups for grad_loc/grad_attn)",
    3: "msda_backward call (zero-fill + binned owner: bin_kernel count/fill, bin_scan_kernel, "
       "bin_acc_kernel for grad_value, then scatter-free bwd_kernel for grad_loc/grad_attn)",
}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _traffic(preset: str, kernel: str):
    """HBM bytes per launch measured offline with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, scaled by a copy-kernel calibration), recorded
    in profiles/traffic_<preset>.txt as `<kernel>: <bytes>` lines."""
    path = ROOT / "profiles" / f"traffic_{preset}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(kernel + ":"):
            try:
                return int(float(line.split(":", 1)[1].split()[0]))
            except ValueError:
                return None
    return None


def _cgroup_cpus():
    """CPUs the cgroup's CFS quota grants (cpu.max), or None without a quota."""
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        return None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        return None


def accuracy(got, ref) -> dict:
    """Norm-relative and max-abs error of the GPU results against the oracle
    (the reference's benchmark reports max_err against its fp32 reference,
    benchmarks/modal_benchmark.py:283-287)."""
    res = {}
    for name, x, r in zip(("out", "grad_value", "grad_loc", "grad_attn"), got, ref):
        x = x.detach().double().cpu().reshape(r.shape)
        r = r.double()
        den = r.norm().item()
        res[name] = {"rel_err": float(f"{(x - r).norm().item() / (den or 1.0):.3e}"),
                     "max_abs_err": float(f"{(x - r).abs().max().item():.3e}")}
    return res


def cpu_baseline(preset: str, max_seconds: float = 25.0, gpu_results=None) -> dict:
    """The oracle (msda_reference restatement: per-level F.grid_sample + torch
    autograd) on fp32 upcasts of the same inputs, fwd+bwd, on this host's
    cores: 1 warm-up, then the median of up to 5 runs within ~max_seconds.
    `gpu_results` (out, grad_value, grad_loc, grad_attn of the timed GPU
    steps, same inputs and grad_out) are compared with the oracle's."""
    import torch

    from msda_triton_amd import presets

    sys.path.insert(0, str(ROOT))
    from oracle import run_reference_fp32

    affinity = len(os.sched_getaffinity(0))
    threads = affinity
    torch.set_num_threads(threads)
    value, shapes, _, loc, attn = presets.make_preset_inputs(preset, device="cpu")
    g = presets.make_grad_out(preset, device="cpu")
    ref_out, ref_grads = run_reference_fp32(value, shapes, loc, attn, g)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < max_seconds:
        t0 = time.perf_counter()
        run_reference_fp32(value, shapes, loc, attn, g)
        times.append(time.perf_counter() - t0)
    fwd_b, bwd_b = presets.algorithmic_bytes(preset)
    t = statistics.median(times)
    res = {
        "value": round((fwd_b + bwd_b) / t / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{preset} preset, full batch, fwd+bwd of the grid_sample oracle in fp32 "
                  f"(median of {len(times)} runs, {t * 1e3:.1f} ms each) on {_cpu_model()}",
        "ms_per_step": round(t * 1e3, 3),
        "affinity_cpus": affinity,
        "cgroup_cpu_quota": _cgroup_cpus(),
    }
    if gpu_results is not None:
        res["gpu_vs_oracle"] = accuracy(gpu_results, (ref_out,) + tuple(ref_grads))
    return res


def _capture(fn, reps, dev):
    """A HIP graph of `reps` back-to-back calls of fn (warmed up on a side
    stream first, as graph capture requires)."""
    import torch

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return graph


def _graph_us(fn, dev, reps=10, replays=5):
    """Device time per call: HIP events on the launch stream around
    `replays` replays of a graph holding `reps` calls."""
    import torch

    graph = _capture(fn, reps, dev)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * replays)


def preset_device_times(preset: str, lib, fp32_grad_accum: bool = False) -> dict:
    """fwd / bwd / fwd+bwd device time of one preset (graph-replayed C-ABI
    calls, see _graph_us)."""
    import torch

    from msda_triton_amd import _native, presets
    from msda_triton_amd.ops import _DTYPE_CODE

    dev = torch.device("cuda", 0)
    c = presets.preset_dims(preset)
    B, S, M, D, Q, L, K = c["B"], c["S"], c["M"], c["D"], c["Q"], c["L"], c["K"]
    value, shapes, starts, loc, attn = presets.make_preset_inputs(preset, device=dev)
    grad_out = presets.make_grad_out(preset, device=dev)
    out = torch.empty(B, Q, M, D, dtype=value.dtype, device=dev)
    gv, gl, ga = torch.empty_like(value), torch.empty_like(loc), torch.empty_like(attn)
    accum = (torch.empty(value.shape, dtype=torch.float32, device=dev)
             if fp32_grad_accum and value.dtype != torch.float32 else None)
    dt = _DTYPE_CODE[value.dtype]
    dims = (B, S, M, D, Q, L, K)

    def fwd():
        _native.check(lib.msda_forward(value.data_ptr(), shapes.data_ptr(), starts.data_ptr(),
                                       loc.data_ptr(), attn.data_ptr(), out.data_ptr(), *dims, dt,
                                       torch.cuda.current_stream().cuda_stream), "msda_forward")

    def bwd():
        _native.check(lib.msda_backward(value.data_ptr(), shapes.data_ptr(), starts.data_ptr(),
                                        loc.data_ptr(), attn.data_ptr(), grad_out.data_ptr(),
                                        gv.data_ptr(), None if accum is None else accum.data_ptr(),
                                        gl.data_ptr(), ga.data_ptr(), *dims, dt,
                                        torch.cuda.current_stream().cuda_stream), "msda_backward")

    f_us, b_us = _graph_us(fwd, dev), _graph_us(bwd, dev)
    bd_us = _graph_us(deterministic_backward(lib, value, shapes, starts, loc, attn, grad_out),
                      dev)
    fb, bb = presets.algorithmic_bytes(preset)
    return {"fwd_us": round(f_us, 2), "bwd_us": round(b_us, 2), "fwd_bwd_us": round(f_us + b_us, 2),
            "fwd_gbps": round(fb / f_us / 1e3, 1), "bwd_gbps": round(bb / b_us / 1e3, 1),
            "fwd_bwd_gbps": round((fb + bb) / (f_us + b_us) / 1e3, 1),
            "bwd_deterministic_us": round(bd_us, 2),
            "grad_value_accum": "fp32" if accum is not None else str(value.dtype).split(".")[-1]}


def deterministic_backward(lib, value, shapes, starts, loc, attn, grad_out):
    """A closure calling msda_backward_deterministic (int64 fixed-point
    grad_value) on preallocated outputs and workspace."""
    import torch

    from msda_triton_amd import _native
    from msda_triton_amd.ops import _DTYPE_CODE, deterministic_workspace

    B, S, M, D = value.shape
    _, Q, _, L, K, _ = loc.shape
    gv, gl, ga = torch.empty_like(value), torch.empty_like(loc), torch.empty_like(attn)
    ws = deterministic_workspace(value, loc)
    dt = _DTYPE_CODE[value.dtype]

    def call():
        _native.check(lib.msda_backward_deterministic(
            value.data_ptr(), shapes.data_ptr(), starts.data_ptr(), loc.data_ptr(),
            attn.data_ptr(), grad_out.data_ptr(), gv.data_ptr(),
            None if ws is None else ws.data_ptr(), gl.data_ptr(),
            ga.data_ptr(), B, S, M, D, Q, L, K, dt, torch.cuda.current_stream().cuda_stream),
            "msda_backward_deterministic")

    return call


def fused_calls(lib, preset: str = "decoder") -> dict:
    """Closures calling msda_fused_forward / msda_fused_backward (per-level
    reference points) on the preset's shapes, with their buffers."""
    import torch

    from msda_triton_amd import _native, presets
    from msda_triton_amd.ops import _DTYPE_CODE

    dev = torch.device("cuda", 0)
    c = presets.preset_dims(preset)
    B, S, M, D, Q, L, K = c["B"], c["S"], c["M"], c["D"], c["Q"], c["L"], c["K"]
    value, shapes, starts, ref, off, logits = presets.make_fused_preset_inputs(preset, dev)
    grad_out = presets.make_grad_out(preset, device=dev)
    dt = _DTYPE_CODE[value.dtype]
    dims = (B, S, M, D, Q, L, K)
    out = torch.empty(B, Q, M, D, dtype=value.dtype, device=dev)
    lse = torch.empty(B, Q, M, dtype=torch.float32, device=dev)
    gv, gref = torch.empty_like(value), torch.empty_like(ref)
    goff, glog = torch.empty_like(off), torch.empty_like(logits)
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def fwd():
        _native.check(lib.msda_fused_forward(
            value.data_ptr(), shapes.data_ptr(), starts.data_ptr(), ref.data_ptr(),
            off.data_ptr(), logits.data_ptr(), out.data_ptr(), lse.data_ptr(), *dims, 1, dt,
            st()), "msda_fused_forward")

    def bwd():
        _native.check(lib.msda_fused_backward(
            value.data_ptr(), shapes.data_ptr(), starts.data_ptr(), ref.data_ptr(),
            off.data_ptr(), logits.data_ptr(), lse.data_ptr(), out.data_ptr(),
            grad_out.data_ptr(), gv.data_ptr(), None, gref.data_ptr(), goff.data_ptr(),
            glog.data_ptr(), *dims, 1, dt, st()), "msda_fused_backward")

    return {"fwd": fwd, "bwd": bwd, "inputs": (value, shapes, starts, ref, off, logits),
            "grad_out": grad_out, "out": out}


def fused_front_end_times(lib, preset: str = "decoder") -> dict:
    """The fused MSDeformAttn front-end (msda_fused_forward / _backward,
    per-level reference points) against the same front-end composed from
    PyTorch ops around the plain operator, as the reference's attention layer
    does it (labs/solutions/lab00.py:201-208; backward: softmax backward,
    offset division and reference-point sum, as autograd runs them).  Both
    graph-replayed; device time per call."""
    import torch

    from msda_triton_amd import _native, presets
    from msda_triton_amd.ops import _DTYPE_CODE

    dev = torch.device("cuda", 0)
    c = presets.preset_dims(preset)
    B, S, M, D, Q, L, K = c["B"], c["S"], c["M"], c["D"], c["Q"], c["L"], c["K"]
    f = fused_calls(lib, preset)
    value, shapes, starts, ref, off, logits = f["inputs"]
    grad_out, out = f["grad_out"], f["out"]
    fused_fwd, fused_bwd = f["fwd"], f["bwd"]
    dt = _DTYPE_CODE[value.dtype]
    dims = (B, S, M, D, Q, L, K)
    gv = torch.empty_like(value)
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    scale = shapes.flip(-1).to(value.dtype)[None, None, None, :, None, :]
    loc = ref[:, :, None, :, None, :] + off / scale
    attn = logits.reshape(B, Q, M, L * K).softmax(-1)
    gloc, gattn = torch.empty_like(off), torch.empty(B, Q, M, L * K, dtype=value.dtype,
                                                        device=dev)

    def composed_fwd():
        lo = ref[:, :, None, :, None, :] + off / scale
        at = logits.reshape(B, Q, M, L * K).softmax(-1)
        _native.check(lib.msda_forward(value.data_ptr(), shapes.data_ptr(), starts.data_ptr(),
                                       lo.data_ptr(), at.data_ptr(), out.data_ptr(), *dims, dt,
                                       st()), "msda_forward")

    def composed_bwd():
        _native.check(lib.msda_backward(value.data_ptr(), shapes.data_ptr(), starts.data_ptr(),
                                        loc.data_ptr(), attn.data_ptr(), grad_out.data_ptr(),
                                        gv.data_ptr(), None, gloc.data_ptr(), gattn.data_ptr(),
                                        *dims, dt, st()), "msda_backward")
        torch._softmax_backward_data(gattn, attn, -1, value.dtype)
        torch.div(gloc, scale)
        gloc.sum((2, 4))

    res = {"preset": preset, "reference_points": "(B, Q, L, 2)",
           "fused_fwd_us": _graph_us(fused_fwd, dev), "fused_bwd_us": _graph_us(fused_bwd, dev),
           "composed_fwd_us": _graph_us(composed_fwd, dev),
           "composed_bwd_us": _graph_us(composed_bwd, dev)}
    res["fused_fwd_bwd_us"] = res["fused_fwd_us"] + res["fused_bwd_us"]
    res["composed_fwd_bwd_us"] = res["composed_fwd_us"] + res["composed_bwd_us"]
    return {k: (round(v, 2) if isinstance(v, float) else v) for k, v in res.items()}


def projection_times(lib, preset: str = "decoder", pad_fraction: float = 0.1) -> dict:
    """The attention layer's projections around the operator
    (labs/solutions/lab00.py:199-208) at the preset's sizes: value_proj over
    the B*S value rows (a `pad_fraction` of rows flagged as padding, zeroed
    after the projection as Deformable-DETR does), the offset + logit
    projections of the B*Q query rows (one split call), out_proj over the B*Q
    operator outputs.  Ours: msda_projection_forward / _backward (grad of
    input, weight and bias).  Torch: F.linear (+ masked_fill), and the
    backward autograd runs for it (masked_fill of the gradient, grad_input,
    grad_weight, grad_bias).  Graph-replayed device time per call."""
    import torch

    from msda_triton_amd import presets
    from msda_triton_amd.ops import _DTYPE_CODE

    dev = torch.device("cuda", 0)
    c = presets.preset_dims(preset)
    B, S, M, D, Q, L, K = c["B"], c["S"], c["M"], c["D"], c["Q"], c["L"], c["K"]
    C = M * D
    dtype = presets.make_preset_inputs(preset, device="cpu")[0].dtype
    code = _DTYPE_CODE[dtype]
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator().manual_seed(3)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def one(name, rows, n1, n2, masked):
        x = torch.randn(rows, C, generator=g).to(dev, dtype)
        w1 = (torch.randn(n1, C, generator=g) / C ** 0.5).to(dev, dtype)
        b1 = torch.randn(n1, generator=g).to(dev, dtype)
        w2 = (torch.randn(n2, C, generator=g) / C ** 0.5).to(dev, dtype) if n2 else None
        b2 = torch.randn(n2, generator=g).to(dev, dtype) if n2 else None
        mask = (torch.rand(rows, generator=g) < pad_fraction).to(dev) if masked else None
        m8 = None if mask is None else mask.view(torch.uint8)
        y1 = torch.empty(rows, n1, device=dev, dtype=dtype)
        y2 = torch.empty(rows, n2, device=dev, dtype=dtype) if n2 else None
        gy1 = torch.randn(rows, n1, generator=g).to(dev, dtype)
        gy2 = torch.randn(rows, n2, generator=g).to(dev, dtype) if n2 else None
        gx, gw1, gb1 = torch.empty_like(x), torch.empty_like(w1), torch.empty_like(b1)
        gw2 = torch.empty_like(w2) if n2 else None
        gb2 = torch.empty_like(b2) if n2 else None
        N = n1 + n2
        ws = torch.empty(lib.msda_projection_workspace_bytes(rows, C, N, code),
                         dtype=torch.uint8, device=dev)

        def ours_fwd():
            assert lib.msda_projection_forward(p(x), p(w1), p(b1), p(w2), p(b2), p(m8), p(y1),
                                               p(y2), rows, C, N, n1, code, st()) == 0

        def ours_bwd():
            assert lib.msda_projection_backward(p(x), p(w1), p(w2), p(m8), p(gy1), p(gy2), p(gx),
                                                p(gw1), p(gb1), p(gw2), p(gb2), p(ws), rows, C, N,
                                                n1, code, st()) == 0

        def torch_fwd():
            o = torch.nn.functional.linear(x, w1, b1)
            if mask is not None:
                o = o.masked_fill(mask[:, None], 0)
            if n2:
                torch.nn.functional.linear(x, w2, b2)

        def torch_bwd():
            gx_ = None
            for gy, w in ((gy1, w1), (gy2, w2)):
                if w is None:
                    continue
                gm = gy.masked_fill(mask[:, None], 0) if mask is not None else gy
                gx_ = gm @ w if gx_ is None else gx_ + gm @ w
                torch.mm(gm.t(), x)
                gm.sum(0)

        r = {"rows": rows, "in": C, "out": N, "masked": masked,
             "fwd_us": _graph_us(ours_fwd, dev), "bwd_us": _graph_us(ours_bwd, dev),
             "torch_fwd_us": _graph_us(torch_fwd, dev), "torch_bwd_us": _graph_us(torch_bwd, dev)}
        # algorithmic bytes: fwd reads x and W, writes y; bwd reads x, W, dy
        # and writes dx, dW, db
        r["fwd_bytes"] = (rows * (C + N) + N * C + N) * e
        r["bwd_bytes"] = (rows * (2 * C + N) + 2 * N * C + N) * e
        r["fwd_GBps"] = r["fwd_bytes"] / r["fwd_us"] / 1e3
        r["bwd_GBps"] = r["bwd_bytes"] / r["bwd_us"] / 1e3
        return name, {k: (round(v, 2) if isinstance(v, float) else v) for k, v in r.items()}

    res = dict([one("value_proj", B * S, C, 0, True),
                one("offset_weight_proj", B * Q, M * L * K * 2, M * L * K, False),
                one("out_proj", B * Q, C, 0, False)])
    tot = {k: round(sum(v[k] for v in res.values()), 2)
           for k in ("fwd_us", "bwd_us", "torch_fwd_us", "torch_bwd_us")}
    return {"preset": preset, "dtype": str(dtype).replace("torch.", ""), **res, "total": tot}


OTHER_PRESETS = ("tiny", "decoder_fp16", "decoder_fp32", "encoder", "high_contention",
                 "mask2former_fp32", "mask2former_bf16")


def main() -> int:
    ap = argparse.ArgumentParser(description="MSDA fwd+bwd benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--preset", default="decoder")
    ap.add_argument("--fp32-grad-accum", action="store_true",
                    help="accumulate grad_value in an fp32 scratch buffer")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-presets", action="store_true",
                    help="skip the other presets and the fused front-end timings")
    ap.add_argument("--pmc-driver", action="store_true",
                    help="for rocprofv3 runs: a few eager fwd/bwd calls plus a 256 MiB "
                         "device copy (counter calibration); prints no JSON")
    ap.add_argument("--calls", choices=("operator", "fused", "deterministic"),
                    default="operator",
                    help="with --pmc-driver: which entry points the calls go through")
    ap.add_argument("--projections-only", action="store_true",
                    help="print only the projection timings (JSON) -- a short run to profile")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the MSDA operator has no multi-GPU path in this "
              "build (batch/head sharding needs no communication; see DESIGN.md). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from msda_triton_amd import _native, presets
    from msda_triton_amd.ops import _DTYPE_CODE

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lib = _native.load()
    if args.projections_only:
        print(json.dumps({"projections": projection_times(lib, args.preset)}), flush=True)
        return 0

    c = presets.preset_dims(args.preset)
    B, S, M, D, Q, L, K = c["B"], c["S"], c["M"], c["D"], c["Q"], c["L"], c["K"]
    value, shapes, starts, loc, attn = presets.make_preset_inputs(args.preset, device=dev)
    grad_out = presets.make_grad_out(args.preset, device=dev)
    out = torch.empty(B, Q, M, D, dtype=value.dtype, device=dev)
    grad_value = torch.empty_like(value)
    grad_loc = torch.empty_like(loc)
    grad_attn = torch.empty_like(attn)
    accum = (torch.empty(value.shape, dtype=torch.float32, device=dev)
             if args.fp32_grad_accum and value.dtype != torch.float32 else None)
    dt = _DTYPE_CODE[value.dtype]
    dims = (B, S, M, D, Q, L, K)

    def fwd():
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.msda_forward(value.data_ptr(), shapes.data_ptr(), starts.data_ptr(),
                              loc.data_ptr(), attn.data_ptr(), out.data_ptr(), *dims, dt, st)
        _native.check(rc, "msda_forward")

    def bwd():
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.msda_backward(value.data_ptr(), shapes.data_ptr(), starts.data_ptr(),
                               loc.data_ptr(), attn.data_ptr(), grad_out.data_ptr(),
                               grad_value.data_ptr(), None if accum is None else accum.data_ptr(),
                               grad_loc.data_ptr(), grad_attn.data_ptr(), *dims, dt, st)
        _native.check(rc, "msda_backward")

    def step():
        fwd()
        bwd()

    if args.pmc_driver:
        if args.calls == "fused":
            f = fused_calls(lib, args.preset)
            fwd, bwd = f["fwd"], f["bwd"]
        elif args.calls == "deterministic":
            bwd = deterministic_backward(lib, value, shapes, starts, loc, attn, grad_out)
        for _ in range(3):
            fwd()
            bwd()
        for _ in range(5):
            fwd()
        for _ in range(5):
            bwd()
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"pmc driver done: {args.preset} ({args.calls}), 5 fwd, 5 bwd, 5 copies of "
              f"{src.numel() * 4} bytes")
        return 0

    def capture(fn, reps):
        return _capture(fn, reps, dev)

    # Steps are replayed from HIP graphs of up to 50 back-to-back steps (the
    # host's per-replay launch cost, ~5 us, is then paid once per 50 steps);
    # a second graph takes the remainder, so exactly K steps run.
    per_graph = max(1, min(50, args.steps))
    step_graph = capture(step, per_graph)
    rest = args.steps % per_graph
    rest_graph = capture(step, rest) if rest else None
    for _ in range(args.warmup // per_graph):  # exactly W warmup steps
        step_graph.replay()
    for _ in range(args.warmup % per_graph):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly K steps, synchronised on both sides.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps // per_graph):
        step_graph.replay()
    if rest_graph is not None:
        rest_graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3

    # Per-call device times: HIP events on the launch stream around replays of
    # graphs holding R back-to-back calls.
    def per_call_us(fn, reps=50, replays=10):
        return _graph_us(fn, dev, reps, replays)

    fwd_us = per_call_us(fwd)
    bwd_us = per_call_us(bwd)
    step_us = per_call_us(step, reps=25)
    bwd_det_us = per_call_us(deterministic_backward(lib, value, shapes, starts, loc, attn,
                                                    grad_out), reps=10, replays=5)

    # Cold variants: a 512 MiB read before every call evicts L2 and the
    # 256 MiB Infinity Cache, so the inputs come from HBM; the flush only
    # reads (row maxima: 512 KiB written), so it leaves no dirty lines to be
    # written back during the timed call.  The flush's own time (measured
    # alone) is subtracted.
    flush_buf = torch.ones(128 << 20, dtype=torch.float32, device=dev).view(-1, 4096)
    flush_max = torch.empty(flush_buf.shape[0], dtype=torch.float32, device=dev)

    def flush():
        torch.amax(flush_buf, dim=1, out=flush_max)

    flush_us = per_call_us(flush, reps=10, replays=5)
    fwd_cold_us = per_call_us(lambda: (flush(), fwd()), reps=10, replays=5) - flush_us
    bwd_cold_us = per_call_us(lambda: (flush(), bwd()), reps=10, replays=5) - flush_us
    del flush_buf, flush_max

    # Through the public autograd operator, eagerly (host launch cost included).
    from msda_triton_amd import multi_scale_deformable_attention as msda

    v_l = value.clone().requires_grad_(True)
    l_l = loc.clone().requires_grad_(True)
    a_l = attn.clone().requires_grad_(True)
    g_flat = grad_out.view(B, Q, M * D)

    def api_step():
        v_l.grad = l_l.grad = a_l.grad = None
        o = msda(v_l, shapes, starts, l_l, a_l, fp32_grad_accum=args.fp32_grad_accum)
        o.backward(g_flat)

    for _ in range(5):
        api_step()
    torch.cuda.synchronize()
    # Peak device memory of one fwd+bwd through the public operator (the
    # reference's peak_mb, benchmarks/modal_benchmark.py:180-190): inputs,
    # output, gradients and any scratch the call allocates.
    v_l.grad = l_l.grad = a_l.grad = None
    torch.cuda.synchronize()
    base_mb = torch.cuda.memory_allocated() / 2 ** 20
    torch.cuda.reset_peak_memory_stats()
    api_step()
    torch.cuda.synchronize()
    peak_mb = torch.cuda.max_memory_allocated() / 2 ** 20
    n_api = 50
    t0 = time.perf_counter()
    for _ in range(n_api):
        api_step()
    torch.cuda.synchronize()
    api_us = (time.perf_counter() - t0) / n_api * 1e6

    fwd_b, bwd_b = presets.algorithmic_bytes(args.preset)
    value_gbps = (fwd_b + bwd_b) / (ms_per_step * 1e-3) / 1e9
    bwd_gbps = bwd_b / (bwd_us * 1e-6) / 1e9
    fwd_gbps = fwd_b / (fwd_us * 1e-6) / 1e9
    dtype_name = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}[value.dtype]

    record = {
        "metric": "MSDA fwd+bwd algorithmic HBM GB/s (with fwd and fwd+bwd ms), "
                  f"{args.preset} preset B{B} Q{Q} {dtype_name} (1 GPU)",
        "value": round(value_gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32-accumulate/" + dtype_name,
        "data": "synthetic (seeded CPU generator, preset distributions)",
        "config": {
            "workload": f"msda_{args.preset}_fwd_bwd",
            "B": B, "Q": Q, "M": M, "D": D, "L": L, "K": K, "S": S,
            "spatial_shapes": c["shapes"],
            "grad_value_accum": "fp32" if accum is not None else dtype_name,
            "timing": "HIP-graph replay of C-ABI calls (50 steps per graph); inputs "
                      "resident in HBM",
        },
        "fwd_us": round(fwd_us, 3),
        "bwd_us": round(bwd_us, 3),
        "fwd_bwd_us": round(step_us, 3),
        "fwd_gbps": round(fwd_gbps, 1),
        "bwd_gbps": round(bwd_gbps, 1),
        "bwd_deterministic_us": round(bwd_det_us, 3),
        # grad_value element updates the reference's backward issues as atomics
        # (4 corners x D per sample), per second of the whole backward call
        "atomic_elem_per_s": round(4 * D * B * Q * M * L * K / (bwd_us * 1e-6), 1),
        "fwd_cold_us": round(fwd_cold_us, 3),
        "bwd_cold_us": round(bwd_cold_us, 3),
        "api_eager_fwd_bwd_us": round(api_us, 1),
        "peak_mb": round(peak_mb, 1),
        "peak_mb_above_resident": round(peak_mb - base_mb, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(bwd_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(bwd_gbps / HBM_PEAK_GBPS, 4),
            "traffic": _traffic(args.preset, "backward"),
            "kernel": BACKWARD_KERNELS.get(
                lib.msda_backward_plan(*dims, dt, 0), "msda_backward call"),
            "algorithmic_bytes": bwd_b,
        },
        "roofline_fwd": {
            "bound": "hbm",
            "achieved": round(fwd_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(fwd_gbps / HBM_PEAK_GBPS, 4),
            "traffic": _traffic(args.preset, "forward"),
            "kernel": "fwd_kernel",
            "algorithmic_bytes": fwd_b,
        },
        "cpu_baseline": None,
    }
    if not args.no_other_presets:
        record["other_presets"] = {
            name: preset_device_times(name, lib)
            for name in OTHER_PRESETS if name != args.preset
        }
        record["fused_front_end"] = fused_front_end_times(lib)
        record["projections"] = projection_times(lib)
    if not args.no_cpu_baseline:
        # The timed steps' results (the last step's; every step computes the
        # same) against the oracle on the same inputs.
        record["cpu_baseline"] = cpu_baseline(
            args.preset, gpu_results=(out, grad_value, grad_loc, grad_attn))
        record["rel_err"] = {k: v["rel_err"]
                             for k, v in record["cpu_baseline"]["gpu_vs_oracle"].items()}
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
