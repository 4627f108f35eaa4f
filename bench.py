#!/usr/bin/env python3
"""STACRLinear save + backward throughput on one MI355X (the north-star layer).

Workload (c_fc layer): GPT-2-medium MLP c_fc as a Transformers Conv1D,
N = 8 x 1024 = 8192 tokens, d_in 1024 -> d_out 4096, bf16, rank 8, residual_budget 0.005,
residual_mode global_topk, int8 residual values.  Synthetic inputs with the configs' generator
(low-rank + noise + 0.1% x20 outliers, per-channel log-normal scale), resident in HBM before
timing.

One step = the two library calls STACRFunction makes for the STAC-R part of a layer-step:
stacr_save_census in forward (coefficients, exact global top-k selection, quantization, and the
entry census it hands to the backward) and stacr_weight_grad_census in backward
(dW = (G^T C) Q^T + G^T R_s).  The layer's other work is the
native nn.Linear / Conv1D arithmetic, unchanged by STAC-R and bit-equal to it (Y = X W^T + b,
grad_input = G W, grad_bias = G.sum(0)); it is not timed, and the time of G.sum(0) is reported
beside the line.  K steps are timed as eager launches and replayed from a HIP graph captured
once (every replay checked against the eager result; a mismatch fails the run); the value is
the faster of the two and both are reported.  Other configured layers (cfg3 c_proj, cfg2 Turbo)
and the basis refresh's Oja step are timed the same way and reported under "other_workloads",
with two whole-layer lines: the drop-in STACRLinear step with its per-step Oja refresh, and
config 4 (2048 <-> 8192, 32768 tokens) through the adaptive engine, and a line for the compact
save outputs (bit-packed index stream, per-row int8 coefficients).  Prints one JSON line.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]
    python bench.py --workload {c_proj,turbo,cfg1,cfg4_up,cfg4_down,oja,cfg4_adaptive_up,cfg4_adaptive_down,
                                drop_in_layer,compact_outputs} [--steps K] [--warmup W]

The second form times one other configured shape alone (cfg1's fp32 nn.Linear, cfg4's 2048 <-> 8192
layers at rank 16 through the projection engine, ...) and prints its own line, for profiling.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "stac-r_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "STACRLinear save+bwd tokens/s (d=1024→4096 bf16) and % of HBM BW roofline"
HBM_PEAK_GBS = 8000.0

# workload (cfg3 c_fc)
N, D_IN, D_OUT, RANK = 8192, 1024, 4096, 8
BUDGET, MODE, CHUNK, BITS = 0.005, "global_topk", 512, 8


def algorithmic_bytes(n, d_in, d_out, rank, k, s_act=2, s_w=2) -> dict:
    """Byte model per layer-step: X, G, C in the activation dtype, U fp32, idx int32, int8 value,
    4 B scale, dW in the weight dtype (save and backward each read the residual entries once)."""
    res = 5 * k + 4 if k else 0
    save = n * d_in * s_act + 4 * d_in * rank + n * rank * s_act + res
    bwd = n * d_out * s_act + n * rank * s_act + res + 4 * d_in * rank + d_out * d_in * s_w
    return {"save": save, "bwd": bwd, "total": save + bwd}


def recorded_traffic(kernel: str):
    """HBM bytes per launch of `kernel` as the committed counter summary records them (rocprofv3
    FETCH_SIZE + WRITE_SIZE, calibrated against a plain copy), or None when none is recorded."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_cfg3_c_fc_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(f"traffic_bytes {kernel}:"):
            return int(line.split(":")[1])
    return None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(x, q, g, budget_s: float = 25.0) -> dict:
    """The reference op sequence as torch CPU library calls (oracle/torch_path.py) on the same
    inputs, on all of this host's cores: 3 warm-up steps, then the median of up to 10."""
    import torch

    from oracle import torch_path

    cores = os.cpu_count() or 1
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    xc, qc, gc = x.cpu(), q.cpu(), g.cpu()

    def one():
        torch_path.layer_step(xc, qc, gc, mode=MODE, budget=BUDGET, chunk_rows=CHUNK, bits=BITS, transposed=True,
                              weight_dtype=torch.bfloat16)

    try:
        for _ in range(3):
            one()
        times, t_start = [], time.perf_counter()
        while len(times) < 10 and time.perf_counter() - t_start < budget_s:
            t0 = time.perf_counter()
            one()
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    per_step = statistics.median(times)
    return {
        "value": N / per_step,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"full c_fc layer-step ({N} tokens, save + dW), median of {len(times)} after 3 warm-up, "
                  f"{per_step * 1e3:.1f} ms/step; torch CPU ops in the reference's order (oracle/torch_path.py)",
        "cpu_model": cpu_model(),
        "torch": torch.__version__,
    }


def time_steps(step, steps: int, warmup: int, check=None):
    """(eager ms, graph ms or None, note) for `steps` calls of `step`; graph replays are checked
    against an eager reference with `check(replay_outputs, eager_outputs)`, which raises."""
    import torch

    ref = step()
    torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / steps
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = step()
    except Exception as exc:  # capture itself unavailable: report eager timing only
        torch.cuda.synchronize()
        return eager_ms, None, f"graph capture unavailable ({exc}); value is eager"
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        fresh = step()  # eager work between replays
        torch.cuda.synchronize()
        if check is not None:
            try:
                check(outs, ref)
            except RuntimeError as exc:  # name the side a fresh eager step agrees with
                agree = [name for name, got in (("the replay", outs), ("the first eager step", ref))
                         if _passes(check, got, fresh)]
                raise RuntimeError(f"{exc}; a later eager step equals {' and '.join(agree) or 'neither'}") from exc
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    return eager_ms, (time.perf_counter() - t0) * 1e3 / steps, None


def _passes(check, outs, ref) -> bool:
    try:
        check(outs, ref)
    except RuntimeError:
        return False
    return True


def _rel(a, b) -> float:
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def check_layer(outs, ref):
    """Every output of a replay equals the eager result bit for bit: the save is deterministic,
    and every timed workload's dW runs on the matrix-core tiles kernels, whose sums have a fixed
    order (a replay reading a stale plan or census would show here)."""
    import torch

    for name, a, b in zip(("coeff", "idx", "data", "scale"), outs[:4], ref[:4]):
        if (a is None) != (b is None) or (a is not None and not torch.equal(a, b)):
            detail = ""
            if a is not None and b is not None and a.shape == b.shape:
                diff = (a != b).reshape(-1)
                first = int(diff.nonzero()[0].item()) if diff.any() else -1
                detail = f": {int(diff.sum().item())} of {diff.numel()} elements, first at {first}"
            raise RuntimeError(f"graph replay of the save differs from the eager result in {name}{detail}")
    if not torch.equal(outs[4], ref[4]):
        raise RuntimeError(f"graph replay of the weight gradient differs from the eager result "
                           f"(rel-L2 {_rel(outs[4], ref[4]):.3g})")


def kernel_breakdown(step, reps: int = 10) -> dict:
    """us per step of each library kernel over `reps` calls of `step` (HIP events on the launch
    stream around every launch, the device kept busy ahead of each)."""
    from stacr_amd import _lib

    with _lib.KernelTimer(max_launches=reps * 64) as timer:
        for _ in range(reps):
            step()
    return {name: round(tot / reps * 1e3, 3) for name, (tot, _cnt) in timer.results.items()}


def layer_workload(name, n, d_in, d_out, rank, budget, mode, steps, warmup, lognormal=True, dtype="bf16",
                   conv1d=True):
    """Timing of one configured layer's save + dW (Conv1D layout unless `conv1d` is False, when dW
    is the nn.Linear d_out x d_in; activations, basis and G in `dtype`, dW in it too)."""
    import torch

    from gpu_cases import make_activation, make_basis, make_grad
    from stacr_amd import kernels

    dev = torch.device("cuda:0")
    tdt = {"bf16": torch.bfloat16, "fp32": torch.float32}[dtype]
    x = make_activation(n, d_in, lognormal=lognormal).to(dev, tdt)
    q = make_basis(d_in, rank).to(dev, tdt)
    g = make_grad(n, d_out).to(dev, tdt)
    k = kernels.residual_plan(n, d_in, mode, budget, CHUNK)[1] if budget > 0 else 0

    def step():
        coeff, idx, data, scale, census = kernels.save_with_census(x, q, mode=mode, budget=budget, chunk_rows=CHUNK,
                                                                   bits=BITS)
        res = (idx, data, scale) if idx is not None else None
        dw, _ = kernels.weight_grad(g, coeff, q, res, BITS, conv1d, tdt, census=census)
        return coeff, idx, data, scale, dw

    eager, graph, note = time_steps(step, steps, warmup, check_layer)
    ms = min(eager, graph) if graph is not None else eager
    s = x.element_size()
    ab = algorithmic_bytes(n, d_in, d_out, rank, k, s_act=s, s_w=s)
    out = {"config": name, "tokens": n, "d_in": d_in, "d_out": d_out, "rank": rank, "k": k, "dtype": dtype,
           "ms_per_step": ms, "tokens_per_s": n / (ms * 1e-3), "eager_ms": eager, "graph_ms": graph,
           "algorithmic_bytes": ab["total"],
           "pct_hbm_roofline": 100.0 * ab["total"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "kernels_us_per_step": kernel_breakdown(step)}
    if note:
        out["note"] = note
    return out


def oja_workload(x, q, steps, warmup):
    """The projection engine's basis refresh (one Oja step per training step by default,
    stacr/layers.py:346-353) on the north-star activation: stacr_oja_step, then the reduced QR."""
    import torch

    from stacr_amd import kernels

    q32 = q.float()

    def step():
        return kernels.oja_step(x, q32, 0.01)

    def check(outs, ref):
        for a, b in zip(outs, ref):
            if not torch.equal(a, b):  # the Oja reductions have a fixed order
                raise RuntimeError("graph replay of the Oja step differs from the eager result")

    eager, graph, note = time_steps(step, steps, warmup, check)
    ms = min(eager, graph) if graph is not None else eager
    byts = N * D_IN * 2 + 2 * 4 * D_IN * RANK  # X once, basis in, update out (one fused pass)
    out = {"config": "oja step on cfg3 c_fc X (8192 x 1024 bf16, rank 8), QR excluded",
           "ms_per_step": ms, "eager_ms": eager, "graph_ms": graph, "algorithmic_bytes": byts,
           "pct_hbm_roofline": 100.0 * byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "kernels_us_per_step": kernel_breakdown(step)}
    if note:
        out["note"] = note
    return out


def adaptive_workload(name, d_in, d_out, steps, warmup):
    """BASELINE config 4 through the adaptive engine: one Pythia-1.4B MLP layer (bf16, 16 x 2048 tokens),
    int8 coefficients and residual values, rank from the sensitivity controller capped at 16, chunk
    top-k 0.005, hybrid refresh every 10 steps (the post-forward Oja step taking Y from the save).
    A step is the layer's whole forward + backward (the dense X W^T and G W products included, as
    the layer runs them), with set_stacr_runtime_state advancing the schedule; eager launches (the
    policy reads the device every step).  Steps cycle through the schedule, so the timed steps
    include their share of refreshes."""
    import torch
    from torch import nn

    from gpu_cases import make_activation, make_grad
    from stacr_amd import _lib, adaptive

    dev = torch.device("cuda:0")
    rows = 16 * 2048
    cfg = adaptive.STACRConfig(rank=16, rank_mode="sensitivity", rank_min=4, rank_max=16, rank_adjust_interval=5,
                               residual_mode="topk", residual_budget=0.005, quantize_coefficients=True,
                               quantize_residuals=True, residual_quantize_bits=8, freeze_basis_after_warmup=True,
                               warmup_steps=0, refresh_trigger="hybrid", refresh_period=10,
                               refresh_energy_threshold=0.1, basis_dtype="bfloat16")
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(d_in, d_out)).to(dev, torch.bfloat16)
    layer = adaptive.apply_adaptive_stacr(model, cfg, surface="all", min_features=1)[0]
    x = make_activation(rows, d_in).to(dev, torch.bfloat16)
    g = make_grad(rows, d_out).to(dev, torch.bfloat16)
    counter = [0]

    def step():
        adaptive.set_stacr_runtime_state(model, counter[0])
        counter[0] += 1
        out = layer(x)
        out.backward(g)
        layer.zero_grad(set_to_none=True)

    for _ in range(max(warmup, 1)):
        step()
    torch.cuda.synchronize()
    refreshes0 = layer.layer_state.get("refresh_count_total", 0)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    refreshes = layer.layer_state.get("refresh_count_total", 0) - refreshes0
    with _lib.KernelTimer(max_launches=64 * 10) as timer:
        for _ in range(10):
            step()
    kern = {n: round(tot / 10 * 1e3, 3) for n, (tot, _c) in timer.results.items()}
    return {"config": name, "tokens": rows, "d_in": d_in, "d_out": d_out, "ms_per_step": ms,
            "tokens_per_s": rows / (ms * 1e-3), "refreshes_in_timed_steps": refreshes,
            "active_rank": layer.layer_state.get("active_rank"),
            "oja_steps_on_the_save_y": layer.layer_state.get("oja_given_y_steps", 0),
            "library_kernels_us_per_step": kern,
            "timing": "eager launches, whole layer step (dense products included)"}


def drop_in_layer_workload(steps, warmup):
    """One training step of the drop-in projection-engine layer as a user runs it: STACRLinear.from_linear
    on the north-star Conv1D shape (1024 -> 4096, bf16, rank 8, global_topk 0.005, int8), default
    update_interval 1, so every step refreshes the basis (Oja step + QR) before the save; forward and
    backward of the layer, dense products included.  Eager launches."""
    import torch

    from gpu_cases import make_activation, make_grad
    from stacr_amd import STACRLinear, _lib

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    lin = torch.nn.Linear(D_IN, D_OUT).to(dev, torch.bfloat16)
    layer = STACRLinear.from_linear(lin, rank=RANK, residual_budget=BUDGET, residual_bits=BITS,
                                    residual_mode=MODE).train()
    x = make_activation(N, D_IN, lognormal=True).to(dev, torch.bfloat16)
    g = make_grad(N, D_OUT).to(dev, torch.bfloat16)
    counter = [0]

    def step():
        layer.set_step(counter[0])
        counter[0] += 1
        y = layer(x)
        y.backward(g)
        lin.weight.grad = None
        lin.bias.grad = None

    for _ in range(max(warmup, 2)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    with _lib.KernelTimer(max_launches=64 * 10) as timer:
        for _ in range(10):
            step()
    kern = {n: round(tot / 10 * 1e3, 3) for n, (tot, _c) in timer.results.items()}
    return {"config": "drop-in STACRLinear step, nn.Linear 1024->4096, N=8192, bf16, r=8, global_topk 0.005, int8, "
                      "Oja refresh every step", "ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3),
            "library_kernels_us_per_step": kern,
            "timing": "eager launches, whole layer step (refresh, dense products included)"}


def compact_outputs_workload(steps, warmup):
    """The north star's compact save outputs on the north-star save's own results (cfg3 c_fc: 41,943
    sorted flat indices, 8192 x 8 bf16 coefficients): the bit-packed index stream (encode, and decode
    back to int32) and the per-row int8 coefficients (quantize, dequantize).  Eager launches; the
    sizes are the stored bytes of each form."""
    import torch

    from gpu_cases import make_activation, make_basis
    from stacr_amd import _lib, kernels
    from stacr_amd.codecs import IndexStream, RowQuantizedCoefficients

    dev = torch.device("cuda:0")
    x = make_activation(N, D_IN, lognormal=True).to(dev, torch.bfloat16)
    q = make_basis(D_IN, RANK).to(dev, torch.bfloat16)
    coeff, idx, _data, _scale = kernels.save(x, q, mode=MODE, budget=BUDGET, chunk_rows=512, bits=BITS)
    stream = IndexStream.encode(idx).check()
    if not torch.equal(stream.decode(idx.dtype), idx):
        raise RuntimeError("compact outputs: the index stream does not decode to the save's indices")

    def encode():
        IndexStream.encode(idx)
        RowQuantizedCoefficients.quantize(coeff)

    rq = RowQuantizedCoefficients.quantize(coeff)

    def decode():
        stream.decode(idx.dtype)
        rq.dequantize()

    out = {"config": "compact save outputs (cfg3 c_fc save: bit-packed index stream, per-row int8 C)"}
    for name, fn in (("encode", encode), ("decode", decode)):
        for _ in range(max(warmup, 2)):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        out[f"{name}_ms"] = (time.perf_counter() - t0) * 1e3 / steps
        with _lib.KernelTimer(max_launches=64 * 10) as timer:
            for _ in range(10):
                fn()
        out[f"{name}_kernels_us"] = {n: round(tot / 10 * 1e3, 3) for n, (tot, _c) in timer.results.items()}
    out.update({"ms_per_step": out["encode_ms"] + out["decode_ms"],
                "index_bytes_int32": int(idx.numel()) * 4, "index_stream_bytes": stream.nbytes(),
                "coeff_bytes_bf16": coeff.numel() * 2, "coeff_int8_bytes": rq.nbytes(),
                "kernels_us_per_step": {**out["encode_kernels_us"], **out["decode_kernels_us"]},
                "timing": "eager launches; encode = stream + row quantizer, decode = their inverses"})
    return out


# The configured layers besides the headline, by name: (description, N, d_in, d_out, rank, budget,
# mode, options).  Each runs through the same save + dW calls; `--workload NAME` times and prints
# one of them alone (a line for profiling, not the contract line).
WORKLOADS = {
    "c_proj": ("cfg3 c_proj: Conv1D 4096->1024, N=8192, bf16, r=8, global_topk 0.005, int8",
               N, 4096, 1024, 8, BUDGET, MODE, {}),
    "turbo": ("cfg2 Turbo: 1280->5120, N=8192, bf16, r=8, no residual",
              N, 1280, 5120, 8, 0.0, "chunk_topk", {"lognormal": False}),
    "cfg1": ("cfg1: nn.Linear 768->3072, N=4096, fp32, r=8, chunk_topk 0.005 (512-row chunks), int8",
             4096, 768, 3072, 8, BUDGET, "chunk_topk", {"lognormal": False, "dtype": "fp32", "conv1d": False}),
    "cfg4_up": ("cfg4 shape: 2048->8192, N=32768, bf16, r=16, chunk_topk 0.005, int8 (projection engine)",
                32768, 2048, 8192, 16, BUDGET, "chunk_topk", {"lognormal": False, "conv1d": False}),
    "cfg4_down": ("cfg4 shape: 8192->2048, N=32768, bf16, r=16, chunk_topk 0.005, int8 (projection engine)",
                  32768, 8192, 2048, 16, BUDGET, "chunk_topk", {"lognormal": False, "conv1d": False}),
}


def run_workload(key, steps, warmup) -> dict:
    name, n, d_in, d_out, rank, budget, mode, opts = WORKLOADS[key]
    return layer_workload(name, n, d_in, d_out, rank, budget, mode, steps, warmup, **opts)


def copy_peak_gbs() -> float:
    """Read + write GB/s of a 1 GiB device-to-device copy on this GPU (a measured stream peak)."""
    import torch

    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    reps = 20
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    gbs = 2 * a.numel() * reps / (time.perf_counter() - t0) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return gbs


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configured workloads")
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["oja", "cfg4_adaptive_up", "cfg4_adaptive_down",
                                                                "drop_in_layer", "compact_outputs"],
                    help="time only this other configured workload and print its line (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2
    if args.workload:
        import torch

        from gpu_cases import make_activation, make_basis

        torch.cuda.set_device(0)
        if args.workload == "oja":
            x = make_activation(N, D_IN, lognormal=True).to("cuda:0", torch.bfloat16)
            w = oja_workload(x, make_basis(D_IN, RANK).to("cuda:0", torch.bfloat16), args.steps, args.warmup)
        elif args.workload.startswith("cfg4_adaptive"):
            up = args.workload.endswith("up")
            w = adaptive_workload("cfg4 adaptive engine, " + ("2048->8192" if up else "8192->2048"),
                                  2048 if up else 8192, 8192 if up else 2048, args.steps, args.warmup)
        elif args.workload == "drop_in_layer":
            w = drop_in_layer_workload(args.steps, args.warmup)
        elif args.workload == "compact_outputs":
            w = compact_outputs_workload(args.steps, args.warmup)
        else:
            w = run_workload(args.workload, args.steps, args.warmup)
        print(json.dumps({"workload": args.workload, **w}), flush=True)
        return 0

    import torch

    from gpu_cases import make_activation, make_basis, make_grad
    from stacr_amd import _lib, kernels

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x = make_activation(N, D_IN, lognormal=True).to(dev, torch.bfloat16)
    q = make_basis(D_IN, RANK).to(dev, torch.bfloat16)
    g = make_grad(N, D_OUT).to(dev, torch.bfloat16)
    k_total, k_saved, _ = kernels.residual_plan(N, D_IN, MODE, BUDGET, CHUNK)

    def step():
        coeff, idx, data, scale, census = kernels.save_with_census(x, q, mode=MODE, budget=BUDGET, chunk_rows=CHUNK,
                                                                   bits=BITS)
        dw, _ = kernels.weight_grad(g, coeff, q, (idx, data, scale), BITS, True, torch.bfloat16, census=census)
        return coeff, idx, data, scale, dw

    print(f"[bench] workload ready: k={k_saved}", file=sys.stderr, flush=True)
    eager_ms, graph_ms, graph_note = time_steps(step, args.steps, args.warmup, check_layer)
    print(f"[bench] eager {eager_ms:.4f} ms/step, graph {graph_ms} ms/step", file=sys.stderr, flush=True)
    use_graph = graph_ms is not None and graph_ms <= eager_ms
    ms = graph_ms if use_graph else eager_ms

    # per-kernel durations (HIP events around each launch on its stream, device kept busy ahead)
    prof_steps = 20
    with _lib.KernelTimer(max_launches=prof_steps * 64) as timer:
        for _ in range(prof_steps):
            step()
    kern = {name: {"avg_us": tot / max(cnt, 1) * 1e3, "per_step_us": tot / prof_steps * 1e3,
                   "launches_per_step": cnt / prof_steps}
            for name, (tot, cnt) in timer.results.items()}
    dominant = max(kern, key=lambda n: kern[n]["per_step_us"])
    ab = algorithmic_bytes(N, D_IN, D_OUT, RANK, k_saved)
    per_kernel_bytes = {"k_tile_grad": ab["bwd"]}
    dom_bytes = per_kernel_bytes.get(dominant)
    avg_s = kern[dominant]["avg_us"] * 1e-6
    achieved = dom_bytes / avg_s / 1e9 if dom_bytes else None
    print("[bench] kernels: " + ", ".join(f"{n}={v['per_step_us']:.1f}us" for n, v in kern.items()),
          file=sys.stderr, flush=True)

    # the layer's native bias gradient (G.sum(0), unchanged from nn.Linear) for reference
    for _ in range(5):
        g.sum(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(50):
        g.sum(0)
    torch.cuda.synchronize()
    bias_us = (time.perf_counter() - t0) * 1e6 / 50

    path_gbs = ab["total"] / (ms * 1e-3) / 1e9
    copy_gbs = copy_peak_gbs()
    out = {
        "metric": METRIC,
        "value": N / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "cfg3 c_fc: STACRLinear save+bwd, Conv1D 1024->4096, N=8192 tokens, bf16, r=8, "
                        "budget 0.005 global_topk, int8 residual",
            "tokens": N, "d_in": D_IN, "d_out": D_OUT, "rank": RANK, "k": k_saved,
            "timing": "hip graph replay" if use_graph else "eager launches",
        },
        "pct_hbm_roofline": 100.0 * path_gbs / HBM_PEAK_GBS,
        "pct_measured_copy_peak": 100.0 * path_gbs / copy_gbs,
        "measured_copy_gbs": copy_gbs,
        "path_algorithmic_bytes": ab["total"],
        "eager_ms_per_step": eager_ms,
        "graph_ms_per_step": graph_ms,
        "native_bias_grad_us": bias_us,
        "roofline": {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS if achieved else None,
            "traffic": recorded_traffic(dominant),
            "algorithmic_bytes_per_launch": dom_bytes,
            "avg_launch_us": kern[dominant]["avg_us"],
        },
        "kernels_us_per_step": {n: round(v["per_step_us"], 3) for n, v in kern.items()},
    }
    if graph_note:
        out["note"] = graph_note
    if not args.no_extra:
        extra_steps, extra_warm = max(10, args.steps // 4), max(3, args.warmup // 4)
        out["other_workloads"] = [run_workload(key, extra_steps, extra_warm) for key in ("c_proj", "turbo")]
        out["other_workloads"].append(oja_workload(x, q, extra_steps, extra_warm))
        out["other_workloads"].append(drop_in_layer_workload(extra_steps, extra_warm))
        out["other_workloads"].append(compact_outputs_workload(extra_steps, extra_warm))
        for up in (True, False):  # config 4 through the adaptive engine (20 steps: two refresh periods)
            out["other_workloads"].append(adaptive_workload(
                "cfg4 adaptive engine, " + ("2048->8192" if up else "8192->2048"), 2048 if up else 8192,
                8192 if up else 2048, 20, 3))
        for w in out["other_workloads"]:
            kern = w.get("kernels_us_per_step", w.get("library_kernels_us_per_step"))
            print(f"[bench] {w['config']}: {w['ms_per_step'] * 1e3:.1f} us {kern}", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(x, q, g)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
