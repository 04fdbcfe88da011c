"""Benchmark: the ApexW 8-bit optimizer step on a Llama-3-8B-shaped parameter set.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config c3|c2|c4|c1|...] [--no-cpu]
    python bench.py --copy-calibration     # 1 GiB device copy, for HBM counter scaling

Prints ONE JSON line (rank 0).  A "step" is one ``ApexW.step()`` over the full
parameter list with synthetic bf16 params ~N(0, 0.02) and grads ~N(0, 1e-3)
already resident in HBM.  ``value`` is parameters updated per second.

``roofline`` prices the fused step kernel against MI355X HBM bandwidth
(8 TB/s): ``achieved`` = algorithmic bytes per launch (read + write of p, g,
moment codes and block scales, computed from the actual state layout) divided
by the average kernel time measured with HIP events on the launch stream.
``traffic`` is the HBM bytes per launch measured with rocprofv3 FETCH_SIZE and
WRITE_SIZE passes (scaled by the same counters on a copy of known size), read
from the committed profile summary of this workload when one exists.
``cpu_baseline`` times the CPU oracle (the reference algorithm restated with
torch CPU ops) on a bounded slice of the same workload on this host's cores.
The default (C3) line also carries ``mfma_roofline``: the C5 hybrid Muon step's
Newton-Schulz GEMMs against the bf16 dense MFMA peak, and ``c4_roofline``: the
C4 compact step over 20,000 ragged tensors with the clip (the whole step, and
its fused step kernel alone), each measured after the earlier tensors are freed.
"""

import argparse
import json
import math
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "optimizer params updated/sec + achieved HBM GB/s (% peak), 8B-param step"


def llama3_8b_shapes():
    s = [(128256, 4096)]
    for _ in range(32):
        s += [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096),
              (4096, 14336), (4096,), (4096,)]
    s += [(4096,), (128256, 4096)]
    return s


def gpt2_small_shapes():
    s = [(50257, 768), (1024, 768)]
    for _ in range(12):
        s += [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,), (768,), (768,),
              (768, 3072), (3072,), (3072, 768), (768,)]
    return s


def ragged_shapes(n=20000, seed=2):
    g = torch.Generator().manual_seed(seed)
    lo, hi = math.log(64), math.log(2 ** 20)
    sizes = torch.exp(torch.rand(n, generator=g, dtype=torch.float64) * (hi - lo) + lo).floor().long().tolist()
    twod = (torch.rand(n, generator=g) < 0.5).tolist()
    shapes = []
    for sz, t in zip(sizes, twod):
        if t and sz >= 64:
            r = 8
            while r * r < sz and sz % (r * 2) == 0:
                r *= 2
            shapes.append((r, sz // r) if sz % r == 0 else (sz,))
        else:
            shapes.append((sz,))
    return shapes


CONFIGS = {
    "c1": dict(workload="C1 compact ApexW step, one fp32 tensor of 2^20", shapes=[(1 << 20,)], dtype=torch.float32,
               kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True)),
    "c2": dict(workload="C2 compact ApexW step, GPT-2-small (124M) bf16", shapes=gpt2_small_shapes(),
               dtype=torch.bfloat16, kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True), per_tensor_scale=True),
    "c3": dict(workload="C3 8-bit ApexW step, Llama-3-8B (8.03B params) bf16, SR on", shapes=llama3_8b_shapes(),
               dtype=torch.bfloat16, kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit")),
    "c3rne": dict(workload="C3 shapes, 8-bit ApexW step with stochastic_rounding=False (the parity mode), bf16",
                  shapes=llama3_8b_shapes(), dtype=torch.bfloat16,
                  kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit",
                              stochastic_rounding=False)),
    "c3fv": dict(workload="C3 shapes, 8-bit ApexW with factored_v=True (INT8 m, fp32 row/column v), bf16, SR on",
                 shapes=llama3_8b_shapes(), dtype=torch.bfloat16, grad_reads=2,
                 kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", factored_v=True)),
    "c3fv6": dict(workload="C3 shapes, 8-bit ApexW with factored_v=True, six_bit=True (6-bit m), bf16, SR on",
                  shapes=llama3_8b_shapes(), dtype=torch.bfloat16, grad_reads=2,
                  kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", factored_v=True,
                              six_bit=True)),
    # the other precision modes on the same shapes
    "c3ultra": dict(workload="C3 shapes, ApexW precision='ultra' (INT8 m blocks, dense bf16 v), bf16, SR on",
                    shapes=llama3_8b_shapes(), dtype=torch.bfloat16,
                    kwargs=dict(lr=1e-3, weight_decay=0.1, precision="ultra")),
    "c2full": dict(workload="C2 shapes, ApexW precision='full' (fp32 m and v), bf16, SR on",
                   shapes=gpt2_small_shapes(), dtype=torch.bfloat16,
                   kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="full"), per_tensor_scale=True),
    "c2auto": dict(workload="C2 shapes, ApexW precision='auto' (bf16 m/v for matrices, fp32 for vectors), bf16, SR on",
                   shapes=gpt2_small_shapes(), dtype=torch.bfloat16,
                   kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="auto"), per_tensor_scale=True),
    # in-backward stepping: a step is opt.zero_grad(), a backward whose graph hands every
    # parameter its synthetic grad (p.view_as(p), no arithmetic), then opt.step(); with
    # hooks the 8-bit kernel runs per batch of 14 layers inside the backward
    "c3hooks": dict(workload="C3 shapes, 8-bit ApexW stepped inside backward (post-accumulate-grad hooks, "
                             "batches of 14), bf16, SR on", shapes=llama3_8b_shapes(), dtype=torch.bfloat16,
                    backward="hooks", kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit")),
    "c3bwd": dict(workload="C3 shapes, 8-bit ApexW, the same backward with the in-backward hooks removed "
                           "(one step after it), bf16, SR on", shapes=llama3_8b_shapes(), dtype=torch.bfloat16,
                  backward="plain", kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit")),
    # grad centralization folded into the 8-bit step: the row means of the dim >= 2 grads are
    # one more read of those grads before the step
    "c3gc": dict(workload="C3 8-bit ApexW step, Llama-3-8B (8.03B params) bf16, SR on, grad_centralization=True",
                 shapes=llama3_8b_shapes(), dtype=torch.bfloat16, row_mean_reads=1,
                 kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit",
                             grad_centralization=True)),
    # the clip's norm pass reads every grad once before the step reads it again (a global
    # norm must be complete before any element is updated): 2 grad reads
    "c4": dict(workload="C4 compact ApexW step, 20k ragged bf16 tensors, clip 1.0", shapes=ragged_shapes(),
               dtype=torch.bfloat16, kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, clip_grad_norm=1.0),
               zero_frac=0.05, grad_reads=2),
    # grad centralization folded into the clip and the step: the row means of the dim >= 2
    # grads are one more read of those grads before the clip and the step
    "c4gc": dict(workload="C4 compact ApexW step, 20k ragged bf16 tensors, clip 1.0, grad_centralization=True",
                 shapes=ragged_shapes(), dtype=torch.bfloat16, grad_reads=2, row_mean_reads=1,
                 kwargs=dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, clip_grad_norm=1.0,
                             grad_centralization=True), zero_frac=0.05),
    "c5": dict(workload="C5 hybrid Muon step (use_muon=True), one Llama-3-8B layer's matrices + 2 RMSNorm, bf16",
               shapes=llama3_8b_shapes()[1:10], dtype=torch.bfloat16,
               kwargs=dict(lr=1e-3, weight_decay=0.1, use_muon=True), mfma=True),
}


def make_params(cfg, device, seed=0):
    g = torch.Generator(device=device).manual_seed(seed)
    params, grads = [], []
    for i, s in enumerate(cfg["shapes"]):
        p = torch.empty(s, dtype=cfg["dtype"], device=device)
        p.normal_(0.0, 0.02, generator=g)
        gr = torch.empty(s, dtype=cfg["dtype"], device=device)
        scale = 1e-3
        if cfg.get("per_tensor_scale"):
            scale *= math.exp((torch.rand((), generator=g, device=device).item() * 2 - 1) * math.log(10.0))
        gr.normal_(0.0, scale, generator=g)
        params.append(torch.nn.Parameter(p))
        grads.append(gr)
    zf = cfg.get("zero_frac", 0.0)
    if zf:
        k = int(len(grads) * zf)
        for i in torch.randperm(len(grads), generator=torch.Generator().manual_seed(seed))[:k].tolist():
            grads[i].zero_()
    for p, gr in zip(params, grads):
        p.grad = gr
    return params


PROFILE_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
# measured HBM bytes per launch: the default line's step kernel (c3) and the C4 step
# kernel of hbm_extra ("c4_step"; the clip's norm pass is not in that figure)
TRAFFIC_FILES = {"c3": "q8_fast_kernel_llama3_8b_traffic.md", "c4_step": "compact_step_kernel_c4_ragged_clip.md"}


def measured_traffic(cfg_name):
    """HBM bytes per launch from the profile summary ('traffic_bytes_per_launch: N'), or None."""
    name = TRAFFIC_FILES.get(cfg_name)
    if not name:
        return None
    try:
        with open(os.path.join(PROFILE_DIR, name)) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip().split()[0])
    except OSError:
        return None
    return None


def copy_calibration():
    """One 1 GiB fp32 device-to-device copy, three times: FETCH_SIZE / WRITE_SIZE of
    this kernel against its known 1 GiB read and 1 GiB write give the counter scale."""
    n = (1 << 30) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read": n * 4, "bytes_written": n * 4, "launches": 3}}), flush=True)


def state_bytes(opt, params, grad_reads=1, grads=None, row_mean_reads=0):
    """Algorithmic HBM bytes of one step: p read+write, g read (twice with a factored
    second moment: its row / column statistics must be complete before any update),
    every state tensor read+write.  grads: the step's grads when p.grad has been
    released (the in-backward steps drop each grad once its batch is stepped).
    row_mean_reads: extra reads of the dim >= 2 grads only (grad centralization's
    row means)."""
    tot = 0
    for i, p in enumerate(params):
        g = p.grad if grads is None else grads[i]
        reads = grad_reads + (row_mean_reads if p.dim() >= 2 else 0)
        tot += 2 * p.numel() * p.element_size() + reads * g.numel() * g.element_size()
        for k, v in opt.state[p].items():
            if torch.is_tensor(v) and k != "step" and v.device.type == "cuda":
                tot += 2 * v.numel() * v.element_size()
    return tot


def ns_roofline(opt, stream, reps=3):
    """MFMA utilisation of the Newton-Schulz GEMMs of one step: the step's
    grouped NS launches are replayed on its own workspaces between HIP events on
    the launch stream.  FLOPs are the algorithmic 4 m^2 n + 2 m^3 per iteration
    per matrix (m <= n), the count of the reference's three matmuls.  The
    kernels compute only the tiles on and above the diagonal of the two
    symmetric products (about 2 m^2 n + m^3 + m^2 n FLOPs); that rate is
    reported as executed_tflops."""
    mu = opt.muon_opt
    plans = list(mu._ns_plans.values())
    steps = int(mu.param_groups[0]["ns_steps"])
    flops = sum(plan.flops for plan in plans)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h = stream.cuda_stream
    for plan in plans:
        plan.run(h)
    ev0.record(stream)
    for _ in range(reps):
        for plan in plans:
            plan.run(h)
    ev1.record(stream)
    torch.cuda.synchronize()
    ns_ms = ev0.elapsed_time(ev1) / reps
    achieved = flops / (ns_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / MFMA_BF16_PEAK_TFLOPS, "traffic": None, "kernel_ms": ns_ms, "flops_per_step": flops,
            "ns_steps": steps, "executed_tflops": sum(plan.exec_flops for plan in plans) / (ns_ms * 1e-3) / 1e12}


def step_kernel_roofline(opt, stream, reps=5):
    """The fused step kernel alone: each group's prepared step launches (the step
    kernel only; the clip's coefficient from the last step stays on the device)
    replayed between HIP events on the launch stream, the step counters restored
    afterwards.  Bytes: p read+write, g read once, the state read+write."""
    import ctypes
    from apexw_amd import _lib as L
    groups = {id(g): g for g in opt.param_groups}
    progs = [(plan, plan.prepare(groups[gid], opt._seed)) for gid, plan in opt._plans.items()]
    h = stream.cuda_stream

    def launch():
        for plan, prog in progs:
            for d_units, n_units, n_fast, n_fast32, hp in prog.launches:
                if plan.kind == "compact":
                    st = plan._lib.apexw_compact_step(plan.d_table.data_ptr(), len(plan.params), d_units.data_ptr(),
                                                      n_units, ctypes.byref(hp), h)
                else:
                    st = plan._lib.apexw_q8_step(plan.d_table.data_ptr(), len(plan.params), d_units.data_ptr(),
                                                 n_units, n_fast, n_fast32, ctypes.byref(hp), h)
                L.check(st, "step kernel replay")
    try:
        launch()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(reps):
            launch()
        ev1.record(stream)
        torch.cuda.synchronize()
    finally:
        for _, prog in progs:
            prog.rollback()
    return ev0.elapsed_time(ev1) / reps


def hbm_extra(cfg_name, steps=10, warmup=3):
    """Another HBM-bound configuration's roofline for the default bench line (C4: the
    compact step over 20,000 ragged tensors with the global-norm clip): the whole
    step (the clip's norm pass reads every grad before the step reads it again),
    then the fused step kernel alone."""
    from apexw_amd import ApexW
    cfg = CONFIGS[cfg_name]
    dev = torch.device("cuda", 0)
    params = make_params(cfg, dev)
    opt = ApexW(params, **cfg["kwargs"])
    for _ in range(warmup):
        opt.step()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        opt.step()
    e1.record(stream)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    step_bytes = state_bytes(opt, params, cfg.get("grad_reads", 1), None, cfg.get("row_mean_reads", 0))
    kern_ms = step_kernel_roofline(opt, stream)
    kern_bytes = state_bytes(opt, params, 1)
    achieved = kern_bytes / (kern_ms * 1e-3) / 1e9
    out = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
           "traffic": measured_traffic(cfg_name + "_step"), "kernel": "compact_step_kernel", "kernel_ms": kern_ms, "bytes_per_launch": kern_bytes,
           "step_ms": step_ms, "step_bytes": step_bytes, "step_gbs": step_bytes / (step_ms * 1e-3) / 1e9,
           "params": sum(p.numel() for p in params), "tensors": len(params), "workload": cfg["workload"]}
    del opt, params
    torch.cuda.empty_cache()
    return out


def cpu_model():
    """The host CPU's model name (first 'model name' line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg_name, budget_s=20.0):
    """Time the CPU oracle on a bounded slice of the workload (whole steps), on every
    core this process may run on."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.optim import OracleApexW
    cfg = CONFIGS[cfg_name]
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    if cfg_name == "c5":
        from oracle.muon import OracleHybrid
        params = make_params(dict(cfg, shapes=[(4096, 4096)]), "cpu")
        opt = OracleHybrid(params, **{k: v for k, v in cfg["kwargs"].items() if k != "use_muon"})
        steps, t0 = 0, time.perf_counter()
        while True:
            opt.step()
            steps += 1
            el = time.perf_counter() - t0
            if el > budget_s or steps >= 20:
                break
        return {"value": params[0].numel() * steps / el, "unit": "params/s", "cores": threads, "kind": "port",
                "cpu_model": cpu_model(),
                "sample": f"the q matrix (4096x4096) of the layer; {steps} Muon steps, fp32 Newton-Schulz "
                          f"(the reference's CPU work dtype); CPU oracle (torch CPU ops)"}
    if cfg_name in ("c3", "c3rne", "c3fv", "c3fv6"):
        shapes = llama3_8b_shapes()[1:10]          # one transformer layer (218M params)
        sample = "one Llama-3-8B layer (q,k,v,o,gate,up,down + 2 RMSNorm, 218.1M params)"
    elif cfg_name == "c4":
        shapes = ragged_shapes()[:500]
        sample = "first 500 of the 20k ragged tensors"
    else:
        shapes = cfg["shapes"]
        sample = "full parameter list"
    sub = dict(cfg, shapes=shapes)
    params = make_params(sub, "cpu")
    n = sum(p.numel() for p in params)
    opt = OracleApexW(params, **cfg["kwargs"])
    opt.step()  # cold step (state allocation)
    steps, t0 = 0, time.perf_counter()
    while True:
        opt.step()
        steps += 1
        el = time.perf_counter() - t0
        if el > budget_s or steps >= 50:
            break
    return {"value": n * steps / el, "unit": "params/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{sample}; {steps} steps after 1 cold step; CPU oracle (torch CPU ops)"}


def mfma_extra(steps=10, warmup=3):
    """The C5 Newton-Schulz roofline, for the default bench line: the hybrid Muon step on
    one Llama-3-8B layer, then the step's grouped NS launches replayed between HIP events."""
    from apexw_amd import ApexW
    cfg = CONFIGS["c5"]
    dev = torch.device("cuda", 0)
    params = make_params(cfg, dev)
    opt = ApexW(params, **cfg["kwargs"])
    for _ in range(warmup):
        opt.step()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        opt.step()
    e1.record(stream)
    torch.cuda.synchronize()
    roof = ns_roofline(opt, stream)
    roof["step_ms"] = e0.elapsed_time(e1) / steps
    roof["workload"] = cfg["workload"]
    del opt, params
    torch.cuda.empty_cache()
    return roof


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--copy-calibration", action="store_true", help="run the counter-calibration copy and exit")
    ap.add_argument("--no-mfma", action="store_true", help="skip the C5 Newton-Schulz roofline of the default line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the optimizer step is data-parallel per shard and this build "
              "has no multi-GPU path; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from apexw_amd import ApexW

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    params = make_params(cfg, dev)
    n = sum(p.numel() for p in params)
    opt = ApexW(params, **cfg["kwargs"])
    step = opt.step
    if cfg.get("backward"):
        grads = [p.grad for p in params]
        for p in params:
            p.grad = None
        if cfg["backward"] == "plain":
            opt._disable_auto_8bit_hooks()

        def step():
            opt.zero_grad(set_to_none=True)
            torch.autograd.backward([p.view_as(p) for p in params], grad_tensors=grads)
            opt.step()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    nbytes = 0 if cfg.get("mfma") else state_bytes(opt, params, cfg.get("grad_reads", 1),
                                                    grads if cfg.get("backward") else None,
                                                    cfg.get("row_mean_reads", 0))
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    host = 0.0
    for _ in range(args.steps):
        h0 = time.perf_counter()
        step()
        host += time.perf_counter() - h0
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1) / args.steps
    ms = wall * 1e3 / args.steps
    achieved = nbytes / (gpu_ms * 1e-3) / 1e9
    if cfg.get("mfma"):
        roofline = ns_roofline(opt, stream)
        roofline["step_ms"] = gpu_ms
    else:
        roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": achieved / HBM_PEAK_GBS, "traffic": measured_traffic(args.config),
                    "kernel_ms": gpu_ms, "bytes_per_launch": nbytes, "bytes_per_param": nbytes / n}
    out = {
        "metric": METRIC, "value": n / (ms * 1e-3), "unit": "params/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "host_ms_per_step": host * 1e3 / args.steps,
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16" if cfg.get("mfma") else "f32", "data": "synthetic",
        "config": {"workload": cfg["workload"], "params": n, "tensors": len(params),
                   "param_dtype": str(cfg["dtype"]).replace("torch.", ""), **{k: v for k, v in cfg["kwargs"].items()}},
        "roofline": roofline,
    }
    if args.config == "c3" and not args.no_mfma:
        # the Muon half of the metric, measured after the C3 tensors are freed
        del step, opt, params
        torch.cuda.empty_cache()
        out["mfma_roofline"] = mfma_extra()
        out["c4_roofline"] = hbm_extra("c4")
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.config, args.cpu_budget)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
