"""Benchmark: fused 2D-RoPE attention fwd+bwd on one MI355X.

Workload (BASELINE metric): ViT-B/16 attention, B=256, H=12, H_img=14 + CLS
(N=197), D=64, bf16, RoPE base 100; q/k/v/dO ~ N(0,1) synthetic.  One step
= forward + backward through the public API (``sdpa_triton_fa_rope`` then
``o.backward(dO)``) with inputs already resident in HBM.

Prints one JSON line (the driver's contract) carrying:
  value          fwd+bwd TFLOP/s (algorithmic 14*B*H*N^2*D per step / wall time)
  roofline       dominant kernel (the backward kernel): algorithmic bytes per
                 launch / its average duration from HIP events on the launch
                 stream, vs 8 TB/s; `traffic` = measured HBM bytes per launch
                 from the committed rocprofv3 counter summary, if present
  cpu_baseline   the PyTorch oracle (Python RoPE + torch SDPA, fp32) on the
                 host CPU at BASELINE.json configs[0] (B=2 H=8 N=197 D=64,
                 loss o.sum()); `workload_slice` adds the same oracle on a
                 bounded slice of the bench workload
  torch_rocm     the same oracle on the GPU in bf16 (torch-ROCm SDPA + RoPE)

The GPU leaves its idle clocks only after some tens of milliseconds of
sustained load (about 30 ms here), so every timed loop is preceded by
PREWARM_S seconds of untimed steps before the `--warmup` steps; without it a
default run would be timed mostly on the clock ramp.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd TFLOP/s at ViT-B/16 (B256 H12 N197 D64 bf16); % of bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")
PREWARM_S = 0.3             # untimed sustained load before each timed loop

WORKLOADS = {
    "vit_b": dict(B=256, H=12, side=14, has_cls=True, D=64, name="vit_b16_attention_fwd_bwd", metric=METRIC),
    "vit_s": dict(B=512, H=6, side=14, has_cls=True, D=64, name="vit_s16_attention_fwd_bwd",
                  metric="fwd+bwd TFLOP/s at ViT-S/16 (B512 H6 N197 D64 bf16); % of bf16 MFMA peak"),
    "vit_l": dict(B=128, H=16, side=16, has_cls=False, D=64, name="vit_l16_256_attention_fwd_bwd",
                  metric="fwd+bwd TFLOP/s at ViT-L/16-256 (B128 H16 N256 D64 bf16, no CLS); % of bf16 MFMA peak"),
    "hires": dict(B=32, H=12, side=32, has_cls=True, D=128, name="hires_n1025_d128_attention_fwd_bwd",
                  metric="fwd+bwd TFLOP/s at high-res ViT (B32 H12 N1025 D128 bf16); % of bf16 MFMA peak"),
}


def prewarm(fn, seconds=PREWARM_S, max_calls=20000):
    """Call ``fn()`` untimed until ``seconds`` of wall time have passed (clock ramp)."""
    import torch

    fn()   # the first call carries one-time set-up (library and code-object loads)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 1
    while n < max_calls:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            break
    return n


def flops(B, H, N, D):
    f = 4.0 * B * H * N * N * D
    return f, 2.5 * f, 3.5 * f   # fwd, bwd (5 GEMMs), fwd+bwd


def hbm_bytes(B, H, N, D, e=2):
    fwd = 4.0 * B * H * N * D * e + 4.0 * B * H * N
    bwd = 8.0 * B * H * N * D * e + 4.0 * B * H * N
    return fwd, bwd


def roofline_time(B, H, N, D):
    ff, fb, _ = flops(B, H, N, D)
    bf, bb = hbm_bytes(B, H, N, D)
    tf = max(ff / (PEAK_BF16_TFLOPS * 1e12), bf / (PEAK_HBM_GBS * 1e9))
    tb = max(fb / (PEAK_BF16_TFLOPS * 1e12), bb / (PEAK_HBM_GBS * 1e9))
    return tf, tb


def make_inputs(wl, device, seed=0, dtype=None):
    import torch

    dtype = dtype or torch.bfloat16
    N = wl["side"] ** 2 + int(wl["has_cls"])
    shape = (wl["B"], wl["H"], N, wl["D"])
    g = torch.Generator().manual_seed(seed)
    ts = [torch.randn(shape, generator=g) for _ in range(4)]
    return [t.to(dtype).to(device) for t in ts]


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _cpu_threads() -> int:
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    return cores


def time_cpu_config0(budget_s=8.0):
    """BASELINE.json configs[0], the reference's CPU-runnable case: Python 2D
    RoPE + torch SDPA (math), fp32, B=2, H=8, H_img=14 + CLS (N=197), D=64,
    q/k/v ~ N(0,1) drawn in that order from seed 0, CosSinTable base 100,
    loss = o.sum() so dO = ones.  Forward and backward are timed separately
    (time.perf_counter), 3 warm-ups, then the median over at least 10 runs
    and about `budget_s` seconds."""
    import torch
    from oracle import torch_ref
    from triton_fused_rope_flash_attn_amd import build_axial_rope_pairs

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    B, H, side, D = 2, 8, 14, 64
    N = side * side + 1
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, H, N, D, generator=g) for _ in range(3))
    cosp, sinp = build_axial_rope_pairs(side, D, torch.device("cpu"), base=100.0)

    def once():
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        t0 = time.perf_counter()
        o = torch_ref.attention(qq, kk, vv, cosp, sinp, True)
        t1 = time.perf_counter()
        o.sum().backward()
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    for _ in range(3):
        once()
    tf, tb = [], []
    t_start = time.perf_counter()
    while len(tf) < 10 or time.perf_counter() - t_start < budget_s:
        a, b = once()
        tf.append(a)
        tb.append(b)
    mf, mb = statistics.median(tf), statistics.median(tb)
    f_fwd, f_bwd, _ = flops(B, H, N, D)
    return {
        "value": (f_fwd + f_bwd) / (mf + mb) / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"BASELINE configs[0]: oracle (Python 2D RoPE + torch SDPA math, fp32, autograd), B={B} H={H} "
            f"N={N} D={D}, q/k/v ~ N(0,1) seed 0, base 100, loss o.sum() (dO = ones); median of {len(tf)} "
            f"runs ({time.perf_counter() - t_start:.1f} s): fwd {mf * 1e3:.2f} ms, bwd {mb * 1e3:.2f} ms; "
            f"{cores} threads; CPU: {_cpu_model()}"
        ),
        "fwd_ms": round(mf * 1e3, 3),
        "bwd_ms": round(mb * 1e3, 3),
    }


def time_cpu_baseline(wl, budget_s=6.0):
    """Oracle fwd+bwd in fp32 on the host over a slice of the bench workload's
    batch (the like-for-like TFLOP/s at the GPU's shape and dO ~ N(0,1)).

    Runs whole fwd+bwd iterations until `budget_s` seconds of CPU work have
    been timed (at least 3), with the thread count capped at the process's
    share of the host (OMP_NUM_THREADS, else the affinity mask)."""
    import torch
    from oracle import torch_ref
    from triton_fused_rope_flash_attn_amd import build_axial_rope_pairs

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    sub = dict(wl, B=4 if wl["D"] == 64 else 1)
    q, k, v, do = make_inputs(sub, "cpu", dtype=torch.float32)
    cosp, sinp = build_axial_rope_pairs(wl["side"], wl["D"], torch.device("cpu"), base=100.0)
    B, H, N, D = q.shape
    times = []
    torch_ref.forward_backward(q, k, v, do, cosp, sinp, wl["has_cls"])  # warm-up
    t_start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        torch_ref.forward_backward(q, k, v, do, cosp, sinp, wl["has_cls"])
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    _, _, fall = flops(B, H, N, D)
    return {
        "value": fall / med / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"oracle (Python 2D RoPE + torch SDPA math, fp32, autograd) fwd+bwd on B={B} of "
            f"{wl['B']} (planes {B * H} of {wl['B'] * H}), N={N}, D={D}, dO ~ N(0,1); median of "
            f"{len(times)} iterations ({sum(times):.1f} s timed), {med * 1e3:.1f} ms each; {cores} "
            f"threads; CPU: {_cpu_model()}"
        ),
    }


def torch_rope(x, cosp, sinp, has_cls):
    """2D RoPE applied in plain torch ops, as the reference README's comparison
    model does (README:125): channel pairs (2p, 2p+1) of token s rotate by
    table row max(s - has_cls, 0), and a CLS token passes through.  This is
    the torch-ROCm comparison's own RoPE, in the input dtype."""
    import torch
    N = x.shape[-2]
    c, s = cosp.to(dtype=x.dtype), sinp.to(dtype=x.dtype)
    if has_cls:   # an identity row (cos 1, sin 0) leaves the CLS token unchanged, exactly
        c = torch.cat([torch.ones_like(c[:1]), c])
        s = torch.cat([torch.zeros_like(s[:1]), s])
    c, s = c[:N], s[:N]
    xe, xo = x[..., 0::2], x[..., 1::2]
    return torch.stack([xe * c - xo * s, xo * c + xe * s], dim=-1).flatten(-2)


def time_torch_rocm(wl, steps, warmup):
    """Python 2D RoPE (bf16) + torch SDPA (flash/efficient backend) fwd+bwd on the GPU."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from triton_fused_rope_flash_attn_amd import CosSinTable

    q, k, v, do = make_inputs(wl, "cuda")
    table = CosSinTable(100.0, wl["side"], wl["D"], device="cuda")
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))

    def step():
        qh = torch_rope(qq, table.COSP, table.SINP, wl["has_cls"])
        kh = torch_rope(kk, table.COSP, table.SINP, wl["has_cls"])
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(qh, kh, vv)
        o.backward(do)

    prewarm(step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    B, H, N, D = q.shape
    _, _, fall = flops(B, H, N, D)
    return {"value": fall / dt / 1e12, "unit": "TFLOP/s", "ms_per_step": dt * 1e3,
            "what": "Python 2D RoPE (bf16) + F.scaled_dot_product_attention (flash/efficient), fwd+bwd"}


def time_block(wl, steps, warmup, compiled=False):
    """ViT attention sub-layer (qkv Linear -> op -> proj), fwd+bwd, bf16:
    ``RoPEAttention`` with the fused op vs the same layer and weights with
    Python RoPE + torch SDPA (flash/efficient) in its place.  ``compiled``:
    both layers under ``torch.compile`` (Inductor), the setting of the
    reference README's compiled comparison (README:165-195); the fused op stays
    one opaque custom op inside the compiled graph."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from triton_fused_rope_flash_attn_amd import RoPEAttention

    def torch_attn(q, k, v, table, H_img=None, has_cls=True):
        cosp, sinp = table.tables()
        qh = torch_rope(q, cosp, sinp, has_cls)
        kh = torch_rope(k, cosp, sinp, has_cls)
        if compiled:
            # Inductor's stride check on torch's flash-attention backward
            # rejects the strided V view of the qkv buffer; a copy avoids it
            v = v.contiguous()
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(qh, kh, v)

    B, H, D, side, has_cls = wl["B"], wl["H"], wl["D"], wl["side"], wl["has_cls"]
    N, C = side * side + int(has_cls), wl["H"] * wl["D"]
    torch.manual_seed(0)
    ours = RoPEAttention(C, H, H_img=side, has_cls=has_cls, device="cuda", dtype=torch.bfloat16)
    ref = RoPEAttention(C, H, H_img=side, has_cls=has_cls, attn=torch_attn, device="cuda",
                        dtype=torch.bfloat16)
    ref.load_state_dict(ours.state_dict())
    x = torch.randn(B, N, C, device="cuda", dtype=torch.bfloat16).requires_grad_(True)
    dy = torch.randn(B, N, C, device="cuda", dtype=torch.bfloat16)
    res = {}
    for name, blk in (("ours", ours), ("torch", ref)):
        fwd = torch.compile(blk) if compiled else blk
        if compiled:
            print(f"bench.py: compiling the {name} layer (Inductor)", file=sys.stderr, flush=True)

        def step():
            x.grad = None
            blk.zero_grad(set_to_none=True)
            fwd(x).backward(dy)

        prewarm(step)
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        res[name] = (time.perf_counter() - t0) / steps * 1e3
    return {"what": f"ViT attention sub-layer fwd+bwd, {'torch.compile (Inductor)' if compiled else 'eager'}, "
                    f"bf16: x [{B},{N},{C}] -> qkv Linear -> "
                    f"{H}-head 2D-RoPE attention -> proj; ours = RoPEAttention, torch = same layer with "
                    "Python RoPE + torch SDPA (flash/efficient)",
            "ours_ms": round(res["ours"], 4), "torch_ms": round(res["torch"], 4),
            "speedup": round(res["torch"] / res["ours"], 3)}


def profile_run(wl, steps, warmup):
    """Kernel launches only: `warmup + steps` x (fwd, bwd) and one calibration copy."""
    import torch
    from triton_fused_rope_flash_attn_amd import CosSinTable
    from triton_fused_rope_flash_attn_amd import _lib

    q, k, v, do = make_inputs(wl, "cuda")
    B, H, N, D = q.shape
    table = CosSinTable(100.0, wl["side"], wl["D"], device="cuda")
    rope = table.packed()
    scale = 1.0 / math.sqrt(D)
    n_pos = N - int(wl["has_cls"])
    # clock ramp on a plain GEMM, so that the traced farope launches are all
    # at steady-state clocks
    a = torch.randn(4096, 4096, dtype=torch.bfloat16, device="cuda")
    b = torch.randn(4096, 4096, dtype=torch.bfloat16, device="cuda")
    prewarm(lambda: torch.mm(a, b))
    del a, b
    for _ in range(warmup + steps):
        o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, n_pos, wl["has_cls"], scale, _lib.BF16)
        torch.ops.farope.attn_bwd(do, q, k, v, o, lse, rope, n_pos, wl["has_cls"], scale, _lib.BF16, res)
    # calibration: a plain copy reads and writes exactly 256 MiB each
    src = torch.empty(128 * 1024 * 1024, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    fb, bb = hbm_bytes(B, H, N, D)
    print(json.dumps({"profile": wl["name"], "launches": warmup + steps, "fwd_alg_bytes": fb,
                      "bwd_alg_bytes": bb, "calib_copy_bytes": 2 * src.numel() * 2}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="vit_b", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch-baseline", action="store_true")
    ap.add_argument("--block", action="store_true",
                    help="also time the ViT attention sub-layer (qkv Linear -> op -> proj) against the "
                         "same layer with torch SDPA + Python RoPE (reported as `vit_block`)")
    ap.add_argument("--compile", action="store_true",
                    help="with --block: also time both layers under torch.compile (Inductor), reported as "
                         "`vit_block_compiled`")
    ap.add_argument("--profile", action="store_true",
                    help="profiling mode for rocprofv3: only the fwd/bwd ops (warmup + steps) and one "
                         "256 MiB device-to-device copy used to calibrate the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this op runs on one GPU (each (b, h) "
            "plane is independent; a multi-GPU run would only split the batch). Use --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch
    from triton_fused_rope_flash_attn_amd import CosSinTable, sdpa_triton_fa_rope
    from triton_fused_rope_flash_attn_amd import _lib

    wl = WORKLOADS[args.workload]
    dev = "cuda"
    if args.profile:
        profile_run(wl, args.steps, args.warmup)
        return
    q, k, v, do = make_inputs(wl, dev)
    B, H, N, D = q.shape
    table = CosSinTable(100.0, wl["side"], wl["D"], device=dev)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))

    def step():
        # gradients are consumed, not accumulated, as after zero_grad(set_to_none=True)
        qq.grad = kk.grad = vv.grad = None
        o = sdpa_triton_fa_rope(qq, kk, vv, table, has_cls=wl["has_cls"])
        o.backward(do)

    prewarm(step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps

    # Per-kernel durations: HIP events on the stream the kernels are launched on.
    stream = torch.cuda.current_stream()
    rope = table.packed()
    scale = 1.0 / math.sqrt(D)
    n_pos = N - int(wl["has_cls"])
    o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, n_pos, wl["has_cls"], scale, _lib.BF16)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for _ in range(3):
        torch.ops.farope.attn_bwd(do, q, k, v, o, lse, rope, n_pos, wl["has_cls"], scale, _lib.BF16, res)
    for a, b, c in ev:
        a.record(stream)
        o, lse, res = torch.ops.farope.attn_fwd(q, k, v, rope, n_pos, wl["has_cls"], scale, _lib.BF16)
        b.record(stream)
        torch.ops.farope.attn_bwd(do, q, k, v, o, lse, rope, n_pos, wl["has_cls"], scale, _lib.BF16, res)
        c.record(stream)
    torch.cuda.synchronize()
    t_fwd = statistics.mean(a.elapsed_time(b) for a, b, c in ev) * 1e-3
    t_bwd = statistics.mean(b.elapsed_time(c) for a, b, c in ev) * 1e-3

    f_fwd, f_bwd, f_all = flops(B, H, N, D)
    by_fwd, by_bwd = hbm_bytes(B, H, N, D)
    tf_star, tb_star = roofline_time(B, H, N, D)
    desc = _lib.make_desc(B, H, N, D, n_pos, wl["has_cls"], _lib.BF16, _lib.BF16, scale)
    bwd_cfg = _lib.tile_config(desc, 1)
    fwd_cfg = _lib.tile_config(desc, 0)
    bwd_kernel = {0: "bwd_plane_kernel", 1: "bwd_dq_kernel + bwd_dkdv_kernel",
                  2: "bwd_dq_kernel + bwd_keys_kernel",
                  3: "bwd_ds_prep_kernel + bwd_keys_kernel + bwd_ds_dq_kernel"}[bwd_cfg[0]]

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        try:
            with open(TRAFFIC_FILE) as fh:
                tr = json.load(fh)
            traffic = tr.get(args.workload, {}).get("bwd_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    value = f_all / dt / 1e12
    achieved_gbs = by_bwd / t_bwd / 1e9
    result = {
        "metric": wl["metric"],   # the BASELINE metric for the default (headline) workload
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_s": PREWARM_S,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q, k, v, dO ~ N(0,1), seed 0)",
        "config": {
            "workload": wl["name"], "B": B, "H": H, "N": N, "D": D, "H_img": wl["side"],
            "has_cls": wl["has_cls"], "rope_base": 100.0, "parallelism": "none (1 GPU)",
        },
        "pct_mfma_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline_fraction_fwd_bwd": round((tf_star + tb_star) / dt, 4),
        "fwd": {"kernel": {0: "fwd_kernel", 1: "fwd_plane_kernel"}[fwd_cfg[0]],
                "ms": round(t_fwd * 1e3, 4), "tflops": round(f_fwd / t_fwd / 1e12, 2),
                "gbs": round(by_fwd / t_fwd / 1e9, 1), "roofline_fraction": round(tf_star / t_fwd, 4),
                "tile": fwd_cfg},
        "bwd": {"ms": round(t_bwd * 1e3, 4), "tflops": round(f_bwd / t_bwd / 1e12, 2),
                "gbs": round(achieved_gbs, 1), "roofline_fraction": round(tb_star / t_bwd, 4),
                "tile": bwd_cfg},
        "roofline": {
            "kernel": bwd_kernel,
            "bound": "hbm" if f_bwd / by_bwd < PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9) else "mfma",
            "achieved": round(achieved_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
        },
    }
    if result["roofline"]["bound"] == "mfma":
        ach = f_bwd / t_bwd / 1e12
        result["roofline"].update(achieved=round(ach, 1), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                                  frac=round(ach / PEAK_BF16_TFLOPS, 4))
    if not args.no_torch_baseline:
        try:
            result["torch_rocm"] = time_torch_rocm(wl, max(5, args.steps // 5), 3)
        except Exception as exc:  # reported, never fatal for the bench line
            result["torch_rocm"] = {"error": repr(exc)[:200]}
    if args.block:
        result["vit_block"] = time_block(wl, max(10, args.steps // 4), 3)
        if args.compile:
            result["vit_block_compiled"] = time_block(wl, max(10, args.steps // 4), 3, compiled=True)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = time_cpu_config0()
        result["cpu_baseline"]["workload_slice"] = time_cpu_baseline(wl)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
