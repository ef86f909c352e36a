"""Benchmark of the MI355X multi-LoRA linear (forward + backward).

One step = forward + backward of the six LoRA linears of one Wan-1.3B DiT
block (q, k, v, o: 1536->1536; ffn.0: 1536->8960; ffn.2: 8960->1536) over
65520 tokens = two roles (generator, fake critic) of 32760 tokens, each with
its own rank-64 adapter on the shared frozen bf16 base,
through the drop-in autograd op with inputs resident in HBM.

Prints one JSON line: metric/value (TFLOP/s of the whole step), the roofline
of the dominant kernel measured with HIP events, the LoRA kernels' HBM GB/s,
and a CPU baseline (the reference per-adapter path in fp32 torch on host
cores, timed on a bounded sample of the same workload).

Other configurations (parity-test cases, measured on request): --config
tiny | wan22_5b | flux | wan13b_fp8 (frozen base stored e4m3 with a per-output-
channel scale: forward on the e4m3 MFMA) | wan13b_roles (the multi-role call site:
teacher conditional + unconditional rows base-only and the fake critic's rows with its
adapter, in one call), --fwd-only for a forward-only step, --per-role to time the
same step as one call per role (this library, and the reference's unfused torch path),
--shared-qkv to feed q, k, v one input and run them as one stacked call (the step
with three separate calls on that input is timed beside it), and --gated-residual to end o
and ffn.2 in the block's gated residual x + y·gate fused into the GEMM epilogue (the step
with the residual as torch ops after the linear is timed beside it).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config wan13b] [--fwd-only] [--per-role] [--shared-qkv] [--gated-residual]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16
MFMA_FP8_PEAK_TFLOPS = 5000.0   # dense fp8


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="wan13b")
    p.add_argument("--fwd-only", action="store_true", help="time forward passes only (no autograd)")
    p.add_argument("--kernel-reps", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bounded CPU-baseline sample budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--shared-qkv", action="store_true",
                   help="q, k, v read one input (as in a DiT block) and run as one stacked call; the same "
                        "step with three separate calls is timed beside it")
    p.add_argument("--gated-residual", action="store_true",
                   help="o and ffn.2 close their branch with the block's gated residual x + y*gate fused into "
                        "the GEMM epilogue; the same step with the residual as torch ops after the linear is "
                        "timed beside it")
    p.add_argument("--per-role", action="store_true",
                   help="also time the same step as one call per segment (role), with this library and with "
                        "the reference's unfused torch path on the GPU")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device copy 4 times (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


TRAFFIC_FILE = ROOT / "profiles" / "gemm_fwd_wan13b_traffic.md"


def recorded_traffic():
    """HBM bytes per launch of the fused forward GEMM, as measured by the rocprofv3
    FETCH_SIZE / WRITE_SIZE passes summarised in profiles/ (None if absent)."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def copy_calibration():
    import torch
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 4}), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the multi-LoRA linear is benchmarked "
                                   "at N=1 (multi-GPU sharding is a design note, not a launched path); "
                                   f"--gpus {args.gpus} / WORLD_SIZE {world} is not supported"}), flush=True)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        copy_calibration()
        return
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    pkg.load_library()
    from dmd_system_amd import kernels, workloads

    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a ROCm GPU")
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    cfg = workloads.CONFIGS[args.config]
    routing = cfg.routing
    scales = [cfg.scale] * len(cfg.ranks)

    fp8 = cfg.base_fp8
    # ---------------- inputs (resident in HBM); an e4m3 base is stored quantised
    lins = []
    for i, (name, K, N) in enumerate(cfg.linears()):
        x, w, b, As, Bs, dy = workloads.make_linear(cfg, K, N, dev, seed=cfg.seed * 100 + i)
        x.requires_grad_(not args.fwd_only)
        for t in As + Bs:
            t.requires_grad_(not args.fwd_only)
        L = dict(name=name, K=K, N=N, x=x, w=w, b=b, As=As, Bs=Bs, dy=dy)
        L["wt"] = w.t().contiguous()  # the frozen base transposed once, for the NT form of dX
        if fp8:
            L["wq"], L["ws"] = kernels.quantize_rows_fp8(w)
            L["wqt"] = L["wq"].t().contiguous()  # the frozen e4m3 base transposed, for the e4m3 dX
        lins.append(L)
    torch.cuda.synchronize()

    if args.shared_qkv:
        if fp8:
            raise SystemExit("--shared-qkv stacks bf16 bases only")
        qkv = lins[:3]
        for L in qkv[1:]:
            L["x"] = qkv[0]["x"]  # one input, as the block's q / k / v read the normed hidden states

    def stacked_step(fwd_only):
        outs = pkg.shared_input_multi_lora(qkv[0]["x"], [L["w"] for L in qkv], [L["b"] for L in qkv],
                                           [L["As"] for L in qkv], [L["Bs"] for L in qkv], scales, routing)
        if not fwd_only:
            torch.autograd.backward(list(outs), [L["dy"] for L in qkv])

    if args.gated_residual:
        if fp8:
            raise SystemExit("--gated-residual fuses into the bf16 GEMM only")
        gen = torch.Generator(device=dev)
        gen.manual_seed(99)
        for L in lins:
            if L["name"] in ("o", "ffn.2"):
                L["res"] = torch.randn(cfg.tokens, L["N"], generator=gen, device=dev).to(torch.bfloat16)
                L["res"].requires_grad_(not args.fwd_only)
                # one gate row per role segment, as Wan's per-sample e[2] / e[5]
                L["gate"] = torch.rand(len(cfg.seg_lengths), L["N"], generator=gen, device=dev) + 0.5
        if len(set(cfg.seg_lengths)) != 1:
            raise SystemExit("--gated-residual needs equal segment lengths (one gate row per segment)")

    def unfused_gated(L):
        y = pkg.multi_lora_linear(L["x"], L["w"], L["b"], L["As"], L["Bs"], scales, routing, weight_t=L["wt"])
        g = L["gate"].repeat_interleave(cfg.tokens // L["gate"].shape[0], dim=0)
        return (L["res"].float() + y.float() * g).to(torch.bfloat16)

    def forward(L, fuse=True):
        if "gate" in L:
            if fuse:
                return pkg.multi_lora_linear_gated(L["x"], L["w"], L["b"], L["As"], L["Bs"], scales, routing,
                                                   L["res"], L["gate"], weight_t=L["wt"])
            return unfused_gated(L)
        if fp8:
            return pkg.multi_lora_linear_fp8(L["x"], L["wq"], L["ws"], L["b"], L["As"], L["Bs"], scales, routing,
                                             wq_t=L["wqt"])
        return pkg.multi_lora_linear(L["x"], L["w"], L["b"], L["As"], L["Bs"], scales, routing, weight_t=L["wt"])

    def step(stack=args.shared_qkv, fuse=True):
        rest = lins[3:] if stack else lins
        if args.fwd_only:
            with torch.no_grad():
                if stack:
                    stacked_step(True)
                for L in rest:
                    forward(L, fuse)
            return
        for L in lins:
            for t in [L["x"], *L["As"], *L["Bs"]] + ([L["res"]] if "res" in L else []):
                t.grad = None
        if stack:
            stacked_step(False)
        for L in rest:
            forward(L, fuse).backward(L["dy"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps
    flops_fn = cfg.flops_fwd if args.fwd_only else cfg.flops_fwd_bwd
    flops_step = sum(flops_fn(L["K"], L["N"]) for L in lins)
    tflops = flops_step / (ms_per_step * 1e-3) / 1e12
    print(f"# step {ms_per_step:.3f} ms, {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)
    def timed_variant(**kw):
        for _ in range(args.warmup):
            step(**kw)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step(**kw)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
        return {"ms_per_step": round(ms, 4), "tflops": round(flops_step / (ms * 1e-3) / 1e12, 2)}

    # the same step, q / k / v as three calls on their one input
    unstacked = timed_variant(stack=False) if args.shared_qkv else None
    # the same step, the gated residual as torch ops after the linear
    unfused = timed_variant(fuse=False) if args.gated_residual else None

    # ---------------- per-kernel timing with HIP events on the launch stream
    reps = args.kernel_reps
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3  # seconds per launch

    from dmd_system_amd.function import _as_operand
    seg = list(zip(cfg.seg_lengths, cfg.seg_adapters))
    R = kernels.padded_rank(cfg.ranks)
    fams = ["gemm_fwd", "gemm_dx", "shrink_x", "shrink_dy", "seg_outer_dB", "seg_outer_dA"]
    if fp8:
        fams += ["quantize_x", "quantize_dy"]
    fam = {k: {"time": 0.0, "flops": 0, "bytes": 0, "launches": 0} for k in fams}
    with torch.no_grad():
        for L in lins:
            M, K, N = cfg.tokens, L["K"], L["N"]
            A_ops = [_as_operand(a) for a in L["As"]]
            B_ops = [_as_operand(v) for v in L["Bs"]]
            x, dy = L["x"].detach(), L["dy"]
            h_rows, h_frag = kernels.shrink(x, A_ops, 0, scales, routing, True, R)
            g_rows, g_frag = kernels.shrink(dy, B_ops, 1, scales, routing, True, R)
            A_t = [a.t().contiguous() for a in A_ops]  # the NT form of dX contracts g with A_aᵀ
            lora_mr = sum(m * cfg.ranks[a] for m, a in seg if a >= 0)
            r_sum = sum(cfg.ranks)
            runs = {
                "gemm_fwd": (lambda: kernels.gemm_fwd(x, L["w"], L["b"], h_rows, B_ops, routing),
                             2 * M * K * N + 2 * lora_mr * N, 0),
                "gemm_dx": (lambda: kernels.gemm_fwd(dy, L["wt"], None, g_rows, A_t, routing),
                            2 * M * K * N + 2 * lora_mr * K, 0),
                "shrink_x": (lambda: kernels.shrink(x, A_ops, 0, scales, routing, True, R),
                             2 * lora_mr * K, M * K * 2 + r_sum * K * 2 + lora_mr * (2 + 4)),
                "shrink_dy": (lambda: kernels.shrink(dy, B_ops, 1, scales, routing, True, R),
                              2 * lora_mr * N, M * N * 2 + r_sum * N * 2 + lora_mr * (2 + 4)),
                "seg_outer_dB": (lambda: kernels.seg_outer(dy, h_frag, R, cfg.ranks, routing, 0,
                                                           [torch.bfloat16] * len(cfg.ranks)),
                                 2 * lora_mr * N, M * N * 2 + lora_mr * 4 + r_sum * N * 2),
                "seg_outer_dA": (lambda: kernels.seg_outer(x, g_frag, R, cfg.ranks, routing, 1,
                                                           [torch.bfloat16] * len(cfg.ranks)),
                                 2 * lora_mr * K, M * K * 2 + lora_mr * 4 + r_sum * K * 2),
            }
            if fp8:
                xq, xs = kernels.quantize_rows_fp8(x)
                runs["gemm_fwd"] = (lambda: kernels.gemm_fwd_fp8(xq, xs, L["wq"], L["ws"], L["b"], h_rows, B_ops,
                                                                 routing), 2 * M * K * N + 2 * lora_mr * N, 0)
                dyq, dys = kernels.quantize_rows_fp8(dy, col_scale=L["ws"])
                g_div, _ = kernels.shrink(dy, B_ops, 1, scales, routing, False, R, row_div=dys)
                a_t = [a.t().contiguous() for a in A_ops]
                runs["gemm_dx"] = (lambda: kernels.gemm_fwd_fp8(dyq, dys, L["wqt"], None, None, g_div, a_t, routing),
                                   2 * M * K * N + 2 * lora_mr * K, 0)
                runs["quantize_x"] = (lambda: kernels.quantize_rows_fp8(x), 0, M * K * 3 + M * 4)
                runs["quantize_dy"] = (lambda: kernels.quantize_rows_fp8(dy, col_scale=L["ws"]), 0,
                                       M * N * 3 + M * 4 + N * 4)
            for k, (fn, fl, by) in runs.items():
                t = timed(fn)
                fam[k]["time"] += t
                fam[k]["flops"] += fl
                fam[k]["bytes"] += by
                fam[k]["launches"] += 1
            del h_rows, h_frag, g_rows, g_frag
    kern = {}
    for k, v in fam.items():
        avg = v["time"] / v["launches"]
        kern[k] = {"avg_us": round(avg * 1e6, 2), "launches_per_step": v["launches"],
                   "tflops": round(v["flops"] / v["time"] / 1e12, 1),
                   "gbs": round(v["bytes"] / v["time"] / 1e9, 1) if v["bytes"] else None}
    gem = fam["gemm_fwd"]
    gem_ach = gem["flops"] / gem["time"] / 1e12
    gem_peak = MFMA_FP8_PEAK_TFLOPS if fp8 else MFMA_BF16_PEAK_TFLOPS
    roofline = {"kernel": ("gemm_kernel NT e4m3 base (fp8 MFMA) + fused dequantise and bf16 LoRA expand"
                           if fp8 else "gemm_kernel NT (base GEMM + fused LoRA expand)")
                + ", avg over the 6 block linears",
                "bound": "mfma", "achieved": round(gem_ach, 1), "peak": gem_peak, "unit": "TFLOP/s",
                "frac": round(gem_ach / gem_peak, 4),
                "traffic": recorded_traffic() if cfg.name == "wan13b" else None,
                "avg_launch_us": round(gem["time"] / gem["launches"] * 1e6, 2),
                "flops_per_launch": gem["flops"] // gem["launches"]}
    lora = {}
    for k in ("shrink_x", "shrink_dy", "seg_outer_dB", "seg_outer_dA") + (("quantize_x", "quantize_dy") if fp8 else ()):
        v = fam[k]
        gbs = v["bytes"] / v["time"] / 1e9
        lora[k] = {"achieved_gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                   "avg_us": kern[k]["avg_us"]}

    # ---------------- vendor GEMM reference (context only): torch bf16 matmul, same shapes
    vendor = {}
    with torch.no_grad():
        for L in lins[3:6]:
            x = L["x"].detach()
            t = timed(lambda: torch.matmul(x, L["w"].T))
            vendor[f"{L['name']} {L['K']}->{L['N']}"] = round(2 * cfg.tokens * L["K"] * L["N"] / t / 1e12, 1)

    per_role = per_role_timing(pkg, cfg, lins, scales, args, flops_step) if args.per_role else None

    # ---------------- CPU baseline: reference per-adapter path, fp32 torch, bounded sample
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_seconds, args.fwd_only)

    pass_name = "fwd" if args.fwd_only else "fwd+bwd"
    shape_name = "Wan-1.3B shape" if cfg.name == "wan13b" else f"{cfg.name} shape"
    out = {
        "metric": f"multi-LoRA linear {pass_name} TFLOP/s at {shape_name}",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("e4m3 base forward (fp32 accumulate), bf16 LoRA and backward" if fp8 else "bf16")
        + ("" if cfg.dtype == "bf16" else f" (config specifies {cfg.dtype}; computed in bf16)"),
        "data": "synthetic (seeded N(0,1) activations, N(0,1/in) frozen base, Kaiming-uniform A, N(0,0.02) B)",
        "config": {"workload": f"{cfg.name}: {pass_name} of the 6 DiT block linears "
                               f"(q,k,v,o {cfg.hidden}->{cfg.hidden}; ffn {cfg.hidden}->{cfg.ffn}->{cfg.hidden}), "
                               f"{cfg.tokens} tokens in segments {list(cfg.seg_lengths)}, ranks {list(cfg.ranks)}, "
                               f"scale {cfg.scale}, bias on" + (", frozen base e4m3 + per-channel scale" if fp8 else "")
                               + ("; q, k, v read one input and run as one stacked call" if args.shared_qkv else "")
                               + ("; o and ffn.2 end in the block's gated residual, fused" if args.gated_residual
                                  else ""),
                   "tokens": cfg.tokens, "flops_per_step": flops_step, "pct_bf16_mfma_peak": round(
                       tflops / MFMA_BF16_PEAK_TFLOPS * 100, 2)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "lora_hbm": lora,
        "kernels": kern,
        "vendor_gemm_tflops": vendor,
        **({"per_role": per_role} if per_role is not None else {}),
        **({"qkv_unstacked": unstacked} if unstacked is not None else {}),
        **({"gated_residual_unfused": unfused} if unfused is not None else {}),
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "gcn_arch": getattr(props, "gcnArchName", "")},
    }
    print(json.dumps(out), flush=True)


def per_role_timing(pkg, cfg, lins, scales, args, flops_step):
    """The step of the batched call, split into one call per segment (one role per call, as
    the reference calls its roles, training/dmd.py:324-345): with this library's op, and
    with the reference's unfused autocast path (low_rank.py:26-28: base GEMM, two skinny
    GEMMs, bf16 scale and add; a base-only role is the plain linear) in torch on the GPU."""
    import torch
    import torch.nn.functional as F
    segs = [(a, b, ad) for a, b, ad in zip(cfg.routing.seg_offsets, cfg.routing.seg_offsets[1:],
                                           cfg.routing.adapter_ids) if b > a]
    # each role owns its input (a leaf of its own, not a slice of the batched one)
    xs = {(id(L), r0): L["x"].detach()[r0:r1].clone().requires_grad_(not args.fwd_only)
          for L in lins for r0, r1, _ in segs}

    def lib_call(L, r0, r1, ad):
        return pkg.multi_lora_linear(xs[id(L), r0], L["w"], L["b"], L["As"], L["Bs"], scales,
                                     pkg.SegmentRouting.single(r1 - r0, ad), weight_t=L["wt"])

    def torch_call(L, r0, r1, ad):
        x = xs[id(L), r0]
        y = F.linear(x, L["w"], L["b"])
        if ad < 0:
            return y
        return y + scales[ad] * F.linear(F.linear(x, L["As"][ad]), L["Bs"][ad])

    def step_of(call):
        def step():
            if args.fwd_only:
                with torch.no_grad():
                    for L in lins:
                        for r0, r1, ad in segs:
                            call(L, r0, r1, ad)
                return
            for L in lins:
                for t in [*L["As"], *L["Bs"]] + [xs[id(L), r0] for r0, _, _ in segs]:
                    t.grad = None
                for r0, r1, ad in segs:
                    call(L, r0, r1, ad).backward(L["dy"][r0:r1])
        return step

    out = {"segments": len(segs)}
    for key, call in (("library", lib_call), ("torch_unfused", torch_call)):
        step = step_of(call)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
        out[key] = {"ms_per_step": round(ms, 4), "tflops": round(flops_step / (ms * 1e-3) / 1e12, 2)}
    return out


def cpu_baseline(cfg, budget_s: float, fwd_only: bool = False):
    """Reference per-adapter path (training/low_rank.py:26-28 per segment + autograd) in fp32 on host cores
    (an e4m3 base is evaluated as its fp32 dequantisation: the reference has no fp8 path)."""
    import torch
    from oracle import torch_reference as TR
    from dmd_system_amd import workloads

    rows_per_seg = max(128, 2048 // len(cfg.seg_lengths))
    sample = workloads.LoraConfig(
        name="cpu-sample", tokens=rows_per_seg * len(cfg.seg_lengths), hidden=cfg.hidden, ffn=cfg.ffn,
        ranks=cfg.ranks, seg_lengths=(rows_per_seg,) * len(cfg.seg_lengths), seg_adapters=cfg.seg_adapters,
        scale=cfg.scale, seed=cfg.seed)
    cpu = torch.device("cpu")
    lin = []
    for i, (name, K, N) in enumerate(sample.linears()):
        x, w, b, As, Bs, dy = workloads.make_linear(sample, K, N, cpu, seed=7 + i, dtype=torch.float32)
        lin.append((K, N, x, w, b, As, Bs, dy))
    off = sample.routing.seg_offsets
    ids = sample.routing.adapter_ids
    scales = [cfg.scale] * len(cfg.ranks)

    def one_block():
        for K, N, x, w, b, As, Bs, dy in lin:
            if fwd_only:
                with torch.no_grad():
                    TR.per_adapter_forward(x, w, b, As, Bs, scales, off, ids)
            else:
                TR.per_adapter_step(x, w, b, As, Bs, scales, off, ids, dy)

    one_block()  # warmup
    t0 = time.perf_counter()
    reps = 0
    while True:
        one_block()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 50:
            break
    flops = sum((sample.flops_fwd if fwd_only else sample.flops_fwd_bwd)(K, N) for _, K, N in sample.linears())
    return {"value": round(flops * reps / el / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{reps} x {'fwd' if fwd_only else 'fwd+bwd'} of the 6 block linears at {sample.tokens} tokens "
                      f"({rows_per_seg} per segment), fp32 torch per-adapter path, {el:.1f} s; "
                      f"host os.cpu_count()={os.cpu_count()}"}


if __name__ == "__main__":
    main()
