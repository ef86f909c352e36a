"""Benchmark of the MI355X multi-LoRA linear (forward + backward).

One step = forward + backward of the six LoRA linears of one Wan-1.3B DiT
block (q, k, v, o: 1536->1536; ffn.0: 1536->8960; ffn.2: 8960->1536) over
65520 tokens = two roles (generator, fake critic) of 32760 tokens, each with
its own rank-64 adapter on the shared frozen bf16 base (config 2, `wan13b`),
through the drop-in autograd op with inputs resident in HBM.

Prints one JSON line: metric/value (TFLOP/s of the whole step), the roofline
of the dominant kernel measured with HIP events, the LoRA kernels' HBM GB/s,
and a CPU baseline (the reference per-adapter path in fp32 torch on host
cores, at the same shapes and token count).

Other configurations (parity-test cases, measured on request): --config
tiny | wan22_5b | flux | wan13b_fp8 (frozen base stored e4m3 with a per-output-
channel scale: forward on the e4m3 MFMA) | wan13b_roles (the multi-role call site:
teacher conditional + unconditional rows base-only and the fake critic's rows with its
adapter, in one call), --fwd-only for a forward-only step, --per-role to time the
same step as one call per role (this library, and the reference's unfused torch path),
--shared-qkv to feed q, k, v one input and run them as one stacked call (the step
with three separate calls on that input is timed beside it), and --gated-residual to end o
and ffn.2 in the block's gated residual x + y·gate on the float32 residual stream, fused
into the GEMM epilogue (the step with the residual as torch ops after the linear is timed
beside it).

Measurement: `value` is the whole-job throughput of exactly K steps after W warmups (one HIP
event pair and wall clock around them, the slower of the two); `step_distribution` times
max(50, K) further steps one by one. Per-kernel rates (roofline, lora_hbm) are the median of
--kernel-reps launches, each reading one of --rotate input sets after a 512 MB read that evicts
L2 and the MALL.

--modulated-norm times only the block's modulated LayerNorm kernel (fused LayerNorm + modulation) at
the configuration's tokens and width, on the float32 residual stream and a bf16 hidden state.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config wan13b] [--fwd-only] [--per-role] [--shared-qkv] [--gated-residual] [--modulated-norm]
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
MFMA_FP32_PEAK_TFLOPS = 157.3   # dense fp32


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="wan13b")
    p.add_argument("--fwd-only", action="store_true", help="time forward passes only (no autograd)")
    p.add_argument("--kernel-reps", type=int, default=50,
                   help="timed launches per kernel and linear (median reported); each launch reads one of "
                        "--rotate input sets and follows a cache scrub")
    p.add_argument("--rotate", type=int, default=3, help="input sets cycled by the per-kernel timing")
    p.add_argument("--scrub-mb", type=int, default=512,
                   help="MB read between timed kernel launches (evicts L2 and the 256 MB MALL)")
    p.add_argument("--median-steps", type=int, default=50,
                   help="extra steps timed one by one (per-step HIP events) for the step median")
    p.add_argument("--cpu-reps", type=int, default=3, help="timed reps (median) per linear of the CPU baseline")
    p.add_argument("--cpu-tokens", type=int, default=0,
                   help="tokens of the CPU baseline (0: the configuration's full token count)")
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
    p.add_argument("--rank", type=int, default=0,
                   help="every adapter of --config at this rank instead of the configuration's (the reference's "
                        "Wan LoRA runs use 128 and 256)")
    p.add_argument("--fp32-masters", action="store_true",
                   help="fp32 adapter masters over the bf16 base outside autocast (the W1 / native layout): the "
                        "shrinks use them at fp32-class precision (hi + lo bf16 parts)")
    p.add_argument("--fp8-dx-bf16", action="store_true",
                   help="with an e4m3 base: dX on the bf16 MFMA against the dequantised base instead of the "
                        "e4m3 MFMA with a quantised dY (closer to the exact dX, slower)")
    p.add_argument("--modulated-norm", action="store_true",
                   help="only time the block's modulated LayerNorm (fused LayerNorm + modulation into the next "
                        "sublayer's bf16 input) at the configuration's tokens and hidden width, on the float32 "
                        "residual stream and on a bf16 hidden state, beside torch's LayerNorm + ops")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device copy 4 times (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    p.add_argument("--profile-kernels", action="store_true",
                   help="only launch each kernel of the step (and torch's bf16 matmul) --kernel-reps times per "
                        "distinct linear shape of --config, each launch after a cache-evicting read, for "
                        "rocprofv3 counter and trace passes; prints the launch schedule")
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


def modulated_norm_bench(args, pkg, cfg, dev):
    """Per-launch time of the fused LayerNorm + modulation (mlora_modulated_norm) at the
    configuration's shape: B samples (one per segment when the segments are equal, as the
    wan13b roles are) of T tokens, width = the block's hidden size. The modulation is Wan's:
    a [1, 6, W] table plus a per-sample [B, 6, W] time embedding (token stride 0). Medians of
    --kernel-reps launches, each after a cache-evicting read, cycling --rotate input sets."""
    import statistics
    import torch
    lengths = cfg.routing.lengths()
    M = sum(lengths)
    B = len(lengths) if len(set(lengths)) == 1 else 1
    T = M // B
    W = cfg.hidden
    scrub = torch.ones(args.scrub_mb << 18, dtype=torch.float32, device=dev)
    table = 0.1 * torch.randn(1, 6, W, device=dev)
    e = 0.1 * torch.randn(B, 6, W, device=dev)
    scale_c, shift_c = e[:, 1:2].expand(B, T, W), e[:, 0:1].expand(B, T, W)

    def time_launches(fn, inputs):
        ts = []
        for i in range(args.kernel_reps + 2):
            x = inputs[i % len(inputs)]
            scrub.amax()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn(x)
            b.record()
            torch.cuda.synchronize()
            if i >= 2:
                ts.append(a.elapsed_time(b) * 1e3)
        return statistics.median(ts)

    res = {}
    for name, dt in (("float32_stream", torch.float32), ("bf16_hidden", torch.bfloat16)):
        inputs = [(3 + 2 * torch.randn(B, T, W, device=dev)).to(dt) for _ in range(args.rotate)]
        out = torch.empty(B, T, W, dtype=torch.bfloat16, device=dev)

        def ours(x):
            pkg.fused_layernorm_modulation(x, table, 1, 0, scale_c, shift_c, out, eps=1e-6)

        def torch_path(x):
            n = torch.nn.functional.layer_norm(x.float(), (W,), eps=1e-6)
            s = (table[:, 1] + e[:, 1]).unsqueeze(1)
            h = (table[:, 0] + e[:, 0]).unsqueeze(1)
            return (n * (1 + s) + h).to(torch.bfloat16)

        us = time_launches(ours, inputs)
        tus = time_launches(torch_path, inputs)
        nbytes = M * W * (inputs[0].element_size() + 2) + 2 * B * W * 4 + 2 * W * 4
        res[name] = {"avg_us": round(us, 2), "bytes_per_launch": nbytes, "achieved_gbs": round(nbytes / us / 1e3, 1),
                     "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "torch_us": round(tus, 2),
                     "speedup_vs_torch": round(tus / us, 2)}
    # backward on the float32 stream (the Wan block): the hidden gradient with the row statistics,
    # the per-sample component gradient, and the whole autograd op (forward + backward) beside torch's
    hidden = [(3 + 2 * torch.randn(B, T, W, device=dev)) for _ in range(args.rotate)]
    up = torch.randn(B, T, W, device=dev).to(torch.bfloat16)
    dx = torch.empty(B, T, W, device=dev)
    mean = torch.empty(B, T, device=dev)
    rstd = torch.empty(B, T, device=dev)
    dcomp = torch.zeros(B, 6, W, device=dev)
    scale4 = e[:, 4:5].expand(B, T, W)

    def hidden_bwd(x):
        pkg.fused_layernorm_modulation_hidden_backward(x, up, table, 4, scale4, dx, mean, rstd, eps=1e-6)

    def comp_bwd(x):
        pkg.fused_reduced_component_gradient(x, up, mean, rstd, dcomp, 4, 3)

    tab_p = table.clone().requires_grad_(True)
    e_p = e.clone().requires_grad_(True)

    def op_fwd_bwd(x):
        x = x.detach().requires_grad_(True)
        pkg.modulated_layer_norm(x, tab_p, e_p, 4, 3, 1e-6).backward(up)

    def torch_fwd_bwd(x):
        x = x.detach().requires_grad_(True)
        mod = tab_p + e_p
        n = torch.nn.functional.layer_norm(x, (W,), eps=1e-6)
        (n * (1 + mod[:, 4:5]) + mod[:, 3:4]).to(torch.bfloat16).backward(up)

    hidden_bwd(hidden[0])
    bus, cus = time_launches(hidden_bwd, hidden), time_launches(comp_bwd, hidden)
    ous, tous = time_launches(op_fwd_bwd, hidden), time_launches(torch_fwd_bwd, hidden)
    hb = M * W * (4 + 2 + 4) + M * 8
    cb = M * W * (4 + 2) + M * 8
    res["backward_float32_stream"] = {
        "hidden_backward_us": round(bus, 2), "hidden_backward_gbs": round(hb / bus / 1e3, 1),
        "component_gradient_us": round(cus, 2), "component_gradient_gbs": round(cb / cus / 1e3, 1),
        "autograd_fwd_bwd_us": round(ous, 2), "torch_autograd_fwd_bwd_us": round(tous, 2),
        "speedup_vs_torch": round(tous / ous, 2)}
    f = res["float32_stream"]
    print(json.dumps({
        "metric": f"modulated LayerNorm GB/s at {cfg.name} shape", "value": f["achieved_gbs"], "unit": "GB/s",
        "higher_is_better": True, "dtype": "f32 -> bf16",
        "config": {"workload": f"fused LayerNorm + Wan modulation into the next sublayer's bf16 input, {B} x {T} "
                               f"tokens, width {W}", "tokens": M},
        "roofline": {"kernel": "modulated_norm_kernel (float32 stream)", "bound": "hbm",
                     "achieved": f["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": f["frac_hbm"], "avg_launch_us": f["avg_us"]},
        "variants": res}), flush=True)


def profile_kernels(args):
    """Launches for rocprofv3: per distinct (K, N) linear shape of the configuration, each kernel
    family `--kernel-reps` times, every launch preceded by a 512 MB read (a torch reduction) that
    evicts L2 and the MALL. The printed schedule lists the launch groups in order (one group =
    the kernels between two reads), so dispatches in a trace or counter file map to
    (shape, family); beside it, each group's algorithmic work ("flop", or "byte": what the
    kernel must move once). Families: gemm_fwd (NT, fused LoRA expand), gemm_dx (NT against the
    transposed base), gemm_dx_nn (NN against the base as stored), shrink_x, shrink_dy,
    seg_outer_dB, seg_outer_dA (main pass + fixed-order reduction), torch_matmul (hipBLASLt, bf16);
    with an e4m3 base instead of the bf16 GEMMs: quantize_x, gemm_fwd_fp8, quantize_dy (dY times
    the channel scales), gemm_dx_fp8 (the e4m3 dX), torch_scaled_mm (hipBLASLt's e4m3 GEMM, where
    torch takes row-wise scales); last, a plain 1 GiB device copy as the reference rate of
    HBM-bound kernels."""
    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    pkg.load_library()
    from dmd_system_amd import kernels, workloads
    from dmd_system_amd.function import _as_operand
    dev = torch.device("cuda:0")
    cfg = workloads.CONFIGS[args.config]
    if args.rank:
        import dataclasses
        cfg = dataclasses.replace(cfg, ranks=(args.rank,) * len(cfg.ranks))
    if cfg.dtype == "fp32":
        raise SystemExit("--profile-kernels covers the bf16 and e4m3 kernels")
    fp8 = cfg.base_fp8
    routing, scales = cfg.routing, [cfg.scale] * len(cfg.ranks)
    R = kernels.padded_rank(cfg.ranks)
    bf = [torch.bfloat16] * len(cfg.ranks)
    M = cfg.tokens
    segs = [(n, a) for n, a in zip(cfg.seg_lengths, cfg.seg_adapters)]
    m_a = sum(n for n, a in segs if a >= 0)                     # rows with an adapter
    mr = sum(n * cfg.ranks[a] for n, a in segs if a >= 0)        # Σ rows·rank
    r_sum = sum(cfg.ranks[a] for a in {a for _, a in segs if a >= 0})

    def algorithmic(fam, K, N):
        return {"gemm_fwd": ("flop", 2 * M * K * N + 2 * mr * N), "gemm_fwd_fp8": ("flop", 2 * M * K * N + 2 * mr * N),
                "gemm_dx": ("flop", 2 * M * K * N + 2 * mr * K), "gemm_dx_nn": ("flop", 2 * M * K * N + 2 * mr * K),
                "gemm_dx_fp8": ("flop", 2 * M * K * N + 2 * mr * K), "torch_matmul": ("flop", 2 * M * K * N),
                "torch_scaled_mm": ("flop", 2 * M * K * N),
                # P rows read once, the adapter operands once, h rows (2 B) and hi/lo fragments (4 B) written
                "shrink_x": ("byte", m_a * K * 2 + r_sum * K * 2 + mr * 6),
                "shrink_dy": ("byte", m_a * N * 2 + r_sum * N * 2 + mr * 6),
                # P rows and the fragments read once, the bf16 gradients written
                "seg_outer_dB": ("byte", m_a * N * 2 + mr * 4 + r_sum * N * 2),
                "seg_outer_dA": ("byte", m_a * K * 2 + mr * 4 + r_sum * K * 2),
                # bf16 rows read, e4m3 rows and one fp32 scale per row written (+ the channel scales)
                "quantize_x": ("byte", M * K * 3 + M * 4), "quantize_dy": ("byte", M * N * 3 + M * 4 + N * 4),
                }[fam]

    scrub = torch.ones(args.scrub_mb << 18, dtype=torch.float32, device=dev)
    schedule, algo = [], {}
    shapes = []
    for name, K, N in cfg.linears():
        if (K, N) not in [(k, n) for _, k, n in shapes]:
            shapes.append((name, K, N))
    with torch.no_grad():
        for i, (name, K, N) in enumerate(shapes):
            x, w, b, As, Bs, dy = workloads.make_linear(cfg, K, N, dev, seed=cfg.seed * 100 + i)
            A_ops, B_ops = [_as_operand(a) for a in As], [_as_operand(v) for v in Bs]
            A_t = [a.t().contiguous() for a in A_ops]
            if fp8:
                wq, ws = kernels.quantize_rows_fp8(w)
                wqt = wq.t().contiguous()
                xq, xs = kernels.quantize_rows_fp8(x)
                dyq, dys = kernels.quantize_rows_fp8(dy, col_scale=ws)
                B_div = [kernels.div_rows_bf16(v, ws) for v in B_ops]
                h_rows, h_frag = kernels.shrink(x, A_ops, 0, scales, routing, True, R, row_div=xs)
                g_rows, g_frag = kernels.shrink(dy, B_ops, 1, scales, routing, True, R, row_div=dys)
                fams = {
                    "quantize_x": lambda: kernels.quantize_rows_fp8(x),
                    "gemm_fwd_fp8": lambda: kernels.gemm_fwd_fp8(xq, xs, wq, ws, b, h_rows, B_div, routing),
                    "quantize_dy": lambda: kernels.quantize_rows_fp8(dy, col_scale=ws),
                    "gemm_dx_fp8": lambda: kernels.gemm_fwd_fp8(dyq, dys, wqt, None, None, g_rows, A_t, routing),
                    "shrink_x": lambda: kernels.shrink(x, A_ops, 0, scales, routing, True, R, row_div=xs),
                    "shrink_dy": lambda: kernels.shrink(dy, B_ops, 1, scales, routing, True, R, row_div=dys),
                }
                # hipBLASLt's e4m3 GEMM (torch._scaled_mm, row-wise scales) on the same operands, context
                # only; left out where this torch build does not take it
                scaled = lambda: torch._scaled_mm(xq, wq.t(), scale_a=xs[:, None], scale_b=ws[None, :],  # noqa: E731
                                                  out_dtype=torch.bfloat16)
                try:
                    scaled()
                    torch.cuda.synchronize()
                    fams["torch_scaled_mm"] = scaled
                except (RuntimeError, TypeError):
                    pass
            else:
                wt = w.t().contiguous()
                h_rows, h_frag = kernels.shrink(x, A_ops, 0, scales, routing, True, R)
                g_rows, g_frag = kernels.shrink(dy, B_ops, 1, scales, routing, True, R)
                fams = {
                    "gemm_fwd": lambda: kernels.gemm_fwd(x, w, b, h_rows, B_ops, routing),
                    "gemm_dx": lambda: kernels.gemm_fwd(dy, wt, None, g_rows, A_t, routing),
                    "gemm_dx_nn": lambda: kernels.gemm_dx(dy, w, g_rows, A_ops, routing),
                    "shrink_x": lambda: kernels.shrink(x, A_ops, 0, scales, routing, True, R),
                    "shrink_dy": lambda: kernels.shrink(dy, B_ops, 1, scales, routing, True, R),
                }
            fams.update({
                "seg_outer_dB": lambda: kernels.seg_outer(dy, h_frag, R, cfg.ranks, routing, 0, bf),
                "seg_outer_dA": lambda: kernels.seg_outer(x, g_frag, R, cfg.ranks, routing, 1, bf),
                "torch_matmul": lambda: torch.matmul(x, w.T),
            })
            for fam, fn in fams.items():
                label = f"{name} {K}->{N} {fam}"
                algo[label] = algorithmic(fam, K, N)
                for rep in range(args.kernel_reps + 1):  # the first group warms up (allocations)
                    scrub.amax()
                    fn()
                    schedule.append(label + (" warm" if rep == 0 else ""))
                torch.cuda.synchronize()
            del x, w, b, As, Bs, dy, A_ops, B_ops, A_t, h_rows, h_frag, g_rows, g_frag, fams
        # reference point for the HBM-bound kernels: a plain 1 GiB device copy (torch's copy kernel)
        src = torch.ones(1 << 29, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        for rep in range(args.kernel_reps + 1):
            scrub.amax()
            dst.copy_(src)
            schedule.append("copy 1GiB copy" + (" warm" if rep == 0 else ""))
        algo["copy 1GiB copy"] = ("byte", 2 << 30)
        torch.cuda.synchronize()
        del src, dst
    print(json.dumps({"profile_kernels": cfg.name, "ranks": list(cfg.ranks), "tokens": M, "reps": args.kernel_reps,
                      "marker": "torch amax reduction before every group", "schedule": schedule,
                      "algorithmic": algo}), flush=True)


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
    if args.profile_kernels:
        profile_kernels(args)
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
    if args.rank:
        import dataclasses
        cfg = dataclasses.replace(cfg, ranks=(args.rank,) * len(cfg.ranks))
    if args.modulated_norm:
        modulated_norm_bench(args, pkg, cfg, dev)
        return
    routing = cfg.routing
    scales = [cfg.scale] * len(cfg.ranks)

    fp8 = cfg.base_fp8
    if args.fp8_dx_bf16 and not fp8:
        raise SystemExit("--fp8-dx-bf16 needs a configuration with an e4m3 base (wan13b_fp8)")
    # a float32 configuration (config 1, the reference's precision='fp32') runs the float32 path:
    # float32 tensors through the same op, on the fp32 MFMA kernels
    f32 = cfg.dtype == "fp32"
    # ---------------- inputs (resident in HBM); an e4m3 base is stored quantised
    lins = []
    for i, (name, K, N) in enumerate(cfg.linears()):
        x, w, b, As, Bs, dy = workloads.make_linear(cfg, K, N, dev, seed=cfg.seed * 100 + i,
                                                    dtype=torch.float32 if f32 else torch.bfloat16)
        if args.fp32_masters:
            if f32 or fp8:
                raise SystemExit("--fp32-masters is for the bf16 base")
            As, Bs = [a.float() for a in As], [b.float() for b in Bs]
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

    if (args.shared_qkv or args.gated_residual) and f32:
        raise SystemExit("--shared-qkv / --gated-residual run the bf16 kernels")
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
                # the Wan block's residual stream is float32 (model.py:305-306,312-313)
                L["res"] = torch.randn(cfg.tokens, L["N"], generator=gen, device=dev)
                L["res"].requires_grad_(not args.fwd_only)
                # one gate row per role segment, as Wan's per-sample e[2] / e[5]
                L["gate"] = torch.rand(len(cfg.seg_lengths), L["N"], generator=gen, device=dev) + 0.5
        if len(set(cfg.seg_lengths)) != 1:
            raise SystemExit("--gated-residual needs equal segment lengths (one gate row per segment)")

    def unfused_gated(L):
        y = pkg.multi_lora_linear(L["x"], L["w"], L["b"], L["As"], L["Bs"], scales, routing, weight_t=L["wt"])
        g = L["gate"].repeat_interleave(cfg.tokens // L["gate"].shape[0], dim=0)
        return L["res"] + y.float() * g

    def forward(L, fuse=True):
        if "gate" in L:
            if fuse:
                return pkg.multi_lora_linear_gated(L["x"], L["w"], L["b"], L["As"], L["Bs"], scales, routing,
                                                   L["res"], L["gate"], weight_t=L["wt"])
            return unfused_gated(L)
        if fp8:
            return pkg.multi_lora_linear_fp8(L["x"], L["wq"], L["ws"], L["b"], L["As"], L["Bs"], scales, routing,
                                             wq_t=L["wqt"], dx_bf16=args.fp8_dx_bf16)
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
    peak_mem = torch.cuda.max_memory_allocated(dev)
    print(f"# step {ms_per_step:.3f} ms, {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)

    # ---------------- per-step distribution: steps timed one by one with HIP events on the
    # launch stream. One step cycles through the six linears' own tensors (~2.5 GB of distinct
    # inputs and outputs), so no step finds the previous use of its operands in the 256 MB MALL.
    n_med = max(args.median_steps, args.steps)
    launch_stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_med)]
    for e0, e1 in evs:
        e0.record(launch_stream)
        step()
        e1.record(launch_stream)
    torch.cuda.synchronize()
    step_ms = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    q = lambda f: step_ms[min(len(step_ms) - 1, int(f * len(step_ms)))]  # noqa: E731
    step_stats = {"steps": n_med, "median_ms": round(q(0.5), 4), "p10_ms": round(q(0.1), 4),
                  "p90_ms": round(q(0.9), 4), "median_tflops": round(flops_step / (q(0.5) * 1e-3) / 1e12, 2)}
    print(f"# step median {q(0.5):.3f} ms over {n_med}", file=sys.stderr, flush=True)
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

    # ---------------- per-kernel timing: HIP events on the launch stream around each launch,
    # every launch reading one of `rotate` input sets (distinct tensors of the linear's shape)
    # and preceded by a read of `scrub_mb` MB (untimed) that evicts L2 and the 256 MB MALL, so
    # a kernel's operands come from HBM as in a real step; the median launch is reported.
    reps = args.kernel_reps
    stream = torch.cuda.current_stream(dev)
    scrub_buf = torch.ones(args.scrub_mb << 18, dtype=torch.float32, device=dev)

    def timed(fns):
        """Median seconds per launch of fns[i % len(fns)]() over `reps` launches. The scrub
        reads (does not write) its buffer, so no dirty lines are left for the timed kernel
        to write back."""
        fns[0]()
        torch.cuda.synchronize()
        pairs = []
        for i in range(reps):
            scrub_buf.amax()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fns[i % len(fns)]()
            e1.record(stream)
            pairs.append((e0, e1))
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in pairs)
        return ms[len(ms) // 2] * 1e-3

    from dmd_system_amd.function import _as_operand
    seg = list(zip(cfg.seg_lengths, cfg.seg_adapters))
    R = kernels.padded_rank(cfg.ranks)
    fams = ["gemm_fwd", "gemm_dx", "shrink_x", "shrink_dy", "seg_outer_dB", "seg_outer_dA"]
    if fp8:
        fams += ["quantize_x", "quantize_dy"]
    fam = {k: {"time": 0.0, "flops": 0, "bytes": 0, "launches": 0} for k in fams}
    gen = torch.Generator(device=dev)
    with torch.no_grad():
        for li, L in enumerate(lins):
            M, K, N = cfg.tokens, L["K"], L["N"]
            A_ops = [_as_operand(a) for a in L["As"]]
            B_ops = [_as_operand(v) for v in L["Bs"]]
            A_t = [a.t().contiguous() for a in A_ops]  # the NT form of dX contracts g with A_aᵀ
            if f32:  # fp32 operands: A_a [r, K], B_a [N, r] (the dY shrink reads B_a as [K=N, r])
                A32 = [a.detach().contiguous() for a in L["As"]]
                B32 = [v.detach().contiguous() for v in L["Bs"]]
            sets = []
            for r in range(max(1, args.rotate)):
                if r == 0:
                    x, dy = L["x"].detach(), L["dy"]
                else:
                    gen.manual_seed(1000 * li + r)
                    dt = torch.float32 if f32 else torch.bfloat16
                    x = torch.randn(M, K, generator=gen, device=dev).to(dt)
                    dy = torch.randn(M, N, generator=gen, device=dev).to(dt)
                if f32:
                    sets.append(dict(x=x, dy=dy, h=kernels.f32_shrink(x, A32, 0, scales, routing, R),
                                     g=kernels.f32_shrink(dy, B32, 1, scales, routing, R)))
                    continue
                h_rows, h_frag = kernels.shrink(x, A_ops, 0, scales, routing, True, R)
                g_rows, g_frag = kernels.shrink(dy, B_ops, 1, scales, routing, True, R)
                S = dict(x=x, dy=dy, h_rows=h_rows, h_frag=h_frag, g_rows=g_rows, g_frag=g_frag)
                if fp8:
                    S["xq"], S["xs"] = kernels.quantize_rows_fp8(x)
                    S["dyq"], S["dys"] = kernels.quantize_rows_fp8(dy, col_scale=L["ws"])
                    S["g_div"], _ = kernels.shrink(dy, B_ops, 1, scales, routing, False, R, row_div=S["dys"])
                sets.append(S)
            lora_mr = sum(m * cfg.ranks[a] for m, a in seg if a >= 0)
            r_sum = sum(cfg.ranks)
            ML = sum(m for m, a in seg if a >= 0)  # rows with an adapter: the LoRA kernels read only these
            bf = [torch.bfloat16] * len(cfg.ranks)
            runs = {
                "gemm_fwd": ([lambda S=S: kernels.gemm_fwd(S["x"], L["w"], L["b"], S["h_rows"], B_ops, routing)
                              for S in sets], 2 * M * K * N + 2 * lora_mr * N, 0),
                "gemm_dx": ([lambda S=S: kernels.gemm_fwd(S["dy"], L["wt"], None, S["g_rows"], A_t, routing)
                             for S in sets], 2 * M * K * N + 2 * lora_mr * K, 0),
                "shrink_x": ([lambda S=S: kernels.shrink(S["x"], A_ops, 0, scales, routing, True, R) for S in sets],
                             2 * lora_mr * K, ML * K * 2 + r_sum * K * 2 + lora_mr * (2 + 4)),
                "shrink_dy": ([lambda S=S: kernels.shrink(S["dy"], B_ops, 1, scales, routing, True, R) for S in sets],
                              2 * lora_mr * N, ML * N * 2 + r_sum * N * 2 + lora_mr * (2 + 4)),
                "seg_outer_dB": ([lambda S=S: kernels.seg_outer(S["dy"], S["h_frag"], R, cfg.ranks, routing, 0, bf)
                                  for S in sets], 2 * lora_mr * N, ML * N * 2 + lora_mr * 4 + r_sum * N * 2),
                "seg_outer_dA": ([lambda S=S: kernels.seg_outer(S["x"], S["g_frag"], R, cfg.ranks, routing, 1, bf)
                                  for S in sets], 2 * lora_mr * K, ML * K * 2 + lora_mr * 4 + r_sum * K * 2),
            }
            if f32:
                runs = {
                    "gemm_fwd": ([lambda S=S: kernels.f32_gemm_fwd(S["x"], L["w"], L["b"], S["h"], B32, routing)
                                  for S in sets], 2 * M * K * N + 2 * lora_mr * N, 0),
                    "gemm_dx": ([lambda S=S: kernels.f32_gemm_dx(S["dy"], L["w"], S["g"], A32, routing)
                                 for S in sets], 2 * M * K * N + 2 * lora_mr * K, 0),
                    "shrink_x": ([lambda S=S: kernels.f32_shrink(S["x"], A32, 0, scales, routing, R) for S in sets],
                                 2 * lora_mr * K, ML * K * 4 + r_sum * K * 4 + lora_mr * 4),
                    "shrink_dy": ([lambda S=S: kernels.f32_shrink(S["dy"], B32, 1, scales, routing, R)
                                   for S in sets], 2 * lora_mr * N, ML * N * 4 + r_sum * N * 4 + lora_mr * 4),
                    "seg_outer_dB": ([lambda S=S: kernels.f32_seg_outer(S["dy"], S["h"], cfg.ranks, routing, 0)
                                      for S in sets], 2 * lora_mr * N, ML * N * 4 + lora_mr * 4 + r_sum * N * 4),
                    "seg_outer_dA": ([lambda S=S: kernels.f32_seg_outer(S["x"], S["g"], cfg.ranks, routing, 1)
                                      for S in sets], 2 * lora_mr * K, ML * K * 4 + lora_mr * 4 + r_sum * K * 4),
                }
            if fp8:
                runs["gemm_fwd"] = ([lambda S=S: kernels.gemm_fwd_fp8(S["xq"], S["xs"], L["wq"], L["ws"], L["b"],
                                                                      S["h_rows"], B_ops, routing) for S in sets],
                                    2 * M * K * N + 2 * lora_mr * N, 0)
                runs["gemm_dx"] = ([lambda S=S: kernels.gemm_fwd_fp8(S["dyq"], S["dys"], L["wqt"], None, None,
                                                                     S["g_div"], A_t, routing) for S in sets],
                                   2 * M * K * N + 2 * lora_mr * K, 0)
                runs["quantize_x"] = ([lambda S=S: kernels.quantize_rows_fp8(S["x"]) for S in sets], 0,
                                      M * K * 3 + M * 4)
                runs["quantize_dy"] = ([lambda S=S: kernels.quantize_rows_fp8(S["dy"], col_scale=L["ws"])
                                        for S in sets], 0, M * N * 3 + M * 4 + N * 4)
            for k, (fns, fl, by) in runs.items():
                t = timed(fns)
                fam[k]["time"] += t
                fam[k]["flops"] += fl
                fam[k]["bytes"] += by
                fam[k]["launches"] += 1
            del sets
    del scrub_buf
    kern = {}
    for k, v in fam.items():
        avg = v["time"] / v["launches"]
        kern[k] = {"avg_us": round(avg * 1e6, 2), "launches_per_step": v["launches"],
                   "tflops": round(v["flops"] / v["time"] / 1e12, 1),
                   "gbs": round(v["bytes"] / v["time"] / 1e9, 1) if v["bytes"] else None}
    gem = fam["gemm_fwd"]
    gem_ach = gem["flops"] / gem["time"] / 1e12
    gem_peak = MFMA_FP8_PEAK_TFLOPS if fp8 else MFMA_FP32_PEAK_TFLOPS if f32 else MFMA_BF16_PEAK_TFLOPS
    roofline = {"kernel": ("gemm_kernel NT e4m3 base (fp8 MFMA) + fused dequantise and bf16 LoRA expand"
                           if fp8 else "f32_linear_kernel (fp32 MFMA base GEMM + fused LoRA expand)" if f32
                           else "gemm_kernel NT (base GEMM + fused LoRA expand)")
                + ", over the 6 block linears (median launch of each, cold caches)",
                "bound": "mfma", "achieved": round(gem_ach, 1), "peak": gem_peak, "unit": "TFLOP/s",
                "frac": round(gem_ach / gem_peak, 4),
                "traffic": recorded_traffic() if cfg.name == "wan13b" else None,
                "avg_launch_us": round(gem["time"] / gem["launches"] * 1e6, 2),
                "flops_per_launch": gem["flops"] // gem["launches"]}
    # the LoRA-side kernels of one step (one launch of each family per linear), from the same
    # per-kernel medians (cold caches; inside a step some operands are still cached)
    lora_side_ms = sum(fam[k]["time"] for k in ("shrink_x", "shrink_dy", "seg_outer_dB", "seg_outer_dA")) * 1e3
    lora = {}
    for k in ("shrink_x", "shrink_dy", "seg_outer_dB", "seg_outer_dA") + (("quantize_x", "quantize_dy") if fp8 else ()):
        v = fam[k]
        gbs = v["bytes"] / v["time"] / 1e9
        lora[k] = {"achieved_gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                   "avg_us": kern[k]["avg_us"]}

    # ---------------- vendor GEMM reference (context only): torch bf16 matmul, same shapes
    vendor = {}
    vendor_fp8 = {}
    scrub_buf = torch.ones(args.scrub_mb << 18, dtype=torch.float32, device=dev)
    with torch.no_grad():
        for L in lins[3:6]:
            x = L["x"].detach()
            t = timed([lambda: torch.matmul(x, L["w"].T)])
            vendor[f"{L['name']} {L['K']}->{L['N']}"] = round(2 * cfg.tokens * L["K"] * L["N"] / t / 1e12, 1)
            if fp8:
                # hipBLASLt's e4m3 GEMM through torch._scaled_mm on the same quantised operands, with
                # row-wise scales (X per token, W per channel) where this torch build takes them
                xq, xs = kernels.quantize_rows_fp8(x)
                key = f"{L['name']} {L['K']}->{L['N']}"
                for form, sa, sb in (("rowwise", xs[:, None], L["ws"][None, :]),
                                     ("tensorwise", xs.max(), L["ws"].max())):
                    try:
                        fn = lambda: torch._scaled_mm(xq, L["wq"].t(), scale_a=sa, scale_b=sb,  # noqa: E731
                                                      out_dtype=torch.bfloat16)
                        fn()
                        torch.cuda.synchronize()
                    except (RuntimeError, TypeError) as exc:
                        vendor_fp8[key + " " + form] = f"unsupported: {str(exc).splitlines()[0][:120]}"
                        continue
                    t = timed([fn])
                    vendor_fp8[key + " " + form] = round(2 * cfg.tokens * L["K"] * L["N"] / t / 1e12, 1)
                    break
                del xq, xs
    del scrub_buf

    per_role = per_role_timing(pkg, cfg, lins, scales, args, flops_step) if args.per_role else None

    # ---------------- CPU baseline: reference per-adapter path, fp32 torch, bounded sample
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_reps, args.cpu_tokens, args.fwd_only)

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
        "step_distribution": step_stats,
        "peak_mem_gb": round(peak_mem / 1e9, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": (("e4m3 base forward (fp32 accumulate), " + ("bf16 dX against the dequantised base"
                                                               if args.fp8_dx_bf16 else "e4m3 dX")
                   + ", bf16 LoRA") if fp8 else "fp32" if f32 else "bf16"),
        "data": "synthetic (seeded N(0,1) activations, N(0,1/in) frozen base, Kaiming-uniform A, N(0,0.02) B)",
        "config": {"workload": f"{cfg.name}: {pass_name} of the 6 DiT block linears "
                               f"(q,k,v,o {cfg.hidden}->{cfg.hidden}; ffn {cfg.hidden}->{cfg.ffn}->{cfg.hidden}), "
                               f"{cfg.tokens} tokens in segments {list(cfg.seg_lengths)}, ranks {list(cfg.ranks)}, "
                               f"scale {cfg.scale}, bias on" + (", frozen base e4m3 + per-channel scale" if fp8 else "")
                               + (", fp32 adapter masters (hi + lo bf16 parts)" if args.fp32_masters else "")
                               + ("; q, k, v read one input and run as one stacked call" if args.shared_qkv else "")
                               + ("; o and ffn.2 end in the block's gated residual, fused" if args.gated_residual
                                  else ""),
                   "tokens": cfg.tokens, "flops_per_step": flops_step, "pct_bf16_mfma_peak": round(
                       tflops / MFMA_BF16_PEAK_TFLOPS * 100, 2)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "lora_hbm": lora,
        "lora_side_ms_per_step": round(lora_side_ms, 3),
        "kernels": kern,
        "vendor_gemm_tflops": vendor,
        **({"vendor_fp8_gemm_tflops": vendor_fp8} if fp8 else {}),
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


def cpu_baseline(cfg, reps: int, tokens: int = 0, fwd_only: bool = False):
    """Reference per-adapter path (training/low_rank.py:26-28 per segment + autograd) in fp32 on host
    cores, at the configuration's shapes (all its tokens unless `tokens` is given, split over the
    segments in proportion): each distinct linear shape timed (1 warmup + median of `reps`), the
    block time the sum over the six linears. An e4m3 base is evaluated as its fp32 dequantisation
    (the reference has no fp8 path)."""
    import torch
    from oracle import torch_reference as TR
    from dmd_system_amd import workloads

    full = tokens <= 0 or tokens >= cfg.tokens
    if full:
        lengths = cfg.seg_lengths
    else:
        lengths = tuple(max(1, round(m * tokens / cfg.tokens)) for m in cfg.seg_lengths)
    sample = workloads.LoraConfig(
        name="cpu-sample", tokens=sum(lengths), hidden=cfg.hidden, ffn=cfg.ffn, ranks=cfg.ranks, seg_lengths=lengths,
        seg_adapters=cfg.seg_adapters, scale=cfg.scale, seed=cfg.seed)
    cpu = torch.device("cpu")
    off, ids = sample.routing.seg_offsets, sample.routing.adapter_ids
    scales = [cfg.scale] * len(cfg.ranks)
    per_shape = {}
    t_all = time.perf_counter()
    for i, (name, K, N) in enumerate(sample.linears()):
        if (K, N) in per_shape:
            continue
        x, w, b, As, Bs, dy = workloads.make_linear(sample, K, N, cpu, seed=7 + i, dtype=torch.float32)

        def once():
            if fwd_only:
                with torch.no_grad():
                    TR.per_adapter_forward(x, w, b, As, Bs, scales, off, ids)
            else:
                TR.per_adapter_step(x, w, b, As, Bs, scales, off, ids, dy)

        once()  # warmup
        ts = []
        for _ in range(max(1, reps)):
            t0 = time.perf_counter()
            once()
            ts.append(time.perf_counter() - t0)
        per_shape[(K, N)] = sorted(ts)[len(ts) // 2]
        del x, w, b, As, Bs, dy
    block_s = sum(per_shape[(K, N)] for _, K, N in sample.linears())
    flops = sum((sample.flops_fwd if fwd_only else sample.flops_fwd_bwd)(K, N) for _, K, N in sample.linears())
    shapes = ", ".join(f"{K}->{N} {t * 1e3:.0f} ms" for (K, N), t in per_shape.items())
    return {"value": round(flops / block_s / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{'fwd' if fwd_only else 'fwd+bwd'} of the 6 block linears at {sample.tokens} tokens "
                      f"({'the full configuration' if full else 'scaled-down token count'}, segments "
                      f"{list(lengths)}), fp32 torch per-adapter path; median of {max(1, reps)} after 1 warmup per "
                      f"linear shape ({shapes}); block {block_s * 1e3:.0f} ms; "
                      f"{time.perf_counter() - t_all:.1f} s of CPU work; host os.cpu_count()={os.cpu_count()}"}


if __name__ == "__main__":
    main()
