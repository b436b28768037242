"""Benchmark: one Wan2.2-A14B DiT forward (40 blocks) at 32760 video tokens on one MI355X.

Workload: 40 Wan2.2-A14B blocks (dim 5120, 40 heads x 128, FFN 13824), S = 32760 tokens
(21x30x52 latent grid, 480x832x81 frames), 512 text tokens, MXFP8 projections and bf16 constant-max
attention, one CFG branch, cross-attention K/V cached (projected once before timing, as the
reference does per generation), the RoPE tables built inside every timed forward (as the reference
builds them per forward). After the metric the same 40 blocks are timed through the reference's own
FP8 recipe (ROW activations, drop-ins composed as its modules call them; ``row_recipe``) and the
40-block forward is measured at 720p (21x45x80 = 75600 tokens; ``p720``). Random N(0, 0.02)
weights (q/k RMSNorm gammas N(1, 0.02)), seeded N(0, 1) latent tokens, text context and timestep
modulation -- synthetic data.

Prints one JSON line. ``value`` is milliseconds per DiT step (lower is better). The roofline entry
is the dominant kernel (self-attention), timed by HIP events around each of its launches inside the
timed steps; the other kernels' times come from events around every launch of one more forward
after the timed steps (events around every launch would add about 2.5 ms to the step). The CPU
baseline is the reference's BF16 eager block (restated in the oracle) timed on this host's cores at
the 1560-token block shape, extrapolated to the step.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

DIM, HEADS, HEAD_DIM, FFN, TXT = 5120, 40, 128, 13824, 512
PEAK_BF16_TFLOPS, PEAK_FP8_TFLOPS, PEAK_HBM_GBS = 2500.0, 5000.0, 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--grid", type=str, default="21,30,52", help="latent patch grid F,H,W")
    p.add_argument("--blocks", type=int, default=40)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-720p", action="store_true", help="skip the 720p (21x45x80) 40-block step timing")
    p.add_argument("--no-row", action="store_true", help="skip the ROW-activation (reference recipe) step timing")
    p.add_argument("--pmc-calibration", action="store_true",
                   help="also run one 256 MiB device copy, the known-size reference for HBM counters")
    return p.parse_args()


def load_traffic(seq_len):
    """HBM bytes per self-attention launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (scaled by the same counters on a known-size copy); committed under profiles/. None unless the
    measurement was taken at this sequence length."""
    path = os.path.join(ROOT, "profiles", "self_attention_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if line.lstrip().startswith("#"):
                continue
            key, _, val = line.partition("=")
            if val.strip():
                vals[key.strip()] = float(val)
    if vals.get("seq_len") != seq_len:
        return None
    return vals.get("self_attention_bytes_per_launch")


class KernelTimer:
    """Records HIP events (on the launching stream) around the kernel calls named in `only` (every
    call when None) while active.

    Events around every launch of the 40-block forward cost about 2.5 ms per step (one process,
    four interleaved two-step runs each: 988.7 ms with events around every launch, 987.0 around the
    self-attention only, 986.1 with none), so the timed steps record only the self-attention (the
    roofline kernel) and the other kernels are timed in one instrumented forward after them
    (`instrumented`)."""

    def __init__(self, only=None):
        self.active = False
        self.only = only
        self.events = {}

    def __call__(self, name, fn):
        if not self.active or (self.only is not None and name not in self.only):
            return fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        r = fn()
        e.record()
        self.events.setdefault(name, []).append((s, e))
        return r

    def summary(self):
        return {k: [s.elapsed_time(e) for s, e in v] for k, v in self.events.items()}


def instrumented(forward):
    """One more forward after the timed steps with events around every kernel call: the components'
    per-launch times (each list holds one entry per launch of that forward)."""
    timer = KernelTimer()
    timer.active = True
    forward(timer)
    torch.cuda.synchronize()
    return timer.summary()


def gemm_flops(S):
    return 2 * S * (DIM * 3 * DIM + DIM * DIM + DIM * DIM + DIM * DIM + 2 * DIM * FFN)


def cpu_baseline(S_full, blocks):
    """Reference BF16 eager block on the host CPU at the 1560-token shape; extrapolated to the
    step: projections/FFN/cross-attention linearly in S, self-attention quadratically."""
    from oracle import block as oblock

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    grid = (1, 30, 52)
    S = 1560
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    raw = {
        "scale_shift_table": torch.randn(6, DIM, generator=g) * 0.02,
        "qkv_w": (torch.randn(DIM, 3 * DIM, generator=g) * 0.02).to(bf), "qkv_b": torch.randn(3 * DIM, generator=g) * 0.02,
        "norm_q": 1 + torch.randn(DIM, generator=g) * 0.02, "norm_k": 1 + torch.randn(DIM, generator=g) * 0.02,
        "o_w": (torch.randn(DIM, DIM, generator=g) * 0.02).to(bf), "o_b": torch.randn(DIM, generator=g) * 0.02,
        "norm2_weight": torch.randn(DIM, generator=g) * 0.02, "norm2_bias": torch.randn(DIM, generator=g) * 0.02,
        "q2_w": (torch.randn(DIM, DIM, generator=g) * 0.02).to(bf), "q2_b": torch.randn(DIM, generator=g) * 0.02,
        "k2_w": (torch.randn(DIM, DIM, generator=g) * 0.02).to(bf), "k2_b": torch.randn(DIM, generator=g) * 0.02,
        "v2_w": (torch.randn(DIM, DIM, generator=g) * 0.02).to(bf), "v2_b": torch.randn(DIM, generator=g) * 0.02,
        "norm_q2": 1 + torch.randn(DIM, generator=g) * 0.02, "norm_k2": 1 + torch.randn(DIM, generator=g) * 0.02,
        "o2_w": (torch.randn(DIM, DIM, generator=g) * 0.02).to(bf), "o2_b": torch.randn(DIM, generator=g) * 0.02,
        "up_w": (torch.randn(DIM, FFN, generator=g) * 0.02).to(bf), "up_b": torch.randn(FFN, generator=g) * 0.02,
        "down_w": (torch.randn(FFN, DIM, generator=g) * 0.02).to(bf), "down_b": torch.randn(DIM, generator=g) * 0.02,
    }
    h = torch.randn(S, DIM, generator=g).to(bf)
    temb = torch.randn(6, DIM, generator=g)
    ctx = torch.randn(TXT, DIM, generator=g).to(bf)

    def run_block():
        return oblock.bf16_eager_block(raw, h, temb, ctx, grid)

    q = torch.randn(1, HEADS, S, HEAD_DIM, generator=g).to(bf)

    def run_self_attn():  # the block's self-attention core alone (_torch_attend on [B, N, S, D])
        sc = torch.matmul(q.float() * HEAD_DIM**-0.5, q.float().transpose(-2, -1))
        return torch.matmul(torch.softmax(sc, dim=-1), q.float()).to(bf)

    def med(fn, n=3):
        fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    t_block = med(run_block)
    t_attn = min(med(run_self_attn), t_block)
    r = S_full / S
    step_ms = blocks * ((t_block - t_attn) * r + t_attn * r * r) * 1000.0
    return {
        "value": round(step_ms, 1),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (f"reference BF16 eager block (oracle restatement: _eager_adaln, torch.matmul, "
                   f"DistributedRMSNorm, RoPE, _torch_attend, GELU-tanh FFN) at S=1560 (1x30x52), 512 text "
                   f"tokens, median of 3 after 1 warm-up: {t_block * 1000:.0f} ms/block, of which self-attention "
                   f"{t_attn * 1000:.0f} ms; extrapolated to {blocks} blocks at S={S_full} (self-attention x{r * r:.0f}, "
                   f"the rest x{r:.1f})"),
    }


def step_720p(pkg, blocks, crosses, tables, temb, dev, steps=2, warmup=1):
    """The 40-block forward at the 720p step's length (21x45x80 = 75600 tokens, 512 text tokens, the
    same weights and cached text K/V), measured after the main metric: `warmup` untimed forwards,
    then `steps` timed ones bracketed by device synchronizations (HIP events around the
    self-attention only), then one instrumented forward for the other kernels' times."""
    blk = pkg.block
    grid = (21, 45, 80)
    S7 = grid[0] * grid[1] * grid[2]
    gen = torch.Generator(device=dev).manual_seed(720)
    h = torch.randn(S7, DIM, device=dev, generator=gen).to(torch.bfloat16)
    for _ in range(warmup):
        blk.dit_forward(blocks, h, temb, grid, crosses, tables=tables)
    timer = KernelTimer(only={"self_attention"})
    timer.active = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = blk.dit_forward(blocks, h, temb, grid, crosses, timer=timer, tables=tables)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite 720p DiT output")
    attn = timer.summary()["self_attention"]
    attn_ms = sum(attn) / len(attn)
    times = instrumented(lambda t: blk.dit_forward(blocks, h, temb, grid, crosses, timer=t, tables=tables))
    comp = {k: round(sum(v), 2) for k, v in sorted(times.items())}
    gemm_ms = sum(sum(v) for k, v in times.items() if k.startswith("gemm_")) / len(blocks)
    return {
        "workload": f"Wan2.2-A14B DiT forward at 720p: {len(blocks)} blocks, 21x45x80 = 75600 tokens, 512 text tokens",
        "seq_len": S7, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 1),
        "self_attention_tflops": round(4.0 * S7 * S7 * HEAD_DIM * HEADS / attn_ms / 1e9, 1),
        "gemm_tflops": round(gemm_flops(S7) / gemm_ms / 1e9, 1),
        "components_ms_per_step": comp,
    }


def row_recipe_step(pkg, row_blocks, row_crosses, tables, temb, h0, grid, steps=2, warmup=1):
    """The reference's own FP8 recipe (ROW activations at every adaLN site, per-tensor FP8 weights
    with per-channel scales, the drop-ins composed as its FP8 modules call them) over the same 40
    blocks at the metric's length: `warmup` untimed forwards, then `steps` timed ones bracketed by
    device synchronizations, then one instrumented forward for the per-drop-in times."""
    rb = pkg.row_block
    for _ in range(warmup):
        rb.row_dit_forward(row_blocks, h0, temb, grid, row_crosses, tables=tables)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = rb.row_dit_forward(row_blocks, h0, temb, grid, row_crosses, tables=tables)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite ROW-recipe DiT output")
    times = instrumented(lambda t: rb.row_dit_forward(row_blocks, h0, temb, grid, row_crosses, timer=t, tables=tables))
    comp = {k: round(sum(v), 2) for k, v in sorted(times.items())}
    return {
        "workload": (f"the reference's FP8 block recipe (ROW activations, per-tensor FP8 weights with per-channel "
                     f"scales, drop-ins composed as row_mx_modules.py calls them), {len(row_blocks)} blocks at "
                     f"S={h0.shape[0]}"),
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 1), "components_ms_per_step": comp,
    }


def copy_ceiling(pkg, traffic_bytes, adaln_gbs, reps=20):
    """The practical HBM streaming rate on this box, beside the nominal 8 TB/s: a copy moving the
    adaLN launch's bytes (half read, half written) through the library's streaming copy kernel
    (16-byte loads, eight per thread in flight, non-temporal stores) and through torch's generic
    device copy for comparison, and the library's read-2-write-1 pass over the same bytes (the
    adaLN pass's own mix), each timed with HIP events over `reps` launches."""
    n = traffic_bytes // 2 // 16 * 16
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)

    def rate(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        return ms, 2 * n / ms / 1e6

    ms_k, gbs_k = rate(lambda: pkg._lib.hbm_stream_copy(dst, src))
    if not torch.equal(dst, src):
        raise RuntimeError("streaming copy mismatch")
    ms_t, gbs_t = rate(lambda: dst.copy_(src))
    del src, dst
    # the adaLN pass's own mix: two bytes read per byte written (bf16 in, e4m3 out)
    nf = traffic_bytes * 2 // 3 // 32768 * 32768
    src = torch.empty(nf, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty(nf // 2, dtype=torch.uint8, device="cuda")
    ms_f, _ = rate(lambda: pkg._lib.hbm_stream_fold(dst, src))
    gbs_f = (nf + nf // 2) / ms_f / 1e6
    del src, dst
    return {"bytes_per_copy": 2 * n, "ms_per_copy": round(ms_k, 4), "gbs": round(gbs_k, 1),
            "adaln_frac_of_copy": round(adaln_gbs / gbs_k, 3), "torch_copy_gbs": round(gbs_t, 1),
            "read2_write1_bytes": nf + nf // 2, "read2_write1_gbs": round(gbs_f, 1),
            "adaln_frac_of_read2_write1": round(adaln_gbs / gbs_f, 3)}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} requested, but this build runs on one GPU only "
              "(no collectives or sharding); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    pkg = __graft_entry__.load_package()

    dev = torch.device("cuda:0")
    grid = tuple(int(x) for x in args.grid.split(","))
    S = grid[0] * grid[1] * grid[2]
    blk, ops = pkg.block, pkg.attention_ops

    gen = torch.Generator(device=dev).manual_seed(2024)
    blocks, row_blocks = [], []
    for _ in range(args.blocks):
        w, raw = blk.random_block_weights(dev, gen, qk_gamma_mean=1.0, keep_raw=not args.no_row)
        blocks.append(w)
        if not args.no_row:  # the same weights as the checkpoint's per-tensor FP8 form
            row_blocks.append(pkg.row_block.row_block_weights(raw)[0])
        del raw
    h0 = torch.randn(S, DIM, device=dev, generator=gen).to(torch.bfloat16)
    temb = torch.randn(6, DIM, device=dev, generator=gen)
    ctx = torch.randn(TXT, DIM, device=dev, generator=gen).to(torch.bfloat16)
    crosses = [blk.project_cross_kv(w, ctx) for w in blocks]
    tables = torch.stack([w.scale_shift_table for w in blocks])
    torch.cuda.synchronize()

    if args.pmc_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    timer = KernelTimer(only={"self_attention"})  # the roofline kernel, timed live in the timed steps
    for _ in range(args.warmup):
        blk.dit_forward(blocks, h0, temb, grid, crosses, tables=tables)
    torch.cuda.synchronize()

    timer.active = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = blk.dit_forward(blocks, h0, temb, grid, crosses, timer=timer, tables=tables)
    torch.cuda.synchronize()
    total_ms = (time.perf_counter() - t0) * 1000.0
    timer.active = False
    ms_step = total_ms / args.steps
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite DiT output")

    attn = timer.summary()["self_attention"]
    attn_flops = 4.0 * S * S * HEAD_DIM * HEADS
    attn_ms = sum(attn) / len(attn)
    attn_tflops = attn_flops / attn_ms / 1e9
    # every other kernel: one instrumented forward after the timed steps
    times = instrumented(lambda t: blk.dit_forward(blocks, h0, temb, grid, crosses, timer=t, tables=tables))
    gemm_names = [k for k in times if k.startswith("gemm_")]
    gemm_ms = sum(sum(times[k]) for k in gemm_names) / args.blocks
    gemm_tflops = gemm_flops(S) / gemm_ms / 1e9
    # adaLN: every launch reads x (bf16) and the two modulation / affine vectors and writes MX codes
    # and scales (the residual adds run in the GEMM epilogues)
    plain = 2 * S * DIM + S * DIM + S * DIM // 32 + 2 * DIM * 4
    ad = times["adaln"]
    adaln_gbs = plain * len(ad) / sum(ad) / 1e6
    first_adaln_us = sum(ad[0::3]) / len(ad[0::3]) * 1000.0
    comp = {k: {"ms_per_launch": round(sum(v) / len(v), 4), "ms_per_step": round(sum(v), 2)}
            for k, v in sorted(times.items())}
    # the self-attention entry from the timed steps' own events
    comp["self_attention"] = {"ms_per_launch": round(attn_ms, 4), "ms_per_step": round(sum(attn) / args.steps, 2)}

    result = {
        "metric": "DiT step ms @32760 tok (A14B); attn+GEMM TFLOP/s; adaLN-quant GB/s",
        "value": round(ms_step, 2),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp8 projections (fp32 acc) + bf16 attention (fp32 acc)",
        "data": "synthetic (seeded N(0,1) activations, random N(0,0.02) weights)",
        "config": {
            "workload": "Wan2.2-A14B DiT forward: 40 blocks, one CFG branch, cross-attn K/V cached",
            "seq_len": S, "grid": list(grid), "blocks": args.blocks, "text_tokens": TXT, "dim": DIM,
            "heads": HEADS, "head_dim": HEAD_DIM, "ffn": FFN, "parallelism": "none (1 GPU)",
        },
        "attn_tflops": round(attn_tflops, 1),
        "gemm_tflops": round(gemm_tflops, 1),
        "adaln_quant_gbs": round(adaln_gbs, 1),
        "adaln_quant_plain_us": round(first_adaln_us, 1),
        "components": comp,
        "roofline": {
            "kernel": f"attention_const_max_kernel (self-attention, S={S}, {HEADS} heads x {HEAD_DIM})",
            "bound": "mfma",
            "achieved": round(attn_tflops, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": load_traffic(S),
        },
    }
    result["hbm_copy_ceiling"] = copy_ceiling(pkg, plain, result["adaln_quant_gbs"])
    if not args.no_row:
        row_crosses = [pkg.row_block.project_cross_kv_row(w, ctx) for w in row_blocks]
        result["row_recipe"] = row_recipe_step(pkg, row_blocks, row_crosses, tables, temb, h0, grid)
        del row_blocks, row_crosses
    if not args.no_720p:
        result["p720"] = step_720p(pkg, blocks, crosses, tables, temb, dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(S, args.blocks)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
