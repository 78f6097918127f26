#!/usr/bin/env python3
"""Benchmark: LoRA fine-tune tokens/s (fwd + bwd + AdamW) on a quantized base, one MI355X.

Workload: Qwen2.5-0.5B architecture (24 layers, d 896, 14/2 heads, QKV bias,
SwiGLU 4864, vocab 151936, NEOX RoPE 1e6), random-init ~N(0, 0.02) quantized on the device with HOS's own
quantizers to Q4_K (Q8_0 for the 896-wide rows a 256-element super-block cannot tile), LoRA r=16 on all
seven projections, batch 4 x 512 uniform-random tokens, AdamW lr 1e-4. One step = one optimizer step over
the whole batch; inputs are resident in HBM before the timed region.

Also reported: the dominant kernel class against its roofline (HIP events around each of its launches in the
last step of the timed region), the isolated configs[1] dX GEMM (4096^3, Q4_K) against bf16/fp16 MFMA peak, and the CPU
baseline (the oracle's restatement of HOS's CPU training path on this host's cores, a bounded sample).
"""
import argparse
import dataclasses
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MFMA_TFLOPS = 2500.0  # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0
METRIC = "fine-tune tokens/sec (fwd+bwd+AdamW) on Q4_K base; dX-GEMM % MFMA peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="qwen2.5-0.5b")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline sample")
    ap.add_argument("--cpu-seq", type=int, default=512, help="tokens in the CPU baseline sample")
    ap.add_argument("--serial-seq", type=int, default=64,
                    help="tokens of the 1-thread configs[0] (SmolLM2-135M) CPU sample (0: skip)")
    ap.add_argument("--rga", action="store_true",
                    help="train RGA adapters (4 genes of bottleneck 4, lambda 1e-3: cmd_peft's defaults) instead of LoRA")
    ap.add_argument("--finetune", action="store_true",
                    help="time the full-parameter finetune step (FtModel: every weight trainable in f32) instead")
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue the step kernel by kernel instead of replaying its captured HIP graph (for profilers)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of known size (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    return ap.parse_args()


COPY_BYTES = 1 << 30


def copy_calibration():
    """A plain device-to-device copy of COPY_BYTES, three times: under rocprofv3 --pmc its FETCH_SIZE and
    WRITE_SIZE per dispatch against COPY_BYTES give the factor that turns those counters into HBM bytes."""
    import torch
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": COPY_BYTES, "dispatches": 3}), flush=True)


def traffic_per_launch(kernel_class, cfg):
    """HBM bytes per launch of `kernel_class` measured by rocprofv3 FETCH_SIZE + WRITE_SIZE (calibrated
    against a plain copy), read from the committed profile summary of this workload when one exists, with where it
    came from: the file, the source revision it was measured on and that run's average launch time (so a tile-rule
    change that moves the live launch time shows the figure as stale)."""
    path = os.path.join(ROOT, "profiles", f"{kernel_class}_traffic_{cfg.name}_b{cfg.batch}x{cfg.seq}.md")
    if not os.path.exists(path):
        return None, None
    meta = {"file": os.path.relpath(path, ROOT)}
    val = None
    for line in open(path):
        for key in ("bytes_per_launch", "measured_at", "avg_launch_us"):
            if line.startswith(key + ":"):
                v = line.split(":", 1)[1].strip()
                if key == "bytes_per_launch":
                    val = float(v)
                else:
                    meta[key] = float(v) if key == "avg_launch_us" else v
    return val, meta


def config1_probe(gpu):
    """configs[1] on its own shapes: W [4096, 4096] ~N(0, 0.02) -> Q4_K; dX = dY·deq(W) with dY [4096, 4096]
    ~N(0, 1e-2), the forward X·deq(W)ᵀ, both at 1 and 3 precision passes (kernel alone, fp16 operand already
    converted, HIP events), and the LoRA r16 A/B gradient on the same shapes (u = x·A, du = s·dY·Bᵀ,
    dB = s·uᵀ·dY, dA = xᵀ·du: hos_hip_lora without the y / dx products), timed on the context stream.
    Parity of every leg at this size: tests/test_gpu_config1.py."""
    from hos_amd.hip_be import GGML_Q4_K
    T = N = K = 4096
    r = 16
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    gpu.upload_quant(0xD0, gpu.quantize(w, GGML_Q4_K), GGML_Q4_K, N, K)
    dy = (rng.standard_normal((T, N), dtype=np.float32) * np.float32(1e-2))
    x = rng.standard_normal((T, K), dtype=np.float32)
    d_dy, d_x, dout = gpu.alloc(T * N * 4), gpu.alloc(T * K * 4), gpu.alloc(T * max(N, K) * 4)
    gpu.h2d(d_dy, dy)
    gpu.h2d(d_x, x)
    flops = 2.0 * T * N * K
    out = {}
    for leg, which, src in (("dx", 1, d_dy), ("fwd", 0, d_x)):
        for passes in (1, 3):
            gpu.set_gemm_passes(passes)
            ms = gpu.time_qgemm(which, 0xD0, src, T, dout, 20)
            tf = flops / (ms * 1e-3) / 1e12
            out[f"{leg}_passes{passes}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                                            "frac_of_peak": round(tf / PEAK_MFMA_TFLOPS, 4),
                                            "timed": "GEMM kernel alone (operand already fp16)"}
            # the same GEMM from the f32 operand, as the per-op entry point runs it: the f32 -> fp16 row-scaled
            # split (hi, and lo for two-plane modes) plus the GEMM, which is what the 4 B/element f32 dY count of
            # the algorithmic bytes starts from
            entry = "qgemm_dx_dev" if which == 1 else "qgemm_fwd_dev"
            gpu.op_async(entry, 0xD0, src, T, dout)  # warm-up
            gpu.timer_begin()
            for _ in range(20):
                gpu.op_async(entry, 0xD0, src, T, dout)
            ms2 = gpu.timer_end() / 20
            tf2 = flops / (ms2 * 1e-3) / 1e12
            out[f"{leg}_passes{passes}_from_f32"] = {"us": round(ms2 * 1e3, 1), "tflops": round(tf2, 1),
                                                     "frac_of_peak": round(tf2 / PEAK_MFMA_TFLOPS, 4),
                                                     "timed": "f32 -> fp16 operand split + GEMM"}
    gpu.set_gemm_passes(1)
    A = gpu.to_dev(rng.standard_normal((K, r), dtype=np.float32) * np.float32(0.02))
    B = gpu.to_dev(rng.standard_normal((r, N), dtype=np.float32) * np.float32(0.02))
    U, DU_A, DB = gpu.empty_dev((T, r)), gpu.empty_dev((K, r)), gpu.empty_dev((r, N))
    args = (d_x, d_dy, T, K, N, r, A, B, 2.0, None, U, DU_A, DB, None)
    gpu.op_async("lora", *args)  # warm-up
    iters = 20
    gpu.timer_begin()
    for _ in range(iters):
        gpu.op_async("lora", *args)
    ms = gpu.timer_end() / iters
    # algorithmic bytes: x and dY read once each (u, du, dA, dB need nothing else of size)
    nbytes = 4.0 * T * (K + N)
    out["lora_r16_dAdB"] = {"us": round(ms * 1e3, 1), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                            "algorithmic_bytes": int(nbytes)}
    for a in (A, B, U, DU_A, DB):
        a.free()
    for p in (d_dy, d_x, dout):
        gpu.free(p)
    gpu.evict(0xD0)
    return out


QNAME = {8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}


def workload(cfg):
    base = QNAME[cfg.quant] + " base"
    if cfg.quant != 8 and cfg.dim % 256:
        base += f" (Q8_0 for {cfg.dim}-wide rows)"
    if cfg.n_experts:
        base += f"; {cfg.n_experts} experts top-{cfg.n_experts_used}, QK-norm" if cfg.qk_norm else \
            f"; {cfg.n_experts} experts top-{cfg.n_experts_used}"
    if cfg.rga_genes:
        return (f"{cfg.name} RGA {cfg.rga_genes} genes x bottleneck {cfg.rga_bottleneck}, lambda {cfg.rga_lambda:g}; "
                f"{base}; AdamW")
    return f"{cfg.name} LoRA r{cfg.lora_rank} on {','.join(cfg.lora_targets)}; {base}; AdamW"


def cpu_baseline(cfg, tensors, seq, threads=0):
    """The oracle (C++ restatement of HOS's CPU path, OpenMP row-parallel, each element's summation order
    serial) on one sequence of `seq` tokens: forward + backward + AdamW, timed on `threads` host threads
    (0: every thread OpenMP is given)."""
    import types
    from oracle import binding as o
    from hos_amd import synth
    oc = types.SimpleNamespace(**{k: getattr(cfg, k) for k in (
        "n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "rms_eps", "rope_base",
        "rope_neox", "attn_bias", "lora_rank", "lora_alpha", "rga_genes", "rga_bottleneck", "rga_lambda")})
    oc.lora_targets = cfg.target_mask
    prev = o.set_threads(0)
    m = o.OracleModel(oc)
    for name, (raw, t, rows, cols) in tensors.items():
        m.set_tensor(name, raw, t, rows, cols)
    if cfg.is_rga:
        for name, v in synth.rga_init(cfg, seed=5).items():
            m.set_rga(name, v)
    for (l, t), (A, B) in synth.lora_init(cfg, seed=5).items():
        m.set_lora(l, ("q", "k", "v", "o", "gate", "up", "down").index(t), A, B)
    ids, tg = synth.tokens(cfg, 1, seq, seed=8)
    cores = o.set_threads(threads)
    t0 = time.perf_counter()
    m.loss_grad(ids, tg)
    m.adamw(cfg.lr, 0.0)
    dt = time.perf_counter() - t0
    o.set_threads(prev)
    return {"value": round(seq / dt, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{cfg.name}: 1 sequence x {seq} tokens (fwd+bwd+AdamW, micro-batch), {dt:.1f} s"}


def finetune_bench(args):
    """Full-parameter finetune (src/finetune.rs FtModel) tokens/s on the same synthetic workload: every
    weight dequantized once to trainable f32, weight GEMMs on fp16 MFMA in 3 precision passes (f32 operands split
    hi/lo), dW for every matrix, AdamW over all."""
    from hos_amd import Gpu, synth
    from hos_amd.finetune import FtModel
    cfg = synth.CONFIGS[args.config]
    gpu = Gpu(0)
    ft = FtModel(gpu, cfg)
    ft.load(synth.build_tensors(gpu, cfg, seed=1234))
    B, T = cfg.batch, cfg.seq
    ids, tg = synth.tokens(cfg, B, T, seed=8)
    ids_dev, tg_dev, loss_dev = gpu.alloc(ids.nbytes), gpu.alloc(tg.nbytes), gpu.alloc(4)
    gpu.h2d(ids_dev, ids)
    gpu.h2d(tg_dev, tg)
    for _ in range(args.warmup):
        ft.step_dev(ids_dev, tg_dev, B, T, 1e-5, 0.0, loss_dev)
    gpu.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ft.step_dev(ids_dev, tg_dev, B, T, 1e-5, 0.0, loss_dev)
    gpu.synchronize()
    dt = time.perf_counter() - t0
    value = B * T * args.steps / dt
    # every weight trains: 6 flops per parameter per token plus attention
    d, qd, kvd, f, v = cfg.dim, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.ffn_dim, cfg.vocab
    p_mat = cfg.n_layers * (d * qd + 2 * d * kvd + qd * d + 3 * d * f) + d * v
    f_tok = 6 * p_mat + 6 * cfg.n_layers * T * qd
    line = {"metric": "full-finetune tokens/sec (fwd+bwd+AdamW, every weight trainable f32)",
            "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(dt / args.steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32 weights; GEMMs fp16 MFMA hi/lo, 3 passes (~2^-22 per product)",
            "data": "synthetic",
            "config": {"workload": f"{cfg.name} full finetune", "global_batch": B, "seq_len": T,
                       "parallelism": "dp1"},
            "tflops_step": round(value * f_tok / 1e12, 2),
            "mfma_frac_step": round(value * f_tok / 1e12 / 2500.0, 4),
            "loss": round(float(gpu.d2h(loss_dev, (1,), np.float32)[0]), 5)}
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.finetune:
        finetune_bench(args)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path shards as data parallel over sequences: one all-reduce of the LoRA gradient arena per step)", file=sys.stderr)
        sys.exit(2)
    from hos_amd import Gpu, synth
    from hos_amd.peft import PeftModel

    cfg = synth.CONFIGS[args.config]
    if args.rga:  # src/main.rs:1017 (PEFT_GENES / PEFT_BOTTLE defaults), :2559-2562 (PEFT_LAMBDA default)
        cfg = dataclasses.replace(cfg, lora_targets=(), rga_genes=4, rga_bottleneck=4, rga_lambda=1e-3)
    gpu = Gpu(0)
    t_setup = time.perf_counter()
    tensors = synth.build_tensors(gpu, cfg, seed=1234)
    pm = PeftModel(gpu, cfg)
    pm.load(tensors)
    if cfg.is_rga:
        for name, v in synth.rga_init(cfg, seed=5).items():
            pm.set_rga(name, v)
    for (l, t), (A, B) in synth.lora_init(cfg, seed=5).items():
        pm.set_lora(l, t, A, B)
    if args.no_graph:
        pm.use_graph(False)
    B, T = cfg.batch, cfg.seq
    ids, tg = synth.tokens(cfg, B, T, seed=8)
    ids_dev, tg_dev, loss_dev = gpu.alloc(ids.nbytes), gpu.alloc(tg.nbytes), gpu.alloc(4)
    gpu.h2d(ids_dev, ids)
    gpu.h2d(tg_dev, tg)
    setup_s = time.perf_counter() - t_setup
    print(f"[bench] setup {setup_s:.1f}s", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        pm.step_dev(ids_dev, tg_dev, B, T, cfg.lr, 0.0, loss_dev)
    gpu.synchronize()

    classes = ["qgemm_fwd", "qgemm_dx", "lora_down", "lora_du", "lora_dab", "attn_fwd", "attn_bwd",
               "rmsnorm", "swiglu", "rope", "ce", "adamw", "embed", "convert", "moe_route", "moe_combine", "rga"]
    # Breakdown pass (every kernel class timed with HIP events; not the timed region): finds the
    # dominant class and gives the per-class split.
    pm.profile(True)
    for _ in range(args.steps):
        pm.step_dev(ids_dev, tg_dev, B, T, cfg.lr, 0.0, loss_dev)
    gpu.synchronize()
    brk = {c: pm.kernel_stats(c) for c in classes}
    pm.profile(False)
    dom = max(brk, key=lambda c: brk[c]["ms"])

    # Timed region. The roofline's kernel class is timed with HIP events around each of its launches in
    # the last timed step (one full step's launches; events in every step would cost ~4% of the step).
    gpu.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if i == args.steps - 1:
            pm.profile(True, only=dom)
        pm.step_dev(ids_dev, tg_dev, B, T, cfg.lr, 0.0, loss_dev)
    gpu.synchronize()
    dt = time.perf_counter() - t0
    loss = float(gpu.d2h(loss_dev, (1,), np.float32)[0])
    ds = pm.kernel_stats(dom)
    pm.profile(False)

    toks = B * T * args.steps
    value = toks / dt
    ms_step = dt / args.steps * 1e3
    f_tok = synth.algorithmic_flops_per_token(cfg, T)
    kernel_ms = {c: round(s["ms"] / args.steps, 3) for c, s in brk.items()}
    avg_launch_s = ds["ms"] / max(ds["launches"], 1) * 1e-3  # over the last timed step
    traffic, tsrc = traffic_per_launch(dom, cfg)
    if tsrc and "avg_launch_us" in tsrc:
        # the counter run's launches against this run's: a >15% move means the kernels changed since the profile
        tsrc["stale"] = abs(avg_launch_s * 1e6 / tsrc["avg_launch_us"] - 1.0) > 0.15
    if ds["flops"] > 0:
        achieved = ds["flops"] / max(ds["launches"], 1) / avg_launch_s / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_MFMA_TFLOPS, 4), "traffic": traffic, "traffic_source": tsrc,
                "kernel": dom, "avg_launch_us": round(avg_launch_s * 1e6, 2), "launches_per_step": ds["launches"]}
    else:
        achieved = ds["bytes"] / max(ds["launches"], 1) / avg_launch_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic, "traffic_source": tsrc,
                "kernel": dom, "avg_launch_us": round(avg_launch_s * 1e6, 2), "launches_per_step": ds["launches"]}

    c1 = config1_probe(gpu)
    cpu = serial = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, tensors, args.cpu_seq)
        if args.serial_seq > 0:  # the reference's training matmul is single-threaded (src/tensor.rs:319-378)
            c0 = synth.CONFIGS["smollm2-135m"]
            serial = cpu_baseline(c0, synth.build_tensors(gpu, c0, seed=1234), args.serial_seq, threads=1)
    line = {
        "metric": METRIC + (" [RGA adapters]" if cfg.is_rga else ""), "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16 MFMA (hi/lo split: 3 passes per layer GEMM, 1-2 on the head) + f32", "data": "synthetic",
        "config": {"workload": workload(cfg), "global_batch": B, "seq_len": T,
                   "parallelism": "dp1", "precision": "layer fwd mode 5 (integer-code kernel for large Q8_0 forwards, else 3-pass: mode-3 precision), "
                                "layer dX 3-pass, head fwd 1-pass, head dX weight-split (mode 4)"},
        "roofline": roof,
        "mfma_roofline_frac_step": round(value * f_tok / 1e12 / PEAK_MFMA_TFLOPS, 4),
        "config1_4096cubed_q4k": c1,
        "cpu_baseline": cpu,
        "cpu_serial_config0": serial,
        "gpu_over_cpu": round(value / cpu["value"], 1) if cpu else None,
        "kernel_ms_per_step": kernel_ms,
        "loss": round(loss, 5),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
