"""Benchmark: GPTQ W4A16-g128 of one 4096 x 4096 layer (Hessian + solve) on
one MI355X, plus MXFP4 quantize+pack bandwidth.

A step is one pass of the hot path over one batch of synthetic input:
``make_empty_hessian`` -> ``accumulate_hessian`` over X [64, 2048, 4096]
(bf16, heavy-tailed) -> weight observer -> GPTQ solve (damping, Cholesky
chain, blocked sweep, lazy trailing updates) -> fake-quantised bf16 weight,
scales and integer codes.  Inputs are generated on the GPU (seeded) and are
resident in HBM before timing starts.

Prints ONE JSON line (rank 0).  ``value`` is ms per layer (lower is better).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llm-compressor_amd"))
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

ROWS = COLS = 4096
BATCHES, SEQ = 64, 2048
GROUP = 128


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=5)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--hessian-calls", type=int, default=1,
                   help="split the 64 x 2048 calibration tokens into this many accumulate_hessian calls")
    return p.parse_args()


def gen_inputs(torch, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    w = torch.randn(ROWS, COLS, generator=g, device=dev) * 0.02
    idx = torch.randperm(ROWS * COLS, generator=g, device=dev)[: ROWS * COLS // 1000]
    w.view(-1)[idx] *= 10.0
    w = w.to(torch.bfloat16)
    c = torch.exp(torch.randn(COLS, generator=g, device=dev))
    x = torch.empty(BATCHES, SEQ, COLS, dtype=torch.bfloat16, device=dev)
    for b in range(BATCHES):  # Student-t(4) * lognormal channel scale
        z = torch.randn(SEQ, COLS, generator=g, device=dev)
        chi = sum(torch.randn(SEQ, COLS, generator=g, device=dev) ** 2 for _ in range(4))
        x[b] = (z / torch.sqrt(chi / 4.0) * c).to(torch.bfloat16)
    return w, x


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (the hot path is measured on "
                                   "one GPU's share; the multi-GPU sharding is described, not run)"}))
        sys.exit(2)
    import torch

    from llmcompressor_amd import _lib, gptq, ops
    from llmcompressor_amd.observers import Observer
    from llmcompressor_amd.quant_args import QuantizationArgs

    _lib.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w, x = gen_inputs(torch, dev)
    lin = torch.nn.Linear(COLS, ROWS, bias=False, device=dev, dtype=torch.bfloat16)
    lin.weight.data = w
    qa = QuantizationArgs(num_bits=4, type="int", symmetric=True, strategy="group", group_size=GROUP)
    chunks = torch.chunk(x, a.hessian_calls, dim=0)
    stream = torch.cuda.current_stream()

    def step(ev=None):
        H = gptq.make_empty_hessian(lin)
        n = torch.zeros((), device=dev)
        if ev: ev[0].record(stream)
        for ch in chunks:
            H, n = gptq.accumulate_hessian(ch, lin, H, n)
        if ev: ev[1].record(stream)
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(lin.weight)
        res = gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(BATCHES))
        if ev: ev[2].record(stream)
        return res

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(a.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        res = step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / a.steps
    hess_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / a.steps
    solve_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / a.steps

    # full-size sanity: codes in range, dequantised weight = bf16(code * scale)
    codes = res.codes
    assert int(codes.min()) >= -8 and int(codes.max()) <= 7
    sc = res.scale.float().repeat_interleave(GROUP, dim=1)
    assert torch.equal((codes.float() * sc).to(torch.bfloat16), res.weight)

    # Hessian kernel alone (syrk + split reduction), HIP events on its stream
    H = torch.zeros(COLS, COLS, device=dev)
    xf = x.reshape(-1, COLS)
    for _ in range(2):
        ops.hessian_syrk_(H, xf)
    reps = 5
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        ops.hessian_syrk_(H, xf)
    e1.record(stream)
    torch.cuda.synchronize()
    syrk_ms = e0.elapsed_time(e1) / reps
    n_tok = BATCHES * SEQ
    syrk_flop = n_tok * COLS * (COLS + 1)  # upper triangle incl. diagonal, 2 flop / MAC
    syrk_tflops = syrk_flop / (syrk_ms * 1e-3) / 1e12

    # MXFP4 quantize + pack (config: W 4096 x 14336, A 8192 x 14336)
    mx = {}
    for name, shape in (("W", (4096, 14336)), ("A", (8192, 14336))):
        g = torch.Generator(device=dev)
        g.manual_seed(2 if name == "W" else 3)
        t = (torch.randn(shape, generator=g, device=dev) * (0.015 if name == "W" else 1.0)).to(torch.bfloat16)
        out = (torch.empty(shape[0], shape[1] // 2, dtype=torch.uint8, device=dev),
               torch.empty(shape[0], shape[1] // 32, dtype=torch.uint8, device=dev))
        for _ in range(3):
            ops.mxfp4_quantize_pack(t, out=out)
        r = 20
        e0.record(stream)
        for _ in range(r):
            ops.mxfp4_quantize_pack(t, out=out)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / r
        nbytes = t.numel() * 2.53125
        mx[name] = {"ms": round(ms, 5), "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": int(nbytes)}
        del t, out

    # plain elementwise copy of 1 GiB (read 1 GiB, write 1 GiB): measured
    # copy bandwidth, and the known-size kernel that scales the FETCH_SIZE /
    # WRITE_SIZE counters
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)
    e0.record(stream)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    e1.record(stream)
    torch.cuda.synchronize()
    copy_ms = e0.elapsed_time(e1) / 3
    copy_gbs = 2 * src.numel() * 4 / (copy_ms * 1e-3) / 1e9
    del src, dst

    traffic = None
    tf = ROOT / "profiles" / "hessian_syrk_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("bytes_per_launch")

    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(torch, w.cpu(), x[:4].cpu())

    line = {
        "metric": "GPTQ ms/layer (W4A16 g128, 4096x4096, Hessian over 64x2048 tokens + solve)",
        "value": round(ms_step, 3),
        "unit": "ms/layer",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 inputs, fp32 accumulate/solve",
        "data": "synthetic (seeded; W 0.02*N(0,1) with 0.1% x10, X Student-t(4) x lognormal channel scale)",
        "config": {"workload": "gptq_w4a16_g128_4096x4096_64x2048tok", "rows": ROWS, "cols": COLS,
                   "tokens": n_tok, "group_size": GROUP, "blocksize": 128, "damp": 0.01, "actorder": None,
                   "hessian_calls": a.hessian_calls},
        "phases_ms": {"hessian": round(hess_ms, 3), "solve": round(solve_ms, 3)},
        "hessian": {"kernel_ms": round(syrk_ms, 4), "tflops": round(syrk_tflops, 1),
                    "frac_fp32_mfma_peak": round(syrk_tflops / PEAK_FP32_MFMA_TFLOPS, 3),
                    "frac_bf16_mfma_peak": round(syrk_tflops / PEAK_BF16_TFLOPS, 4)},
        "mxfp4_quantize_pack": mx,
        "copy_1GiB_GB_s": round(copy_gbs, 1),
        "roofline": {"bound": "mfma", "achieved": round(syrk_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(syrk_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "kernel": "syrk_stream_kernel + syrk_reduce_kernel (Hessian, 131072 tokens)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(torch, w_cpu, x_sample):
    """The oracle (torch-CPU restatement of the reference) on the host cores.

    Sample: Hessian over 4 x 2048 tokens (scaled to the layer's 64 x 2048)
    plus one full 4096 x 4096 oracle solve."""
    from oracle import gptq as og
    from oracle.qargs import OArgs

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t0 = time.perf_counter()
    H, n = og.accumulate_hessian(x_sample, og.make_empty_hessian(COLS), torch.zeros(()))
    t_h = time.perf_counter() - t0
    scale = (BATCHES * SEQ) / (x_sample.shape[0] * x_sample.shape[1])
    t0 = time.perf_counter()
    og.quantize_weight(w_cpu, OArgs(num_bits=4, strategy="group", group_size=GROUP), og.normalise_hessian(H, n))
    t_s = time.perf_counter() - t0
    return {"value": round((t_h * scale + t_s) * 1e3, 1), "unit": "ms/layer", "cores": cores, "kind": "port",
            "sample": f"Hessian over {x_sample.shape[0]}x{x_sample.shape[1]} tokens x{scale:g} + one full "
                      f"{ROWS}x{COLS} GPTQ solve (oracle, torch-CPU MKL)",
            "hessian_ms_scaled": round(t_h * scale * 1e3, 1), "solve_ms": round(t_s * 1e3, 1)}


if __name__ == "__main__":
    main()
