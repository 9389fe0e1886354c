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
    p.add_argument("--headline-only", action="store_true",
                   help="skip the W8A8, MoE and decoder-layer workloads the default line also reports")
    p.add_argument("--hessian-calls", type=int, default=1,
                   help="split the 64 x 2048 calibration tokens into this many accumulate_hessian calls")
    p.add_argument("--workload", default="gptq_w4a16",
                   choices=["gptq_w4a16", "mxfp4", "gptq_w8a8", "moe", "decoder", "sparsegpt", "mse_observer",
                            "pipeline", "torch_reference"],
                   help="gptq_w4a16 (default): the headline line; the others measure the remaining "
                        "calibration workloads (MXFP4 pack, W8A8 channel + actorder, MoE experts, "
                        "Llama-3-8B-shaped decoder layer, SparseGPT 50 %% / 2:4 on a 4096x4096 layer, "
                        "MSE weight observer on 4096x4096 and 14336x4096, sequential pipeline over two "
                        "Llama-3-8B-shaped layers); torch_reference times the reference's algorithm as "
                        "plain torch ops on the same GPU beside this library on the headline layer")
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
    if a.workload != "gptq_w4a16":
        OTHER_WORKLOADS[a.workload](a)
        return
    import torch

    from llmcompressor_amd import _lib, gptq, ops
    from llmcompressor_amd.observers import Observer
    from llmcompressor_amd.quant_args import QuantizationArgs
    from llmcompressor_amd.staging import HessianStage

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
        return res, H

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(a.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        res, H_last = step(evs[i])
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

    # the dominant kernel: the Hessian call (stream + reduction kernels) of
    # each timed step, HIP events on the kernels' stream around it
    n_tok = BATCHES * SEQ
    syrk_flop = n_tok * COLS * (COLS + 1)  # upper triangle incl. diagonal, 2 flop / MAC
    syrk_ms = hess_ms
    syrk_tflops = syrk_flop / (syrk_ms * 1e-3) / 1e12
    xf = x.reshape(-1, COLS)
    reps = 5

    # the reference's per-batch calling pattern (batch_size=1 calibration:
    # one accumulate_hessian call per 2048-token sample, 64 calls)
    chunks64 = torch.chunk(x, BATCHES, dim=0)
    H64 = gptq.make_empty_hessian(lin)
    n64 = torch.zeros((), device=dev)
    for ch in chunks64:
        H64, n64 = gptq.accumulate_hessian(ch, lin, H64, n64)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps64 = 10   # each pass is a few ms: fewer repetitions time the clock ramp more than the path
    e0.record(stream)
    for _ in range(reps64):
        H64.zero_()
        for ch in chunks64:
            H64, n64 = gptq.accumulate_hessian(ch, lin, H64, n64)
    e1.record(stream)
    torch.cuda.synchronize()
    h64_ms = e0.elapsed_time(e1) / reps64
    h64_rel = ((torch.triu(H64) - torch.triu(H_last)).norm() / torch.triu(H_last).norm()).item()
    del H64

    # the same 64 calls through the modifiers' forward hook, which holds the
    # calls' rows (by reference) and accumulates them 131072 rows at a time in
    # one segmented syrk; each call's input is a tensor of its own, as a
    # forward pass makes it (a view into one 1 GiB tensor would be copied)
    calls64 = [ch.clone() for ch in chunks64]
    Hs = gptq.make_empty_hessian(lin)
    ns = torch.zeros((), device=dev)
    stage = HessianStage()

    def flush(segs, samples):
        ops.hessian_syrk_segments_(Hs, segs, alpha=2.0)
        ns.add_(samples)

    def staged_calls():
        for ch in calls64:
            rows, added = gptq.hessian_rows(ch, lin, dev)
            stage.add(rows, added, flush)
        stage.flush(flush)

    for _ in range(2):
        staged_calls()
    e0.record(stream)
    for _ in range(reps64):
        Hs.zero_()
        staged_calls()
    e1.record(stream)
    torch.cuda.synchronize()
    hs_ms = e0.elapsed_time(e1) / reps64
    hs_rel = ((torch.triu(Hs) - torch.triu(H_last)).norm() / torch.triu(H_last).norm()).item()
    stage.release()
    del Hs, calls64

    # vendor GEMM on the same product: torch.mm (hipBLASLt) of X^T X as the
    # full 4096 x 4096 square with a bf16 result (twice the multiply-adds of
    # the triangle, half the output precision)
    xt = xf.t().contiguous()
    for _ in range(2):
        torch.mm(xt, xf)
    e0.record(stream)
    for _ in range(reps):
        torch.mm(xt, xf)
    e1.record(stream)
    torch.cuda.synchronize()
    mm_ms = e0.elapsed_time(e1) / reps
    mm_tflops = 2 * n_tok * COLS * COLS / (mm_ms * 1e-3) / 1e12
    del xt

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

    # counters of the same kernels (rocprofv3 --pmc passes, commands in the file)
    traffic = counters = None
    tf = ROOT / "profiles" / "hessian_syrk_counters.json"
    if tf.exists():
        pmc = json.loads(tf.read_text())
        traffic = pmc.get("bytes_per_launch")
        counters = {"file": "profiles/hessian_syrk_counters.json",
                    **{k: pmc.get(k) for k in ("algorithmic_bytes_per_launch", "mfma_busy_frac", "sclk_ghz_avg",
                                               "mfma_instructions", "mfma_bf16_flop_issued",
                                               "lds_instructions_per_mfma", "lds_bank_conflict_cycles")}}

    cpu = parity = None
    if not a.no_cpu_baseline:
        cpu, parity = cpu_baseline(torch, w.cpu(), x[:16].cpu(), H_last.cpu(), res)

    # the W8A8, MoE and decoder-layer configurations, two timed steps each
    # after one warm-up, reported inside this line (each also has its own
    # --workload line)
    others = None
    if not a.headline_only:
        global _COLLECT
        del x, xf, w, lin, res, H_last, chunks, chunks64
        torch.cuda.empty_cache()
        _COLLECT = []
        sub = argparse.Namespace(**{**vars(a), "steps": 2, "warmup": 1})
        for fn in (bench_w8a8, bench_moe, bench_decoder):
            fn(sub)
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        others = {}
        for ln in _COLLECT:
            others[ln["config"]["workload"]] = {k: ln[k] for k in ("metric", "value", "unit", "steps", "warmup")
                                                if k in ln}
            for k in ("phases_ms", "hessian", "act_quant_int8_per_token", "tokens_per_expert", "modifier_path"):
                if k in ln:
                    others[ln["config"]["workload"]][k] = ln[k]
        _COLLECT = None

    line = {
        "metric": ("GPTQ ms/layer (W4A16 g128, 4096x4096: Hessian of 64x2048 tokens in "
                   + ("one accumulate_hessian call" if a.hessian_calls == 1 else f"{a.hessian_calls} calls")
                   + " + solve)"),
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
        # the same layer calibrated through the modifiers' forward hook (64
        # calls of one 2048-token sample, staged): its Hessian time plus the solve
        "hook_path_ms_per_layer": round(hs_ms + solve_ms, 3),
        "hessian": {"ms": round(syrk_ms, 4), "tflops": round(syrk_tflops, 1),
                    "frac_fp32_mfma_peak": round(syrk_tflops / PEAK_FP32_MFMA_TFLOPS, 3),
                    "frac_bf16_mfma_peak": round(syrk_tflops / PEAK_BF16_TFLOPS, 4),
                    "vendor_gemm_full_square_bf16_out": {"ms": round(mm_ms, 4), "tflops": round(mm_tflops, 1)},
                    "calls_64x2048": {"ms": round(h64_ms, 4),
                                      "tflops": round(syrk_flop / (h64_ms * 1e-3) / 1e12, 1),
                                      "frac_bf16_mfma_peak": round(syrk_flop / (h64_ms * 1e-3) / 1e12
                                                                   / PEAK_BF16_TFLOPS, 4),
                                      "rel_diff_vs_one_call": float(f"{h64_rel:.3g}")},
                    "hook_staged_64x2048": {"ms": round(hs_ms, 4),
                                            "tflops": round(syrk_flop / (hs_ms * 1e-3) / 1e12, 1),
                                            "frac_bf16_mfma_peak": round(syrk_flop / (hs_ms * 1e-3) / 1e12
                                                                         / PEAK_BF16_TFLOPS, 4),
                                            "rel_diff_vs_one_call": float(f"{hs_rel:.3g}")}},
        "mxfp4_quantize_pack": mx,
        "copy_1GiB_GB_s": round(copy_gbs, 1),
        "roofline": {"bound": "mfma", "achieved": round(syrk_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(syrk_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "counters": counters,
                     "kernel": "syrk_stream_kernel + syrk_stream_reduce_kernel (the Hessian call of each timed step, "
                               "131072 tokens)"},
        "cpu_baseline": cpu,
        "parity": parity,
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)


def _host_info(torch):
    """CPU model (lscpu's model name with vendor, family, model and stepping,
    and /proc/cpuinfo's model name where it says more) and the BLAS / LAPACK
    backends torch was built with."""
    import re
    import subprocess
    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for key in ("Vendor ID", "Model name", "CPU family", "Model", "Stepping", "Socket(s)",
                    "Core(s) per socket", "Thread(s) per core", "CPU max MHz"):
            m = re.search(rf"^\s*{re.escape(key)}:\s*(.+)$", out, re.M)
            if m:
                fields[key] = m.group(1).strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            m = re.search(r"^model name\s*:\s*(.+)$", f.read(), re.M)
        if m and m.group(1).strip() != fields.get("Model name"):
            fields["cpuinfo model name"] = m.group(1).strip()
    except OSError:
        pass
    model = None
    if fields:
        model = fields.get("Model name", "?") + " (" + ", ".join(
            f"{k} {v}" for k, v in fields.items() if k != "Model name") + ")"
    cfg = torch.__config__.show()
    blas = re.search(r"BLAS_INFO=(\w+)", cfg)
    lapack = re.search(r"LAPACK_INFO=(\w+)", cfg)
    return {"cpu_model": model, "blas": blas.group(1) if blas else None,
            "lapack": lapack.group(1) if lapack else None}


def _median_ms(fn, runs=5, warmup=1):
    """Median of ``runs`` timed calls after ``warmup`` untimed ones (ms), and
    the last call's result."""
    for _ in range(warmup):
        out = fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        out = fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return sorted(times)[len(times) // 2], out


def cpu_baseline(torch, w_cpu, x_sample, h_gpu, res):
    """The oracle (torch-CPU restatement of the reference) on the host cores.

    Sample, each phase the median of 5 runs after one warm-up: the Hessian
    over 16 x 2048 tokens (scaled x4 to the layer's 64 x 2048) and the full
    4096 x 4096 oracle solve.  The solve runs on the GPU's own Hessian of the
    timed step (upper triangle mirrored, / num_samples), so its integer codes
    compare with the GPU's: code agreement, the largest code difference, and
    the layer output error ||X (W - Q)|| of both on 2048 of the tokens."""
    from oracle import gptq as og
    from oracle.qargs import OArgs

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t_h, _h = _median_ms(lambda: og.accumulate_hessian(x_sample, og.make_empty_hessian(COLS), torch.zeros(())))
    del _h
    scale = (BATCHES * SEQ) / (x_sample.shape[0] * x_sample.shape[1])
    Hf = torch.triu(h_gpu) + torch.triu(h_gpu, 1).t()
    t_s, (_, out_o, ex) = _median_ms(lambda: og.quantize_weight(
        w_cpu, OArgs(num_bits=4, strategy="group", group_size=GROUP), Hf / float(BATCHES), return_codes=True))
    cpu = {"value": round(t_h * scale + t_s, 1), "unit": "ms/layer", "cores": cores, "kind": "port",
           "sample": f"median of 5 runs after one warm-up per phase: Hessian over {x_sample.shape[0]}x"
                     f"{x_sample.shape[1]} tokens x{scale:g} + the full {ROWS}x{COLS} GPTQ solve (oracle, "
                     f"torch-CPU) on the GPU's Hessian",
           "hessian_ms_scaled": round(t_h * scale, 1), "solve_ms": round(t_s, 1), **_host_info(torch)}
    a, b = res.codes.cpu().to(torch.int32), ex["codes"]
    d = (a - b).abs()
    nz = d != 0
    first = torch.where(nz.any(1), d.gather(1, nz.int().argmax(1, keepdim=True))[:, 0], torch.zeros_like(d[:, 0]))
    xs = x_sample[0].reshape(-1, COLS).float()
    e_gpu = (xs @ (w_cpu.float() - res.weight.cpu().float()).t()).norm().item()
    e_ora = (xs @ (w_cpu.float() - out_o["weight"].float()).t()).norm().item()
    parity = {"vs": "oracle solve on the GPU's Hessian", "code_agreement": round(1.0 - nz.float().mean().item(), 7),
              "mismatches": int(nz.sum()), "rows_diverged": int(nz.any(1).sum()), "max_code_diff": int(d.max()),
              "first_divergence_max": int(first.max()), "codes_beyond_1": int((d > 1).sum()),
              "layer_err_gpu": round(e_gpu, 4), "layer_err_oracle": round(e_ora, 4),
              "layer_err_ratio": round(e_gpu / e_ora, 6),
              "scales_equal": bool(torch.equal(res.scale.cpu(), out_o["weight_scale"].reshape(res.scale.shape)))}
    return cpu, parity


# ---------------------------------------------------------------- other workloads
def _setup():
    import torch
    from llmcompressor_amd import _lib
    _lib.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    return torch, dev


def _gpu_heavy(torch, dev, rows, cols, seed, nu=4, lognormal=True, chunk=8192):
    """Student-t(nu) [x lognormal(0,1) per column] bf16 [rows, cols], generated on the GPU."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    c = torch.exp(torch.randn(cols, generator=g, device=dev)) if lognormal else None
    out = torch.empty(rows, cols, dtype=torch.bfloat16, device=dev)
    for r0 in range(0, rows, chunk):
        m = min(chunk, rows - r0)
        z = torch.randn(m, cols, generator=g, device=dev)
        chi = torch.zeros(m, cols, device=dev)
        for _ in range(nu):
            chi += torch.randn(m, cols, generator=g, device=dev) ** 2
        t = z / torch.sqrt(chi / nu)
        if c is not None:
            t *= c
        out[r0:r0 + m] = t.to(torch.bfloat16)
    return out


def _timed(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps, out


_COLLECT = None   # a list while the default line gathers the other workloads' lines


def _line(metric, value, unit, a, ms, workload, extra, higher=False, dtype="bf16 inputs, fp32 accumulate/solve"):
    line = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": round(ms, 3), "higher_is_better": higher, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded, generated on the GPU)",
            "config": {"workload": workload}}
    line.update(extra)
    if _COLLECT is not None:
        _COLLECT.append(line)
    else:
        print(json.dumps(line), flush=True)


def bench_mxfp4(a):
    """MXFP4 W4A4 quantize + pack: W [4096, 14336] and A [8192, 14336] bf16."""
    torch, dev = _setup()
    from llmcompressor_amd import ops
    res = {}
    tot_ms = tot_b = 0.0
    for name, shape, seed in (("W", (4096, 14336), 2), ("A", (8192, 14336), 3)):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        t = (torch.randn(shape, generator=g, device=dev) * 0.015).to(torch.bfloat16) if name == "W" else \
            _gpu_heavy(torch, dev, shape[0], shape[1], seed, nu=3, lognormal=False)
        out = (torch.empty(shape[0], shape[1] // 2, dtype=torch.uint8, device=dev),
               torch.empty(shape[0], shape[1] // 32, dtype=torch.uint8, device=dev))
        ms, _ = _timed(torch, lambda: ops.mxfp4_quantize_pack(t, out=out), max(a.steps, 20), max(a.warmup, 3))
        nbytes = t.numel() * 2.53125
        res[name] = {"ms": round(ms, 5), "GB_s": round(nbytes / ms / 1e6, 1),
                     "frac_hbm_peak": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4), "bytes": int(nbytes)}
        tot_ms += ms
        tot_b += nbytes
    gbs = tot_b / tot_ms / 1e6
    _line("MXFP4 quantize+pack GB/s (W 4096x14336 + A 8192x14336)", gbs, "GB/s", a, tot_ms, "mxfp4_w4a4_pack",
          {"per_tensor": res, "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                           "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}},
          higher=True, dtype="bf16 in, e2m1 + e8m0 out")


def bench_w8a8(a):
    """GPTQ W8A8: int8 channel-symmetric weights, actorder=weight, W [14336, 4096], X 128 x 2048 tokens,
    plus per-token dynamic int8 quantization of X."""
    torch, dev = _setup()
    from llmcompressor_amd import gptq, ops
    from llmcompressor_amd.observers import Observer
    from llmcompressor_amd.quant_args import QuantizationArgs
    rows, cols, batches, seq = 14336, 4096, 128, 2048
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    w = (torch.randn(rows, cols, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = _gpu_heavy(torch, dev, batches * seq, cols, 5)
    lin = torch.nn.Linear(cols, rows, bias=False, device=dev, dtype=torch.bfloat16)
    lin.weight.data = w
    qa = QuantizationArgs(num_bits=8, type="int", symmetric=True, strategy="channel", actorder="weight")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    def step():
        H = gptq.make_empty_hessian(lin)
        n = torch.zeros((), device=dev)
        ev[0].record()
        H, n = gptq.accumulate_hessian(x.view(batches, seq, cols), lin, H, n)
        ev[1].record()
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(lin.weight)
        r = gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(batches))
        ev[2].record()
        return r

    ms, res = _timed(torch, step, a.steps, a.warmup)
    torch.cuda.synchronize()
    hess_ms, solve_ms = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])
    assert int(res.codes.min()) >= -128 and int(res.codes.max()) <= 127
    act_ms, _ = _timed(torch, lambda: ops.quantize_int8_per_token(x), 5, 2)
    act_bytes = x.numel() * 2 + x.numel() + x.shape[0] * 2
    flop = batches * seq * cols * (cols + 1)
    _line("GPTQ ms/layer (W8A8 int8 channel, actorder=weight, 14336x4096, Hessian over 128x2048 tokens + solve)",
          ms, "ms/layer", a, ms, "gptq_w8a8_channel_actorder_14336x4096_128x2048tok",
          {"phases_ms": {"hessian": round(hess_ms, 3), "solve": round(solve_ms, 3)},
           "hessian": {"tflops": round(flop / hess_ms / 1e9, 1),
                       "frac_bf16_mfma_peak": round(flop / hess_ms / 1e9 / PEAK_BF16_TFLOPS, 4)},
           "act_quant_int8_per_token": {"ms": round(act_ms, 4), "GB_s": round(act_bytes / act_ms / 1e6, 1),
                                        "frac_hbm_peak": round(act_bytes / act_ms / 1e6 / PEAK_HBM_GBS, 4)}})


def bench_moe(a):
    """MoE expert GPTQ W4A16 g128: 128 experts (gate/up 768x2048, down 2048x768), 32768 tokens routed
    top-8 (Zipf 1.1 prior + Gumbel): grouped per-expert Hessians + 384 solves."""
    torch, dev = _setup()
    from llmcompressor_amd import gptq, moe, workloads
    from llmcompressor_amd.quant_args import QuantizationArgs
    E, hid, inter, tokens, k = 128, 2048, 768, 32768, 8
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    gate = (torch.randn(E, inter, hid, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    up = (torch.randn(E, inter, hid, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    down = (torch.randn(E, hid, inter, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    hs = _gpu_heavy(torch, dev, tokens, hid, 7)
    idx, wts = workloads.moe_routing(tokens, E, k)
    rows, offsets, _ = moe.route_tokens(idx.to(dev), E)
    counts = [offsets[e + 1] - offsets[e] for e in range(E)]
    inter_x = moe.expert_intermediate(hs, rows, offsets, gate, up)   # calibration forward (untimed)
    off_dev = torch.tensor(offsets, dtype=torch.int64, device=dev)
    qa = QuantizationArgs(num_bits=4, type="int", symmetric=True, strategy="group", group_size=128)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    def step():
        # uncleared: the grouped syrk writes every upper triangle (fresh=True)
        Hgu = torch.empty(E, hid, hid, device=dev)
        Hd = torch.empty(E, inter, inter, device=dev)
        ns = torch.zeros(E, device=dev)
        ev[0].record()
        moe.accumulate_expert_hessians(hs, rows, off_dev, Hgu, ns, fresh=True)
        moe.accumulate_expert_hessians(inter_x, None, off_dev, Hd, ns.clone(), fresh=True)
        ev[1].record()
        # all experts of one projection solved together (one launch per step);
        # gate and up share their input, hence their Hessian and its Cholesky chain
        # (gate and up: one stack of 1536 rows per expert, rows being
        # independent given Hinv and their own scales)
        pgu = gptq.prepare_hessians_batched(Hgu, qa, ns)
        gptq.gptq_quantize_batched(torch.cat([gate, up], dim=1), qa, Hgu, num_samples=ns, prepared=pgu)
        gptq.gptq_quantize_batched(down, qa, Hd, num_samples=ns)
        ev[2].record()

    ms, _ = _timed(torch, step, a.steps, a.warmup)
    torch.cuda.synchronize()
    hess_ms, solve_ms = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])
    flop = sum(c * (hid * (hid + 1) + inter * (inter + 1)) for c in counts)
    del inter_x

    # the same layer through GPTQModifier: a LinearExperts forward (the
    # reference's per-expert loop) with the modifier's hooks on its 384 expert
    # Linears (grouped accumulation per family), then the batched solves; the
    # modifier's own cost is that time less the same forward without hooks
    from llmcompressor_amd import GPTQModifier
    from llmcompressor_amd.moe import LinearExperts
    idx_d = idx.to(dev)
    wts_d = wts.to(dev).to(torch.bfloat16)

    def block():
        return LinearExperts.from_stacked(gate.clone(), up.clone(), down.clone())

    def plain():
        m = block()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            m(hs, idx_d, wts_d)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    def modifier():
        m = block()
        mod = GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), actorder=None)
        mod.on_initialize(m)
        mod.on_calibration_start(m)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            m(hs, idx_d, wts_d)
        mod.on_calibration_end()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        mod.on_sequential_epoch_end(list(mod._modules))
        mod.on_finalize()
        torch.cuda.synchronize()
        return (t1 - t0) * 1e3, (time.perf_counter() - t1) * 1e3

    plain()   # warm-up
    plain_ms = sum(plain() for _ in range(max(1, a.steps))) / max(1, a.steps)
    modifier()   # warm-up
    runs = [modifier() for _ in range(max(1, a.steps))]
    fwd_ms = sum(r[0] for r in runs) / len(runs)
    comp_ms = sum(r[1] for r in runs) / len(runs)
    mod_ms = fwd_ms - plain_ms + comp_ms
    _line("MoE GPTQ ms/layer (128 experts W4A16 g128, 32768 tokens top-8: grouped Hessians + 384 solves)",
          ms, "ms/layer", a, ms, "moe_128x(768x2048,2048x768)_32768tok_top8",
          {"phases_ms": {"grouped_hessians": round(hess_ms, 3), "solves": round(solve_ms, 3)},
           "modifier_path": {"ms": round(mod_ms, 3), "ratio_to_direct": round(mod_ms / ms, 3),
                             "calibration_forward_with_hooks_ms": round(fwd_ms, 3),
                             "forward_without_hooks_ms": round(plain_ms, 3), "compress_ms": round(comp_ms, 3)},
           "hessian": {"tflops": round(flop / hess_ms / 1e9, 1),
                       "frac_bf16_mfma_peak": round(flop / hess_ms / 1e9 / PEAK_BF16_TFLOPS, 4)},
           "tokens_per_expert": {"min": min(counts), "max": max(counts), "mean": sum(counts) / E}})


def bench_decoder(a):
    """Llama-3-8B-shaped decoder layer, sequential GPTQ W4A16 g128 over 256 x 2048 tokens: four Hessians
    (q/k/v shared, o, gate/up shared, down d=14336) and seven solves."""
    torch, dev = _setup()
    from llmcompressor_amd import gptq
    from llmcompressor_amd.observers import Observer
    from llmcompressor_amd.quant_args import QuantizationArgs
    hidden, inter, kv, batches, seq = 4096, 14336, 1024, 256, 2048
    ntok = batches * seq
    g = torch.Generator(device=dev)
    g.manual_seed(9)

    def w(r, c):
        return (torch.randn(r, c, generator=g, device=dev) * 0.02).to(torch.bfloat16)

    W = {"q_proj": w(hidden, hidden), "k_proj": w(kv, hidden), "v_proj": w(kv, hidden),
         "o_proj": w(hidden, hidden), "gate_proj": w(inter, hidden), "up_proj": w(inter, hidden),
         "down_proj": w(hidden, inter)}
    # module inputs the calibration hooks see (generated / computed untimed)
    x_attn = _gpu_heavy(torch, dev, ntok, hidden, 10)
    x_o = _gpu_heavy(torch, dev, ntok, hidden, 11)
    x_mlp = _gpu_heavy(torch, dev, ntok, hidden, 12)
    x_down = torch.empty(ntok, inter, dtype=torch.bfloat16, device=dev)
    for r0 in range(0, ntok, 32768):
        xm = x_mlp[r0:r0 + 32768]
        x_down[r0:r0 + 32768] = torch.nn.functional.silu(xm @ W["gate_proj"].t()) * (xm @ W["up_proj"].t())
    qa = QuantizationArgs(num_bits=4, type="int", symmetric=True, strategy="group", group_size=128)
    lin = {}
    for name, wt in W.items():
        m = torch.nn.Linear(wt.shape[1], wt.shape[0], bias=False, device=dev, dtype=torch.bfloat16)
        m.weight.data = wt
        lin[name] = m
    groups = [(("q_proj", "k_proj", "v_proj"), x_attn), (("o_proj",), x_o), (("gate_proj", "up_proj"), x_mlp),
              (("down_proj",), x_down)]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    def step():
        Hs = []
        ev[0].record()
        for names, xin in groups:
            m = lin[names[0]]
            H = gptq.make_empty_hessian(m)
            n = torch.zeros((), device=dev)
            H, n = gptq.accumulate_hessian(xin.view(batches, seq, -1), m, H, n)
            Hs.append(H)
        ev[1].record()
        for (names, _), H in zip(groups, Hs):
            # modules with the same input share the Hessian and its Cholesky
            # chain, and are solved as one stack of rows (rows are independent
            # given Hinv and their own scales)
            prep = gptq.prepare_hessian(H, qa, float(batches))
            w = lin[names[0]].weight if len(names) == 1 else torch.cat([lin[nm].weight for nm in names])
            obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
            obs(w)
            gptq.gptq_quantize(w, qa, H, obs, num_samples=float(batches), prepared=prep)
        ev[2].record()

    ms, _ = _timed(torch, step, a.steps, a.warmup)
    torch.cuda.synchronize()
    hess_ms, solve_ms = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])
    flop = 3 * ntok * hidden * (hidden + 1) + ntok * inter * (inter + 1)
    _line("Decoder-layer GPTQ ms (Llama-3-8B-shaped, W4A16 g128, 256x2048 tokens: 4 Hessians + 7 solves)",
          ms, "ms/layer", a, ms, "llama3_8b_decoder_layer_w4a16_256x2048tok",
          {"phases_ms": {"hessians": round(hess_ms, 3), "solves": round(solve_ms, 3)},
           "hessian": {"tflops": round(flop / hess_ms / 1e9, 1),
                       "frac_bf16_mfma_peak": round(flop / hess_ms / 1e9 / PEAK_BF16_TFLOPS, 4)}})


def bench_sparsegpt(a):
    """SparseGPT on a 4096 x 4096 layer: running-mean Hessian over 64 x 2048 tokens, then the 50 %
    unstructured solve (the step); the 2:4 solve on the same Hessian is timed beside it."""
    torch, dev = _setup()
    from llmcompressor_amd import sparsegpt
    rows = cols = 4096
    batches, seq = 64, 2048
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    w = (torch.randn(rows, cols, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = _gpu_heavy(torch, dev, batches * seq, cols, 1)
    lin = torch.nn.Linear(cols, rows, bias=False, device=dev, dtype=torch.bfloat16)
    lin.weight.data = w
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    def step():
        H = sparsegpt.make_empty_hessian(lin)
        ev[0].record()
        H, n = sparsegpt.accumulate_hessian(x.view(batches, seq, cols), lin, H, 0)
        ev[1].record()
        r = sparsegpt.sparsegpt_prune(lin.weight, H, 0.5)
        ev[2].record()
        return r, H

    ms, (res, H) = _timed(torch, step, a.steps, a.warmup)
    torch.cuda.synchronize()
    hess_ms, solve_ms = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])
    nm_ms, res24 = _timed(torch, lambda: sparsegpt.sparsegpt_prune(lin.weight, H, 0.5, 2, 4), a.steps, a.warmup)
    z = float((res.weight == 0).float().mean())
    z24 = float((res24.weight == 0).float().mean())
    assert 0.5 <= z < 0.51 and 0.5 <= z24 < 0.51
    flop = batches * seq * cols * (cols + 1)
    _line("SparseGPT ms/layer (50 % unstructured, 4096x4096, Hessian over 64x2048 tokens + solve)",
          ms, "ms/layer", a, ms, "sparsegpt_50pct_4096x4096_64x2048tok",
          {"phases_ms": {"hessian": round(hess_ms, 3), "solve": round(solve_ms, 3)},
           "solve_2of4_ms": round(nm_ms, 3), "sparsity": {"unstructured": round(z, 6), "2of4": round(z24, 6)},
           "hessian": {"tflops": round(flop / hess_ms / 1e9, 1),
                       "frac_bf16_mfma_peak": round(flop / hess_ms / 1e9 / PEAK_BF16_TFLOPS, 4)}})


def bench_mse_observer(a):
    """memoryless_mse weight observer (20 shrink candidates, norm 2.4): W 4096x4096 int4 group 128 (the step)
    and W 14336x4096 int8 channel, bf16; the min-max observer beside them."""
    torch, dev = _setup()
    from llmcompressor_amd.observers import Observer
    from llmcompressor_amd.quant_args import QuantizationArgs
    res = {}
    for name, shape, kw in (("w4_g128_4096x4096", (4096, 4096), dict(num_bits=4, strategy="group", group_size=128)),
                            ("w8_channel_14336x4096", (14336, 4096), dict(num_bits=8, strategy="channel"))):
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        w = (torch.randn(shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)

        def run(obs_name):
            o = Observer.load_from_registry(obs_name, base_name="weight", args=QuantizationArgs(observer=obs_name, **kw))
            return o(w).get_qparams()

        ms, _ = _timed(torch, lambda: run("memoryless_mse"), max(a.steps, 10), max(a.warmup, 2))
        mm_ms, _ = _timed(torch, lambda: run("memoryless_minmax"), max(a.steps, 10), max(a.warmup, 2))
        evals = w.numel() * 20
        res[name] = {"ms": round(ms, 4), "minmax_ms": round(mm_ms, 4),
                     "candidate_evals_per_s": round(evals / ms * 1e3 / 1e9, 2), "unit_evals": "1e9/s"}
    ms = res["w4_g128_4096x4096"]["ms"]
    _line("MSE weight observer ms (memoryless_mse, W 4096x4096 bf16, int4 group 128, 20 shrink candidates)", ms,
          "ms", a, ms, "mse_observer_w4_g128_4096x4096", {"per_shape": res}, dtype="bf16 in, fp32 error sums")


def bench_pipeline(a):
    """Sequential pipeline, GPTQ W4A16 g128 over two Llama-3-8B-shaped MLP+projection layers (q/k/v/o 4096,
    gate/up/down 14336), 64 x 2048 calibration tokens in 8 batches: activation cache on the GPU vs offloaded
    to pinned host memory with prefetch."""
    torch, dev = _setup()
    import copy

    import torch.nn.functional as F

    from llmcompressor_amd import GPTQModifier
    from llmcompressor_amd.pipeline import sequential_calibrate

    hidden, inter, nb, bs, seq = 4096, 14336, 8, 8, 2048

    class Layer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            L = lambda i, o: torch.nn.Linear(i, o, bias=False)  # noqa: E731
            self.q, self.k, self.v, self.o = L(hidden, hidden), L(hidden, 1024), L(hidden, 1024), L(hidden, hidden)
            self.gate, self.up, self.down = L(hidden, inter), L(hidden, inter), L(inter, hidden)

        def forward(self, x):
            a = self.q(x) + F.pad(self.k(x) * self.v(x), (0, hidden - 1024))
            h = x + self.o(torch.tanh(a))
            return h + self.down(F.silu(self.gate(h)) * self.up(h))

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = torch.nn.ModuleList(Layer() for _ in range(2))

        def forward(self, x):
            for layer in self.layers:
                x = layer(x)
            return x

    torch.manual_seed(9)
    base = Model().to(dev).to(torch.bfloat16)
    for p_ in base.parameters():
        p_.data.mul_(0.5)
    xs = [_gpu_heavy(torch, dev, bs * seq, hidden, 10 + b).view(bs, seq, hidden) for b in range(nb)]
    res = {}
    for name, off, pre in (("gpu_cache", None, False), ("host_offload_prefetch", "cpu", True)):
        times = []
        for it in range(1 + max(1, a.steps // 2)):   # the first run warms the libraries up
            m = copy.deepcopy(base)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            sequential_calibrate(m, m.layers, xs, GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=()),
                                 offload_device=off, prefetch=pre)
            torch.cuda.synchronize()
            if it:
                times.append((time.perf_counter() - t0) * 1e3)
        res[name] = round(min(times), 2)
    act_bytes = nb * bs * seq * hidden * 2
    _line("Sequential pipeline ms (GPTQ W4A16 g128, 2 Llama-3-8B-shaped layers, 64x2048 tokens, host-offloaded "
          "activation cache with prefetch)", res["host_offload_prefetch"], "ms", a, res["host_offload_prefetch"],
          "sequential_pipeline_2_layers_64x2048tok",
          {"ms_gpu_cache": res["gpu_cache"], "activation_bytes_per_layer_pass": act_bytes,
           "offload_overhead_ms": round(res["host_offload_prefetch"] - res["gpu_cache"], 2)})


def _torch_gptq_w4a16(torch, w, x, num_samples, group, blocksize=128, percdamp=0.01):
    """The reference's own algorithm as torch ops on the GPU, the way it runs
    on a ROCm device today (timing comparator only): fp32 GEMM Hessian
    (modifiers/gptq/gptq_quantize.py:22-32, 63-97; base.py:594), memoryless
    min-max group scales in the weight dtype (observers/min_max.py:16-25,
    observers/base.py:99-123), damping and the three-call Cholesky chain
    (gptq_quantize.py:181-196), and the per-column loop with its lazy block
    update (:199-277), each column a channel-wise fake quantize with the
    dequantised value in the scale's dtype.  Returns (hessian_ms, solve_ms,
    Q fp32, scale bf16)."""
    import math

    sync = torch.cuda.synchronize
    sync()
    t0 = time.perf_counter()
    H = torch.zeros(w.shape[1], w.shape[1], dtype=torch.float32, device=w.device)
    inp = x.reshape(-1, x.shape[-1]).t().to(torch.float32)
    inp = math.sqrt(2) * inp
    H += inp.matmul(inp.t())
    del inp
    H = H / num_samples
    sync()
    t1 = time.perf_counter()
    rows, cols = w.shape
    g = w.view(rows, cols // group, group)
    mn = torch.clamp(torch.amin(g, dim=-1), max=0)
    mx = torch.clamp(torch.amax(g, dim=-1), min=0)
    scale = torch.clamp(torch.maximum(mn.abs(), mx.abs()) / 7.5, min=torch.finfo(torch.float32).eps)
    W = w.clone().to(torch.float32)
    g_idx = torch.arange(cols, device=w.device, dtype=torch.int) // group
    dead = torch.diag(H) == 0
    H[dead, dead] = 1
    W[:, dead] = 0
    damp = percdamp * torch.mean(torch.diag(H))
    diag = torch.arange(cols, device=w.device)
    H[diag, diag] += damp
    H = torch.linalg.cholesky(H)
    H = torch.cholesky_inverse(H)
    Hinv = torch.linalg.cholesky(H, upper=True)
    losses = torch.zeros(rows, device=w.device)
    for i1 in range(0, cols, blocksize):
        i2 = min(i1 + blocksize, cols)
        W1 = W[:, i1:i2].clone()
        Q1 = torch.zeros_like(W1)
        Err1 = torch.zeros_like(W1)
        losses1 = torch.zeros_like(W1)
        Hinv1 = Hinv[i1:i2, i1:i2]
        for i in range(i2 - i1):
            wc = W1[:, i]
            d = Hinv1[i, i]
            s = scale[:, g_idx[i1 + i]]
            q = (torch.round(torch.clamp(wc / s, -8, 7)).to(s.dtype) * s).to(torch.float32)
            Q1[:, i] = q
            losses1[:, i] = (wc - q) ** 2 / d ** 2
            err1 = (wc - q) / d
            W1[:, i:] -= err1.unsqueeze(1).matmul(Hinv1[i, i:].unsqueeze(0))
            Err1[:, i] = err1
        W[:, i1:i2] = Q1
        losses += torch.sum(losses1, 1) / 2
        W[:, i2:] -= Err1.matmul(Hinv[i1:i2, i2:])
    torch.sum(losses).item()
    sync()
    t2 = time.perf_counter()
    return (t1 - t0) * 1e3, (t2 - t1) * 1e3, W, scale


def _torch_mxfp4(torch, t):
    """MXFP4 quantize + pack as torch ops (the compressed-tensors path the
    reference calls: group absmax, e8m0 exponent of the bf16-rounded absmax,
    division by the power-of-two scale, the e2m1 thresholds of
    ``cast_to_fp4``, two codes per byte)."""
    rows, cols = t.shape
    g = t.view(rows, cols // 32, 32)
    amax = torch.amax(torch.abs(g), dim=-1)
    bits = ((amax.view(torch.int16).to(torch.int32) & 0xFFFF) + 32) & 0xFF80
    e8 = torch.clamp(((bits >> 7) & 0xFF) - 2, 0, 254)
    e8 = torch.where(bits == 0, torch.zeros_like(e8), e8)
    v = g.to(torch.float32) / torch.pow(2.0, (e8 - 127).to(torch.float32))[..., None]
    a = torch.abs(v)
    idx = sum((a > th).to(torch.uint8) for th in (0.25, 1.25, 2.5, 5.0)) + \
        sum((a >= th).to(torch.uint8) for th in (0.75, 1.75, 3.5))
    code = (idx | ((v < 0).to(torch.uint8) << 3)).view(rows, cols)
    return code[:, 0::2] | (code[:, 1::2] << 4), e8.to(torch.uint8)


def bench_torch_reference(a):
    """The headline layer (W4A16 g128, 4096 x 4096, 64 x 2048 tokens) through
    the reference's algorithm as plain torch ops on the same GPU, beside this
    library's step on the same inputs; the integer codes of the two are
    compared.  One timed pass of the torch path after a warm-up on a
    256-column slice (library initialisation)."""
    torch, dev = _setup()
    from llmcompressor_amd import gptq
    from llmcompressor_amd.observers import Observer
    from llmcompressor_amd.quant_args import QuantizationArgs

    w, x = gen_inputs(torch, dev)
    _torch_gptq_w4a16(torch, w[:256, :256].contiguous(), x[:2, :, :256].contiguous(), 2, GROUP)
    h_ms, s_ms, Q, scale = _torch_gptq_w4a16(torch, w, x, BATCHES, GROUP)
    ref_codes = torch.round(Q / scale.float().repeat_interleave(GROUP, dim=1)).to(torch.int32)
    del Q

    lin = torch.nn.Linear(COLS, ROWS, bias=False, device=dev, dtype=torch.bfloat16)
    lin.weight.data = w
    qa = QuantizationArgs(num_bits=4, type="int", symmetric=True, strategy="group", group_size=GROUP)

    def step():
        H = gptq.make_empty_hessian(lin)
        H, n = gptq.accumulate_hessian(x, lin, H, torch.zeros((), device=dev))
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(lin.weight)
        return gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(BATCHES))

    ms, res = _timed(torch, step, a.steps, a.warmup)

    # MXFP4 quantize + pack of W 4096 x 14336 (the MXFP4 configuration's weight)
    from llmcompressor_amd import ops
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    t = (torch.randn((4096, 14336), generator=gen, device=dev) * 0.015).to(torch.bfloat16)
    mx_ref_ms, (p_ref, e_ref) = _timed(torch, lambda: _torch_mxfp4(torch, t), 3, 1)
    mx_ms, (p_us, e_us) = _timed(torch, lambda: ops.mxfp4_quantize_pack(t), 20, 3)
    mx = {"torch_ms": round(mx_ref_ms, 4), "mi355q_ms": round(mx_ms, 4), "speedup": round(mx_ref_ms / mx_ms, 1),
          "bit_equal": bool(torch.equal(p_ref, p_us) and torch.equal(e_ref, e_us))}
    del t

    same = (res.codes.to(torch.int32) == ref_codes)
    diff = (res.codes.to(torch.int32) - ref_codes).abs()
    ref_ms = h_ms + s_ms
    _line("GPTQ ms/layer of the reference's algorithm as torch ops on this GPU (W4A16 g128, 4096x4096, "
          "64x2048 tokens)", ref_ms, "ms/layer", a, ref_ms, "torch_reference_gptq_w4a16_g128_4096x4096",
          {"phases_ms": {"hessian": round(h_ms, 2), "solve": round(s_ms, 2)},
           "mi355q_ms_per_layer": round(ms, 3), "speedup": round(ref_ms / ms, 1),
           "scale_equal": bool(torch.equal(res.scale, scale)),
           "code_agreement": round(float(same.float().mean()), 6), "max_code_diff": int(diff.max()),
           "mxfp4_quantize_pack_4096x14336": mx},
          dtype="fp32 (torch reference path)")


OTHER_WORKLOADS = {"mxfp4": bench_mxfp4, "gptq_w8a8": bench_w8a8, "moe": bench_moe, "decoder": bench_decoder,
                   "sparsegpt": bench_sparsegpt, "mse_observer": bench_mse_observer,
                   "pipeline": bench_pipeline, "torch_reference": bench_torch_reference}


if __name__ == "__main__":
    main()
