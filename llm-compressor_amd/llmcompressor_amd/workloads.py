"""Seeded synthetic inputs for the five calibration workloads.

Every tensor is drawn on the CPU from its own ``torch.Generator`` seed in
fp32 and rounded to bf16 (RNE), so a GPU run and a CPU check consume
identical bytes; ``sha256_bf16`` fingerprints them.  Heavy tails follow
Student-t(nu) = z / sqrt(chi2_nu / nu) and per-channel scales
lognormal(0, 1) = exp(z).

Workloads (sizes are the full ones; every generator takes smaller sizes for
tests):

* ``gptq_w4a16``  - W [4096, 4096] = 0.02 N(0,1) with 0.1 % of entries x10
  (seed 0); X [64, 2048, 4096] = t4 * c_j (seed 1).
* ``mxfp4``       - W [4096, 14336] = 0.015 N(0,1) (seed 2); A [8192, 14336]
  = t3 (seed 3).
* ``gptq_w8a8``   - W [14336, 4096] = 0.02 N(0,1) (seed 4); X [128, 2048,
  4096] heavy-tailed as above (seed 5).
* ``moe``         - 128 experts, gate/up [768, 2048], down [2048, 768]
  (seed 6); hidden [32768, 2048] (seed 7); Zipf(1.1) router prior + Gumbel
  noise, top-8 (seed 8).
* ``decoder``     - Llama-3-8B-shaped layer weights (seed 9); X [256, 2048,
  4096] (seed 10).
"""
from __future__ import annotations

import hashlib

import torch


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def normal(shape, std: float, seed: int) -> torch.Tensor:
    return (torch.randn(shape, generator=_gen(seed)) * std).to(torch.bfloat16)


def student_t(shape, nu: float, g: torch.Generator, chunk: int = 1 << 24) -> torch.Tensor:
    """Student-t(nu) samples in fp32, generated in chunks to bound memory."""
    n = 1
    for s in shape:
        n *= s
    out = torch.empty(n, dtype=torch.float32)
    gamma_shape = torch.tensor([nu / 2.0])
    for o in range(0, n, chunk):
        m = min(chunk, n - o)
        z = torch.randn(m, generator=g)
        # chi2_nu = 2 * Gamma(nu/2, 1); torch._standard_gamma takes no
        # generator, so build chi2 from nu normal squares for integer nu.
        if float(nu).is_integer():
            c = torch.zeros(m)
            for _ in range(int(nu)):
                c += torch.randn(m, generator=g) ** 2
        else:  # pragma: no cover - all workloads use integer nu
            c = 2.0 * torch._standard_gamma(gamma_shape.expand(m))
        out[o:o + m] = z / torch.sqrt(c / nu)
    return out.reshape(shape)


def heavy_tailed_activations(shape, seed: int, nu: float = 4.0,
                             channel_lognormal: bool = True) -> torch.Tensor:
    """t_nu times a per-channel lognormal(0,1) scale, as bf16."""
    g = _gen(seed)
    cols = shape[-1]
    c = torch.exp(torch.randn(cols, generator=g)) if channel_lognormal else torch.ones(cols)
    x = student_t(shape, nu, g)
    x.mul_(c)
    return x.to(torch.bfloat16)


def gptq_weight(rows: int, cols: int, seed: int = 0, std: float = 0.02,
                outlier_frac: float = 0.001, outlier_mult: float = 10.0) -> torch.Tensor:
    g = _gen(seed)
    w = torch.randn(rows, cols, generator=g) * std
    n_out = int(round(outlier_frac * rows * cols))
    if n_out:
        idx = torch.randperm(rows * cols, generator=g)[:n_out]
        w.view(-1)[idx] *= outlier_mult
    return w.to(torch.bfloat16)


def gptq_w4a16(rows=4096, cols=4096, batches=64, seq=2048):
    """Single Linear, W4A16 group 128: returns (W, X[batches, seq, cols])."""
    return gptq_weight(rows, cols, seed=0), heavy_tailed_activations((batches, seq, cols), seed=1)


def mxfp4(w_rows=4096, cols=14336, a_rows=8192):
    w = normal((w_rows, cols), 0.015, seed=2)
    a = student_t((a_rows, cols), 3.0, _gen(3)).to(torch.bfloat16)
    return w, a


def gptq_w8a8(rows=14336, cols=4096, batches=128, seq=2048):
    return normal((rows, cols), 0.02, seed=4), heavy_tailed_activations((batches, seq, cols), seed=5)


def moe_routing(tokens: int, experts: int, top_k: int, seed: int = 8, zipf_s: float = 1.1):
    """Router: log Zipf(s) expert prior + Gumbel noise, top-k distinct experts.

    Returns (top_k_index [tokens, top_k] int64, top_k_weights [tokens, top_k] fp32
    softmax over the selected logits).
    """
    g = _gen(seed)
    ranks = torch.randperm(experts, generator=g).to(torch.float32) + 1.0
    prior = -zipf_s * torch.log(ranks)
    u = torch.rand(tokens, experts, generator=g).clamp_(1e-20, 1.0 - 1e-7)
    logits = prior.unsqueeze(0) - torch.log(-torch.log(u))
    vals, idx = torch.topk(logits, top_k, dim=-1)
    return idx, torch.softmax(vals, dim=-1)


def moe(experts=128, hidden=2048, inter=768, tokens=32768, top_k=8):
    g = _gen(6)
    gate = (torch.randn(experts, inter, hidden, generator=g) * 0.02).to(torch.bfloat16)
    up = (torch.randn(experts, inter, hidden, generator=g) * 0.02).to(torch.bfloat16)
    down = (torch.randn(experts, hidden, inter, generator=g) * 0.02).to(torch.bfloat16)
    hs = heavy_tailed_activations((tokens, hidden), seed=7)
    idx, wts = moe_routing(tokens, experts, top_k)
    return gate, up, down, hs, idx, wts


def decoder_layer(hidden=4096, inter=14336, kv_dim=1024, seed=9):
    g = _gen(seed)
    std = 0.02

    def w(r, c):
        return (torch.randn(r, c, generator=g) * std).to(torch.bfloat16)

    return {
        "q_proj": w(hidden, hidden), "k_proj": w(kv_dim, hidden), "v_proj": w(kv_dim, hidden),
        "o_proj": w(hidden, hidden), "gate_proj": w(inter, hidden), "up_proj": w(inter, hidden),
        "down_proj": w(hidden, inter),
    }


def sha256_bf16(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.int16).numpy().tobytes()).hexdigest()
