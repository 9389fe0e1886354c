"""GPU: whole-layer GPTQ at the decoder-layer and MoE configurations' shapes
(reduced where the oracle would take minutes) against the oracle.

* A Llama-shaped decoder layer (hidden 1024, 16 query and 4 key/value heads
  of 64, intermediate 8192, so the down projection's Hessian has 528 tiles and
  its 4096-token calls take the two-split path) calibrated on 4 x 2 x 2048
  tokens (twice the intermediate width, as calibration sets exceed the
  widths they calibrate) by GPTQModifier
  with shared Hessians (q/k/v and gate/up), modules.py's basic pipeline: one
  pass over the batches, then every module compressed.  Each module's input is
  captured in the same forward; the oracle accumulates its own Hessian from
  it (checked against the GPU's to 1e-5) and solves on the GPU's Hessian, so
  the codes compare the solves (modifiers/gptq/base.py:255-289,578-601).
* The Cholesky chain at d = 14336 (the Llama-3-8B down projection) against the
  oracle's three-call chain on the same Hessian.
* One batched solve of 128 experts of 768 x 2048 (an MoE gate/up projection)
  against oracle solves of sampled experts.

GPTQ code bars as in test_gpu_parity.py's end-to-end tests.
"""
import pytest
import torch
import torch.nn.functional as F

from llmcompressor_amd import GPTQModifier, gptq, ops
from llmcompressor_amd.staging import HessianStage
from llmcompressor_amd.quant_args import QuantizationArgs
from oracle import gptq as og
from oracle.qargs import OArgs
from parity_util import code_agreement, code_bar

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def rel_fro(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _full(Hu):
    return torch.triu(Hu) + torch.triu(Hu, 1).t()


def _gpu_heavy(shape, seed, dev, nu=4):
    """Student-t(nu) x lognormal(0, 1) per column, bf16, generated on the GPU."""
    g = torch.Generator(device=dev).manual_seed(seed)
    c = torch.exp(torch.randn(shape[-1], generator=g, device=dev))
    z = torch.randn(shape, generator=g, device=dev)
    chi = sum(torch.randn(shape, generator=g, device=dev) ** 2 for _ in range(nu))
    return (z / torch.sqrt(chi / nu) * c).to(torch.bfloat16)


def _check_codes(tag, codes, ex_codes, W, Q, Q_oracle, X):
    st = code_agreement(codes.cpu().to(torch.int32), ex_codes)
    Xf = X.reshape(-1, X.shape[-1]).float()
    e_gpu = (Xf @ (W.float() - Q.cpu().float()).t()).norm().item()
    e_ora = (Xf @ (W.float() - Q_oracle.float()).t()).norm().item()
    say(f"  {tag}: {st} err {e_gpu:.6g} vs {e_ora:.6g}")
    assert code_bar(st, codes.shape[0]), tag
    assert abs(e_gpu - e_ora) <= 0.005 * e_ora, tag


class LlamaLayer(torch.nn.Module):
    def __init__(self, hidden=1024, heads=16, kv_heads=4, inter=8192, seed=9):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.heads, self.kv_heads, self.hd = heads, kv_heads, hidden // heads

        def lin(i, o):
            m = torch.nn.Linear(i, o, bias=False)
            m.weight.data = (torch.randn(o, i, generator=g) * 0.02).to(torch.bfloat16)
            return m

        self.q_proj, self.k_proj = lin(hidden, hidden), lin(hidden, kv_heads * self.hd)
        self.v_proj, self.o_proj = lin(hidden, kv_heads * self.hd), lin(hidden, hidden)
        self.gate_proj, self.up_proj, self.down_proj = lin(hidden, inter), lin(hidden, inter), lin(inter, hidden)

    @staticmethod
    def _rms(x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype)

    def forward(self, x):
        B, T, D = x.shape
        h = self._rms(x)
        q = self.q_proj(h).view(B, T, self.heads, self.hd).transpose(1, 2).float()
        k = self.k_proj(h).view(B, T, self.kv_heads, self.hd).transpose(1, 2).float()
        v = self.v_proj(h).view(B, T, self.kv_heads, self.hd).transpose(1, 2).float()
        rep = self.heads // self.kv_heads
        k, v = k.repeat_interleave(rep, dim=1).contiguous(), v.repeat_interleave(rep, dim=1).contiguous()
        a = F.scaled_dot_product_attention(q, k, v, is_causal=True)      # fp32 attention
        x = x + self.o_proj(a.transpose(1, 2).reshape(B, T, D).to(x.dtype))
        h = self._rms(x)
        return x + self.down_proj(F.silu(self.gate_proj(h)) * self.up_proj(h))


def test_decoder_layer_gptq_modifier_vs_oracle(dev):
    say("decoder layer (hidden 1024, inter 8192) through GPTQModifier vs the oracle")
    layer = LlamaLayer().to(dev)
    W0 = {n: m.weight.detach().cpu().clone() for n, m in layer.named_children()}
    seen = {n: [] for n in W0}

    def capture(name):
        return lambda mod, args: seen[name].append(args[0].detach().cpu())

    hooks = [m.register_forward_pre_hook(capture(n)) for n, m in layer.named_children()]
    batches = [_gpu_heavy((2, 2048, 1024), 100 + b, dev) for b in range(4)]
    mod = GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=())   # actorder static -> weight
    mod.apply(layer, batches)
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    oa = OArgs(num_bits=4, strategy="group", group_size=128, actorder="weight")
    for name, m in layer.named_children():
        xs = seen[name]
        cols = xs[0].shape[-1]
        # the GPU Hessian the modifier accumulated (same kernel, rows and
        # staged calls: the same bits)
        lin = torch.nn.Linear(cols, 1, bias=False, device=dev)
        Hg, ng = gptq.make_empty_hessian(lin), torch.zeros((), device=dev)
        Ho, no = og.make_empty_hessian(cols), torch.zeros(())
        stage = HessianStage()
        for x in xs:
            rows, added = gptq.hessian_rows(x, lin, dev)
            ng += added
            stage.add(rows, added, lambda r, _s: ops.hessian_syrk_(Hg, r, alpha=2.0))
            Ho, no = og.accumulate_hessian(x, Ho, no)
        stage.flush(lambda r, _s: ops.hessian_syrk_(Hg, r, alpha=2.0))
        Hg = Hg.cpu()
        assert float(ng) == float(no) == 8.0
        r = rel_fro(torch.triu(Hg), torch.triu(Ho))
        assert r <= 1e-5, (name, r)
        _, out_o, ex = og.quantize_weight(W0[name], oa, _full(Hg) / float(no), return_codes=True)
        assert torch.equal(m.weight_scale.detach().cpu(), out_o["weight_scale"]), name
        _check_codes(f"{name} {tuple(W0[name].shape)} H rel {r:.2e}", m.gptq_codes, ex["codes"], W0[name],
                     m.weight.detach(), out_o["weight"], xs[0][:1])


def test_hinv_d14336_vs_oracle_chain(dev):
    d, n = 14336, 16384
    say(f"cholesky chain d={d} ({n} tokens) vs the oracle's chain")
    x = _gpu_heavy((n, d), 7, dev)
    H = torch.zeros(d, d, device=dev)
    ops.hessian_syrk_(H, x, alpha=2.0)
    del x
    hinv, dead, ok = ops.gptq_hinv(H, None, float(n), 0.01)
    assert ok and int(dead.sum()) == 0
    hinv = hinv.cpu()
    Hc = _full(H.cpu()) / float(n)
    del H
    U, ok_o = og.cholesky_chain(Hc, 0.01)
    assert ok_o
    r = rel_fro(hinv, U)
    say(f"  rel {r:.3e}")
    assert r <= 1e-4
    assert torch.equal(hinv, torch.triu(hinv))


def test_moe_batched_solve_128_experts_vs_oracle(dev):
    B, rows, cols, tok = 128, 768, 2048, 1024
    say(f"batched GPTQ of {B} experts {rows}x{cols} vs oracle solves of sampled experts")
    g = torch.Generator(device=dev).manual_seed(6)
    W = (torch.randn(B, rows, cols, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    X = _gpu_heavy((B, tok, cols), 8, dev)
    H = torch.zeros(B, cols, cols, device=dev)
    for b in range(B):
        ops.hessian_syrk_(H[b], X[b], alpha=2.0)
    qa = QuantizationArgs(num_bits=4, type="int", symmetric=True, strategy="group", group_size=128,
                          actorder="weight")
    res = gptq.gptq_quantize_batched(W, qa, H.clone(), num_samples=1.0)
    oa = OArgs(num_bits=4, strategy="group", group_size=128, actorder="weight")
    for b in (0, 37, 90, 127):
        Xb, Hb = X[b].cpu(), H[b].cpu()
        Ho, no = og.accumulate_hessian(Xb, og.make_empty_hessian(cols), torch.zeros(()))
        r = rel_fro(torch.triu(Hb), torch.triu(Ho))
        assert r <= 1e-5, (b, r)
        assert res[b].hinv_ok
        _, out_o, ex = og.quantize_weight(W[b].cpu(), oa, _full(Hb), return_codes=True)
        assert torch.equal(res[b].scale.cpu().to(torch.bfloat16).reshape(out_o["weight_scale"].shape),
                           out_o["weight_scale"])
        _check_codes(f"expert {b}", res[b].codes, ex["codes"], W[b].cpu(), res[b].weight, out_o["weight"], Xb[:512])
