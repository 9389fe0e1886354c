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
  and of 2048 x 768 (the down projection) against oracle solves of sampled
  experts.
* NVFP4 through GPTQModifier on a Llama-shaped layer: q/k/v and gate/up
  share their global scales, as the oracle computes them.

GPTQ code bars as in test_gpu_parity.py's end-to-end tests.
"""
import pytest
import torch
import torch.nn.functional as F

from llmcompressor_amd import GPTQModifier, gptq, ops
from llmcompressor_amd.staging import HessianStage
from llmcompressor_amd.quant_args import QuantizationArgs
from oracle import gptq as og
from oracle.fake_quant import signed_grid_index
from oracle.observers import OMinMax, global_scale_from_stats
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


def _modifier_hessian(xs, dev, name):
    """The Hessian GPTQModifier accumulated from the inputs ``xs`` (same
    kernel, rows and staged calls: the same bits), on the host, checked
    against the oracle's to 1e-5: (H upper, num_samples, relative error)."""
    cols = xs[0].shape[-1]
    lin = torch.nn.Linear(cols, 1, bias=False, device=dev)
    Hg, ng = gptq.make_empty_hessian(lin), torch.zeros((), device=dev)
    Ho, no = og.make_empty_hessian(cols), torch.zeros(())
    stage = HessianStage()
    for x in xs:
        rows, added = gptq.hessian_rows(x, lin, dev)
        ng += added
        stage.add(rows, added, lambda segs, _s: ops.hessian_syrk_segments_(Hg, segs, alpha=2.0))
        Ho, no = og.accumulate_hessian(x, Ho, no)
    stage.flush(lambda segs, _s: ops.hessian_syrk_segments_(Hg, segs, alpha=2.0))
    Hg = Hg.cpu()
    assert float(ng) == float(no)
    r = rel_fro(torch.triu(Hg), torch.triu(Ho))
    assert r <= 1e-5, (name, r)
    return Hg, float(no), r


def _capture_inputs(layer):
    seen = {n: [] for n, _ in layer.named_children()}

    def capture(name):
        return lambda mod, args: seen[name].append(args[0].detach().cpu())

    hooks = [m.register_forward_pre_hook(capture(n)) for n, m in layer.named_children()]
    return seen, hooks


def test_decoder_layer_gptq_modifier_vs_oracle(dev):
    say("decoder layer (hidden 1024, inter 8192) through GPTQModifier vs the oracle")
    layer = LlamaLayer().to(dev)
    W0 = {n: m.weight.detach().cpu().clone() for n, m in layer.named_children()}
    seen, hooks = _capture_inputs(layer)
    batches = [_gpu_heavy((2, 2048, 1024), 100 + b, dev) for b in range(4)]
    mod = GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=())   # actorder static -> weight
    mod.apply(layer, batches)
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    oa = OArgs(num_bits=4, strategy="group", group_size=128, actorder="weight")
    for name, m in layer.named_children():
        Hg, no, r = _modifier_hessian(seen[name], dev, name)
        assert no == 8.0
        _, out_o, ex = og.quantize_weight(W0[name], oa, _full(Hg) / no, return_codes=True)
        assert torch.equal(m.weight_scale.detach().cpu(), out_o["weight_scale"]), name
        _check_codes(f"{name} {tuple(W0[name].shape)} H rel {r:.2e}", m.gptq_codes, ex["codes"], W0[name],
                     m.weight.detach(), out_o["weight"], seen[name][0][:1])


FUSED = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


def test_decoder_layer_nvfp4_fused_global_scales_vs_oracle(dev):
    """NVFP4 (tensor-group 16, fp8 group scales, one global scale) through
    GPTQModifier on a Llama-shaped layer: q/k/v and gate/up share one global
    scale each (observers/fusion.py:17-105, observers/helpers.py:161-215,
    wired at modifiers/quantization/quantization/mixin.py:381-382; the
    reference's test_gptq_quantize.py:179-213 asserts the equalities), equal
    to the oracle's generate_gparam over the group's combined statistics,
    rounded to bf16 as quantize_weight returns it and held in the fp32
    parameter; o and down keep their own.  Codes pass the bar against oracle
    solves with the fused global scale."""
    say("decoder layer NVFP4 through GPTQModifier: fused global scales")
    layer = LlamaLayer(hidden=512, heads=8, kv_heads=2, inter=1536, seed=19).to(dev)
    with torch.no_grad():   # members of one set with different ranges
        layer.k_proj.weight.mul_(3)
        layer.up_proj.weight.mul_(2)
    W0 = {n: m.weight.detach().cpu().clone() for n, m in layer.named_children()}
    seen, hooks = _capture_inputs(layer)
    batches = [_gpu_heavy((2, 1024, 512), 200 + b, dev) for b in range(2)]
    GPTQModifier(scheme="NVFP4A16", targets=("Linear",), ignore=()).apply(layer, batches)
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    E4 = torch.float8_e4m3fn
    oa = OArgs(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=E4,
               actorder="weight")
    stats = {}
    for n, w in W0.items():
        o = OMinMax("memoryless_minmax", "weight", oa)
        o(w)
        stats[n] = (o.min_vals, o.max_vals)
    gs = {n: getattr(layer, n).weight_global_scale for n in W0}
    assert all(v.dtype == torch.float32 and v.shape == (1,) for v in gs.values())
    group_of = {n: grp for grp in FUSED for n in grp}
    for n in W0:
        grp = group_of.get(n, (n,))
        want = global_scale_from_stats([stats[m] for m in grp]).to(torch.bfloat16).float()
        assert float(gs[n]) == float(want), n
        assert float(gs[n]) == float(gs[grp[0]]), n
    assert float(gs["q_proj"]) != float(gs["gate_proj"])
    # fused scales differ from what each member alone would get
    own_k = global_scale_from_stats([stats["k_proj"]]).to(torch.bfloat16).float()
    own_q = global_scale_from_stats([stats["q_proj"]]).to(torch.bfloat16).float()
    assert float(own_q) != float(gs["q_proj"]) and float(own_k) == float(gs["q_proj"])
    for name, m in layer.named_children():
        Hg, no, r = _modifier_hessian(seen[name], dev, name)
        obs = OMinMax("memoryless_minmax", "weight", oa)
        obs(W0[name])
        obs.fused_stats = [stats[o] for o in group_of.get(name, (name,)) if o != name]
        _, out_o, ex = og.quantize_weight(W0[name], oa, _full(Hg) / no, observer=obs, return_codes=True)
        assert torch.equal(m.weight_scale.detach().cpu().float(), out_o["weight_scale"].float()), name
        gi = signed_grid_index(m.gptq_codes.cpu().to(torch.int32), oa)
        gio = signed_grid_index(ex["codes"], oa)
        st = code_agreement(gi, gio)
        Xf = seen[name][0][:1].reshape(-1, W0[name].shape[1]).float()
        e_gpu = (Xf @ (W0[name].float() - m.weight.detach().cpu().float()).t()).norm().item()
        e_ora = (Xf @ (W0[name].float() - out_o["weight"].float()).t()).norm().item()
        say(f"  {name}: gs {float(gs[name]):.6g} {st} err {e_gpu:.6g} vs {e_ora:.6g}")
        assert code_bar(st, W0[name].shape[0]), name
        assert abs(e_gpu - e_ora) <= 0.005 * e_ora, name


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


@pytest.mark.parametrize("rows,cols,tok", [(768, 2048, 1024), (2048, 768, 512)], ids=["gate_up", "down"])
def test_moe_batched_solve_128_experts_vs_oracle(dev, rows, cols, tok):
    """One batched solve of 128 experts of an MoE projection: gate / up
    (768 x 2048) and down (2048 x 768, the 262144-row batch)."""
    B = 128
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
