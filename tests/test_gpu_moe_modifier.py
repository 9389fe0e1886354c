"""MoE experts through GPTQModifier against the oracle.

A block of 16 gated experts (``LinearExperts``: the reference's
``LinearExperts2D`` forward, ``modeling/moe/linear_experts.py:244-277``)
routed top-2 with a skewed router and one expert that receives no token,
calibrated by ``GPTQModifier`` over two forwards.  The expert projections
form families: each forward's routed rows go to one grouped syrk per family
(gate and up share their input, hence one Hessian), and each family is
solved in one batched solve per projection.  Per expert and projection the
oracle accumulates its own Hessian from the rows the expert's hook received
(``gptq_quantize.py:63-97``: one sample per 2-D call, also for an empty
call) and solves it (``:100-296``): Hessians within 1e-5, sample counts
equal, scales equal, every row's first code divergence +-1 and layer error
within 0.5 % per expert, and the end-to-end code bar over each projection
of the layer (all experts' codes together: one row that diverges in a
256-row expert is already 0.2 % of that expert's codes).  The empty expert's Hessian is zero, so every column is dead and its
weight quantizes to zero, as in the reference.
"""
import pytest
import torch

from llmcompressor_amd import GPTQModifier, modifiers
from llmcompressor_amd.moe import LinearExperts, moe_calibration_context
from oracle import gptq as og
from oracle.qargs import OArgs
from parity_util import code_agreement, code_bar

pytestmark = pytest.mark.gpu

E, HIDDEN, INTER, TOKENS, TOPK, EMPTY = 16, 512, 256, 2048, 2, 5


def say(*a):
    print(*a, flush=True)


class MoEBlock(torch.nn.Module):
    def __init__(self, dev, seed=3):
        super().__init__()
        g = torch.Generator(device=dev).manual_seed(seed)
        gate = (torch.randn(E, INTER, HIDDEN, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        up = (torch.randn(E, INTER, HIDDEN, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        down = (torch.randn(E, HIDDEN, INTER, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        self.experts = LinearExperts.from_stacked(gate, up, down)
        # a Zipf-skewed prior; one expert never chosen
        prior = torch.log(1.0 / torch.arange(1, E + 1, dtype=torch.float32, device=dev) ** 1.1)
        prior[EMPTY] = -1e4
        self.register_buffer("prior", prior)
        self.register_buffer("router", torch.randn(E, HIDDEN, generator=g, device=dev) * 0.05)

    def forward(self, x):
        h = x.reshape(-1, x.shape[-1])
        logits = h.float() @ self.router.t() + self.prior
        w, idx = torch.topk(torch.softmax(logits, -1), TOPK, dim=-1)
        return self.experts(h, idx, (w / w.sum(-1, keepdim=True)).to(h.dtype)).reshape(x.shape)


def _heavy(dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    z = torch.randn(TOKENS, HIDDEN, generator=g, device=dev)
    chi = sum(torch.randn(TOKENS, HIDDEN, generator=g, device=dev) ** 2 for _ in range(4))
    c = torch.exp(torch.randn(HIDDEN, generator=g, device=dev))
    return (z / torch.sqrt(chi / 4) * c).to(torch.bfloat16).reshape(1, TOKENS, HIDDEN)


@pytest.mark.parametrize("calibrate_all", [False, True], ids=["routed", "all_experts"])
def test_moe_experts_through_gptq_modifier_vs_oracle(dev, monkeypatch, calibrate_all):
    say(f"MoE {E} experts through GPTQModifier (calibrate all experts: {calibrate_all})")
    block = MoEBlock(dev)
    W0 = {n: m.weight.detach().cpu().clone() for n, m in block.named_modules() if isinstance(m, torch.nn.Linear)}
    seen = {n: [] for n in W0}
    hooks = [m.register_forward_pre_hook(lambda mod, a, _n=n: seen[_n].append(a[0].detach().cpu()))
             for n, m in block.named_modules() if isinstance(m, torch.nn.Linear)]
    batched = []
    real = modifiers.gptq_quantize_batched

    def counting(weights, *a, **k):
        batched.append(tuple(weights.shape))
        return real(weights, *a, **k)

    monkeypatch.setattr(modifiers, "gptq_quantize_batched", counting)
    mod = GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=())
    mod.on_initialize(block)
    fams = {id(f): f for f in mod._families.values()}
    assert sorted(f.key for f in fams.values()) == ["experts.*.down_proj", "experts.*.gate_proj",
                                                  "experts.*.up_proj"]
    hess = {}
    for f in fams.values():
        flush = f.flush

        def snap(f=f, flush=flush):
            flush()
            if f.H is not None:
                hess[f.key] = f.H.detach().cpu().clone()
        f.flush = snap
    mod.on_calibration_start(block)
    batches = [_heavy(dev, 10 + b) for b in range(2)]
    with torch.no_grad():
        if calibrate_all:
            with moe_calibration_context():
                for b in batches:
                    block(b)
        else:
            for b in batches:
                block(b)
    mod.on_calibration_end()
    mod.on_sequential_epoch_end(list(mod._modules))
    mod.on_finalize()
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    # gate and up (one shared Hessian) as one stack of rows, then down
    assert batched == [(E, 2 * INTER, HIDDEN), (E, HIDDEN, INTER)]
    assert set(hess) == {"experts.*.gate_proj", "experts.*.down_proj"}   # up shares gate's
    oa = OArgs(num_bits=4, strategy="group", group_size=128, actorder="weight")
    counts = [seen[f"experts.{e}.gate_proj"] for e in range(E)]
    say("  routed rows per expert: " + " ".join(str(sum(x.shape[0] for x in c)) for c in counts))
    assert sum(x.shape[0] for x in counts[EMPTY]) == (2 * TOKENS if calibrate_all else 0)
    layer_codes = {p: ([], []) for p in ("gate_proj", "up_proj", "down_proj")}
    for e in range(E):
        for proj, fam_key in (("gate_proj", "gate_proj"), ("up_proj", "gate_proj"), ("down_proj", "down_proj")):
            name = f"experts.{e}.{proj}"
            m = block.get_submodule(name)
            xs = seen[name]
            cols = W0[name].shape[1]
            Ho, no = og.make_empty_hessian(cols), torch.zeros(())
            for x in xs:
                Ho, no = og.accumulate_hessian(x, Ho, no)
            assert float(no) == 2.0
            Hg = torch.triu(hess[f"experts.*.{fam_key}"][e])
            if float(Ho.abs().max()) == 0:
                assert float(Hg.abs().max()) == 0, name
                r = 0.0
            else:
                r = ((Hg.double() - torch.triu(Ho).double()).norm() / torch.triu(Ho).double().norm()).item()
            assert r <= 1e-5, (name, r)
            _, out_o, ex = og.quantize_weight(W0[name], oa, og.normalise_hessian(Ho, no), return_codes=True)
            assert torch.equal(m.weight_scale.detach().cpu(), out_o["weight_scale"]), name
            st = code_agreement(m.gptq_codes.cpu().to(torch.int32), ex["codes"])
            layer_codes[proj][0].append(m.gptq_codes.cpu().to(torch.int32))
            layer_codes[proj][1].append(ex["codes"])
            X = torch.cat([x.reshape(-1, cols) for x in xs]).float()
            if X.shape[0] == 0:
                assert torch.equal(m.weight.detach().cpu(), out_o["weight"]), name
                assert int(m.gptq_codes.abs().sum()) == 0
                continue
            e_gpu = (X @ (W0[name].float() - m.weight.detach().cpu().float()).t()).norm().item()
            e_ora = (X @ (W0[name].float() - out_o["weight"].float()).t()).norm().item()
            if st["mismatches"] or e == 0:
                say(f"  {name}: rows {X.shape[0]} H rel {r:.2e} {st} err {e_gpu:.6g} vs {e_ora:.6g}")
            assert st["first_divergence_max"] <= 1, name
            assert abs(e_gpu - e_ora) <= 0.005 * e_ora + 1e-12, name
    for proj, (ours, theirs) in layer_codes.items():
        st = code_agreement(torch.cat(ours), torch.cat(theirs))
        say(f"  {proj} over all experts: {st}")
        assert code_bar(st, sum(c.shape[0] for c in ours)), proj
