"""GPU: Hessians accumulated through the modifiers' staging (calibration
calls gathered into longer syrk calls) equal the per-call accumulation up to
the order of fp32 additions - both the GPTQ sum (H += 2 X^T X) and the
SparseGPT running mean - and match the oracle."""
import pytest
import torch

from llmcompressor_amd import gptq, ops, sparsegpt, workloads
from llmcompressor_amd.staging import HessianStage
from oracle import gptq as og

pytestmark = pytest.mark.gpu

SIZES = [2048] * 7 + [12000] + [2048] * 3 + [1000]   # one call past half the buffer, a ragged tail


def _rel(a, b):
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def _batches(d, dev):
    return [workloads.heavy_tailed_activations((1, n, d), seed=300 + i).to(dev) for i, n in enumerate(SIZES)]


def test_gptq_staged_hessian_matches_per_call(dev):
    print("GPTQ Hessian: staged calls vs one syrk per call vs the oracle", flush=True)
    d = 1024
    lin = torch.nn.Linear(d, 1, bias=False, device=dev)
    xs = _batches(d, dev)
    H1, n1 = gptq.make_empty_hessian(lin), torch.zeros((), device=dev)
    for x in xs:
        H1, n1 = gptq.accumulate_hessian(x, lin, H1, n1)
    H2, n2 = gptq.make_empty_hessian(lin), torch.zeros((), device=dev)
    stage, calls = HessianStage(16384), []

    def flush(segs, samples):
        calls.append(sum(s.shape[0] for s in segs))
        ops.hessian_syrk_segments_(H2, segs, alpha=2.0)
    for x in xs:
        rows, added = gptq.hessian_rows(x, lin, dev)
        n2 += added
        stage.add(rows, added, flush)
    stage.flush(flush)
    assert calls == [14336, 12000, 7144], calls
    assert float(n1) == float(n2) == len(SIZES)
    r = _rel(torch.triu(H2), torch.triu(H1))
    assert r <= 2e-6, r
    Ho, no = og.make_empty_hessian(d), torch.zeros(())
    for x in xs:
        Ho, no = og.accumulate_hessian(x.cpu(), Ho, no)
    assert _rel(torch.triu(H2).cpu(), torch.triu(Ho)) <= 1e-5


def test_sparsegpt_staged_running_mean_matches_per_call(dev):
    print("SparseGPT running-mean Hessian: staged calls vs one syrk per call", flush=True)
    d = 768
    lin = torch.nn.Linear(d, 1, bias=False, device=dev)
    xs = _batches(d, dev)
    H1, n1 = sparsegpt.make_empty_hessian(lin), 0
    for x in xs:
        H1, n1 = sparsegpt.accumulate_hessian(x, lin, H1, n1)
    H2, n2, folded = sparsegpt.make_empty_hessian(lin), 0, [0]
    stage = HessianStage()

    def flush(segs, samples):
        folded[0] = sparsegpt.fold_rows(H2, segs, folded[0], samples)
    for x in xs:
        rows, added = sparsegpt.hessian_rows(x, lin, dev)
        n2 += added
        stage.add(rows, added, flush)
    stage.flush(flush)
    assert n1 == n2 == folded[0] == len(SIZES)
    r = _rel(torch.triu(H2), torch.triu(H1))
    assert r <= 2e-6, r


def test_gptq_modifier_staged_matches_unstaged(dev):
    """Three layers fed different inputs, six 2048-token batches; a budget
    for one stage (the other two layers accumulate per call), against the
    modifier without staging: the same scales, codes within the GPTQ code
    bar (the Hessians differ in the order of fp32 additions)."""
    print("GPTQModifier: staged (one stage in the budget) vs per-call Hessians", flush=True)
    import copy
    from llmcompressor_amd import GPTQModifier
    from parity_util import code_agreement, code_bar
    torch.manual_seed(0)
    model = torch.nn.Sequential(*[torch.nn.Linear(512, 512, bias=False) for _ in range(3)]).to(dev).to(torch.bfloat16)
    batches = [workloads.heavy_tailed_activations((1, 2048, 512), seed=400 + i).to(dev) for i in range(6)]
    ref = copy.deepcopy(model)
    # no activation ordering: a permutation from diag(H) could swap two near-equal entries
    GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), actorder=None,
                 hessian_batch_tokens=0).apply(ref, batches)
    mod = GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), actorder=None,
                       hessian_stage_bytes=65536 * 512 * 2)
    mod.apply(model, batches)
    assert mod._stage_held == 0 and not mod._stages
    for a, b in zip(model, ref):
        assert torch.equal(a.weight_scale, b.weight_scale)
        st = code_agreement(a.gptq_codes.cpu().int(), b.gptq_codes.cpu().int())
        assert code_bar(st, a.weight.shape[0]), st
