"""GPU parity: every kernel against the CPU oracle on the same seeded inputs.

Bars: bit-exact for observers / quantize / pack; Hessian relative Frobenius
error <= 1e-5 (upper triangle); Cholesky chain within 1e-4 relative.

GPTQ codes: given the oracle's own Hinv, the GPU sweep reproduces the
oracle's codes with every mismatch within 1 LSB (only the lazy-update GEMMs'
summation order differs).  End to end (the GPU's own Cholesky chain), codes
agree on >= 99.9 % of entries, every row's first divergence is +-1, at most
1 % of the rows diverge, and ||WX - Q(W)X|| is within 0.5 % of the oracle's
(parity_util.code_bar).  Codes after a row's first flip can differ by more
than one: GPTQ feeds each rounding error into the row's later columns, and
the oracle against itself with its BLAS on 1 thread instead of all cores
gives codes up to 3 apart at 4096 x 4096 (tests/gptq_code_spread.py), so a
+-1 bound on every code holds for no fp32 implementation that is not
bit-identical to the oracle's LAPACK.
"""
import numpy as np
import pytest
import torch

from llmcompressor_amd import gptq, moe, ops, workloads
from llmcompressor_amd.calibration import initialize_module_for_quantization, initialize_observer, observe
from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs, QuantizationScheme
from oracle import fake_quant as ofq
from oracle import gptq as og
from oracle import moe as omoe
from oracle import observers as oobs
from oracle import pack as opack
from oracle.qargs import OArgs
from parity_util import code_agreement, code_bar

pytestmark = pytest.mark.gpu

HESS_TOL = 1e-5


def say(*a):
    print(*a, flush=True)


def rel_fro(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


# ---------------------------------------------------------------- Hessian
# (16384, 512): every tile split into parts; (16500, 2304) and (16384, 4096):
# full tiles plus split tail tiles
@pytest.mark.parametrize("n,d", [(300, 64), (2048, 256), (5000, 384), (16384, 512), (4100, 1000), (16500, 2304),
                                 (16384, 4096)])
def test_hessian_syrk_parity(dev, n, d):
    say(f"hessian syrk n={n} d={d}")
    x = workloads.heavy_tailed_activations((n, d), seed=n + d)
    g = torch.Generator().manual_seed(1)
    h0 = torch.randn(d, d, generator=g)
    H = h0.clone().to(dev)
    ops.hessian_syrk_(H, x.to(dev), alpha=2.0)
    Ho, _ = og.accumulate_hessian(x, h0.clone(), torch.zeros(()))
    got = H.cpu()
    iu = torch.triu_indices(d, d)
    r = rel_fro(got[iu[0], iu[1]], Ho[iu[0], iu[1]])
    assert r <= HESS_TOL, r
    il = torch.tril_indices(d, d, -1)
    assert torch.equal(got[il[0], il[1]], h0[il[0], il[1]])  # strictly-lower part untouched
    H2 = h0.clone().to(dev)
    ops.hessian_syrk_(H2, x.to(dev), alpha=2.0)
    assert torch.equal(H2.cpu(), got)  # deterministic


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64], ids=["fp16", "fp32", "fp64"])
@pytest.mark.parametrize("n,d", [(777, 200), (5000, 384), (16384, 1024), (3000, 100)])
def test_hessian_other_input_dtypes(dev, dtype, n, d):
    """Calibration activations in fp16 / fp32 / fp64 through the drop-in
    accumulate_hessian (the reference casts every input to fp32,
    gptq_quantize.py:93): fp16 on the 16-bit MFMA kernels (exact products),
    fp32 on the fp32 MFMA product, fp64 converted to fp32 first; d = 100 is
    not a multiple of 8 (fp16 then also takes the fp32 product)."""
    say(f"hessian {dtype} n={n} d={d}")
    g = torch.Generator().manual_seed(n + d)
    x = (torch.randn(n, d, generator=g) * torch.exp(torch.randn(d, generator=g))).to(dtype)
    lin = torch.nn.Linear(d, 8, bias=False).to(dev)
    H, cnt = gptq.make_empty_hessian(lin), torch.zeros((), device=dev)
    H, cnt = gptq.accumulate_hessian(x.unsqueeze(0).to(dev), lin, H, cnt)
    H, cnt = gptq.accumulate_hessian(x[: n // 3].unsqueeze(0).to(dev), lin, H, cnt)
    Ho, no = og.accumulate_hessian(x.unsqueeze(0), og.make_empty_hessian(d), torch.zeros(()))
    Ho, no = og.accumulate_hessian(x[: n // 3].unsqueeze(0), Ho, no)
    assert float(cnt) == float(no) == 2.0
    r = rel_fro(torch.triu(H.cpu()), torch.triu(Ho))
    assert r <= HESS_TOL, r
    assert torch.count_nonzero(torch.tril(H, -1)) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
def test_hessian_grouped_other_dtypes(dev, dtype):
    say(f"grouped hessian {dtype}")
    T, d, E = 2000, 256, 5
    g = torch.Generator().manual_seed(13)
    hs = (torch.randn(T, d, generator=g) * 3).to(dtype)
    idx = torch.randint(0, E, (T, 2), generator=g)
    idx[:, 1] = (idx[:, 0] + 1 + torch.randint(0, E - 1, (T,), generator=g)) % E
    rows, offsets, _ = moe.route_tokens(idx.to(dev), E)
    H = torch.zeros(E, d, d, device=dev)
    ns = torch.zeros(E, device=dev)
    moe.accumulate_expert_hessians(hs.to(dev), rows, offsets, H, ns)
    Ho, no = omoe.expert_hessians(hs, idx, E)
    for e in range(E):
        assert rel_fro(torch.triu(H[e].cpu()), torch.triu(Ho[e])) <= HESS_TOL, e


def test_hessian_running_mean_fp16(dev):
    """SparseGPT's running-mean Hessian (sgpt_sparsify.py:48-53) on fp16 input."""
    from llmcompressor_amd import sparsegpt
    from oracle import sparsegpt as osg
    say("sparsegpt running-mean hessian fp16")
    g = torch.Generator().manual_seed(3)
    xs = [(torch.randn(2, 300, 256, generator=g) * 2).to(torch.float16) for _ in range(3)]
    lin = torch.nn.Linear(256, 8, bias=False).to(dev)
    H, n = sparsegpt.make_empty_hessian(lin), 0
    Ho, no = osg.make_empty_hessian(256), 0
    for x in xs:
        H, n = sparsegpt.accumulate_hessian(x.to(dev), lin, H, n)
        Ho, no = osg.accumulate_hessian(x, Ho, no)
    assert rel_fro(torch.triu(H.cpu()), torch.triu(Ho)) <= HESS_TOL


def test_hessian_syrk_many_tiles(dev):
    """d = 8192 (528 tiles, so at most two token splits): upper triangle
    against an fp64 product on the GPU."""
    n, d = 16384, 8192
    say(f"hessian syrk n={n} d={d} (fp64 GPU reference)")
    x = workloads.heavy_tailed_activations((n, d), seed=5).to(dev)
    H = torch.zeros(d, d, device=dev)
    ops.hessian_syrk_(H, x, alpha=2.0)
    xd = x.double()
    ref = 2.0 * (xd.t().contiguous() @ xd)
    up = torch.triu(torch.ones(d, d, dtype=torch.bool, device=dev))
    r = ((H.double() - ref)[up].norm() / ref[up].norm()).item()
    assert r <= HESS_TOL, r
    assert torch.count_nonzero(torch.tril(H, -1)) == 0


def test_hessian_dropin_counts_and_strided_input(dev):
    say("accumulate_hessian drop-in")
    lin = torch.nn.Linear(128, 16, bias=False).to(dev)
    H = gptq.make_empty_hessian(lin)
    n = torch.zeros((), device=dev)
    x3 = workloads.heavy_tailed_activations((3, 40, 128), seed=3)
    x2 = workloads.heavy_tailed_activations((17, 256), seed=4)[:, ::2]  # strided 2-D view
    H, n = gptq.accumulate_hessian(x3.to(dev), lin, H, n)
    H, n = gptq.accumulate_hessian(x2.to(dev), lin, H, n)
    assert n.item() == 4
    Ho = og.make_empty_hessian(128)
    no = torch.zeros(())
    Ho, no = og.accumulate_hessian(x3, Ho, no)
    Ho, no = og.accumulate_hessian(x2, Ho, no)
    assert rel_fro(torch.triu(H.cpu()), torch.triu(Ho)) <= HESS_TOL
    gptq.symmetrize_hessian(H)
    assert rel_fro(H.cpu(), Ho) <= HESS_TOL


@pytest.mark.parametrize("k,stride,pad,dil", [(1, 1, 0, 1), (3, 1, 1, 1), (3, 2, 1, 2)])
def test_hessian_conv2d_unfold(dev, k, stride, pad, dil):
    """Conv2d inputs through the drop-in accumulate_hessian (gptq_quantize.py:
    80-89): the unfolded patches' Hessian against the oracle's, the batch as
    the sample count; the 1 x 1 kernel with make_empty_hessian's size."""
    say(f"conv2d hessian k={k} stride={stride} pad={pad} dil={dil}")
    C = 96
    conv = torch.nn.Conv2d(C, 16, k, stride=stride, padding=pad, dilation=dil).to(dev)
    d = C * k * k
    x = workloads.heavy_tailed_activations((4 * 20 * 24, C), seed=k + stride).reshape(4, 20, 24, C)
    x = x.permute(0, 3, 1, 2).contiguous()        # [B, C, h, w] bf16
    H = gptq.make_empty_hessian(conv) if k == 1 else torch.zeros(d, d, device=dev)
    n = torch.zeros((), device=dev)
    H, n = gptq.accumulate_hessian(x.to(dev), conv, H, n)
    Ho, no = og.accumulate_hessian_conv2d(x, torch.zeros(d, d), torch.zeros(()), k, dil, pad, stride)
    assert float(n) == float(no) == 4.0
    assert rel_fro(torch.triu(H.cpu()), torch.triu(Ho)) <= HESS_TOL


def test_sparsegpt_hessian_conv2d_unfold(dev):
    """The running-mean Hessian of a 1 x 1 Conv2d (sgpt_sparsify.py:37-45)."""
    from llmcompressor_amd import sparsegpt
    from oracle import sparsegpt as osg
    say("sparsegpt conv2d hessian")
    C = 64
    conv = torch.nn.Conv2d(C, 8, 1).to(dev)
    xs = [workloads.heavy_tailed_activations((2 * 10 * 12, C), seed=40 + i).reshape(2, 10, 12, C)
          .permute(0, 3, 1, 2).contiguous() for i in range(3)]
    H, n = sparsegpt.make_empty_hessian(conv), 0
    Ho, no = osg.make_empty_hessian(C), 0
    for x in xs:
        H, n = sparsegpt.accumulate_hessian(x.to(dev), conv, H, n)
        # the 1 x 1 patches are the pixels' channel vectors: the Linear form of the oracle
        Ho, no = osg.accumulate_hessian(x.permute(0, 2, 3, 1).reshape(2, -1, C), Ho, no)
    assert n == no == 6
    assert rel_fro(torch.triu(H.cpu()), torch.triu(Ho)) <= HESS_TOL


def test_hessian_grouped_parity(dev):
    say("grouped hessian")
    T, d, E = 3000, 256, 6
    hs = workloads.heavy_tailed_activations((T, d), seed=11)
    g = torch.Generator().manual_seed(12)
    idx = torch.randint(0, E, (T, 2), generator=g)
    idx[:, 1] = (idx[:, 0] + 1 + torch.randint(0, E - 1, (T,), generator=g)) % E
    idx[idx == 4] = 0  # expert 4 receives nothing
    rows, offsets, _ = moe.route_tokens(idx.to(dev), E)
    H = torch.zeros(E, d, d, device=dev)
    ns = torch.zeros(E, device=dev)
    moe.accumulate_expert_hessians(hs.to(dev), rows, offsets, H, ns)
    Ho, no = omoe.expert_hessians(hs, idx, E)
    assert torch.equal(ns.cpu(), no)
    lists = omoe.expert_token_lists(idx, E)
    for e in range(E):
        assert torch.equal(rows[offsets[e]:offsets[e + 1]].cpu().long(), lists[e])
        if offsets[e + 1] == offsets[e]:
            assert torch.count_nonzero(H[e]) == 0
            continue
        assert rel_fro(torch.triu(H[e].cpu()), torch.triu(Ho[e])) <= HESS_TOL, e


def _grouped_case(counts, n_x, d, dtype, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = (torch.randn(n_x, d, generator=g, device=dev) * torch.exp(torch.randn(d, generator=g, device=dev))).to(dtype)
    rows = torch.cat([torch.randint(0, n_x, (c,), generator=g, device=dev) for c in counts]).to(torch.int32)
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    return x, rows, offsets


def _grouped_check(H, x, rows, offsets, alpha=2.0):
    for e in range(len(offsets) - 1):
        a, b = offsets[e], offsets[e + 1]
        if a == b:
            assert torch.count_nonzero(H[e]) == 0, e
            continue
        xe = (x[a:b] if rows is None else x[rows[a:b].long()]).double()
        ref = alpha * (xe.t().contiguous() @ xe)
        up = torch.triu(torch.ones_like(ref, dtype=torch.bool))
        r = ((H[e].double() - ref)[up].norm() / ref[up].norm()).item()
        assert r <= HESS_TOL, (e, b - a, r)
        assert torch.count_nonzero(torch.tril(H[e], -1)) == 0, e


@pytest.mark.parametrize("d,dtype", [(2048, torch.bfloat16), (1000, torch.bfloat16), (768, torch.float16)],
                         ids=["d2048-bf16", "d1000-bf16", "d768-fp16"])
def test_hessian_grouped_multichunk(dev, d, dtype):
    """Experts of 0 .. 9000 routed rows (1, 2 and 3 chunks of 4096, an empty
    expert, one row): the device-built work table, the gathering DMA, the
    direct first-chunk update and the ordered slot reduction, against an fp64
    product per expert; a second call adds the same again and is bitwise
    equal to twice the first (deterministic)."""
    counts = [9000, 5000, 0, 100, 4096, 4097, 1, 2000, 300, 8192]
    say(f"grouped hessian multi-chunk d={d} {dtype}")
    x, rows, offsets = _grouped_case(counts, 7000, d, dtype, 21, dev)
    H = torch.zeros(len(counts), d, d, device=dev)
    ops.hessian_grouped_syrk_(H, x, rows, offsets, alpha=2.0)
    _grouped_check(H, x, rows, offsets)
    H1 = H.clone()
    ops.hessian_grouped_syrk_(H, x, rows, torch.tensor(offsets, device=dev), alpha=2.0)
    H2 = torch.zeros_like(H)
    ops.hessian_grouped_syrk_(H2, x, rows, offsets, alpha=2.0)
    assert torch.equal(H2, H1)
    assert ((H - 2 * H1).norm() / H1.norm()).item() <= 1e-6


@pytest.mark.parametrize("gather", [True, False], ids=["gathered", "grouped"])
def test_hessian_grouped_fresh_h_is_written_not_read(dev, gather):
    """beta = 0 (a freshly allocated, uncleared stack): every expert's upper
    triangle equals the add-to-zeros result bit for bit (zeros for an expert
    without rows, a second chunk still reduced after the first), and the
    strictly-lower triangle keeps whatever it held."""
    counts = [9000, 0, 100, 4097, 1]
    d = 768
    say(f"grouped hessian beta=0 gather={gather}")
    x, rows, offsets = _grouped_case(counts, 7000, d, torch.bfloat16, 23, dev)
    if not gather:
        x, rows = x[rows.long()].contiguous(), None
    ref = torch.zeros(len(counts), d, d, device=dev)
    ops.hessian_grouped_syrk_(ref, x, rows, offsets, alpha=2.0)
    H = torch.full((len(counts), d, d), float("nan"), device=dev)
    ops.hessian_grouped_syrk_(H, x, rows, torch.tensor(offsets, device=dev), alpha=2.0, beta=0.0)
    up = torch.triu(torch.ones(d, d, dtype=torch.bool, device=dev))
    for e in range(len(counts)):
        assert torch.equal(H[e][up], ref[e][up]), e
        assert bool(torch.isnan(H[e][~up]).all()), e
    with pytest.raises(ValueError):
        ops.hessian_grouped_syrk_(H, x, rows, offsets, alpha=2.0, beta=0.5)


def test_hessian_grouped_contiguous_rows(dev):
    """rows None: x already grouped by expert (the down projection's inputs),
    offsets given on the device."""
    counts = [5000, 0, 4096, 33, 12000]
    d = 768
    say("grouped hessian contiguous rows")
    g = torch.Generator(device=dev).manual_seed(22)
    x = torch.randn(sum(counts) + 10, d, generator=g, device=dev).to(torch.bfloat16)
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    H = torch.zeros(len(counts), d, d, device=dev)
    moe.accumulate_expert_hessians(x, None, torch.tensor(offsets, device=dev), H, torch.zeros(len(counts),
                                                                                              device=dev))
    _grouped_check(H, x, None, offsets)


# ---------------------------------------------------------------- observers / quant / pack
W_CASES = [
    dict(num_bits=4, strategy="group", group_size=128),
    dict(num_bits=4, strategy="group", group_size=32),
    dict(num_bits=4, strategy="group", group_size=16, symmetric=False),
    dict(num_bits=4, strategy="group", group_size=3),
    dict(num_bits=8, strategy="channel"),
    dict(num_bits=8, strategy="channel", symmetric=False),
    dict(num_bits=4, strategy="tensor"),
    dict(num_bits=8, strategy="block", block_structure=[16, 32]),
]


@pytest.mark.parametrize("case", W_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_observer_qparams_and_codes_exact(dev, case):
    say(f"observer {case}")
    cols = 384 if case.get("group_size") == 3 else 512
    w = workloads.gptq_weight(96, cols, seed=21)
    if case.get("symmetric", True):
        # an all-zero row / group: scale 0 -> the dtype's epsilon.  (Asymmetric
        # zero groups give zp = qmin - 0/0, a NaN whose integer conversion is
        # platform-defined in the reference; not exercised.)
        w[0, :] = 0
    qa = QuantizationArgs(**case)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    qp = obs(w.to(dev)).get_qparams()
    oa = OArgs(**case)
    oo = oobs.OMinMax("memoryless_minmax", "weight", oa)
    oq = oo(w).get_qparams()
    assert qp["scale"].dtype == oq["scale"].dtype
    assert torch.equal(qp["scale"].cpu().reshape(oq["scale"].shape), oq["scale"])
    assert torch.equal(qp["zero_point"].cpu().reshape(oq["zero_point"].shape), oq["zero_point"])
    codes = ops.quantize_int(w.to(dev), qp["scale"], None if qa.symmetric else qp["zero_point"], qa.strategy.value,
                             qa.num_bits, qa.group_size, block_structure=qa.block_structure)
    s = ofq.expand_qparams(oq["scale"], w.shape, oa)
    z = ofq.expand_qparams(oq["zero_point"], w.shape, oa)
    ocodes = ofq.quantize(w, s, None if oa.symmetric else z, oa)
    assert torch.equal(codes.cpu().float(), ocodes.float())


def test_strict_symmetric_on_gpu(dev):
    """strict_symmetric_minmax (observers/min_max.py:28-55) on the GPU: the
    reference's known answers (test_strict_symmetric.py:13-71: fp32 scale
    absmax / 127, clamped at 1e-8 after the division, int8 codes
    round(x / scale).clamp(-128, 127)) and random weights against the oracle."""
    say("strict symmetric observer")
    import json
    from pathlib import Path
    g = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())["strict_symmetric"]
    qa = QuantizationArgs(num_bits=8, type="int", strategy="channel", symmetric=True,
                          observer="strict_symmetric_minmax")
    obs = Observer.load_from_registry("strict_symmetric_minmax", base_name="weight", args=qa)
    x = torch.tensor(g["observed"], dtype=torch.float32)
    sc = obs(x.to(dev)).get_qparams()["scale"]
    assert sc.dtype == torch.float32
    assert sc.cpu().flatten().tolist() == pytest.approx(g["scale"])
    obs = Observer.load_from_registry("strict_symmetric_minmax", base_name="weight", args=qa)
    assert obs(torch.zeros(2, 3, device=dev)).get_qparams()["scale"].cpu().flatten().tolist() == \
        pytest.approx(g["zeros_scale"])
    xb = x.to(torch.bfloat16)   # the model-free path: bf16 weight, fp32 scale, fp32 division
    obs = Observer.load_from_registry("strict_symmetric_minmax", base_name="weight", args=qa)
    sc = obs(xb.to(dev)).get_qparams()["scale"]
    codes = ops.quantize_int(xb.to(dev), sc, None, "channel", 8, div_dtype=torch.float32).cpu()
    exp = torch.round(xb.float() / sc.cpu().reshape(-1, 1)).clamp(-128, 127).to(torch.int8)
    assert torch.equal(codes, exp)
    oa = OArgs(num_bits=8, strategy="channel")
    for dtype in (torch.bfloat16, torch.float32):
        w = workloads.gptq_weight(200, 640, seed=71).to(dtype)
        w[3] = 0
        obs = Observer.load_from_registry("strict_symmetric_minmax", base_name="weight", args=qa)
        sc = obs(w.to(dev)).get_qparams()["scale"].cpu()
        osc = oobs.OMinMax("strict_symmetric_minmax", "weight", oa)(w.float()).get_qparams()["scale"]
        assert torch.equal(sc.reshape(osc.shape), osc)
        codes = ops.quantize_int(w.to(dev), sc.to(dev), None, "channel", 8, div_dtype=torch.float32).cpu()
        assert torch.equal(codes, torch.round(w.float() / osc.reshape(-1, 1)).clamp(-128, 127).to(torch.int8))


def test_lifecycle_table_on_gpu(dev):
    """The reference's weight known-answer table, through the GPU kernels."""
    say("lifecycle table")
    import json
    from pathlib import Path
    gold = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
    w = torch.arange(24, dtype=torch.bfloat16).reshape(4, 6)
    for case in gold["static_weight_quantization"]["cases"]:
        a = dict(case["args"])
        if a["type"] != "int":
            continue
        qa = QuantizationArgs(**a)
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(w.to(dev))
        assert torch.equal(obs.min_vals.float().cpu().reshape(-1), torch.tensor(case["min"]).float().reshape(-1))
        qp = obs.get_qparams()
        codes = ops.quantize_int(w.to(dev), qp["scale"], None, qa.strategy.value, qa.num_bits, qa.group_size,
                                 block_structure=qa.block_structure).cpu()
        s = ofq.expand_qparams(qp["scale"].cpu(), w.shape, OArgs(**a))
        deq = (codes.to(torch.bfloat16) * s).to(torch.bfloat16)
        assert torch.allclose(deq.float(), torch.tensor(case["quant"], dtype=torch.bfloat16).float()), a


def test_pack_int4_exact(dev):
    say("pack int4")
    r = np.random.default_rng(1).integers(-8, 8, size=(64, 256)).astype(np.int8)
    t = torch.from_numpy(r).to(dev)
    assert np.array_equal(ops.pack_int4_int32(t).cpu().numpy(), opack.pack_to_int32(r))
    assert np.array_equal(ops.pack_int4_int8(t).cpu().numpy(), opack.pack_int4_to_int8(r))
    with pytest.raises(ValueError, match="even number of columns"):
        ops.pack_int4_int8(t[:, :3])


def _all_bf16_groups():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = (b.astype(np.uint32) << 16).view(np.float32)
    b = b[np.isfinite(f)]
    b = b[: (len(b) // 32) * 32]
    return b.reshape(-1, 32)


@pytest.mark.parametrize("rule", ["ct", "ocp"])
def test_mxfp4_exact(dev, rule):
    say(f"mxfp4 {rule}")
    w, _ = workloads.mxfp4(w_rows=128, cols=1024, a_rows=8)
    a = workloads.student_t((128, 1024), 3.0, torch.Generator().manual_seed(3)).to(torch.bfloat16)
    special = torch.tensor([0.0, -0.0, 0.25, -0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -5.0, 6.0, 7.0, 1e-30,
                            -1e-30, 3.0e38, 0.1, -0.3] + [0.0] * 14, dtype=torch.bfloat16)
    allb = torch.from_numpy(_all_bf16_groups().view(np.int16)).view(torch.bfloat16)
    for x in (w, a, special.reshape(1, 32), allb):
        c, s = ops.mxfp4_quantize_pack(x.to(dev), rule)
        oc, os_ = opack.mxfp4_quantize_pack(x.view(torch.int16).numpy().view(np.uint16), rule)
        assert np.array_equal(c.cpu().numpy(), oc)
        assert np.array_equal(s.cpu().numpy(), os_)
        back = ops.mxfp4_dequantize(c, s).cpu().float().numpy()
        ob = opack.mxfp4_unpack(oc, os_)
        fin = np.isfinite(ob) & (np.abs(ob) < 3e38)
        assert np.array_equal(back[fin], torch.from_numpy(ob[fin]).to(torch.bfloat16).float().numpy())


def test_fp8_exact_all_bf16(dev):
    say("fp8")
    b = _all_bf16_groups().reshape(-1, 64)
    x = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    for scale in (1.0, 0.37):
        s = torch.full((x.shape[0], 1), scale, dtype=torch.bfloat16)
        q = ops.quantize_fp8(x.to(dev), s.to(dev), "channel").cpu()
        oq = ofq.round_to_type(x / s, OArgs(num_bits=8, type="float"), -448.0, 448.0).to(torch.float8_e4m3fn)
        assert torch.equal(q.view(torch.uint8), oq.view(torch.uint8)), scale


@pytest.mark.parametrize("cols", [1024, 4096, 14336, 1000])
def test_int8_per_token_exact(dev, cols):
    say(f"int8 per token cols={cols}")
    x = workloads.heavy_tailed_activations((333, cols), seed=8)
    x[5] = 0
    codes, scale = ops.quantize_int8_per_token(x.to(dev))
    oa = OArgs(num_bits=8, strategy="token")
    mn, mx = x.amin(dim=1, keepdim=True), x.amax(dim=1, keepdim=True)
    os_, oz = oobs.calculate_qparams(mn, mx, oa)
    oc = ofq.quantize(x, os_, None, oa)
    assert torch.equal(scale.cpu(), os_)
    assert torch.equal(codes.cpu().float(), oc.float())


def test_int8_per_token_quotients_all_bf16(dev):
    """Every finite bf16 value divided by 257 different row scales."""
    say("int8 per token, all bf16 quotients")
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = (b.astype(np.uint32) << 16).view(np.float32)
    vals = torch.from_numpy(f[np.isfinite(f)].copy()).reshape(8, -1)   # 8 rows of 8160 values
    g = torch.Generator().manual_seed(11)
    amax = torch.cat([torch.tensor([1.0, 127.5, 3.0e38, 1e-30, 0.0078125 * 127.5]),
                      torch.exp(torch.randn(252, generator=g) * 8.0)])
    x = vals.unsqueeze(0).repeat(amax.numel(), 1, 1)
    lim = amax.view(-1, 1, 1)
    x = torch.maximum(torch.minimum(x, lim), -lim)
    x[:, :, 0] = lim[:, :, 0]
    x = x.reshape(-1, vals.shape[1])
    x = x.to(torch.bfloat16)
    codes, scale = ops.quantize_int8_per_token(x.to(dev))
    oa = OArgs(num_bits=8, strategy="token")
    mn, mx = x.amin(dim=1, keepdim=True), x.amax(dim=1, keepdim=True)
    os_, oz = oobs.calculate_qparams(mn, mx, oa)
    oc = ofq.quantize(x, os_, None, oa)
    assert torch.equal(scale.cpu(), os_)
    assert torch.equal(codes.cpu().float(), oc.float())


# ---------------------------------------------------------------- GPTQ
def _spd_from_tokens(d, tokens, seed):
    x = workloads.heavy_tailed_activations((tokens, d), seed=seed)
    H, n = og.accumulate_hessian(x, og.make_empty_hessian(d), torch.zeros(()))
    return H / n


@pytest.mark.parametrize("d,batch", [(1000, 1), (384, 1), (2048, 16)], ids=["ragged-1000", "3-blocks-384",
                                                                          "batch16-2048"])
def test_blocked_chain_reads_no_uninitialised_workspace(dev, d, batch):
    """The blocked chain (orders not a multiple of 128, fewer than 4 blocks,
    batches over 8) builds X = L^-1 in its workspace without clearing it:
    every element it reads was written first.  With the workspace filled
    with NaN beforehand, hinv equals bit for bit the one from a zeroed
    workspace."""
    import ctypes as C
    from llmcompressor_amd import _lib as L
    say(f"blocked chain on a NaN workspace d={d} batch={batch}")
    Hs = torch.stack([torch.triu(_spd_from_tokens(d, 2 * d, seed=70 + b)) for b in range(batch)]).to(dev)
    ns = torch.ones(batch, dtype=torch.float32, device=dev)
    lib = L.lib()
    nbytes = lib.mi355q_gptq_hinv_workspace_size(d) * batch
    out = []
    for fill in (0.0, float("nan")):
        ws = torch.full(((nbytes + 3) // 4,), fill, dtype=torch.float32, device=dev)
        hinv = torch.empty((batch, d, d), dtype=torch.float32, device=dev)
        dead = torch.empty((batch, d), dtype=torch.int32, device=dev)
        status = torch.zeros(batch, dtype=torch.int32, device=dev)
        L.check(lib.mi355q_gptq_hinv_batched(Hs.data_ptr(), Hs.stride(1), Hs.stride(0), d, batch, None, 0,
                                             ns.data_ptr(), C.c_float(0.01), hinv.data_ptr(), d * d,
                                             dead.data_ptr(), status.data_ptr(), ws.data_ptr(), nbytes,
                                             L.stream_of(Hs)))
        torch.cuda.synchronize()
        assert int(status.abs().sum()) == 0
        out.append(hinv.cpu())
    assert torch.isfinite(out[1]).all()
    assert torch.equal(out[0], out[1])


# d = 256, 384, 1000: the blocked chain; 512, 1024, 2048 (multiples of 128
# with at least 4 blocks): the dataflow factorisation
@pytest.mark.parametrize("d,perm", [(256, False), (1000, False), (384, True), (512, False), (1024, True),
                                    (2048, False)])
def test_gptq_hinv_matches_oracle_chain(dev, d, perm):
    say(f"hinv d={d} perm={perm}")
    H = _spd_from_tokens(d, 4 * d, seed=d)
    H[7, :] = 0
    H[:, 7] = 0  # a dead column
    p = torch.argsort(torch.diag(H), descending=True, stable=True) if perm else None
    Hu = torch.triu(H).to(dev)
    hinv, dead, ok = ops.gptq_hinv(Hu, None if p is None else p.to(dev), 1.0, 0.01)
    assert ok
    Hp = H[p][:, p] if perm else H.clone()
    dd = torch.diag(Hp) == 0
    assert torch.equal(dead.cpu().bool(), dd)
    Hp[dd, dd] = 1
    U, ok_o = og.cholesky_chain(Hp, 0.01)
    assert ok_o
    assert rel_fro(hinv.cpu(), U) <= 1e-4
    assert torch.equal(hinv.cpu(), torch.triu(hinv.cpu()))


def test_gptq_hinv_non_pd_reports_status(dev):
    say("hinv non-PD")
    H = _spd_from_tokens(128, 512, seed=5)
    H[9, 9] = -1e6
    _, _, ok = ops.gptq_hinv(torch.triu(H).to(dev), None, 1.0, 0.0)
    assert not ok


def test_gptq_non_pd_falls_back_to_rtn_on_device(dev):
    """A Hessian that is not positive definite gets Hinv = identity on the
    device (no host synchronisation before the sweep), so the solve is
    round-to-nearest, as the reference's LinAlgError branch
    (gptq_quantize.py:189-196)."""
    say("gptq non-PD -> RTN on the device")
    d, rows = 256, 64
    qa = QuantizationArgs(type="int", num_bits=4, strategy="group", group_size=128)
    H = torch.triu(_spd_from_tokens(d, 1024, seed=61))
    H[5, 5] = -1e3
    prep = gptq.prepare_hessian(H.to(dev), qa, 1.0)
    assert torch.equal(prep.hinv.cpu(), torch.eye(d))
    assert prep.ok is False
    W = workloads.gptq_weight(rows, d, seed=62).to(dev)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(W)
    res = gptq.gptq_quantize(W, qa, H.to(dev), obs, prepared=prep)
    assert res.hinv_ok is False
    s = res.scale.float().repeat_interleave(128, dim=1)
    rtn = torch.clamp(torch.round(W.float() / s), -8, 7)
    assert torch.equal(res.codes.float().cpu(), rtn.cpu())
    ok_prep = gptq.prepare_hessian(torch.triu(_spd_from_tokens(d, 1024, seed=63)).to(dev), qa, 1.0)
    assert ok_prep.ok is True


GPTQ_CASES = [
    dict(num_bits=4, strategy="group", group_size=128),
    dict(num_bits=4, strategy="group", group_size=128, symmetric=False),
    dict(num_bits=4, strategy="group", group_size=128, actorder="weight"),
    dict(num_bits=4, strategy="group", group_size=64, actorder="group"),
    dict(num_bits=8, strategy="channel", actorder="weight"),
    dict(num_bits=8, strategy="block", block_structure=[64, 128]),
    dict(num_bits=4, strategy="tensor"),
]


@pytest.mark.parametrize("case", GPTQ_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_gptq_batched_equals_single(dev, case):
    """The batched solve (one launch per step for all experts) gives each
    module exactly what its own solve gives, including a non-PD member."""
    say(f"gptq batched {case}")
    B, rows, d = 3, 200, 384
    qa = QuantizationArgs(type="int", **case)
    Ws, Hs = [], []
    for b in range(B):
        Ws.append(workloads.gptq_weight(rows, d, seed=20 + b))
        Hs.append(torch.triu(_spd_from_tokens(d, 1024, seed=30 + b)) * (b + 1))
    Hs[2][7, 7] = -1e3        # not positive definite: RTN fallback for this member only
    W = torch.stack(Ws).to(dev)
    H = torch.stack(Hs).to(dev)
    ns = torch.tensor([1.0, 2.0, 3.0])
    res = gptq.gptq_quantize_batched(W, qa, H.clone(), num_samples=ns)
    for b in range(B):
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(W[b])
        single = gptq.gptq_quantize(W[b], qa, H[b].clone(), obs, num_samples=float(ns[b]))
        assert res[b].hinv_ok == single.hinv_ok == (b != 2)
        assert torch.equal(res[b].codes, single.codes)
        assert torch.equal(res[b].weight, single.weight)
        assert torch.equal(res[b].scale.reshape(single.scale.shape), single.scale)
        assert abs(res[b].loss - single.loss) <= 1e-5 * abs(single.loss) + 1e-12


@pytest.mark.parametrize("symmetric", [True, False])
def test_gptq_pulled_updates_equal_pushed(dev, symmetric):
    """A 4096-row solve fills at most two sweep workgroups per CU, so each
    block applies the K = 128 updates of the earlier blocks of its mid-block
    itself; the same matrix in a batch of three (768 workgroups) gets them
    from separate K = 128 products after each block.  Both form each product
    in the same MFMA order, so the results agree bit for bit."""
    say(f"gptq pulled vs pushed mid-block updates, symmetric={symmetric}")
    rows, d = 4096, 512
    qa = QuantizationArgs(type="int", num_bits=4, strategy="group", group_size=128, symmetric=symmetric)
    W = workloads.gptq_weight(rows, d, seed=41).to(dev)
    H = torch.triu(_spd_from_tokens(d, 2048, seed=42)).to(dev)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(W)
    single = gptq.gptq_quantize(W, qa, H.clone(), obs, num_samples=1.0)
    res = gptq.gptq_quantize_batched(W.unsqueeze(0).repeat(3, 1, 1).contiguous(), qa,
                                     H.unsqueeze(0).repeat(3, 1, 1).contiguous(), num_samples=1.0)
    for b in range(3):
        assert torch.equal(res[b].codes, single.codes), b
        assert torch.equal(res[b].weight, single.weight), b


@pytest.mark.parametrize("cols,kw", [(128, dict(num_bits=8, strategy="channel")),
                                     (256, dict(num_bits=4, strategy="group", group_size=64)),
                                     (256, dict(num_bits=4, strategy="group", group_size=64, symmetric=False))])
def test_gptq_wide_sweep_equals_single(dev, cols, kw):
    """A batch of eight 4096-row matrices (2048 sixteen-lane workgroups) is
    swept with 4 lanes per row when its scales are symmetric; each matrix
    alone with 16.  Every element sees the same operations in the same order
    either way, so codes and weights agree bit for bit (the per-row losses
    are summed in another order).  Zero points keep the 16-lane sweep."""
    say(f"gptq 4-lane batched sweep vs single 16-lane sweeps, cols={cols} {kw}")
    _wide_vs_single(dev, 8, 4096, cols, kw, seed=60)


def test_gptq_wide_sweep_ragged_rows(dev):
    """Forty 1000-row matrices (2520 sixteen-lane workgroups): the 4-lane
    sweep's last workgroup of each matrix holds 40 live rows of 64."""
    say("gptq 4-lane batched sweep, 40 x 1000 rows")
    _wide_vs_single(dev, 40, 1000, 128, dict(num_bits=4, strategy="group", group_size=128), seed=90)


def _wide_vs_single(dev, B, rows, cols, kw, seed):
    qa = QuantizationArgs(type="int", **kw)
    Ws = [workloads.gptq_weight(rows, cols, seed=seed + b) for b in range(B)]
    Hs = [torch.triu(_spd_from_tokens(cols, 1024, seed=seed + 100 + b)) for b in range(B)]
    W = torch.stack(Ws).to(dev)
    H = torch.stack(Hs).to(dev)
    res = gptq.gptq_quantize_batched(W, qa, H.clone(), num_samples=1.0)
    for b in range(B):
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(W[b])
        single = gptq.gptq_quantize(W[b], qa, H[b].clone(), obs, num_samples=1.0)
        assert torch.equal(res[b].codes, single.codes), b
        assert torch.equal(res[b].weight, single.weight), b
        assert abs(res[b].loss - single.loss) <= 1e-5 * abs(single.loss) + 1e-12


def test_gptq_prepared_hessian_shared(dev):
    """Modules with the same input (q/k/v, gate/up) may share the Cholesky
    chain: a prepared Hessian gives exactly the results of separate solves."""
    say("gptq shared prepared Hessian")
    d = 384
    qa = QuantizationArgs(type="int", num_bits=4, strategy="group", group_size=128, actorder="weight")
    H = torch.triu(_spd_from_tokens(d, 1024, seed=41)).to(dev)
    prep = gptq.prepare_hessian(H, qa, 2.0)
    for seed, rows in ((50, 128), (51, 200)):
        W = workloads.gptq_weight(rows, d, seed=seed).to(dev)
        outs = []
        for p in (prep, None):
            obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
            obs(W)
            outs.append(gptq.gptq_quantize(W, qa, H.clone(), obs, num_samples=2.0, prepared=p))
        assert torch.equal(outs[0].codes, outs[1].codes)
        assert torch.equal(outs[0].weight, outs[1].weight)
        assert torch.equal(outs[0].g_idx, outs[1].g_idx)


def _layer_err(W, Q, X):
    Xf = X.reshape(-1, X.shape[-1]).float()
    return (Xf @ (W.float() - Q.float()).t()).norm().item()


@pytest.mark.parametrize("case", GPTQ_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_gptq_sweep_given_oracle_hinv(dev, case):
    """The sweep, lazy updates, actorder and dead-column handling on the GPU
    with the oracle's own Hinv (the chain replaced by the oracle's LAPACK
    result): every code within 1 LSB of the oracle's."""
    rows, cols, tokens = 384, 1024, 4096
    say(f"gptq sweep given the oracle's hinv {case}")
    W = workloads.gptq_weight(rows, cols, seed=33)
    X = workloads.heavy_tailed_activations((2, tokens // 2, cols), seed=34)
    Ho, no = og.accumulate_hessian(X, og.make_empty_hessian(cols), torch.zeros(()))
    Ho = og.normalise_hessian(Ho, no)
    Ho[5, :] = 0
    Ho[:, 5] = 0   # a dead column
    oa = OArgs(**case)
    loss_o, out_o, ex = og.quantize_weight(W, oa, Ho, return_codes=True)
    qa = QuantizationArgs(**case)
    actorder = gptq._effective_actorder(qa)
    perm = None if ex["perm"] is None else ex["perm"].to(dev)
    Hp = Ho if perm is None else Ho[ex["perm"]][:, ex["perm"]]
    dead = (torch.diag(Hp) == 0).to(torch.int32).to(dev)
    prep = gptq.PreparedHessian(actorder, perm, None if perm is None else torch.argsort(perm), ex["hinv"].to(dev),
                                dead, torch.zeros(1, dtype=torch.int32, device=dev))
    Wd = W.to(dev)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(Wd)
    res = gptq.gptq_quantize(Wd, qa, torch.triu(Ho).to(dev), obs, prepared=prep)
    st = code_agreement(res.codes.cpu().to(torch.int32), ex["codes"])
    say(f"  {st} loss {res.loss:.6g} vs {loss_o:.6g}")
    assert st["max_diff"] <= 1 and st["agree"] >= 0.9999
    assert abs(res.loss - loss_o) <= 1e-4 * abs(loss_o) + 1e-6


@pytest.mark.parametrize("case", GPTQ_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_gptq_end_to_end_parity(dev, case):
    rows, cols, tokens = 384, 1024, 4096
    say(f"gptq e2e {case} rows={rows} cols={cols} tokens={tokens}")
    W = workloads.gptq_weight(rows, cols, seed=31)
    X = workloads.heavy_tailed_activations((2, tokens // 2, cols), seed=32)
    qa = QuantizationArgs(**case)
    lin = torch.nn.Linear(cols, rows, bias=False).to(dev)
    lin.weight.data = W.to(dev)
    H = gptq.make_empty_hessian(lin)
    n = torch.zeros((), device=dev)
    H, n = gptq.accumulate_hessian(X.to(dev), lin, H, n)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(lin.weight)
    res = gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(n.item()))
    Ho, no = og.accumulate_hessian(X, og.make_empty_hessian(cols), torch.zeros(()))
    loss_o, out_o, ex = og.quantize_weight(W, OArgs(**case), og.normalise_hessian(Ho, no), return_codes=True)
    st = code_agreement(res.codes.cpu().to(torch.int32), ex["codes"])
    e_gpu = _layer_err(W, res.weight.cpu(), X)
    e_ora = _layer_err(W, out_o["weight"], X)
    say(f"  {st} err_gpu={e_gpu:.6g} err_oracle={e_ora:.6g} loss {res.loss:.6g} vs {loss_o:.6g}")
    assert code_bar(st, rows)
    assert abs(e_gpu - e_ora) <= 0.005 * e_ora
    assert abs(res.loss - loss_o) <= 1e-3 * abs(loss_o) + 1e-6
    assert torch.equal(res.scale.cpu(), ex["scale_used"].to(res.scale.dtype).reshape(res.scale.shape))


@pytest.mark.parametrize("actorder", [None, "weight", "group"])
def test_reference_shape_contracts_on_gpu(dev, actorder):
    """test_gptq_quantize.py:21-60 through the drop-in quantize_weight."""
    say(f"shape contract actorder={actorder}")
    module = torch.nn.Linear(8, 6, bias=False).to(dev)
    qa = QuantizationArgs(num_bits=4, symmetric=True, strategy="group", group_size=2, actorder=actorder)
    initialize_module_for_quantization(module, QuantizationScheme(targets=["Linear"], weights=qa))
    initialize_observer(module, "weight")
    observe(module, "weight")
    H = gptq.make_empty_hessian(module)
    H += torch.diag(torch.arange(1, 9, dtype=H.dtype, device=dev))
    loss, q = gptq.quantize_weight(module=module, quant_args=qa, hessian=H)
    assert loss >= 0
    assert q["weight"].shape == module.weight.shape
    assert q["weight_scale"].shape == (6, 4) and q["weight_zero_point"].shape == (6, 4)
    assert ("weight_g_idx" in q) == (actorder == "group")


def test_block_strategy_shape_contract_on_gpu(dev):
    """test_gptq_quantize.py:63-97 (7 columns, block [2, 4], blocksize 3)."""
    say("block shape contract")
    module = torch.nn.Linear(7, 5, bias=False).to(dev)
    qa = QuantizationArgs(num_bits=8, symmetric=True, strategy="block", block_structure=[2, 4])
    initialize_module_for_quantization(module, QuantizationScheme(targets=["Linear"], weights=qa))
    initialize_observer(module, "weight")
    observe(module, "weight")
    H = gptq.make_empty_hessian(module) + torch.eye(7, device=dev)
    loss, q = gptq.quantize_weight(module=module, quant_args=qa, hessian=H, blocksize=3)
    assert loss >= 0 and q["weight_scale"].shape == (3, 2) and "weight_g_idx" not in q
