"""Pin the GPTQ oracle (Hessian, Cholesky chain, sweep) by mathematics (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import gptq as og
from oracle.observers import OMinMax
from oracle.qargs import OArgs


def _x(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * torch.exp(torch.randn(shape[-1], generator=g))).to(torch.bfloat16)


def test_hessian_closed_form_and_sample_count():
    x = _x((3, 50, 16), 0)
    H = og.make_empty_hessian(16)
    n = torch.zeros(())
    H, n = og.accumulate_hessian(x, H, n)
    assert n.item() == 3
    x2 = _x((7, 16), 1)
    H, n = og.accumulate_hessian(x2, H, n)          # 2-D input counts as one sample
    assert n.item() == 4
    xs = torch.cat([x.reshape(-1, 16), x2]).double()
    exact = 2.0 * xs.t() @ xs
    rel = ((H.double() - exact).norm() / exact.norm()).item()
    assert rel < 1e-6
    assert torch.equal(H, H.t())


def _spd(d, seed, tokens=None):
    x = _x((tokens or 4 * d, d), seed).float()
    return x.t() @ x / x.shape[0]


def test_cholesky_chain_identity_and_fp64():
    H = _spd(64, 2)
    U, ok = og.cholesky_chain(H, 0.01)
    assert ok
    assert torch.equal(U, torch.triu(U))
    Hd = H.double() + 0.01 * torch.mean(torch.diag(H.double())) * torch.eye(64, dtype=torch.float64)
    I = U.double().t() @ U.double() @ Hd
    assert (I - torch.eye(64, dtype=torch.float64)).abs().max().item() < 1e-3
    U64 = torch.linalg.cholesky(torch.linalg.inv(Hd), upper=True)
    assert ((U.double() - U64).norm() / U64.norm()).item() < 1e-4


def test_cholesky_chain_non_pd_falls_back_to_identity():
    H = _spd(16, 3)
    H[5, 5] = -50.0
    U, ok = og.cholesky_chain(H, 0.0)
    assert not ok and torch.equal(U, torch.eye(16))


def _weight(r, c, seed):
    return (torch.randn(r, c, generator=torch.Generator().manual_seed(seed)) * 0.02).to(torch.bfloat16)


def test_diagonal_hessian_is_round_to_nearest():
    """Diagonal H -> diagonal Hinv -> no cross-column error feedback -> GPTQ == RTN."""
    W = _weight(12, 64, 4)
    H = torch.diag(torch.arange(1, 65, dtype=torch.float32))
    args = OArgs(num_bits=4, strategy="group", group_size=16)
    _, out, ex = og.quantize_weight(W, args, H, return_codes=True)
    s = ex["scale_used"].float().repeat_interleave(16, 1)
    rtn = torch.clamp(torch.round(W.float() / s), -8, 7).to(torch.int32)
    assert torch.equal(ex["codes"], rtn)


def test_blocksize_invariance():
    W = _weight(16, 48, 5)
    H = _spd(48, 6)
    args = OArgs(num_bits=4, strategy="group", group_size=16)
    outs = [og.quantize_weight(W, args, H, blocksize=b, return_codes=True) for b in (3, 16, 128)]
    for o in outs[1:]:
        assert torch.equal(o[2]["codes"], outs[0][2]["codes"])
        assert abs(o[0] - outs[0][0]) <= 1e-4 * abs(outs[0][0]) + 1e-9


def _obq_fp64(W, H, scale, qmin, qmax, percdamp=0.01):
    """Optimal Brain Quantization with explicit inverse downdates, fp64, column order.

    After quantizing the first remaining column q, the remaining weights move by
    -(w_q - q) / [H_F^-1]_qq * [H_F^-1]_{q, :} with H_F the Hessian restricted
    to the not-yet-quantized columns (recomputed by a full inverse each step).
    """
    W = W.astype(np.float64).copy()
    r, c = W.shape
    Hd = H.astype(np.float64) + percdamp * np.mean(np.diag(H)) * np.eye(c)
    codes = np.zeros((r, c), dtype=np.int64)
    for i in range(c):
        F = list(range(i, c))
        Hi = np.linalg.inv(Hd[np.ix_(F, F)])
        w = W[:, i]
        q = np.clip(np.round(w / scale[:, i]), qmin, qmax)
        codes[:, i] = q
        deq = q * scale[:, i]
        W[:, i + 1:] -= np.outer((w - deq) / Hi[0, 0], Hi[0, 1:])
    return codes


def test_sweep_matches_brute_force_obq_fp64():
    W = _weight(32, 24, 7)
    H = _spd(24, 8, tokens=200)
    args = OArgs(num_bits=4, strategy="channel")
    _, _, ex = og.quantize_weight(W, args, H, blocksize=8, return_codes=True,
                                  dequant_in_scale_dtype=False)
    s = ex["scale_used"].float().expand(32, 24).double().numpy()
    ref = _obq_fp64(W.float().numpy(), H.numpy(), s, -8, 7)
    agree = (ex["codes"].numpy() == ref).mean()
    assert agree >= 0.99 and np.abs(ex["codes"].numpy() - ref).max() <= 1


@pytest.mark.parametrize("actorder", [None, "weight", "group"])
def test_shapes_group_actorder(actorder):
    """test_gptq_quantize.py:21-60."""
    W = _weight(6, 8, 9)
    H = torch.diag(torch.arange(1, 9, dtype=torch.float32))
    args = OArgs(num_bits=4, strategy="group", group_size=2, actorder=actorder)
    loss, q = og.quantize_weight(W, args, H)
    assert loss >= 0
    assert q["weight"].shape == W.shape
    assert q["weight_scale"].shape == (6, 4) and q["weight_zero_point"].shape == (6, 4)
    assert ("weight_g_idx" in q) == (actorder == "group")
    if actorder == "group":
        assert q["weight_g_idx"].shape == (8,)


@pytest.mark.parametrize("actorder", [None, "weight"])
def test_shapes_block_strategy(actorder):
    """test_gptq_quantize.py:63-97."""
    W = _weight(5, 7, 10)
    args = OArgs(num_bits=8, strategy="block", block_structure=[2, 4], actorder=actorder)
    loss, q = og.quantize_weight(W, args, torch.eye(7), blocksize=3)
    assert loss >= 0 and q["weight"].shape == W.shape
    assert q["weight_scale"].shape == (3, 2) and "weight_g_idx" not in q


def test_channel_actorder_weight():
    """test_gptq_quantize.py:100-132."""
    W = _weight(4, 8, 11)
    args = OArgs(num_bits=4, strategy="channel", actorder="weight")
    loss, q = og.quantize_weight(W, args, torch.diag(torch.arange(1, 9, dtype=torch.float32)), blocksize=4)
    assert loss >= 0 and q["weight"].shape == W.shape and q["weight_scale"].shape[0] == 4
    assert "weight_g_idx" not in q


def test_dead_columns_are_zeroed():
    W = _weight(8, 16, 12)
    H = _spd(16, 13)
    H[3, :] = 0
    H[:, 3] = 0
    args = OArgs(num_bits=4, strategy="channel")
    _, q, ex = og.quantize_weight(W, args, H, return_codes=True)
    assert torch.all(q["weight"][:, 3] == 0) and torch.all(ex["codes"][:, 3] == 0)


FLOAT_ARGS = [OArgs(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=torch.float8_e4m3fn),
              OArgs(num_bits=4, type="float", strategy="group", group_size=32, is_mx=True),
              OArgs(num_bits=8, type="float", strategy="channel"),
              OArgs(num_bits=8, type="float", strategy="tensor")]


@pytest.mark.parametrize("args", FLOAT_ARGS, ids=["nvfp4", "mxfp4", "fp8-channel", "fp8-tensor"])
def test_float_diagonal_hessian_is_round_to_nearest(args):
    """Float weights (gptq_quantize.py:215-247 with global_scale): a diagonal
    Hessian gives GPTQ == CT fake_quantize of the fp32 weight with the same
    qparams, and the codes dequantise back to the weight."""
    from oracle import fake_quant as ofq
    W = _weight(24, 128, 9)
    W[0, :5] = torch.tensor([0.0, -0.0, 1e-6, -1e-6, 0.3], dtype=torch.bfloat16)
    H = torch.diag(torch.linspace(1.0, 4.0, 128))
    _, out, ex = og.quantize_weight(W, args, H, return_codes=True)
    obs = OMinMax("memoryless_minmax", "weight", args)
    qp = obs(W).get_qparams()
    s = ofq.expand_qparams(qp["scale"], W.shape, args)
    rtn = ofq.fake_quantize(W.float(), s, None, args, qp["global_scale"]).to(W.dtype)
    assert torch.equal(out["weight"], rtn)
    # codes: grid value x effective scale = the dequantised weight (bf16)
    s_eff = s.float() if qp["global_scale"] is None else s.float() / qp["global_scale"]
    gi = ofq.signed_grid_index(ex["codes"], args)
    if args.num_bits == 8:
        vals = (ex["codes"] & 0xFF).to(torch.uint8).view(torch.float8_e4m3fn).float()
    else:
        grid = torch.tensor(ofq.FP4_GRID)
        vals = grid[(ex["codes"] & 7).long()] * torch.where((ex["codes"] >> 3) & 1 == 1, -1.0, 1.0)
    assert torch.equal((vals * s_eff).to(W.dtype), out["weight"])
    assert int(gi.abs().max()) <= (126 if args.num_bits == 8 else 7)


def test_nvfp4_global_scale_in_outputs():
    """weight_global_scale (gptq_quantize.py:292-293) and fp8 group scales."""
    W = _weight(16, 64, 10)
    args = FLOAT_ARGS[0]
    _, out, ex = og.quantize_weight(W, args, _spd(64, 11), return_codes=True)
    gs = out["weight_global_scale"]
    assert gs.dtype == W.dtype and gs.numel() == 1
    assert float(gs) == pytest.approx(448 * 6 / float(W.abs().max()), rel=1e-2)


@pytest.mark.parametrize("k,stride,pad,dil", [(3, 1, 1, 1), (3, 2, 0, 2), (1, 1, 0, 1), (2, 3, 1, 1)])
def test_conv2d_hessian_is_the_patch_gram_matrix(k, stride, pad, dil):
    """The oracle's Conv2d branch (unfold, permute, flatten) against patches
    cut out by explicit loops: H = 2 sum over (image, position) of p p^T,
    p the (channel, ky, kx)-ordered receptive field, zero outside the image."""
    g = torch.Generator().manual_seed(k * 7 + stride)
    B, C, h, w = 2, 3, 6, 5
    x = torch.randn(B, C, h, w, generator=g, dtype=torch.float64)
    d = C * k * k
    H, n = og.accumulate_hessian_conv2d(x.float(), torch.zeros(d, d), torch.zeros(()), k, dil, pad, stride)
    ho = (h + 2 * pad - dil * (k - 1) - 1) // stride + 1
    wo = (w + 2 * pad - dil * (k - 1) - 1) // stride + 1
    ref = torch.zeros(d, d, dtype=torch.float64)
    for b in range(B):
        for oy in range(ho):
            for ox in range(wo):
                p = torch.zeros(d, dtype=torch.float64)
                for c in range(C):
                    for ky in range(k):
                        for kx in range(k):
                            iy, ix = oy * stride - pad + ky * dil, ox * stride - pad + kx * dil
                            if 0 <= iy < h and 0 <= ix < w:
                                p[(c * k + ky) * k + kx] = x[b, c, iy, ix]
                ref += 2 * torch.outer(p, p)
    assert float(n) == B
    assert torch.allclose(H.double(), ref, rtol=1e-5, atol=1e-5)


def test_nvfp4_fused_global_scale_is_the_groups_absmax():
    """observers/base.py:78-96 over a fused set (q/k/v): every member's
    global scale is 448 * 6 / the absmax over all members' weights (so the
    largest member sets it and each member's own scale is at least it), the
    same for every member whatever its own range, and a member fused with
    nothing gets its own."""
    args = FLOAT_ARGS[0]
    ws = [_weight(16, 64, 20), _weight(8, 64, 21) * 3, _weight(8, 64, 22)]
    obs = []
    for w in ws:
        o = OMinMax("memoryless_minmax", "weight", args)
        o(w)
        obs.append(o)
    stats = [(o.min_vals, o.max_vals) for o in obs]
    gss = []
    for i, o in enumerate(obs):
        o.fused_stats = [s for j, s in enumerate(stats) if j != i]
        gss.append(float(o.get_qparams()["global_scale"]))
    absmax = max(float(w.abs().max()) for w in ws)
    assert gss[0] == gss[1] == gss[2]
    # torch evaluates the scalar quotient as reciprocal(absmax) * 2688 in the
    # statistics' dtype (bf16 here)
    want = (torch.tensor(absmax, dtype=torch.bfloat16).reciprocal() * 2688.0).to(torch.bfloat16)
    assert gss[0] == float(want)
    own = []
    for w in ws:
        o = OMinMax("memoryless_minmax", "weight", args)
        own.append(float(o(w).get_qparams()["global_scale"]))
    assert all(g >= gss[0] for g in own) and gss[0] == min(own)
