"""Pin the SparseGPT oracle (running-mean Hessian, masks, compensation) by
mathematics (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import sparsegpt as osg


def _x(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * torch.exp(torch.randn(shape[-1], generator=g))).to(torch.bfloat16)


def _weight(r, c, seed):
    return (torch.randn(r, c, generator=torch.Generator().manual_seed(seed)) * 0.02).to(torch.bfloat16)


def _spd(d, seed, tokens=None):
    x = _x((tokens or 4 * d, d), seed).float()
    return x.t() @ x / x.shape[0]


def test_hessian_running_mean_closed_form():
    """H = (2 / N) sum x x^T with N counting samples (2-D input = one sample)."""
    H = osg.make_empty_hessian(16)
    n = 0
    parts = [_x((3, 40, 16), 0), _x((9, 16), 1), _x((2, 25, 16), 2)]
    for p in parts:
        H, n = osg.accumulate_hessian(p, H, n)
    assert n == 6
    xs = torch.cat([p.reshape(-1, 16) for p in parts]).double()
    exact = 2.0 / 6 * xs.t() @ xs
    assert ((H.double() - exact).norm() / exact.norm()).item() < 1e-6


def _brute(W, H, frac, sparsity, n, m, block, preserve=False):
    """fp64 sequential optimal-brain-surgeon pruning.  Column c of a row is
    removed (if selected) by the closed-form update over the columns not yet
    processed, w[c:] -= w_c / T[0, 0] * T[0, :], with T the explicit inverse of
    the damped Hessian's trailing block H[c:, c:]; its saliency is
    w_c^2 / T[0, 0].  No Cholesky factor is used.  Returns (W, loss).

    With a preserved mask and N:M groups, the reference weighs the group that
    starts at block column j by the live mask of matrix columns [j, j + m)
    (``sgpt_sparsify.py:181-182`` indexes the whole-matrix mask with the
    block-relative i), i.e. by the first block's mask including the groups it
    has already pruned; ``live`` is that mask here."""
    W = W.double().numpy().copy()
    H = H.double().numpy().copy()
    rows, d = W.shape
    dead = np.diag(H) == 0
    H[dead, dead] = 1
    W[:, dead] = 0
    H = H + frac * np.mean(np.diag(H)) * np.eye(d)
    T = [np.linalg.inv(H[c:, c:]) for c in range(d)]
    sal = np.array([T[c][0, 0] for c in range(d)])
    base = (W == 0) if preserve else None
    live = base.copy() if preserve else None
    loss = 0.0
    for i1 in range(0, d, block):
        i2 = min(i1 + block, d)
        if n == 0:
            tmp = W[:, i1:i2] ** 2 / sal[None, i1:i2]
            k = int(tmp.size * sparsity)
            if base is not None:
                tmp = tmp * ~base[:, i1:i2]
                sel = base[:, i1:i2].copy()
                if k > sel.sum():
                    sel = tmp <= np.sort(tmp.ravel())[k]
            else:
                sel = tmp <= np.sort(tmp.ravel())[k]
        else:
            sel = base[:, i1:i2].copy() if base is not None else np.zeros((rows, i2 - i1), bool)
        for c in range(i1, i2):
            j = c - i1
            if n and j % m == 0:
                g1 = min(c + m, i2)
                tmp = W[:, c:g1] ** 2 / sal[None, c:g1]
                if base is not None:
                    tmp = tmp * ~live[:, j:j + g1 - c]
                idx = np.argsort(tmp, axis=1, kind="stable")[:, :n]
                for r in range(rows):
                    sel[r, j + idx[r]] = True
                if live is not None and n:
                    live[:, i1:i2] |= sel
            for r in np.nonzero(sel[:, j])[0]:
                wc = W[r, c]
                loss += wc * wc / T[c][0, 0] / 2
                upd = wc / T[c][0, 0] * T[c][0, :]
                if base is not None:   # later blocks keep their masked entries
                    upd[i2 - c:] *= ~base[r, i2:]
                W[r, c:] -= upd
                W[r, c] = 0.0
    return W, loss


@pytest.mark.parametrize("sparsity,n,m,block,cols", [(0.5, 0, 0, 16, 64), (0.7, 0, 0, 32, 50), (0.0, 0, 0, 16, 48),
                                                      (0.5, 2, 4, 16, 64), (0.5, 4, 8, 24, 72), (0.5, 1, 3, 16, 47)])
def test_sweep_matches_sequential_obs_brute_force(sparsity, n, m, block, cols):
    rows = 24
    W = _weight(rows, cols, 10 + cols)
    H = _spd(cols, 20 + cols)
    loss, out, _, ok = osg.sparsify_weight(W.float(), H, sparsity, n, m, block, 0.01, False)
    assert ok
    Wb, loss_b = _brute(W, H, 0.01, sparsity, n, m, block)
    out = out.double().numpy()
    assert np.array_equal(out == 0, Wb == 0), "pruned sets differ"
    scale = np.abs(Wb).max()
    assert np.abs(out - Wb).max() <= 2e-5 * scale
    assert abs(loss - loss_b) <= 1e-4 * loss_b


def test_sweep_brute_force_with_preserved_mask():
    rows, cols = 24, 64
    W = _weight(rows, cols, 3).float()
    W[torch.rand(rows, cols, generator=torch.Generator().manual_seed(4)) < 0.3] = 0
    H = _spd(cols, 5)
    for n, m in ((0, 0), (2, 4)):
        loss, out, _, _ = osg.sparsify_weight(W, H, 0.5, n, m, 16, 0.01, True)
        Wb, loss_b = _brute(W, H, 0.01, 0.5, n, m, 16, preserve=True)
        out = out.double().numpy()
        assert np.array_equal(out == 0, Wb == 0)
        assert np.abs(out - Wb).max() <= 2e-5 * np.abs(Wb).max()
        assert abs(loss - loss_b) <= 1e-4 * loss_b
        assert torch.all((W == 0) <= (torch.from_numpy(out) == 0))


def test_identity_hessian_is_magnitude_pruning():
    """H = I: no cross-column feedback, equal saliency denominators, so each
    block keeps exactly the entries above its k-th smallest magnitude, and N:M
    prunes the n smallest magnitudes of every group (lower column on ties)."""
    rows, cols, block = 16, 40, 16
    W = _weight(rows, cols, 7).float()
    H = torch.eye(cols)
    _, out, _, _ = osg.sparsify_weight(W, H, 0.5, 0, 0, block, 0.01, False)
    exp = W.clone()
    for i1 in range(0, cols, block):
        b = W[:, i1:i1 + block]
        a = (b * b).flatten()
        thr = torch.sort(a)[0][int(a.numel() * 0.5)]
        exp[:, i1:i1 + block] = torch.where(b * b <= thr, torch.zeros_like(b), b)
    assert torch.equal(out, exp)
    _, out, _, _ = osg.sparsify_weight(W, H, 0.5, 2, 4, block, 0.01, False)
    exp = W.clone().reshape(rows, -1, 4)
    idx = torch.sort(exp.abs(), dim=2, stable=True)[1][:, :, :2]
    exp.scatter_(2, idx, 0.0)
    assert torch.equal(out, exp.reshape(rows, cols))


def test_mask_invariants_and_dead_columns():
    rows, cols, block = 32, 96, 32
    W = _weight(rows, cols, 8).float()
    H = _spd(cols, 9)
    H[:, 5] = 0
    H[5, :] = 0
    _, out, _, _ = osg.sparsify_weight(W, H, 0.6, 0, 0, block, 0.01, False)
    assert torch.all(out[:, 5] == 0)
    for i1 in range(0, cols, block):
        z = int((out[:, i1:i1 + block] == 0).sum())
        assert z == int(rows * block * 0.6) + 1   # every value at or below the k-th smallest
    _, out, _, _ = osg.sparsify_weight(W, H, 0.5, 2, 4, block, 0.01, False)
    assert torch.all((out.reshape(rows, -1, 4) == 0).sum(-1) == 2)


def test_preserve_mask_rejects_lower_target():
    W = _weight(8, 32, 1).float()
    W[:, :20] = 0
    with pytest.raises(ValueError):
        osg.sparsify_weight(W, _spd(32, 2), 0.5, 0, 0, 16, 0.01, True)


def test_non_pd_falls_back_to_identity():
    H = _spd(16, 3)
    H[4, 4] = -100.0
    _, _, hinv, ok = osg.sparsify_weight(_weight(4, 16, 2).float(), H, 0.5, 0, 0, 16, 0.0, False)
    assert not ok and torch.equal(hinv, torch.eye(16))
