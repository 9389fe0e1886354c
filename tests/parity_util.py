"""Shared helpers of the GPU parity tests (code agreement statistics)."""
import torch


def code_agreement(a: torch.Tensor, b: torch.Tensor) -> dict:
    """Agreement statistics of two code matrices [rows, cols].

    GPTQ feeds each column's rounding error into the later columns of its
    row, so a value that sits on a rounding boundary in one implementation
    and just off it in another flips by one code, and the row then diverges
    (the oracle run against itself with only the Cholesky chain's fp32
    operation order changed shows the same cascades).  The first divergence
    of every row is therefore the meaningful check: it must be a +-1 flip.
    """
    d = (a - b).abs()
    nz = d != 0
    first = torch.zeros(a.shape[0], dtype=torch.int32)
    rows = nz.any(1)
    if bool(rows.any()):
        idx = nz.int().argmax(1)
        first = torch.where(rows, d.gather(1, idx[:, None])[:, 0], first)
    return {"agree": 1.0 - nz.float().mean().item(), "mismatches": int(nz.sum()), "rows_diverged": int(rows.sum()),
            "max_diff": int(d.max()), "first_divergence_max": int(first.max()),
            "frac_beyond_1": (d > 1).float().mean().item()}


def code_bar(st: dict, rows: int, rows_frac: float = 0.01) -> bool:
    """The end-to-end GPTQ code bar: >= 99.9 % of codes agree, every row's
    first divergence is a one-code flip, and at most ``rows_frac`` of the rows
    (1 %) diverge at all (codes after a row's first flip may differ by more
    than one, as they do between two runs of the oracle itself under a
    different BLAS thread count).  FP8 weights take 2 %: e4m3's grid step is
    relative to each value rather than to the group's range, so more values
    sit near a boundary; the oracle against itself with only the Hessian's
    fp32 summation changed diverges in up to 3 of 384 rows at 384 x 1024
    (``gptq_code_spread.py --formats``), where int4 diverges in at most one."""
    return (st["agree"] >= 0.999 and st["first_divergence_max"] <= 1
            and st["rows_diverged"] <= max(1, int(rows * rows_frac)))
