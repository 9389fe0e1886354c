"""Host logic of the Hessian staging (no GPU): every row reaches the
accumulation exactly once, in call order, with the calls' sample counts;
16-bit rows at least 512 wide are handed over as the callers' own tensors
(no copy) unless they are small, cannot be held, or were modified in place."""
import torch
import pytest

from llmcompressor_amd.staging import HessianStage


class Recorder:
    def __init__(self):
        self.calls = []
        self.segs = []

    def __call__(self, segs, samples):
        assert isinstance(segs, list) and segs
        self.segs.append(list(segs))
        self.calls.append((torch.cat([s.clone() for s in segs]), samples))


def _run(sizes, tokens, dtypes=None, d=8):
    rec, stage = Recorder(), HessianStage(tokens)
    sent, total = [], 0
    for i, n in enumerate(sizes):
        dt = dtypes[i] if dtypes else torch.float32
        x = (torch.arange(n * d, dtype=torch.float32).reshape(n, d) + 1000 * i).to(dt)
        sent.append(x)
        stage.add(x, i + 1, rec)
        total += i + 1
    stage.flush(rec)
    return rec, sent, total


@pytest.mark.parametrize("sizes", [[3, 3, 3, 3, 3], [8, 8, 1], [2, 9, 2, 2], [16], [5, 11, 4, 4, 4, 4]],
                         ids=["small", "exact-fill", "pass-through", "one-big", "mixed"])
def test_rows_in_order_once(sizes):
    tokens = 16
    rec, sent, total = _run(sizes, tokens)
    got = torch.cat([r for r, _ in rec.calls])
    assert torch.equal(got, torch.cat(sent))
    assert sum(s for _, s in rec.calls) == total
    for rows, _ in rec.calls:
        assert rows.shape[0] <= max(tokens, max(sizes))


def test_full_buffer_flushes_at_once():
    rec, stage = Recorder(), HessianStage(8)
    for i in range(4):
        stage.add(torch.ones(2, 4) * i, 1, rec)
    assert len(rec.calls) == 1 and rec.calls[0][0].shape[0] == 8 and rec.calls[0][1] == 4
    stage.flush(rec)
    assert len(rec.calls) == 1           # nothing left


def test_large_call_goes_through_after_staged_rows():
    rec, stage = Recorder(), HessianStage(16)
    stage.add(torch.zeros(3, 4), 1, rec)
    stage.add(torch.ones(9, 4), 2, rec)   # more than half the buffer
    assert [c[0].shape[0] for c in rec.calls] == [3, 9] and [c[1] for c in rec.calls] == [1, 2]


def test_dtype_or_width_change_flushes_first():
    rec, _, _ = _run([3, 3, 3], 16, dtypes=[torch.float32, torch.bfloat16, torch.bfloat16])
    assert [c[0].dtype for c in rec.calls] == [torch.float32, torch.bfloat16]
    assert [c[0].shape[0] for c in rec.calls] == [3, 6]
    rec, stage = Recorder(), HessianStage(16)
    stage.add(torch.zeros(2, 4), 1, rec)
    stage.add(torch.zeros(2, 6), 1, rec)
    stage.flush(rec)
    assert [tuple(c[0].shape) for c in rec.calls] == [(2, 4), (2, 6)]


def test_rejects_empty_buffer():
    with pytest.raises(ValueError):
        HessianStage(0)


def test_modifier_stage_budget():
    """A module gets a stage while the stages held fit in the budget; the
    rest accumulate every call at once, and a dropped stage frees its share."""
    from llmcompressor_amd.modifiers import _Staging

    class M(_Staging):
        pass

    m = M()
    m._init_staging(tokens=1024, budget=3 * 1024 * 64 * 2)   # three stages of 1024 x 64 bf16
    x = torch.zeros(16, 64, dtype=torch.bfloat16)
    mods = [object() for _ in range(5)]
    got = [m._stage_for(k, x) for k in mods]
    assert [g is not None for g in got] == [True, True, True, False, False]
    assert m._stage_for(mods[3], x) is None and m._stage_held == 3 * 1024 * 64 * 2
    rec = Recorder()
    got[0].add(x, 1, rec)
    m._drop_stage(mods[0], rec)
    assert len(rec.calls) == 1 and rec.calls[0][0].shape == (16, 64)
    assert m._stage_held == 2 * 1024 * 64 * 2 and mods[0] not in m._stages
    assert m._stage_for(mods[0], x) is not None            # room again


def test_stage_rows_capped_at_1_gib():
    from llmcompressor_amd.staging import DEFAULT_TOKENS, stage_tokens
    assert DEFAULT_TOKENS == 131072
    assert stage_tokens(DEFAULT_TOKENS, 4096, 2) == 131072       # 1 GiB: 64 calls of 2048 rows
    assert stage_tokens(DEFAULT_TOKENS, 14336, 2) == 36864       # 1008 MiB
    assert stage_tokens(DEFAULT_TOKENS, 14336, 4) == 18432
    assert stage_tokens(1024, 64, 2) == 1024
    assert stage_tokens(DEFAULT_TOKENS, 1 << 20, 4) == 2048      # never below one 2048-row sample


def _bf(n, d=512, tag=0):
    return (torch.arange(n * d, dtype=torch.float32).reshape(n, d) % 251 + tag).to(torch.bfloat16)


def test_wide_16bit_calls_held_by_reference():
    """2048-row bf16 calls are the segments themselves (no copy), in call
    order; small calls are copied into one buffer segment after them."""
    rec, stage = Recorder(), HessianStage(8192)
    xs = [_bf(2048, tag=i) for i in range(3)]
    small = [_bf(100, tag=10 + i) for i in range(2)]
    stage.add(xs[0], 1, rec)
    stage.add(small[0], 1, rec)
    stage.add(xs[1], 1, rec)
    stage.add(small[1], 1, rec)
    stage.add(xs[2], 1, rec)
    stage.flush(rec)
    assert len(rec.segs) == 1 and rec.calls[0][1] == 5
    segs = rec.segs[0]
    assert [s.data_ptr() for s in segs[:3]] == [x.data_ptr() for x in xs]
    assert torch.equal(segs[3], torch.cat(small))
    assert stage.fill == 0 and not stage._segs


def test_held_rows_modified_in_place_raise():
    rec, stage = Recorder(), HessianStage(8192)
    x = _bf(1024)
    stage.add(x, 1, rec)
    x.add_(1)
    with pytest.raises(RuntimeError, match="modified in place"):
        stage.flush(rec)
    assert not rec.calls


def test_unholdable_calls_are_copied():
    """A view into a much larger tensor, another row stride and an inference
    tensor are held as copies (still one segment each)."""
    rec, stage = Recorder(), HessianStage(16384)
    big = _bf(8192)
    view = big[:1024]                     # storage eight times the rows
    strided = _bf(1024, d=1024)[:, :512]  # row stride 1024
    with torch.inference_mode():
        inf = _bf(1024, tag=3)
    for x in (view, strided, inf):
        stage.add(x, 1, rec)
    stage.flush(rec)
    segs = rec.segs[0]
    assert len(segs) == 3
    for s, x in zip(segs, (view, strided, inf)):
        assert s.data_ptr() != x.data_ptr() and s.is_contiguous() and torch.equal(s, x)


def test_segment_count_flushes():
    from llmcompressor_amd.staging import MAX_SEGMENTS
    rec, stage = Recorder(), HessianStage(1 << 20)
    for i in range(MAX_SEGMENTS + 3):
        stage.add(_bf(256, tag=i % 7), 1, rec)
    stage.flush(rec)
    assert [len(s) for s in rec.segs] == [MAX_SEGMENTS, 3]
    assert [c[1] for c in rec.calls] == [MAX_SEGMENTS, 3]


def test_narrow_or_fp32_rows_stay_copied():
    rec, stage = Recorder(), HessianStage(8192)
    xs = [_bf(1024, d=256, tag=i) for i in range(3)]
    for x in xs:
        stage.add(x, 1, rec)
    stage.flush(rec)
    assert len(rec.segs[0]) == 1 and torch.equal(rec.segs[0][0], torch.cat(xs))
