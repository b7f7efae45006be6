"""Host work-list plans (prefixlm.plan): layout, coverage, ordering and errors.

The plan is this build's own format (the reference sizes its FA3 grids from the
max_seqlen scalars, models/flash_attention_prefixlm_v2.py:115-128), so it is pinned
by what the kernels need from it: every (segment, tile) pair exactly once, ordered
by a cost that equals the kernels' inner trip count, which is recounted here by
brute force from the mask rule (query i sees key j iff j <= i or j < p).
"""
import numpy as np
import pytest

from prefixlm import build_plan, compute_aux_seq_tensors_scalars, plan_size

MAGIC = 0x50524C32
# (tile rows, inner tile) of the three lists: forward 128-query tiles over 32-key
# tiles, backward 128-key tiles over 32-row query tiles, backward 128-query tiles
# over 32-key tiles
LISTS = (("fwd", 128, 32), ("kv", 128, 32), ("q", 128, 32))


def _align(x):
    return (x + 255) // 256 * 256


def _layout(total, nseq):
    """Three lists (header, items), then int32 ds_base[nseq + 1]."""
    off, out = 0, []
    for _, tile, _ in LISTS:
        nmax = (total + tile - 1) // tile + nseq
        out.append((off, off + 256, nmax))
        off += 256 + _align(8 * nmax)
    return out, off + _align(4 * (nseq + 1))


def _sees(i, j, p, causal):
    return j <= i or (not causal and j < p)


def _brute_cost(kind, t, tile, inner, p, L, causal):
    """Inner trip count of one work item, from the mask rule alone."""
    if kind in ("fwd", "q"):
        rows = range(t * tile, min((t + 1) * tile, L))
        kend = max(j for i in rows for j in range(L) if _sees(i, j, p, causal)) + 1
        return -(-kend // inner)
    keys = range(t * tile, min((t + 1) * tile, L))
    qmin = min(i for i in range(L) for j in keys if _sees(i, j, p, causal))
    return -(-(L - qmin // inner * inner) // inner)


def _parse(plan, total, nseq):
    lay, nbytes = _layout(total, nseq)
    assert plan.nbytes == nbytes
    raw = plan.view(np.int32)
    lists = []
    for (hoff, ioff, nmax), (_, tile, _) in zip(lay, LISTS):
        h = raw[hoff // 4: hoff // 4 + 16]
        assert h[2] == MAGIC and h[3] == nseq and h[4] == total and h[5] == tile
        assert h[1] == 0
        n = int(h[0])
        assert n <= nmax
        items = raw[ioff // 4: ioff // 4 + 2 * n].reshape(n, 2)
        lists.append(items)
    return lists


def _batch(prefix, causal, T):
    prefix = np.asarray(prefix, dtype=np.int32)
    causal = np.asarray(causal, dtype=np.int32)
    return compute_aux_seq_tensors_scalars(prefix, causal, T)


CASES = [
    ([3, 2], [1, 4], 16),                       # the reference helper's example shape
    ([0, 200, 1, 130], [300, 0, 0, 127], 1024),  # pure causal, pure prefix, one token, tile edges
    ([128, 64, 0], [128, 200, 129], 700),
]


@pytest.mark.parametrize("prefix,causal,T", CASES)
@pytest.mark.parametrize("is_causal", [False, True])
def test_plan_covers_every_tile_once_in_cost_order(prefix, causal, T, is_causal):
    tensors, scalars = _batch(prefix, causal, T)
    plan = build_plan(tensors, scalars, is_causal)
    assert plan.dtype == np.int32 and plan.nbytes == plan_size(scalars["total_seqlen"], scalars["numseqs"])
    lists = _parse(plan, scalars["total_seqlen"], scalars["numseqs"])
    for (kind, tile, inner), items in zip(LISTS, lists):
        want = {(s, t) for s, (p, c) in enumerate(zip(prefix, causal)) for t in range(-(-(p + c) // tile))}
        got = [tuple(x) for x in items.tolist()]
        assert len(got) == len(set(got)) and set(got) == want, kind
        costs = [_brute_cost(kind, t, tile, inner, prefix[s], prefix[s] + causal[s], is_causal) for s, t in got]
        assert all(a >= b for a, b in zip(costs, costs[1:])), (kind, costs)
        # ties keep (segment, tile) order: the plan is a function of the metadata
        for k in range(len(got) - 1):
            if costs[k] == costs[k + 1]:
                assert got[k] < got[k + 1]


def test_plan_is_deterministic_and_accepts_tensors():
    import torch
    tensors, scalars = _batch([5, 300, 0], [20, 1, 77], 512)
    a = build_plan(tensors, scalars)
    b = build_plan({k: torch.from_numpy(v) for k, v in tensors.items()},
                   {k: torch.tensor(v) for k, v in scalars.items()})
    assert np.array_equal(a, b)


def test_causal_flag_changes_order_only():
    tensors, scalars = _batch([100, 7], [28, 300], 512)
    a = _parse(build_plan(tensors, scalars, False), scalars["total_seqlen"], 2)
    b = _parse(build_plan(tensors, scalars, True), scalars["total_seqlen"], 2)
    for x, y in zip(a, b):
        assert sorted(map(tuple, x.tolist())) == sorted(map(tuple, y.tolist()))


def test_empty_batch_plan():
    tensors = {n: np.zeros(8, dtype=np.int32) for n in ("prefix_lens", "causal_lens", "cu_seqlens")}
    plan = build_plan(tensors, {"numseqs": 0, "total_seqlen": 0})
    for items in _parse(plan, 0, 0):
        assert items.shape == (0, 2)


def test_plan_rejects_inconsistent_metadata():
    tensors, scalars = _batch([3, 2], [1, 4], 16)
    bad = dict(tensors)
    bad["cu_seqlens"] = tensors["cu_seqlens"].copy()
    bad["cu_seqlens"][2] += 1
    with pytest.raises(RuntimeError, match="inconsistent metadata"):
        build_plan(bad, scalars)
    with pytest.raises(RuntimeError):
        build_plan(tensors, dict(scalars, total_seqlen=99))


@pytest.mark.parametrize("prefix,causal,T", CASES)
@pytest.mark.parametrize("is_causal", [False, True])
def test_plan_ds_bases(prefix, causal, T, is_causal):
    """The stored-dS section: ds_base[s + 1] - ds_base[s] is the number of (32-row query
    tile, 64-key group) pairs of segment s with an attended pair (brute force over the
    mask with the segment's prefix, whatever is_causal), and ds_base[numseqs] is the
    blocks per head the headers carry."""
    tensors, scalars = _batch(prefix, causal, T)
    nseq, total = scalars["numseqs"], scalars["total_seqlen"]
    plan = build_plan(tensors, scalars, is_causal)
    lay, nbytes = _layout(total, nseq)
    raw = plan.view(np.int32)
    ds_off = (nbytes - _align(4 * (nseq + 1))) // 4
    base = raw[ds_off: ds_off + nseq + 1]
    want = [0]
    for p, c in zip(prefix, causal):
        L = p + c
        n = sum(1 for qt in range(-(-L // 32)) for kg in range(-(-L // 64))
                if any(_sees(i, 64 * kg, p, False) for i in range(32 * qt, min(L, 32 * qt + 32))))
        want.append(want[-1] + n)
    assert base.tolist() == want
    for hoff, _, _ in lay:
        assert raw[hoff // 4 + 2 + 4] == want[-1]
