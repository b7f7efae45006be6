"""Metadata helper (reference models/flash_attention_prefixlm_v2.py:10-24) and
useful-work counting."""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle.prefixlm_oracle import allowed_two_pass, aux_seq_ref
from prefixlm.metadata import compute_aux_seq_tensors_scalars, useful_entries, useful_flops


def test_known_answer():
    # hand-computed: two segments of lengths 4 and 6 in an 8-token pack
    t, s = compute_aux_seq_tensors_scalars(np.array([3, 2], np.int32), np.array([1, 4], np.int32), 8)
    assert t["prefix_lens"].tolist() == [3, 2, 0, 0, 0, 0, 0, 0]
    assert t["causal_lens"].tolist() == [1, 4, 0, 0, 0, 0, 0, 0]
    # the tail after the last boundary is 0, not the total
    assert t["cu_seqlens"].tolist() == [0, 4, 10, 0, 0, 0, 0, 0]
    assert s == {"total_seqlen": 10, "numseqs": 2, "max_seqlen_prefix": 3,
                 "max_seqlen_causal": 4, "max_seqlen_all": 6}
    for v in t.values():
        assert v.dtype == np.int32 and v.shape == (8,)
    rt, rs = aux_seq_ref([3, 2], [1, 4], 8)
    assert rs == s
    assert all(rt[k] == t[k].tolist() for k in rt)


@settings(max_examples=200, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 50), st.integers(0, 50)), min_size=1, max_size=12),
       st.integers(0, 20))
def test_matches_loop_restatement(segs, extra):
    pre = np.array([a for a, _ in segs], np.int32)
    cau = np.array([b for _, b in segs], np.int32)
    T = len(segs) + 1 + extra
    t, s = compute_aux_seq_tensors_scalars(pre, cau, T)
    rt, rs = aux_seq_ref(pre, cau, T)
    assert s == rs
    for k in rt:
        assert t[k].tolist() == rt[k]
        assert t[k].dtype == np.int32


def test_too_many_segments_rejected():
    with pytest.raises(ValueError):
        compute_aux_seq_tensors_scalars(np.array([1, 1], np.int32), np.array([1, 1], np.int32), 2)


@settings(max_examples=60, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 9), st.integers(0, 9)), min_size=1, max_size=5),
       st.booleans())
def test_useful_entries_brute_force(segs, is_causal):
    pre = [a for a, _ in segs]
    cau = [b for _, b in segs]
    n = 0
    for p, c in segs:
        L = p + c
        n += sum(allowed_two_pass(i, j, p, L, is_causal) for i in range(L) for j in range(L))
    assert useful_entries(pre, cau, is_causal) == n


def test_useful_flops_config3_figure():
    # 8 x 8192 with prefixes {0,512,...,8192}: 361,514,496 attended pairs per head
    pre = [0, 512, 1024, 2048, 4096, 6144, 7680, 8192]
    cau = [8192 - p for p in pre]
    assert useful_entries(pre, cau) == 361_514_496
    assert useful_flops(pre, cau, 16, 128) == 14 * 128 * 16 * 361_514_496
