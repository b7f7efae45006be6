"""Synthetic config generators follow the configuration text."""
import numpy as np
import torch

from prefixlm.synth import CONFIG_SHAPES, make_batch, segments_for_config


def test_config1():
    pre, cau = segments_for_config(1)
    L = pre + cau
    assert len(L) == 4 and L.sum() == 4096 and L[-1] >= 1
    assert ((L[:3] >= 256) & (L[:3] <= 2048)).all()
    assert ((pre >= 0) & (pre <= L // 2)).all()


def test_config2():
    pre, cau = segments_for_config(2)
    L = pre + cau
    assert L.sum() == 16384
    assert ((L[:-1] >= 64) & (L[:-1] <= 4096)).all() and 1 <= L[-1] <= 4096
    assert ((pre >= 0) & (pre <= 0.6 * L)).all()
    assert 8 <= len(L) <= 40
    p5, c5 = segments_for_config(5)
    assert (p5 == pre).all() and (c5 == cau).all()


def test_config3():
    pre, cau = segments_for_config(3)
    assert ((pre + cau) == 8192).all()
    assert pre.tolist() == [0, 512, 1024, 2048, 4096, 6144, 7680, 8192]


def test_config4():
    pre, cau = segments_for_config(4)
    L = pre + cau
    assert L.sum() == 32768 and (L == 4096).sum() == 1
    short = L[L != 4096]
    assert ((short[:-1] >= 32) & (short[:-1] <= 256)).all()
    assert ((pre >= np.floor(0.7 * L)) & (pre <= 0.9 * L)).all()


def test_batches_are_seeded_and_bf16():
    a = make_batch([3, 2], [4, 1], 16, 2, 128, seed=5)
    b = make_batch([3, 2], [4, 1], 16, 2, 128, seed=5)
    assert a.q.dtype == torch.bfloat16 and torch.equal(a.q, b.q) and torch.equal(a.dout, b.dout)
    assert a.seq_scalars["total_seqlen"].item() == 10 and a.seq_scalars["numseqs"].item() == 2
    assert a.seq_tensors["cu_seqlens"].tolist()[:4] == [0, 7, 10, 0]
    assert set(CONFIG_SHAPES) == {1, 2, 3, 4, 5}
