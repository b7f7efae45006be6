"""GPU: size-independent properties of the forward and backward at the benchmark sizes,
checked bitwise (no oracle: these hold for the kernels exactly, whatever the size).

* Scaling dO by a power of two scales dQ, dK and dV by it exactly: every fp16 operand
  scale in the backward (dO's, the stored dS's, dP's) is a power of two chosen from the
  per-head maxima, which move by the same power of two, so the fp16 operands and the
  MFMA results are unchanged and only the exact power-of-two epilogue factors differ.
* Scaling V by a power of two scales O by it (LSE and the residual codes unchanged),
  leaves dV unchanged and scales dQ and dK by it, for the same reason.
* Permuting the segments of a packed batch permutes the rows of every output: work
  items are per (segment, tile, head) and every scale is either per segment or a
  per-head maximum over all rows, so no result depends on where a segment sits.
The reference computes each of these in fp32 (models/flash_attention_prefixlm_v2.py:
115-128, 186-206), where they hold up to rounding; here they hold bitwise.
"""
import numpy as np
import pytest
import torch

from prefixlm import flash_attn_varlen_prefixlm, op
from prefixlm.synth import make_config_batch, metadata_tensors

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _run(b, q=None, k=None, v=None, dout=None, seq=None):
    q, k, v = ((b.q if q is None else q), (b.k if k is None else k), (b.v if v is None else v))
    q, k, v = (t.detach().clone().requires_grad_() for t in (q, k, v))
    seq = b.seq_info if seq is None else seq
    out = flash_attn_varlen_prefixlm(q, k, v, False, **seq)
    out.backward(b.dout if dout is None else dout)
    sc = 1.0 / np.sqrt(b.q.shape[-1])
    _, lse, lo, _ = op.varlen_fwd(q.detach(), k.detach(), v.detach(), False, *seq.values(), sc)
    torch.cuda.synchronize()
    return out.detach(), lse, lo, q.grad, k.grad, v.grad


def _scaled(x, f):
    y = (x.float() * f).to(x.dtype)
    assert torch.equal(y.float(), x.float() * f), "the scaled tensor must be exact"
    return y


@pytest.mark.parametrize("cfg", [2, 4])
@pytest.mark.parametrize("f", [4.0, 0.125])
def test_gradients_scale_with_dout(cfg, f):
    print(f"[prop] config {cfg}: dO x {f}", flush=True)
    b = make_config_batch(cfg, device=DEV, gen_device="cuda")
    base = _run(b)
    got = _run(b, dout=_scaled(b.dout, f))
    for name, x, y in zip(("out", "lse", "out_lo"), base[:3], got[:3]):
        assert torch.equal(x, y), name
    for name, x, y in zip(("dq", "dk", "dv"), base[3:], got[3:]):
        assert torch.equal(_scaled(x, f), y), name


@pytest.mark.parametrize("cfg", [2, 4])
def test_outputs_scale_with_v(cfg):
    f = 8.0
    print(f"[prop] config {cfg}: V x {f}", flush=True)
    b = make_config_batch(cfg, device=DEV, gen_device="cuda")
    base = _run(b)
    got = _run(b, v=_scaled(b.v, f))
    assert torch.equal(_scaled(base[0], f), got[0]), "out"
    assert torch.equal(base[1], got[1]), "lse"
    assert torch.equal(base[2], got[2]), "out_lo"
    assert torch.equal(_scaled(base[3], f), got[3]), "dq"
    assert torch.equal(_scaled(base[4], f), got[4]), "dk"
    assert torch.equal(base[5], got[5]), "dv"


def test_segment_permutation_permutes_outputs():
    """Config 4 (199 segments) with its segments in a random order."""
    print("[prop] config 4: segments permuted", flush=True)
    b = make_config_batch(4, device=DEV, gen_device="cuda")
    T = b.q.shape[0]
    L = b.prefix + b.causal
    cu = np.concatenate([[0], np.cumsum(L)])
    total = int(cu[-1])
    perm = np.random.default_rng(3).permutation(len(L))
    rows = np.concatenate([np.arange(cu[s], cu[s + 1]) for s in perm] + [np.arange(total, T)])
    idx = torch.from_numpy(rows).to(DEV)
    st, ss = metadata_tensors(b.prefix[perm], b.causal[perm], T, DEV)
    seq = {**st, **ss}
    base = _run(b)
    got = _run(b, q=b.q[idx], k=b.k[idx], v=b.v[idx], dout=b.dout[idx], seq=seq)
    for name, x, y in zip(("out", "out_lo", "dq", "dk", "dv"), (base[0], base[2], *base[3:]),
                          (got[0], got[2], *got[3:])):
        assert torch.equal(x[idx], y), name
    assert torch.equal(base[1][:, idx[:total]], got[1][:, :total]), "lse"
