"""Host-side operator plumbing without a GPU: signature, fake (meta) shapes,
autograd wiring, torch.compile tracing, and loud failure without the library."""
import inspect

import pytest
import torch

import prefixlm
from prefixlm import _capi, op
from prefixlm.flash_attention_prefixlm_v2 import (compute_aux_seq_tensors_scalars,
                                                  flash_attn_varlen_prefixlm)

REF_PARAMS = ["q", "k", "v", "is_causal", "prefix_lens", "causal_lens", "cu_seqlens", "total_seqlen",
              "numseqs", "max_seqlen_prefix", "max_seqlen_causal", "max_seqlen_all"]


def test_signature_is_reference_plus_optional_scale_and_plan():
    params = list(inspect.signature(flash_attn_varlen_prefixlm).parameters)
    assert params == REF_PARAMS + ["softmax_scale", "plan", "plan_ds_blocks"]
    assert inspect.signature(flash_attn_varlen_prefixlm).parameters["softmax_scale"].default is None
    assert inspect.signature(flash_attn_varlen_prefixlm).parameters["plan"].default is None
    assert prefixlm.compute_aux_seq_tensors_scalars is compute_aux_seq_tensors_scalars


def _meta_inputs(T=256, H=4, D=128):
    q, k, v = (torch.empty((T, H, D), dtype=torch.bfloat16, device="meta", requires_grad=True)
               for _ in range(3))
    seq = {n: torch.empty((T,), dtype=torch.int32, device="meta")
           for n in ("prefix_lens", "causal_lens", "cu_seqlens")}
    for n, val in (("total_seqlen", 200), ("numseqs", 2), ("max_seqlen_prefix", 50),
                   ("max_seqlen_causal", 100), ("max_seqlen_all", 150)):
        seq[n] = torch.tensor(val)
    return q, k, v, seq


def test_fake_shapes_and_autograd_on_meta():
    q, k, v, seq = _meta_inputs()
    out, lse, lo, qa = op.varlen_fwd(q, k, v, False, *seq.values(), 0.1)
    assert lo.shape == q.shape and lo.dtype == torch.int8
    assert qa.dim() == 1 and qa.dtype == torch.float32 and qa.numel() == op._q_amax_count(q.shape[0], q.shape[1])
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    assert lse.shape == (4, 256) and lse.dtype == torch.float32
    o = flash_attn_varlen_prefixlm(q, k, v, False, **seq)
    assert o.shape == q.shape
    o.backward(torch.empty_like(o))
    for t in (q, k, v):
        assert t.grad is not None and t.grad.shape == t.shape and t.grad.device.type == "meta"


def test_torch_compile_traces_the_op():
    q, k, v, seq = _meta_inputs()
    q, k, v = (t.detach() for t in (q, k, v))

    def f(q, k, v):
        return flash_attn_varlen_prefixlm(q, k, v, False, **seq) * 2

    out = torch.compile(f, backend="eager", dynamic=False, fullgraph=True)(q, k, v)
    assert out.shape == q.shape


def test_scalars_must_be_on_cpu():
    q, k, v, seq = _meta_inputs()
    seq["total_seqlen"] = torch.tensor(200, device="meta")
    with pytest.raises(AssertionError, match="CPU"):
        op._cpu_scalar(seq["total_seqlen"], "total_seqlen")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setenv("PREFIXLM_LIB", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_capi, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _capi.load()


def test_meta_tensor_conversion_helpers():
    t = torch.arange(5, dtype=torch.int64)
    m = op._meta(t, torch.device("cpu"))
    assert m.dtype == torch.int32 and m.tolist() == [0, 1, 2, 3, 4]
    with pytest.raises(TypeError):
        op._as_kernel_operand(torch.zeros(4, 2, 128), "q")


def test_residual_operand_is_int8_shaped_like_out():
    """out_lo holds int8 codes: a bf16 residual (an older layout, twice the bytes) or a
    tensor of another shape is refused before any launch; strides that are multiples of
    16 pass as they are, others are made dense."""
    out = torch.zeros(8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="int8"):
        op._as_residual_operand(torch.zeros(8, 2, 128, dtype=torch.bfloat16), out)
    with pytest.raises(ValueError):
        op._as_residual_operand(torch.zeros(8, 2, 64, dtype=torch.int8), out)
    base = torch.zeros(8, 4, 128 + 16, dtype=torch.int8)
    view = base[:, ::2, :128]   # strides (576, 288, 1)
    assert op._as_residual_operand(view, out) is view
    odd = torch.zeros(8, 2, 136, dtype=torch.int8)[:, :, :128]   # strides (272, 136, 1)
    dense = op._as_residual_operand(odd, out)
    assert dense.is_contiguous() and torch.equal(dense, odd)


def test_library_of_another_version_is_refused(monkeypatch):
    """A library whose major.minor version differs from the package's is not used."""
    class Old:
        def __getattr__(self, name):
            return _Fn(100 if name == "prefixlm_version" else 0)

    class _Fn:
        def __init__(self, v):
            self.v = v
        def __call__(self, *a):
            return self.v

    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setattr(_capi.ctypes, "CDLL", lambda path: Old())
    monkeypatch.setattr(_capi.os.path, "exists", lambda path: True)
    with pytest.raises(RuntimeError, match="version 100"):
        _capi.load()
