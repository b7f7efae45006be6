"""The C-ABI library: it loads, exports every symbol include/prefixlm.h declares,
its argument structs match the header's layout, and host-side validation rejects
bad arguments before touching the GPU (no compute calls here)."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from prefixlm import _build, _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "prefixlm.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    return _capi.load()


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*[\w\s\*]*?\b(prefixlm_\w+)\s*\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
        assert n in _capi.SIGNATURES, f"{n} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", _build.LIB_PATH], capture_output=True, text=True)
    exported = set(l.split()[-1] for l in out.stdout.splitlines() if " T " in l)
    assert set(names) <= exported


def test_struct_layout_matches_header():
    fields = {"prefixlm_fwd_args": _capi.FwdArgs, "prefixlm_bwd_args": _capi.BwdArgs,
              "prefixlm_rope_args": _capi.RopeArgs, "prefixlm_kvcache_args": _capi.KvcacheArgs,
              "prefixlm_swiglu_args": _capi.SwigluArgs, "prefixlm_rmsnorm_args": _capi.RmsnormArgs,
              "prefixlm_proj_gemm_args": _capi.ProjGemmArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "prefixlm.h"', "int main(void){"]
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c99", "-I", os.path.dirname(HEADER), src, "-o", exe], check=True)
        res = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    got = {}
    for line in res.splitlines():
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for cname, cls in fields.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert got[(cname, f)] == getattr(cls, f).offset, (cname, f)


def test_workspace_sizes(lib):
    # forward: 64-byte header + one int2 per possible 128-row tile, each 256-aligned
    items = (16384 + 127) // 128 + 16
    assert lib.prefixlm_fwd_workspace_size(16384, 16, 128, 16384, 16) == 256 + ((8 * items + 255) // 256) * 256
    # backward: two (header + items) work lists (128-key and 128-query tiles), the
    # stored-dS block base of every segment, the per-head and per-(segment, head)
    # statistics with 16 work counters, and delta [H, T]; no dQ accumulator
    def al(x):
        return (x + 255) // 256 * 256
    kv_items = (16384 + 127) // 128 + 16
    q_items = (16384 + 127) // 128 + 16
    want = (al(4 * 17) + 256 + al(8 * kv_items) + 256 + al(8 * q_items) + al(4 * (16 * 4 + 16 * 16 * 2 + 16))
            + al(4 * 16 * 16384))
    assert lib.prefixlm_bwd_workspace_size(16384, 16, 128, 16384, 16) == want
    # head_dim 64 runs kernels of its own over the same work lists and statistics
    assert (lib.prefixlm_fwd_workspace_size(16384, 16, 64, 16384, 16)
            == lib.prefixlm_fwd_workspace_size(16384, 16, 128, 16384, 16))
    assert lib.prefixlm_bwd_workspace_size(16384, 16, 64, 16384, 16) == want
    assert lib.prefixlm_version() >= 100


def test_version_matches_header_and_loader(lib):
    """The loader refuses a library of another major.minor version (its buffers, out_lo
    above all, have another layout); header, library and loader agree on it."""
    hdr = open(HEADER).read()
    want = int(re.search(r"#define PREFIXLM_VERSION (\d+)", hdr).group(1))
    assert lib.prefixlm_version() == want == _capi.LIB_VERSION


def test_ds_buffer_size(lib):
    # fp16 dS blocks of 32 queries x 64 keys per head, then one fp32 scale per (128-key
    # tile slot, head), T/128 + numseqs + 1 slots. The scalars' bound: (T/32 + numseqs + 1)
    # query tiles x ceil(max_seqlen_all / 64) key groups; or a given block count
    def al(x):
        return (x + 255) // 256 * 256
    for T, H, n, mx in ((16384, 16, 13, 4096), (65536, 16, 8, 8192), (800, 2, 3, 300), (64, 1, 1, 1)):
        blocks = (T // 32 + n + 1) * ((mx + 63) // 64)
        want = al(H * blocks * 4096) + al(4 * H * (T // 128 + n + 1))
        assert lib.prefixlm_bwd_ds_bytes(T, H, n, mx) == want
        assert lib.prefixlm_bwd_ds_bytes_blocks(T, H, n, blocks) == want
        assert lib.prefixlm_bwd_ds_bytes_blocks(T, H, n, 7) == al(H * 7 * 4096) + al(4 * H * (T // 128 + n + 1))
    # 2.2 GB for config 2's shape at max_seqlen_all 4096
    assert 2.1e9 < lib.prefixlm_bwd_ds_bytes(16384, 16, 13, 4096) < 2.3e9
    # no dS path: segments past 32768 rows, one head's blocks past 2 GiB, empty batches
    assert lib.prefixlm_bwd_ds_bytes(65536, 16, 1, 32769) == 0
    assert lib.prefixlm_bwd_ds_bytes(1 << 20, 1, 1, 32768) == 0
    assert lib.prefixlm_bwd_ds_bytes(64, 1, 0, 0) == 0
    assert lib.prefixlm_bwd_ds_bytes_blocks(64, 1, 1, 0) == 0
    assert lib.prefixlm_bwd_ds_bytes_blocks(64, 1, 1, 1 << 19) == 0


def _attended_blocks(prefix, causal):
    """Brute force: (32-row query tile, 64-key group) pairs of each segment with at least
    one allowed (query, key) pair under the mask j <= i or j < prefix."""
    n = 0
    for p, c in zip(prefix, causal):
        L = p + c
        for qt in range((L + 31) // 32):
            for kg in range((L + 63) // 64):
                q1 = min(L, 32 * qt + 32)               # queries 32 qt .. q1 - 1
                k0 = 64 * kg
                if k0 < p or k0 <= q1 - 1:             # key k0 is seen by the last query
                    n += 1
    return n


def test_plan_ds_blocks_count_the_attended_blocks(lib):
    """The plan's stored-dS block count equals a brute-force count of the attended
    (query tile, key group) pairs, on edge packings and on the benchmark's configs."""
    import numpy as np
    from prefixlm import plan_ds_blocks, build_plan
    from prefixlm.synth import metadata_tensors, segments_for_config
    cases = [([0], [1]), ([1], [0]), ([64], [0]), ([0], [64]), ([63], [2]), ([65], [63]), ([0, 100, 5], [300, 0, 27]),
             ([129], [1000]), ([4096], [0]), ([0], [4096])]
    rng = np.random.default_rng(5)
    for _ in range(20):
        m = int(rng.integers(1, 6))
        L = rng.integers(1, 700, m)
        p = (rng.random(m) * (L + 1)).astype(int)
        cases.append((p.tolist(), (L - p).tolist()))
    for cfg in (2, 4):
        cases.append(segments_for_config(cfg))
    for pre, cau in cases:
        T = sum(pre) + sum(cau) + 5
        st, ss = metadata_tensors(pre, cau, T, "cpu")
        got = plan_ds_blocks(build_plan(st, ss))
        assert got == _attended_blocks(pre, cau), (pre, cau)
    with pytest.raises(ValueError):
        plan_ds_blocks(np.zeros(64, dtype=np.int32))


def test_struct_size_is_checked(lib):
    """A caller compiled against another header (another struct size) is rejected."""
    a = _valid_fwd_args()
    a.struct_size = ctypes.sizeof(_capi.FwdArgs) - 8
    assert lib.prefixlm_fwd(ctypes.byref(a), None) == 1 and "struct_size" in _capi.last_error()
    b = _capi.BwdArgs()
    b.struct_size = ctypes.sizeof(_capi.BwdArgs) + 8
    assert lib.prefixlm_bwd(ctypes.byref(b), None) == 1 and "struct_size" in _capi.last_error()


def _valid_fwd_args():
    a = _capi.FwdArgs()
    fake = 1 << 20  # never dereferenced: validation fails first in every case below
    a.q = a.k = a.v = a.out = a.lse = a.workspace = fake
    a.prefix_lens = a.causal_lens = a.cu_seqlens = fake
    for n in ("q", "k", "v", "out"):
        setattr(a, f"{n}_stride_t", 16 * 128)
        setattr(a, f"{n}_stride_h", 128)
    a.meta_len = 64
    a.num_tokens, a.num_heads, a.head_dim = 64, 16, 128
    a.total_seqlen, a.numseqs, a.max_seqlen_all = 64, 2, 40
    a.softmax_scale = 0.088
    a.workspace_bytes = 1 << 20
    return a


@pytest.mark.parametrize("field,value,needle", [
    ("head_dim", 96, "head_dim"),
    ("total_seqlen", 65, "total_seqlen"),
    ("numseqs", 64, "cu_seqlens entries"),
    ("max_seqlen_all", 65, "max_seqlen_all"),
    ("q_stride_t", 100, "strides"),
    ("v_stride_h", 4, "strides"),
    ("workspace_bytes", 16, "workspace"),
    ("q", (1 << 20) + 2, "aligned"),
    ("out", 0, "null"),
])
def test_fwd_validation_rejects(lib, field, value, needle):
    a = _valid_fwd_args()
    setattr(a, field, value)
    rc = lib.prefixlm_fwd(ctypes.byref(a), None)
    assert rc == 1
    assert needle in _capi.last_error()


def test_bwd_validation_rejects(lib):
    a = _capi.BwdArgs()
    a.head_dim = 128
    a.num_tokens = 8
    a.num_heads = 1
    rc = lib.prefixlm_bwd(ctypes.byref(a), None)
    assert rc == 1 and "null" in _capi.last_error()
    assert lib.prefixlm_fwd(None, None) == 1


def test_timer_is_caller_owned(lib):
    """A timer handle holds its own records: reading a fresh one reports no launches
    (no GPU call is made), and two timers are independent objects."""
    t1, t2 = _capi.Timer(), _capi.Timer()
    assert t1._h and t2._h and t1._h != t2._h
    r = t1.read()
    assert set(r) == set(_capi.KERNEL_NAMES) and all(v == (0.0, 0) for v in r.values())
    assert _capi.active_timer().value is None
    with t2:
        assert _capi.active_timer().value == t2._h
    assert _capi.active_timer().value is None
    t1.close()
    t2.close()
    assert lib.prefixlm_timer_read(None, None, None) == 1 and "null" in _capi.last_error()


@pytest.mark.parametrize("field,value,needle", [
    ("K", 100, "multiple"), ("N", 300, "multiple"), ("x_stride", 100, "strides"), ("eps", -1.0, "eps"),
    ("y", 0, "null"),
])
def test_proj_gemm_validation_rejects(lib, field, value, needle):
    a = _capi.ProjGemmArgs(x=1 << 20, w=1 << 20, y=1 << 20, x_stride=2048, w_stride=2048, y_stride=8192,
                           M=16, K=2048, N=8192, swiglu=0, norm=1, eps=1e-6)
    setattr(a, field, value)
    assert lib.prefixlm_proj_gemm(ctypes.byref(a), None) == 1
    assert needle in _capi.last_error()
