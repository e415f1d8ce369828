"""The C-ABI library (include/frisk_hip.h) on the CPU: it loads, exports
every declared entry point, and rejects invalid requests before any device
work (so these calls need no GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

from frisk_amd import runtime as rt

HEADER = Path(__file__).resolve().parents[1] / "include" / "frisk_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+[\s*]+(frisk_\w+)\s*\(", text, re.M)))


def test_header_declares_the_runtime_exports():
    assert declared_functions() == sorted(rt.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = rt.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.frisk_abi_version() == rt.ABI_VERSION


def gemm_call(**over):
    d = rt.GemmDesc(m=64, n=64, k=64, trans_a=0, trans_b=1, a_type=rt.BF16, b_type=rt.BF16,
                    c_type=rt.BF16, clear_accum=1, a=16, lda=64, b=16, ldb=64, c=16, ldc=64,
                    scale_a=1.0, scale_b=1.0)
    for key, val in over.items():
        setattr(d, key, val)
    lib = rt.load()
    rc = lib.frisk_gemm(ctypes.byref(d), None)
    return rc, lib.frisk_last_error().decode()


@pytest.mark.parametrize("over,code,prefix", [
    (dict(m=0), rt.EINVAL, "legacy-gemm-shape"),
    (dict(k=-3), rt.EINVAL, "legacy-gemm-shape"),
    (dict(b_type=rt.F16), rt.EINVAL, "legacy-gemm-type"),
    (dict(a_type=rt.I8, b_type=rt.I8, c_type=rt.F32), rt.EINVAL, "legacy-gemm-type"),
    (dict(a_type=rt.F32, b_type=rt.F32, c_type=rt.BF16), rt.EINVAL, "legacy-gemm-type"),
    (dict(a=0), rt.EINVAL, "frisk_gemm: null"),
    (dict(ldb=32), rt.EINVAL, "frisk_gemm: leading dimension"),
    (dict(scale_a=2.0), rt.EINVAL, "frisk_gemm: scale"),
    (dict(a_type=rt.I8, b_type=rt.I8, c_type=rt.I32, k=200000, lda=200000, ldb=200000),
     rt.EUNSUP, "frisk_gemm: int8"),
])
def test_gemm_rejects_invalid_requests(over, code, prefix):
    rc, msg = gemm_call(**over)
    assert rc == code and msg.startswith(prefix), (rc, msg)


def attn_call(**over):
    d = rt.AttnDesc(batch=1, heads=1, seq_q=64, seq_k=64, head_dim=128, dtype=rt.BF16, causal=0,
                    sm_scale=0.088, q=16, q_stride_b=8192, q_stride_h=8192, q_stride_s=128,
                    k=16, k_stride_b=8192, k_stride_h=8192, k_stride_s=128,
                    v=16, v_stride_b=8192, v_stride_h=8192, v_stride_s=128,
                    o=16, o_stride_b=8192, o_stride_h=8192, o_stride_s=128, lse=None,
                    o_dtype=rt.BF16)
    for key, val in over.items():
        setattr(d, key, val)
    lib = rt.load()
    rc = lib.frisk_attn_fwd(ctypes.byref(d), None)
    return rc, lib.frisk_last_error().decode()


@pytest.mark.parametrize("over,code,prefix", [
    (dict(seq_q=0), rt.EINVAL, "frisk_attn_fwd: sizes"),
    (dict(dtype=rt.F32), rt.EINVAL, "frisk_attn_fwd: dtype"),
    (dict(head_dim=96, q_stride_s=96, k_stride_s=96, v_stride_s=96, o_stride_s=96), rt.EUNSUP,
     "frisk_attn_fwd: head_dim"),
    (dict(o_dtype=rt.F16), rt.EINVAL, "frisk_attn_fwd: o_dtype"),
    (dict(q=24), rt.EINVAL, "frisk_attn_fwd: Q/K/V/O must be 16-byte"),
    (dict(k_stride_s=100), rt.EINVAL, "frisk_attn_fwd: strides"),
    (dict(v_stride_s=64), rt.EINVAL, "frisk_attn_fwd: sequence stride"),
    (dict(sm_scale=0.0), rt.EINVAL, "frisk_attn_fwd: sm_scale"),
    (dict(o=0), rt.EINVAL, "frisk_attn_fwd: null"),
])
def test_attn_rejects_invalid_requests(over, code, prefix):
    rc, msg = attn_call(**over)
    assert rc == code and msg.startswith(prefix), (rc, msg)


def test_null_descriptor():
    lib = rt.load()
    assert lib.frisk_gemm(None, None) == rt.EINVAL
    assert lib.frisk_attn_fwd(None, None) == rt.EINVAL


def test_python_binding_rejects_host_tensors_and_bad_shapes():
    import torch
    a = torch.zeros(4, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device tensor"):
        rt.gemm(a, a, torch.zeros(4, 4, dtype=torch.bfloat16), trans_b=True)
    with pytest.raises(ValueError, match="rank-2"):
        rt.gemm_desc(torch.zeros(4, dtype=torch.bfloat16), a, a)
