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
    # |a b| <= 128 * 128 = 2^14: K = 131072 could reach 2^31 (all -128).
    (dict(a_type=rt.I8, b_type=rt.I8, c_type=rt.I32, k=131072, lda=131072, ldb=131072),
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
    (dict(k_transposed=2), rt.EINVAL, "frisk_attn_fwd: k_transposed must be 0 or 1"),
    # K stored [b, h, head_dim, seq_k]: its row stride runs over keys.
    (dict(k_transposed=1, seq_k=4096, k_stride_s=2048, k_stride_h=262144, k_stride_b=262144),
     rt.EINVAL, "frisk_attn_fwd: transposed K needs a head_dim row stride of at least seq_k"),
    (dict(k_transposed=1, seq_k=65, seq_q=65, k_stride_s=72, k_stride_h=9216, k_stride_b=9216),
     rt.EUNSUP, "frisk_attn_fwd: transposed K needs an even seq_k"),
    (dict(k_transposed=1, seq_k=64, k_stride_s=(1 << 24), k_stride_h=(1 << 31),
          k_stride_b=(1 << 31)), rt.EUNSUP, "frisk_attn_fwd: K/V rows span"),
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


def reduce_call(**over):
    d = rt.ReduceDesc(rows=64, cols=64, dtype=rt.F32, kind=rt.REDUCE_SUM, axis=1, clear=1,
                      src=16, ld_src=64, dst=16, dst_stride=1)
    for key, val in over.items():
        setattr(d, key, val)
    lib = rt.load()
    return lib.frisk_reduce(ctypes.byref(d), None), lib.frisk_last_error().decode()


@pytest.mark.parametrize("over,code,prefix", [
    (dict(rows=0), rt.EINVAL, "frisk_reduce: rows and cols"),
    (dict(dtype=rt.I32), rt.EINVAL, "frisk_reduce: dtype"),
    (dict(dtype=rt.E4M3), rt.EINVAL, "frisk_reduce: dtype"),
    (dict(kind=3), rt.EINVAL, "frisk_reduce: unknown reduction kind"),
    (dict(axis=2), rt.EINVAL, "frisk_reduce: axis"),
    (dict(src=0), rt.EINVAL, "frisk_reduce: null"),
    (dict(src=18), rt.EINVAL, "frisk_reduce: pointers must be element-aligned"),
    (dict(ld_src=32), rt.EINVAL, "frisk_reduce: ld_src"),
    (dict(dst_stride=0), rt.EINVAL, "frisk_reduce: ld_src"),
    (dict(axis=0, rows=1 << 23, ld_src=64), rt.EUNSUP, "frisk_reduce: size"),
    (dict(leaf_order_bits=5), rt.EINVAL, "frisk_reduce: a leaf order of 5 bits"),
    (dict(leaf_order_bits=31), rt.EINVAL, "frisk_reduce: leaf_order_bits"),
    (dict(leaf_order_bits=6, leaf_order=(ctypes.c_uint8 * 32)(0, 1, 2, 3, 4, 4)), rt.EINVAL,
     "frisk_reduce: leaf_order is not a permutation"),
    (dict(leaf_order_bits=6, leaf_order=(ctypes.c_uint8 * 32)(0, 1, 2, 3, 4, 6)), rt.EINVAL,
     "frisk_reduce: leaf_order is not a permutation"),
])
def test_reduce_rejects_invalid_requests(over, code, prefix):
    rc, msg = reduce_call(**over)
    assert rc == code and msg.startswith(prefix), (rc, msg)


def copy_call(**over):
    d = rt.CopyDesc(rows=8, cols=8, src_type=rt.F32, dst_type=rt.BF16, src=16, ld_src=8, dst=16,
                    ld_dst=8)
    for key, val in over.items():
        setattr(d, key, val)
    lib = rt.load()
    return lib.frisk_copy(ctypes.byref(d), None), lib.frisk_last_error().decode()


@pytest.mark.parametrize("over,code,prefix", [
    (dict(cols=0), rt.EINVAL, "frisk_copy: rows and cols"),
    (dict(src_type=9), rt.EINVAL, "frisk_copy: unknown element type"),
    (dict(src_type=rt.I8), rt.EINVAL, "frisk_copy: no conversion i8 -> bf16"),
    (dict(dst_type=rt.I32), rt.EINVAL, "frisk_copy: no conversion f32 -> i32"),
    (dict(dst=0), rt.EINVAL, "frisk_copy: null"),
    (dict(src=18), rt.EINVAL, "frisk_copy: pointers"),
    (dict(ld_dst=4), rt.EINVAL, "frisk_copy: row stride"),
])
def test_copy_rejects_invalid_requests(over, code, prefix):
    rc, msg = copy_call(**over)
    assert rc == code and msg.startswith(prefix), (rc, msg)


def fill_call(**over):
    d = rt.FillDesc(rows=8, cols=8, dtype=rt.F32, value=1.0, dst=16, ld=8)
    for key, val in over.items():
        setattr(d, key, val)
    lib = rt.load()
    return lib.frisk_fill(ctypes.byref(d), None), lib.frisk_last_error().decode()


@pytest.mark.parametrize("over,code,prefix", [
    (dict(rows=-1), rt.EINVAL, "frisk_fill: rows and cols"),
    (dict(dtype=11), rt.EINVAL, "frisk_fill: unknown element type"),
    (dict(dst=0), rt.EINVAL, "frisk_fill: null"),
    (dict(dtype=rt.I32, dst=18), rt.EINVAL, "frisk_fill: pointer"),
    (dict(ld=7), rt.EINVAL, "frisk_fill: row stride"),
    (dict(dtype=rt.I8, value=128.0), rt.EINVAL, "frisk_fill: value"),
    (dict(dtype=rt.I32, value=0.5), rt.EINVAL, "frisk_fill: value"),
])
def test_fill_rejects_invalid_requests(over, code, prefix):
    rc, msg = fill_call(**over)
    assert rc == code and msg.startswith(prefix), (rc, msg)


def test_tileop_null_descriptors():
    lib = rt.load()
    assert lib.frisk_reduce(None, None) == rt.EINVAL
    assert lib.frisk_copy(None, None) == rt.EINVAL
    assert lib.frisk_fill(None, None) == rt.EINVAL


def test_descriptor_layouts_match_the_header(tmp_path):
    """sizeof / offsetof of every descriptor as a C compiler lays out
    include/frisk_hip.h, against the ctypes mirrors."""
    import subprocess
    structs = {"frisk_gemm_desc": rt.GemmDesc, "frisk_attn_desc": rt.AttnDesc,
               "frisk_reduce_desc": rt.ReduceDesc, "frisk_copy_desc": rt.CopyDesc,
               "frisk_fill_desc": rt.FillDesc}
    lines = ['#include <stddef.h>', '#include <stdio.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict((" ".join(l.split()[:2]), int(l.split()[2])) for l in out if l)
    for cname, py in structs.items():
        assert got[f"{cname} size"] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[f"{cname} {field}"] == getattr(py, field).offset, (cname, field)


def test_reduce_workspace_size_query():
    lib = rt.load()

    def size(**over):
        d = rt.ReduceDesc(rows=64, cols=64, dtype=rt.F32, kind=rt.REDUCE_SUM, axis=1, clear=1,
                          src=16, ld_src=64, dst=16, dst_stride=1)
        for key, val in over.items():
            setattr(d, key, val)
        return lib.frisk_reduce_workspace_size(ctypes.byref(d))

    assert size() == 0                                           # axis 1: one pass
    assert size(axis=0, rows=255) == 0                           # few rows: one pass
    # 16384 columns = 128 strips of 128; 1024 workgroups -> 8 row blocks of 1024
    assert size(axis=0, rows=8192, cols=16384, ld_src=16384) == 8 * 16384 * 4
    # 32 strips: 32 blocks wanted; blocks are capped at 2^15 rows (8 groups x 2^12)
    assert size(axis=0, rows=1 << 22, cols=4096, ld_src=4096) == 128 * 4096 * 4
    # 64 columns = 16 slots: one strip, 16 row groups, 1024 blocks of at least 128 rows
    assert size(axis=0, rows=4096, cols=64, ld_src=64) == 32 * 64 * 4
    assert size(axis=0, rows=8192, cols=16384, ld_src=16384, leaf_order_bits=13,
                leaf_order=(ctypes.c_uint8 * 32)(*range(13))) == 0
    assert size(rows=0) == rt.EINVAL
    assert lib.frisk_reduce_workspace_size(None) == rt.EINVAL


def test_reduce_rejects_a_short_workspace():
    rc, msg = reduce_call(axis=0, rows=8192, cols=16384, ld_src=16384, workspace=16,
                          workspace_bytes=1000)
    assert rc == rt.EINVAL and msg.startswith("frisk_reduce: workspace of 1000 bytes"), msg
    rc, msg = reduce_call(axis=0, rows=8192, cols=16384, ld_src=16384, workspace=24,
                          workspace_bytes=8 * 16384 * 4)
    assert rc == rt.EINVAL and "16-byte aligned" in msg, msg


def gemm_size(**over):
    d = rt.GemmDesc(m=128, n=4096, k=4096, trans_a=0, trans_b=1, a_type=rt.BF16, b_type=rt.BF16,
                    c_type=rt.BF16, clear_accum=1, a=16, lda=4096, b=16, ldb=4096, c=16,
                    ldc=4096, scale_a=1.0, scale_b=1.0)
    for key, val in over.items():
        setattr(d, key, val)
    return rt.load().frisk_gemm_workspace_size(ctypes.byref(d))


def test_gemm_workspace_size_query():
    # The plan assumes 256 CUs where no device answers (and MI355X has 256).
    # 128 x 4096 x 4096 on 128 x 128 tiles: 32 tiles; 8 slices of 1 KiB of
    # K (one workgroup per CU; f32 partials at most the bytes of A and B),
    # summed by a second launch: slices x M x N f32.
    assert gemm_size() == 8 * 128 * 4096 * 4
    # 256 x 4096 x 4096: 64 tiles, 4 slices.
    assert gemm_size(m=256) == 4 * 256 * 4096 * 4
    # 512 x 4096 x 4096: 128 tiles in 2 slices, summed inside the GEMM
    # launch: a 128x128 f32 partial per (tile, slice), then 64 arrival
    # words of 8 bytes per tile.
    assert gemm_size(m=512) == 128 * 2 * 128 * 128 * 4 + 128 * 64 * 8
    # 1024 x 4096 x 14336: 64 256x256 tiles in 4 slices (slice sum).
    assert gemm_size(m=1024, k=14336, lda=14336, ldb=14336) == 4 * 1024 * 4096 * 4
    # 1024 x 4096 x 4096: 256 128x128 tiles already fill the CUs; no split.
    assert gemm_size(m=1024) == 0
    # 16 x 2048 x 16384 on the small-M kernel: 64-column tiles -> 32 tiles,
    # 8 slices (one workgroup per CU).
    assert gemm_size(m=16, n=2048, k=16384, lda=16384, ldb=16384, ldc=2048) == 8 * 16 * 2048 * 4
    # 16 x 4096 x 14336: 256 unsplit 16-column tiles fill the CUs in one
    # round, so it does not split; 16 x 5120 x 14336 (320 tiles) does.
    assert gemm_size(m=16, k=14336, lda=14336, ldb=14336) == 0
    assert gemm_size(m=16, n=5120, k=14336, lda=14336, ldb=14336, ldc=5120) == 4 * 16 * 5120 * 4
    # 16 x 14336 x 4096: 224 tiles fill 7/8 of 256 CUs in one round, no split
    # (also at M = 64); 16 x 8192 x 8192: 256 unsplit 32-column tiles, no
    # split; M = 32 there: 128 tiles, 2 slices.
    assert gemm_size(m=16, n=14336, ldc=14336) == 0
    assert gemm_size(m=64, n=14336, ldc=14336) == 0
    assert gemm_size(m=16, n=8192, k=8192, lda=8192, ldb=8192, ldc=8192) == 0
    assert gemm_size(m=32, n=8192, k=8192, lda=8192, ldb=8192, ldc=8192) == 2 * 32 * 8192 * 4
    # 16 x 4096 x 4096: W below 64 MiB, no split.
    assert gemm_size(m=16) == 0
    # No split: grids of at least CUs / 2 256x256 tiles, K too short to
    # slice, layouts and types without a split kernel.
    assert gemm_size(m=4096) == 0
    assert gemm_size(k=256, lda=256, ldb=256) == 0
    # Every storage order splits alike (the kernels take all four).
    assert gemm_size(trans_b=0) == 8 * 128 * 4096 * 4
    assert gemm_size(trans_a=1, lda=128) == 8 * 128 * 4096 * 4
    assert gemm_size(a_type=rt.E4M3, b_type=rt.E4M3) == 0
    assert gemm_size(m=0) == rt.EINVAL
    assert rt.load().frisk_gemm_workspace_size(None) == rt.EINVAL


def test_gemm_rejects_a_short_or_misaligned_workspace():
    rc, msg = gemm_call(m=128, n=4096, k=4096, lda=4096, ldb=4096, ldc=4096, workspace=16,
                        workspace_bytes=1000)
    assert rc == rt.EINVAL and msg.startswith("frisk_gemm: workspace of 1000 bytes"), msg
    rc, msg = gemm_call(m=128, n=4096, k=4096, lda=4096, ldb=4096, ldc=4096, workspace=24,
                        workspace_bytes=1 << 30)
    assert rc == rt.EINVAL and "16-byte aligned" in msg, msg
    rc, msg = gemm_call(workspace=16, workspace_bytes=-1)
    assert rc == rt.EINVAL and "negative workspace_bytes" in msg, msg


def plan(**over):
    d = rt.GemmDesc(m=4096, n=4096, k=4096, trans_a=0, trans_b=1, a_type=rt.BF16, b_type=rt.BF16,
                    c_type=rt.BF16, clear_accum=1, a=16, lda=4096, b=16, ldb=4096, c=16,
                    ldc=4096, scale_a=1.0, scale_b=1.0)
    for key, val in over.items():
        setattr(d, key, val)
    return rt.plan_of(d)


def test_gemm_plan_every_layout_runs_on_the_matrix_cores():
    # 4096^3 in each storage order: the 256x256-tile kernel; M/N-major
    # operands are read from LDS with the transposing reads.
    for ta in (0, 1):
        for tb in (0, 1):
            p = plan(trans_a=ta, trans_b=tb)
            assert p["kernel"] == "gemm_w4" and p["tile_m"] == 256, p
            assert p["atom"] == "v_mfma_f32_32x32x16_bf16" and p["waves"] == [2, 2]
            assert p["a_major"] == ("m" if ta else "k") and p["b_major"] == ("k" if tb else "n")
            assert p["lds_read_a"] == ("ds_read_b64_tr_b16" if ta else "ds_read_b128")
            assert p["lds_read_b"] == ("ds_read_b128" if tb else "ds_read_b64_tr_b16")
    p = plan(trans_b=0, a_type=rt.E4M3, b_type=rt.E4M3, c_type=rt.BF16)
    assert p["atom"] == "v_mfma_f32_32x32x64_f8f6f4" and p["lds_read_b"] == "ds_read_b64_tr_b8"
    p = plan(trans_a=1, a_type=rt.I8, b_type=rt.I8, c_type=rt.I32)
    assert p["atom"] == "v_mfma_i32_32x32x32_i8" and p["lds_read_a"] == "ds_read_b64_tr_b8"
    # Fewer than 128 256x256 tiles: 128x128 tiles, in every layout.
    assert plan(m=1024, trans_b=0)["kernel"] == "gemm_128"
    assert plan(m=1024, trans_a=1, lda=1024)["kernel"] == "gemm_128"
    # Small M with K-contiguous operands: the small-M kernel.
    p = plan(m=16)
    assert p["kernel"] == "gemm_skinny" and p["atom"] == "v_mfma_f32_16x16x32_bf16"
    # Split-K shows up in the plan when the workspace is there.
    p = plan(m=128, trans_b=0, workspace_bytes=1 << 30)
    assert p["kernel"] == "gemm_128" and p["slices"] == 8 and p["slice_sum"] == "second_launch"
    assert p["workspace_bytes"] == 8 * 128 * 4096 * 4
    p = plan(m=512, trans_b=0, workspace_bytes=1 << 30)
    assert p["kernel"] == "gemm_128" and p["slices"] == 2 and p["slice_sum"] == "in_launch"
    assert p["workspace_bytes"] == 128 * 2 * 128 * 128 * 4 + 128 * 64 * 8
    p = plan(m=128, trans_b=0)
    assert p["slices"] == 1 and p["slice_sum"] == "none"


def test_gemm_plan_generic_cases():
    # A 16 B misalignment of a pitch, a K-contiguous operand without whole
    # 16 B pieces of K, and a pitch whose tile reaches past 2^31 bytes run the
    # generic kernel.
    # f32 runs on the matrix cores (v_mfma_f32_32x32x2_f32); an N-major f32
    # B is read with four ds_read_b32 (there is no 32-bit transposing read).
    p = plan(a_type=rt.F32, b_type=rt.F32, c_type=rt.F32)
    assert p["kernel"] == "gemm_w4" and p["atom"] == "v_mfma_f32_32x32x2_f32", p
    p = plan(m=512, n=512, k=512, lda=512, ldb=512, ldc=512, trans_b=0, a_type=rt.F32,
             b_type=rt.F32, c_type=rt.F32)
    assert p["kernel"] == "gemm_128" and p["lds_read_b"] == "ds_read_b32", p
    assert plan(a_type=rt.F32, b_type=rt.F32, c_type=rt.F32, lda=4098)["kernel"] == "gemm_generic"
    assert plan(lda=4100)["kernel"] == "gemm_generic"
    assert plan(k=4092, lda=4096, ldb=4096)["kernel"] == "gemm_generic"
    # ...but an M/N-major operand takes any K (its K tail is per k-row).
    assert plan(k=4092, lda=4096, trans_a=1, trans_b=0)["kernel"] == "gemm_w4"
    big = (1 << 31) // (255 * 2) + 8
    assert plan(lda=big - big % 8)["kernel"] == "gemm_generic"
    assert plan(lda=(1 << 31) // (256 * 2) - 4096)["kernel"] == "gemm_w4"
    # M/N-major: (K - 1) pitches plus a tile row.
    assert plan(trans_b=0, ldb=(1 << 31) // (4095 * 2) + 8)["kernel"] == "gemm_generic"
    # Ragged N with a 16 B pitch of C stays on the matrix cores.
    assert plan(n=4090, ldb=4096)["kernel"] == "gemm_w4"
    assert plan(n=4090, ldb=4096, ldc=4090)["kernel"] == "gemm_generic"
    with pytest.raises(ValueError, match="legacy-gemm-shape"):
        plan(m=0)


def test_gemm_variant_requests():
    # frisk_gemm_desc.tile / wave_m / wave_n name the kernel that runs; the
    # plan reports it with its instruction contract in the solver's syntax.
    p = plan(tile=128, wave_m=4, wave_n=1)
    assert p["kernel"] == "gemm_128" and p["requested"] and p["waves"] == [4, 1]
    assert p["wave_tile"] == [32, 128] and p["slices"] == 1
    assert p["mma_contract"] == ('{atom = "v_mfma_f32_32x32x16_bf16", wave_grid = [4, 1], '
                                 'repeats = [1, 4, 2], policy = "FullRow", swapped = false}')
    p = plan(tile=256)
    assert p["kernel"] == "gemm_w4" and p["requested"] and "swapped = true" in p["mma_contract"]
    assert plan(tile=128)["waves"] == [2, 2]
    # The library's own choice is reported unrequested, with its contract.
    p = plan()
    assert not p["requested"] and 'repeats = [4, 4, 4], policy = "Square"' in p["mma_contract"]
    # A requested variant runs unsplit: no workspace is asked for.
    d = rt.GemmDesc(m=128, n=4096, k=4096, trans_a=0, trans_b=0, a_type=rt.BF16, b_type=rt.BF16,
                    c_type=rt.BF16, clear_accum=1, a=16, lda=4096, b=16, ldb=4096, c=16,
                    ldc=4096, scale_a=1.0, scale_b=1.0, tile=128)
    assert rt.load().frisk_gemm_workspace_size(ctypes.byref(d)) == 0
    d.tile = 0
    assert rt.load().frisk_gemm_workspace_size(ctypes.byref(d)) > 0
    # Small M requested on 128x128 tiles runs there, not on the small-M kernel.
    assert plan(m=16, tile=128, wave_m=2, wave_n=1)["kernel"] == "gemm_128"
    for bad in (dict(tile=128, wave_m=3, wave_n=1), dict(tile=256, wave_m=4, wave_n=1),
                dict(tile=64), dict(wave_m=2, wave_n=2), dict(tile=128, wave_m=2),
                dict(tile=128, variant_flags=1)):
        with pytest.raises(ValueError, match="no kernel variant"):
            plan(**bad)
    # Valid variant, but the request is not matrix-core work.
    for bad in (dict(a_type=rt.F32, b_type=rt.F32, c_type=rt.F32, lda=4098), dict(lda=4100)):
        with pytest.raises(ValueError, match="runs on the matrix cores only"):
            plan(tile=128, **bad)
    rc, msg = gemm_call(tile=256, lda=4100)
    assert rc == rt.EUNSUP and "256x256-tile variant" in msg, msg


def test_attn_rejects_kv_rows_beyond_32bit_offsets():
    # 32 heads x 128 dims viewed [b, s, h, d] -> [b, h, s, d]: a key row is
    # 8 KiB apart, so key 2^18 (the 2^18 + 1st) starts at 2 GiB.
    rc, msg = attn_call(seq_q=64, seq_k=262145, k_stride_s=4096, v_stride_s=4096,
                        k_stride_b=4096 * 262145, v_stride_b=4096 * 262145, k_stride_h=128,
                        v_stride_h=128)
    assert rc == rt.EUNSUP and "2^31 - 1 bytes" in msg, msg


def noalloc_call(**over):
    d = rt.GemmDesc(m=64, n=64, k=64, trans_a=0, trans_b=1, a_type=rt.BF16, b_type=rt.BF16,
                    c_type=rt.BF16, clear_accum=1, a=16, lda=64, b=16, ldb=64, c=16, ldc=64,
                    scale_a=1.0, scale_b=1.0)
    for key, val in over.items():
        setattr(d, key, val)
    lib = rt.load()
    rc = lib.frisk_gemm_noalloc(ctypes.byref(d), None)
    return rc, lib.frisk_last_error().decode()


def test_gemm_noalloc_rejects_before_any_device_work():
    # The usual contract checks, a caller workspace, and a split whose
    # partials exceed the library's scratch (768 x 8192 x 28672 splits into
    # 120 MiB of partials; the scratch holds 64 MiB).
    rc, msg = noalloc_call(m=0)
    assert rc == rt.EINVAL and msg.startswith("legacy-gemm-shape"), msg
    rc, msg = noalloc_call(workspace=16, workspace_bytes=1 << 20)
    assert rc == rt.EINVAL and "takes no workspace" in msg, msg
    # The descriptor carries fake device pointers: it may only reach the
    # call if the size check is certain to reject it before any launch, so
    # the split's workspace is checked to exceed the scratch first (on a
    # device with another CU count the plan could differ).
    big = dict(m=768, n=8192, k=28672, lda=28672, ldb=28672, ldc=8192)
    d = rt.GemmDesc(big["m"], big["n"], big["k"], 0, 1, rt.BF16, rt.BF16, rt.BF16, 1, 16,
                    big["lda"], 16, big["ldb"], 16, big["ldc"], 1.0, 1.0, None, 0, 0, 0, 0, 0)
    need = rt.load().frisk_gemm_workspace_size(ctypes.byref(d))
    if need <= rt.NOALLOC_SCRATCH_BYTES:
        pytest.skip(f"this device splits 768x8192x28672 into {need} bytes, within the scratch")
    rc, msg = noalloc_call(**big)
    assert rc == rt.EUNSUP and "beyond the 67108864-byte scratch" in msg, msg
    assert rt.NOALLOC_SCRATCH_BYTES == 64 << 20
    assert "#define FRISK_GEMM_NOALLOC_SCRATCH_BYTES (64ll << 20)" in HEADER.read_text()


def test_last_error_is_per_thread():
    # Two host threads fail in lockstep with different errors; after both
    # have failed, each reads back its own message (thread-local
    # frisk_last_error), across many rounds.
    import threading
    rounds = 200
    barrier = threading.Barrier(2)
    seen = {0: [], 1: []}
    bad = {0: dict(m=0), 1: dict(b_type=rt.F16)}
    prefix = {0: "legacy-gemm-shape", 1: "legacy-gemm-type"}

    def work(t):
        lib = rt.load()
        for _ in range(rounds):
            d = rt.GemmDesc(m=64, n=64, k=64, trans_a=0, trans_b=1, a_type=rt.BF16, b_type=rt.BF16,
                            c_type=rt.BF16, clear_accum=1, a=16, lda=64, b=16, ldb=64, c=16,
                            ldc=64, scale_a=1.0, scale_b=1.0)
            for key, val in bad[t].items():
                setattr(d, key, val)
            rc = lib.frisk_gemm(ctypes.byref(d), None)
            barrier.wait()
            seen[t].append((rc, lib.frisk_last_error().decode()))
            barrier.wait()

    ths = [threading.Thread(target=work, args=(t,)) for t in (0, 1)]
    for th in ths:
        th.start()
    for th in ths:
        th.join(timeout=60)
    for t in (0, 1):
        assert len(seen[t]) == rounds
        assert all(rc == rt.EINVAL and msg.startswith(prefix[t]) for rc, msg in seen[t]), seen[t][:3]
