"""ctypes binding of libfrisk_hip.so (include/frisk_hip.h).

This is the Python side of the C-ABI: it fills the descriptors from torch
device tensors and calls frisk_gemm / frisk_attn_fwd / frisk_reduce /
frisk_copy / frisk_fill on the current HIP stream.  There is no fallback: if the library is missing or a call fails,
a RuntimeError (or ValueError for rejected requests, matching the
reference's ValueError on contract violations, ffi/ir.cpp:333-341) is raised.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfrisk_hip.so"

F32, F16, BF16, E4M3, I8, I32, F64 = 0, 1, 2, 3, 4, 5, 6
OK, EINVAL, EUNSUP, EHIP = 0, -1, -2, -3

DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", E4M3: "e4m3", I8: "i8", I32: "i32", F64: "f64"}

# Exported symbols declared by include/frisk_hip.h.
EXPORTS = ("frisk_gemm", "frisk_gemm_workspace_size", "frisk_gemm_plan", "frisk_gemm_noalloc",
           "frisk_attn_fwd",
           "frisk_reduce", "frisk_reduce_workspace_size",
           "frisk_copy", "frisk_fill",
           "frisk_last_error", "frisk_abi_version", "frisk_probe_mfma_layout",
           "frisk_probe_lds_transpose")
ABI_VERSION = 7

REDUCE_SUM, REDUCE_MAX, REDUCE_MIN = 0, 1, 2
REDUCE_KINDS = {"sum": REDUCE_SUM, "add": REDUCE_SUM, "max": REDUCE_MAX, "min": REDUCE_MIN}


class GemmDesc(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
        ("trans_a", ctypes.c_int32), ("trans_b", ctypes.c_int32),
        ("a_type", ctypes.c_int32), ("b_type", ctypes.c_int32), ("c_type", ctypes.c_int32),
        ("clear_accum", ctypes.c_int32),
        ("a", ctypes.c_void_p), ("lda", ctypes.c_int64),
        ("b", ctypes.c_void_p), ("ldb", ctypes.c_int64),
        ("c", ctypes.c_void_p), ("ldc", ctypes.c_int64),
        ("scale_a", ctypes.c_float), ("scale_b", ctypes.c_float),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("tile", ctypes.c_int32), ("wave_m", ctypes.c_int32), ("wave_n", ctypes.c_int32),
        ("variant_flags", ctypes.c_int32), ("slices", ctypes.c_int32),
    ]


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64), ("heads", ctypes.c_int64), ("seq_q", ctypes.c_int64),
        ("seq_k", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32), ("sm_scale", ctypes.c_float),
        ("q", ctypes.c_void_p), ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("q_stride_s", ctypes.c_int64),
        ("k", ctypes.c_void_p), ("k_stride_b", ctypes.c_int64), ("k_stride_h", ctypes.c_int64),
        ("k_stride_s", ctypes.c_int64),
        ("v", ctypes.c_void_p), ("v_stride_b", ctypes.c_int64), ("v_stride_h", ctypes.c_int64),
        ("v_stride_s", ctypes.c_int64),
        ("o", ctypes.c_void_p), ("o_stride_b", ctypes.c_int64), ("o_stride_h", ctypes.c_int64),
        ("o_stride_s", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
        ("o_dtype", ctypes.c_int32),
        ("k_transposed", ctypes.c_int32), ("waves", ctypes.c_int32),
    ]


class ReduceDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("kind", ctypes.c_int32), ("axis", ctypes.c_int32),
        ("clear", ctypes.c_int32),
        ("src", ctypes.c_void_p), ("ld_src", ctypes.c_int64),
        ("dst", ctypes.c_void_p), ("dst_stride", ctypes.c_int64),
        ("leaf_order_bits", ctypes.c_int32), ("leaf_order", ctypes.c_uint8 * 32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


class CopyDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
        ("src_type", ctypes.c_int32), ("dst_type", ctypes.c_int32),
        ("src", ctypes.c_void_p), ("ld_src", ctypes.c_int64),
        ("dst", ctypes.c_void_p), ("ld_dst", ctypes.c_int64),
    ]


class FillDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("value", ctypes.c_double),
        ("dst", ctypes.c_void_p), ("ld", ctypes.c_int64),
    ]


_lib = None


def load() -> ctypes.CDLL:
    """Load libfrisk_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m frisk_amd.build` "
            "(there is no CPU fallback for the GEMM/attention path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.frisk_gemm.argtypes = [ctypes.POINTER(GemmDesc), ctypes.c_void_p]
    lib.frisk_gemm.restype = ctypes.c_int
    lib.frisk_gemm_workspace_size.argtypes = [ctypes.POINTER(GemmDesc)]
    lib.frisk_gemm_workspace_size.restype = ctypes.c_int64
    lib.frisk_gemm_plan.argtypes = [ctypes.POINTER(GemmDesc), ctypes.c_char_p, ctypes.c_int64]
    lib.frisk_gemm_plan.restype = ctypes.c_int
    lib.frisk_gemm_noalloc.argtypes = [ctypes.POINTER(GemmDesc), ctypes.c_void_p]
    lib.frisk_gemm_noalloc.restype = ctypes.c_int
    lib.frisk_attn_fwd.argtypes = [ctypes.POINTER(AttnDesc), ctypes.c_void_p]
    lib.frisk_attn_fwd.restype = ctypes.c_int
    lib.frisk_reduce.argtypes = [ctypes.POINTER(ReduceDesc), ctypes.c_void_p]
    lib.frisk_reduce.restype = ctypes.c_int
    lib.frisk_reduce_workspace_size.argtypes = [ctypes.POINTER(ReduceDesc)]
    lib.frisk_reduce_workspace_size.restype = ctypes.c_int64
    lib.frisk_copy.argtypes = [ctypes.POINTER(CopyDesc), ctypes.c_void_p]
    lib.frisk_copy.restype = ctypes.c_int
    lib.frisk_fill.argtypes = [ctypes.POINTER(FillDesc), ctypes.c_void_p]
    lib.frisk_fill.restype = ctypes.c_int
    lib.frisk_last_error.argtypes = []
    lib.frisk_last_error.restype = ctypes.c_char_p
    lib.frisk_abi_version.argtypes = []
    lib.frisk_abi_version.restype = ctypes.c_int
    lib.frisk_probe_mfma_layout.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                            ctypes.c_void_p]
    lib.frisk_probe_mfma_layout.restype = ctypes.c_int
    lib.frisk_probe_lds_transpose.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                              ctypes.c_void_p]
    lib.frisk_probe_lds_transpose.restype = ctypes.c_int
    if lib.frisk_abi_version() != ABI_VERSION:
        raise RuntimeError("libfrisk_hip.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def _check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = load().frisk_last_error().decode()
    if rc in (EINVAL, EUNSUP):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def torch_dtype_code(dt) -> int:
    import torch
    table = {
        torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
        torch.float8_e4m3fn: E4M3, torch.int8: I8, torch.int32: I32, torch.float64: F64,
    }
    if dt not in table:
        raise ValueError(f"unsupported tensor dtype {dt}")
    return table[dt]


def _stream_handle(stream) -> int:
    import torch
    if stream is None:
        # torch's raw accessor returns the current stream's handle without
        # building a Stream object (0.1 us against 3 us per launch); the
        # public path stays as the fallback.
        raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if raw is not None:
            return int(raw(torch.cuda.current_device()))
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream) if hasattr(stream, "cuda_stream") else int(stream)


def _row_major(t, name: str) -> int:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a rank-2 tensor with unit column stride")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    return t.stride(0)


def gemm_desc(a, b, c, *, trans_a=False, trans_b=False, clear_accum=True,
              scale_a=1.0, scale_b=1.0, variant=None) -> GemmDesc:
    """Describe C (+)= op(A).op(B) for row-major device tensors (see frisk_hip.h).
    `variant` = (tile, wave_m, wave_n) or (tile, wave_m, wave_n, slices)
    requests a kernel variant (frisk_gemm_desc.tile ... slices)."""
    lda, ldb, ldc = _row_major(a, "A"), _row_major(b, "B"), _row_major(c, "C")
    m = a.shape[1] if trans_a else a.shape[0]
    k = a.shape[0] if trans_a else a.shape[1]
    kb = b.shape[1] if trans_b else b.shape[0]
    n = b.shape[0] if trans_b else b.shape[1]
    if kb != k or tuple(c.shape) != (m, n):
        raise ValueError(f"legacy-gemm-shape: effective shapes A{tuple(a.shape)} B{tuple(b.shape)} "
                         f"C{tuple(c.shape)} do not form an MxK . KxN -> MxN product")
    return GemmDesc(m, n, k, int(bool(trans_a)), int(bool(trans_b)),
                    torch_dtype_code(a.dtype), torch_dtype_code(b.dtype), torch_dtype_code(c.dtype),
                    int(bool(clear_accum)), a.data_ptr(), lda, b.data_ptr(), ldb,
                    c.data_ptr(), ldc, float(scale_a), float(scale_b), None, 0,
                    *(tuple(variant[:3]) if variant else (0, 0, 0)), 0,
                    int(variant[3]) if variant and len(variant) > 3 else 0)


def gemm_workspace_bytes(a, b, c, *, trans_a=False, trans_b=False) -> int:
    """frisk_gemm_workspace_size for gemm(a, b, c, ...): 0 when no split-K applies."""
    d = gemm_desc(a, b, c, trans_a=trans_a, trans_b=trans_b)
    need = int(load().frisk_gemm_workspace_size(ctypes.byref(d)))
    _check(need if need < 0 else OK, "frisk_gemm_workspace_size")
    return need


def plan_of(desc: GemmDesc) -> dict:
    """frisk_gemm_plan for a descriptor: the launch frisk_gemm would make."""
    import json
    buf = ctypes.create_string_buffer(1024)
    _check(load().frisk_gemm_plan(ctypes.byref(desc), buf, len(buf)), "frisk_gemm_plan")
    return json.loads(buf.value.decode())


def gemm_plan(a, b, c, *, trans_a=False, trans_b=False, workspace=True, variant=None) -> dict:
    """The launch gemm(a, b, c, ..., workspace=workspace, variant=variant) makes
    (frisk_gemm_plan): kernel, tiles, MFMA atom, wave grid, operand storage
    order and LDS reads, split-K, and the kernel's instruction contract."""
    d = gemm_desc(a, b, c, trans_a=trans_a, trans_b=trans_b, variant=variant)
    if workspace is not False:
        need = int(load().frisk_gemm_workspace_size(ctypes.byref(d)))
        _check(need if need < 0 else OK, "frisk_gemm_workspace_size")
        d.workspace_bytes = need if workspace is True else workspace.numel() * workspace.element_size()
    return plan_of(d)


def gemm(a, b, c, *, trans_a=False, trans_b=False, clear_accum=True,
         scale_a=1.0, scale_b=1.0, workspace=True, stream=None, variant=None):
    """C = op(A).op(B) (or C += ... with clear_accum=False) on the GPU.

    `workspace`: True allocates the scratch frisk_gemm_workspace_size asks
    for (torch's caching allocator), a device tensor supplies it, False runs
    the unsplit kernels.  `variant` = (tile, wave_m, wave_n[, slices]) runs
    that kernel variant: (256, 2, 2), or (128, gm, gn) with the wave grid
    2x2, 4x1, 1x4, 2x1 or 1x2, unsplit or (2x2 grid) in `slices` K slices."""
    d = gemm_desc(a, b, c, trans_a=trans_a, trans_b=trans_b, clear_accum=clear_accum,
                  scale_a=scale_a, scale_b=scale_b, variant=variant)
    ws = None
    if workspace is not False:
        need = load().frisk_gemm_workspace_size(ctypes.byref(d))
        _check(int(need) if need < 0 else OK, "frisk_gemm_workspace_size")
        if need > 0:
            import torch
            ws = workspace if workspace is not True else \
                torch.empty(need, dtype=torch.uint8, device=c.device)
            d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
    _check(load().frisk_gemm(ctypes.byref(d), ctypes.c_void_p(_stream_handle(stream))),
           "frisk_gemm")
    return c


# FRISK_GEMM_NOALLOC_SCRATCH_BYTES of include/frisk_hip.h.
NOALLOC_SCRATCH_BYTES = 64 << 20


def gemm_noalloc(a, b, c, *, trans_a=False, trans_b=False, clear_accum=True,
                 scale_a=1.0, scale_b=1.0, stream=None):
    """frisk_gemm_noalloc: gemm() with the split-K partials in the library's
    own device scratch; nothing is allocated."""
    d = gemm_desc(a, b, c, trans_a=trans_a, trans_b=trans_b, clear_accum=clear_accum,
                  scale_a=scale_a, scale_b=scale_b)
    _check(load().frisk_gemm_noalloc(ctypes.byref(d), ctypes.c_void_p(_stream_handle(stream))),
           "frisk_gemm_noalloc")
    return c


# Atom codes of frisk_probe_mfma_layout: (mfma name, K, accumulators per lane, S).
PROBE_ATOMS = {0: ("v_mfma_f32_32x32x16_bf16", 16, 16, 64),
               1: ("v_mfma_f32_16x16x32_bf16", 32, 4, 64),
               2: ("v_mfma_i32_32x32x32_i8", 32, 16, 32)}


def probe_mfma_layout(atom: int, out, stream=None):
    """Run the MFMA layout probe into the f32 device tensor `out`."""
    if out.dtype.is_floating_point is False or out.element_size() != 4 or not out.is_contiguous() \
            or not out.is_cuda:
        raise ValueError("out must be a contiguous f32 device tensor")
    _check(load().frisk_probe_mfma_layout(int(atom), ctypes.c_void_p(out.data_ptr()), out.numel(),
                                          ctypes.c_void_p(_stream_handle(stream))),
           "frisk_probe_mfma_layout")
    return out


def probe_lds_transpose(bits: int, out, stream=None):
    """Run the transposing LDS read probe into the int16/uint16 device tensor `out`."""
    if out.element_size() != 2 or not out.is_contiguous() or not out.is_cuda:
        raise ValueError("out must be a contiguous 16-bit device tensor")
    _check(load().frisk_probe_lds_transpose(int(bits), ctypes.c_void_p(out.data_ptr()), out.numel(),
                                            ctypes.c_void_p(_stream_handle(stream))),
           "frisk_probe_lds_transpose")
    return out


def attn_desc(q, k, v, o, *, causal=False, sm_scale=None, lse=None,
              k_transposed=False, waves=0) -> AttnDesc:
    """Describe the attention forward of [batch, heads, seq, head_dim] device
    tensors; with k_transposed, K is [batch, heads, head_dim, seq_k] with unit
    key stride (read in place, not copied)."""
    shapes, strides = [], []
    for name, t in (("Q", q), ("K", k), ("V", v), ("O", o)):
        sh, st = t.shape, t.stride()
        if len(sh) != 4 or st[3] != 1 or not t.is_cuda:
            inner = "seq_k" if name == "K" and k_transposed else "head_dim"
            raise ValueError(f"{name} must be a rank-4 device tensor with unit {inner} stride")
        shapes.append(tuple(sh))
        strides.append(st)
    b, h, sq, d = shapes[0]
    sk = shapes[1][3] if k_transposed else shapes[1][2]
    k_shape = (b, h, d, sk) if k_transposed else (b, h, sk, d)
    if shapes[1] != k_shape or shapes[2] != (b, h, sk, d) or shapes[3] != (b, h, sq, d):
        raise ValueError("attention shapes disagree")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("Q/K/V must share one dtype")
    import torch
    if o.dtype not in (q.dtype, torch.float32):
        raise ValueError("O must have the Q/K/V dtype or float32")
    if lse is not None and (tuple(lse.shape) != (b, h, sq) or not lse.is_contiguous()
                            or lse.dtype.is_floating_point is False or lse.element_size() != 4):
        raise ValueError("lse must be a contiguous f32 [batch, heads, seq_q] tensor")
    if sm_scale is None:
        sm_scale = d ** -0.5
    qs, ks, vs, os_ = strides
    return AttnDesc(b, h, sq, sk, d, torch_dtype_code(q.dtype), int(bool(causal)),
                    float(sm_scale),
                    q.data_ptr(), qs[0], qs[1], qs[2],
                    k.data_ptr(), ks[0], ks[1], ks[2],
                    v.data_ptr(), vs[0], vs[1], vs[2],
                    o.data_ptr(), os_[0], os_[1], os_[2],
                    lse.data_ptr() if lse is not None else None, torch_dtype_code(o.dtype),
                    int(bool(k_transposed)), int(waves))


def attn_fwd(q, k, v, o, *, causal=False, sm_scale=None, lse=None, stream=None,
             k_transposed=False, waves=0):
    """O = softmax(sm_scale . Q K^T [causal mask]) V on the GPU.  K is
    [batch, heads, seq_k, head_dim], or [batch, heads, head_dim, seq_k] with
    k_transposed=True (read in place).  `waves` (4 or 8) requests the
    workgroup shape; 0 lets the library choose."""
    d = attn_desc(q, k, v, o, causal=causal, sm_scale=sm_scale, lse=lse, k_transposed=k_transposed,
                  waves=waves)
    _check(load().frisk_attn_fwd(ctypes.byref(d), ctypes.c_void_p(_stream_handle(stream))),
           "frisk_attn_fwd")
    return o


def _matrix(t, name: str):
    """(rows, cols, row stride) of a rank-1 or rank-2 device tensor with unit
    innermost stride; a rank-1 tensor is one row."""
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dim() == 1:
        if t.stride(0) != 1 and t.numel() > 1:
            raise ValueError(f"{name} must have unit stride")
        return 1, t.shape[0], max(t.shape[0], 1)
    if t.dim() != 2 or (t.stride(1) != 1 and t.shape[1] > 1):
        raise ValueError(f"{name} must be a rank-1 or rank-2 tensor with unit column stride")
    return t.shape[0], t.shape[1], max(t.stride(0), t.shape[1])


def reduce_workspace_bytes(src, dst, kind="sum", *, axis=1) -> int:
    """frisk_reduce_workspace_size for reduce(src, dst, kind, axis=axis)."""
    rows, cols, ld = _matrix(src, "src")
    d = ReduceDesc(rows, cols, torch_dtype_code(src.dtype), REDUCE_KINDS[kind], axis, 1,
                   src.data_ptr(), ld, dst.data_ptr(), max(dst.stride(0), 1))
    need = int(load().frisk_reduce_workspace_size(ctypes.byref(d)))
    _check(need if need < 0 else OK, "frisk_reduce_workspace_size")
    return need


def reduce(src, dst, kind="sum", *, axis=1, clear=True, leaf_order=None, workspace=True,
           stream=None):
    """frisk.reduce: dst = reduce(src) along `axis` of the [rows, cols] tensor
    src (or dst = combine(dst, reduce(src)) with clear=False).  dst is a
    rank-1 tensor of the kept extent, any stride, same dtype.  `leaf_order`
    (a permutation of the reduced index bits, tree level j along bit
    leaf_order[j]) replaces the ascending leaf order.  `workspace`: True
    allocates the scratch frisk_reduce_workspace_size asks for (torch's
    caching allocator), a uint8 device tensor supplies it, False runs the
    single-pass kernels."""
    rows, cols, ld = _matrix(src, "src")
    if src.dim() != 2:
        raise ValueError("src must be rank 2")
    if kind not in REDUCE_KINDS:
        raise ValueError(f"unknown reduction kind {kind!r} (sum/add, max, min)")
    if axis not in (0, 1):
        raise ValueError("axis must be 0 or 1")
    n = rows if axis == 1 else cols
    if dst.dim() != 1 or dst.shape[0] != n or not dst.is_cuda:
        raise ValueError(f"dst must be a rank-1 device tensor of {n} elements")
    if dst.dtype != src.dtype:
        raise ValueError("src and dst must share one dtype")
    order = list(leaf_order or [])
    if len(order) > 32:
        raise ValueError("leaf_order has more than 32 bits")
    d = ReduceDesc(rows, cols, torch_dtype_code(src.dtype), REDUCE_KINDS[kind], axis,
                   int(bool(clear)), src.data_ptr(), ld, dst.data_ptr(), max(dst.stride(0), 1),
                   len(order), (ctypes.c_uint8 * 32)(*order), None, 0)
    ws = None
    if workspace is not False:
        need = load().frisk_reduce_workspace_size(ctypes.byref(d))
        _check(int(need) if need < 0 else OK, "frisk_reduce_workspace_size")
        if need > 0:
            import torch
            ws = workspace if workspace is not True else \
                torch.empty(need, dtype=torch.uint8, device=src.device)
            d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
    _check(load().frisk_reduce(ctypes.byref(d), ctypes.c_void_p(_stream_handle(stream))),
           "frisk_reduce")
    return dst


def copy(src, dst, *, stream=None):
    """frisk.copy of a whole tile: dst = src converted to dst's dtype."""
    rows, cols, lds = _matrix(src, "src")
    drows, dcols, ldd = _matrix(dst, "dst")
    if (rows, cols) != (drows, dcols):
        raise ValueError(f"copy shapes differ: {tuple(src.shape)} -> {tuple(dst.shape)}")
    d = CopyDesc(rows, cols, torch_dtype_code(src.dtype), torch_dtype_code(dst.dtype),
                 src.data_ptr(), lds, dst.data_ptr(), ldd)
    _check(load().frisk_copy(ctypes.byref(d), ctypes.c_void_p(_stream_handle(stream))),
           "frisk_copy")
    return dst


def fill(dst, value, *, stream=None):
    """frisk.fill: every element of dst = value rounded to dst's dtype."""
    rows, cols, ld = _matrix(dst, "dst")
    d = FillDesc(rows, cols, torch_dtype_code(dst.dtype), float(value), dst.data_ptr(), ld)
    _check(load().frisk_fill(ctypes.byref(d), ctypes.c_void_p(_stream_handle(stream))),
           "frisk_fill")
    return dst
