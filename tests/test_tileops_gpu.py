"""GPU parity of the tile ops (frisk_reduce, frisk_copy, frisk_fill) against
the CPU oracle (oracle/tileops.py): bit-exact for every dtype, kind, axis,
clear/merge mode, shape class (one slot, one chunk, many chunks, tall
columns), stride, unaligned pointer and special value (NaN, +-0, +-inf;
NaN results only need to be NaN).  Outputs sit between guard bytes, so a
write outside the tile fails the test."""
import zlib

import numpy as np
import pytest
import torch

from frisk_amd import runtime as rt
from oracle import tileops as T
from tests.gpu_util import Guarded

pytestmark = pytest.mark.gpu

TORCH = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
         "e4m3": torch.float8_e4m3fn}
RAW = {"f32": (np.uint32, np.int32, torch.int32), "f16": (np.uint16, np.int16, torch.int16),
       "bf16": (np.uint16, np.int16, torch.int16), "e4m3": (np.uint8, np.uint8, torch.uint8)}


def device_from_bits(dtype, bits):
    _, signed, _ = RAW[dtype]
    return torch.from_numpy(np.ascontiguousarray(bits).view(signed).copy()).cuda().view(TORCH[dtype])


def bits_of(dtype, t):
    unsigned, _, tint = RAW[dtype]
    return t.contiguous().view(tint).cpu().numpy().view(unsigned)


def assert_same_bits(dtype, got_bits, want_bits, what=""):
    got_v, want_v = T.from_bits(dtype, got_bits), T.from_bits(dtype, want_bits)
    nan = np.isnan(want_v)
    assert np.array_equal(np.isnan(got_v), nan), f"{what}: NaN positions differ"
    bad = np.nonzero(got_bits[~nan] != want_bits[~nan])[0]
    assert bad.size == 0, (f"{what}: {bad.size} mismatches, first at {bad[0]}: "
                           f"{got_v[~nan][bad[0]]!r} vs {want_v[~nan][bad[0]]!r}")


def seed_of(*key):
    return zlib.crc32(repr(key).encode())


def values(dtype, shape, seed, specials=False):
    """Association-sensitive values of `dtype` (as float32)."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    span = 10 if dtype == "f16" else 20
    x = rng.standard_normal(n) * np.exp2(rng.integers(-span, span + 1, n))
    if specials:
        idx = rng.choice(n, size=max(1, n // 50), replace=False)
        x[idx] = rng.choice([np.nan, np.inf, -np.inf, 0.0, -0.0], size=idx.size)
    return T.round_to(dtype, x.astype(np.float32)).reshape(shape)


SHAPES = [(1, 1), (3, 5), (64, 64), (17, 1000), (5, 70000), (3000, 7), (1025, 129)]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("kind", ["sum", "max", "min"])
@pytest.mark.parametrize("axis", [1, 0])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_reduce_matches_oracle(dtype, kind, axis, shape):
    src = values(dtype, shape, seed=seed_of(dtype, kind, axis, shape))
    n = shape[0] if axis == 1 else shape[1]
    old = values(dtype, (n,), seed=7)
    for clear in (True, False):
        dst = Guarded((n,), TORCH[dtype])
        dst.t.copy_(device_from_bits(dtype, T.to_bits(dtype, old)))
        rt.reduce(device_from_bits(dtype, T.to_bits(dtype, src)), dst.t, kind, axis=axis,
                  clear=clear)
        torch.cuda.synchronize()
        want = T.reduce(src, kind, axis, dtype, clear=clear, old=old)
        assert_same_bits(dtype, bits_of(dtype, dst.t), T.to_bits(dtype, want),
                         f"{dtype} {kind} axis{axis} {shape} clear={clear}")
        assert dst.guards_intact()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("kind", ["sum", "max", "min"])
@pytest.mark.parametrize("axis", [1, 0])
def test_reduce_special_values(dtype, kind, axis):
    shape = (96, 300)
    src = values(dtype, shape, seed=11, specials=True)
    n = shape[0] if axis == 1 else shape[1]
    dst = torch.empty(n, dtype=TORCH[dtype], device="cuda")
    rt.reduce(device_from_bits(dtype, T.to_bits(dtype, src)), dst, kind, axis=axis)
    assert_same_bits(dtype, bits_of(dtype, dst), T.to_bits(dtype, T.reduce(src, kind, axis, dtype)))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("axis", [1, 0])
def test_reduce_strided_and_unaligned(dtype, axis):
    """src is a column window of a wider tensor starting one element past a
    16-byte boundary (element loads instead of vectors); dst has stride 3."""
    rows, cols = 70, 531
    base = values(dtype, (rows, cols + 9), seed=13)
    big = device_from_bits(dtype, T.to_bits(dtype, base))
    view = big[:, 1:1 + cols]
    assert view.data_ptr() % 16 != 0 and view.stride(0) == cols + 9
    n = rows if axis == 1 else cols
    out = torch.zeros(3 * n, dtype=TORCH[dtype], device="cuda")
    rt.reduce(view, out[::3], "sum", axis=axis)
    want = T.reduce(base[:, 1:1 + cols], "sum", axis, dtype)
    got = bits_of(dtype, out)
    assert_same_bits(dtype, got[::3], T.to_bits(dtype, want))
    assert not np.any(got.reshape(n, 3)[:, 1:])


def test_reduce_large_rows_property():
    """The bench shape (32768 x 4096 f32): exact small-integer sums equal
    torch's, max equals torch.amax, and sampled rows match the oracle bit for
    bit on association-sensitive values."""
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    x = torch.randint(-8, 9, (32768, 4096), generator=g, device="cuda").float()
    out = torch.empty(32768, device="cuda")
    rt.reduce(x, out, "sum", axis=1)
    assert torch.equal(out, x.sum(dim=1))
    rt.reduce(x, out, "max", axis=1)
    assert torch.equal(out, x.amax(dim=1))
    col = torch.empty(4096, device="cuda")
    rt.reduce(x, col, "sum", axis=0)
    assert torch.equal(col, x.sum(dim=0))
    vals = values("f32", (256, 4096), seed=22)
    rt.reduce(torch.from_numpy(vals).cuda(), out[:256], "sum", axis=1)
    assert_same_bits("f32", bits_of("f32", out[:256]), T.to_bits("f32", T.reduce(vals, "sum", 1, "f32")))


def random_bits(dtype, shape, seed):
    rng = np.random.default_rng(seed)
    unsigned = RAW[dtype][0]
    width = np.dtype(unsigned).itemsize * 8
    return rng.integers(0, 1 << width, size=shape, dtype=np.uint64).astype(unsigned)


COPY_SHAPES = [(1, 1), (3, 13), (64, 64), (129, 1000), (1, 100003)]


@pytest.mark.parametrize("src", T.DTYPES)
@pytest.mark.parametrize("dst", T.DTYPES)
@pytest.mark.parametrize("shape", COPY_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_copy_converts_like_the_oracle(src, dst, shape):
    bits = random_bits(src, shape, seed=seed_of(src, dst, shape))
    out = Guarded(shape, TORCH[dst])
    rt.copy(device_from_bits(src, bits), out.t)
    torch.cuda.synchronize()
    assert_same_bits(dst, bits_of(dst, out.t).reshape(-1), T.convert(src, dst, bits).reshape(-1),
                     f"{src}->{dst} {shape}")
    assert out.guards_intact()


@pytest.mark.parametrize("src,dst", [("f32", "bf16"), ("bf16", "f32"), ("f16", "e4m3"),
                                     ("f32", "f32")])
def test_copy_strided_and_unaligned(src, dst):
    rows, cols = 77, 301
    bits = random_bits(src, (rows, cols + 5), seed=31)
    sbig = device_from_bits(src, bits)
    dbig = torch.zeros(rows, cols + 11, dtype=TORCH[dst], device="cuda")
    rt.copy(sbig[:, 1:1 + cols], dbig[:, 3:3 + cols])
    got = bits_of(dst, dbig)
    assert_same_bits(dst, got[:, 3:3 + cols].reshape(-1),
                     T.convert(src, dst, bits[:, 1:1 + cols]).reshape(-1))
    assert not np.any(got[:, :3]) and not np.any(got[:, 3 + cols:])


@pytest.mark.parametrize("tdt", [torch.int8, torch.int32, torch.float64])
def test_copy_raw_types(tdt):
    g = torch.Generator(device="cuda")
    g.manual_seed(41)
    x = torch.randint(-100, 100, (333, 517), generator=g, device="cuda").to(tdt)
    y = torch.empty_like(x)
    rt.copy(x, y)
    assert torch.equal(x, y)
    z = torch.zeros(333, 600, dtype=tdt, device="cuda")
    rt.copy(x[:, 1:], z[:, 2:518])
    assert torch.equal(z[:, 2:518], x[:, 1:]) and not z[:, :2].any() and not z[:, 518:].any()


FILL_VALUES = {
    "f32": [0.0, -0.0, 1.0, 1 / 3, -2.5e-42, 1e39, float("nan")],
    "f16": [0.0, -0.0, 1 / 3, 65519.0, 65520.0, 2.0 ** -25 + 2.0 ** -40, float("-inf")],
    "bf16": [1.0 + 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -40, -3.0e38, 1e-40],
    "e4m3": [464.0, 465.0, -0.001, 1.5 * 2.0 ** -10, 240.0],
    "i8": [-128.0, 127.0, 0.0],
    "i32": [-2147483648.0, 2147483647.0, 7.0],
    "f64": [1 / 3, -0.0],
}
FILL_TORCH = dict(TORCH, i8=torch.int8, i32=torch.int32, f64=torch.float64)
FILL_RAW = {"f32": (np.uint32, torch.int32), "f16": (np.uint16, torch.int16),
            "bf16": (np.uint16, torch.int16), "e4m3": (np.uint8, torch.uint8),
            "i8": (np.uint8, torch.uint8), "i32": (np.uint32, torch.int32),
            "f64": (np.uint64, torch.int64)}


@pytest.mark.parametrize("dtype", sorted(FILL_VALUES))
@pytest.mark.parametrize("shape", [(1, 1), (7, 9), (1000, 1000)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_fill_matches_oracle(dtype, shape):
    unsigned, tint = FILL_RAW[dtype]
    for v in FILL_VALUES[dtype]:
        out = Guarded(shape, FILL_TORCH[dtype])
        rt.fill(out.t, v)
        torch.cuda.synchronize()
        got = out.t.view(tint).cpu().numpy().view(unsigned)
        want = T.fill_bits(dtype, v)
        assert np.all(got == unsigned(want)), (dtype, v, hex(int(got.flat[0])), hex(want))
        assert out.guards_intact()


def test_fill_strided_window():
    z = torch.zeros(50, 70, dtype=torch.bfloat16, device="cuda")
    rt.fill(z[3:40, 5:66], -1.5)
    want = torch.zeros_like(z)
    want[3:40, 5:66] = -1.5
    assert torch.equal(z, want)


# ---- tile programs through execute() ---------------------------------------------
def _run(built, tensors):
    import re
    import frisk_amd as F
    s, _ = built
    name = re.search(r"frisk.kernel @(\w+)", str(s.module)).group(1)
    F.execute(s.module, name, tensors)
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind,init", [("max", None), ("add", None), ("min", float("inf")),
                                       ("add", 0.0)])
@pytest.mark.parametrize("dtype", ["fp32", "fp16"])
def test_execute_row_reduce_program(kind, init, dtype):
    from tests import programs as P
    dt = {"fp32": "f32", "fp16": "f16"}[dtype]
    R, C = 512, 96
    x = values(dt, (R, C), seed=seed_of("rowprog", kind, dtype))
    y = torch.full((R,), 7.0, dtype=TORCH[dt], device="cuda")
    _run(P.row_reduce(R, C, BR=64, kind=kind, dtype=dtype, init=init),
         [device_from_bits(dt, T.to_bits(dt, x)), y])
    want = T.reduce(x, kind, 1, dt) if init is None else \
        T.reduce(x, kind, 1, dt, clear=False, old=np.full(R, init, dtype=np.float32))
    assert_same_bits(dt, bits_of(dt, y), T.to_bits(dt, want))


def test_execute_column_strip_program():
    from tests import programs as P
    R, C = 300, 256
    x = values("f32", (R, C), seed=51)
    y = torch.empty(C, device="cuda")
    _run(P.col_reduce_tiles(R, C, BC=64), [torch.from_numpy(x).cuda(), y])
    assert_same_bits("f32", bits_of("f32", y), T.to_bits("f32", T.reduce(x, "sum", 0, "f32")))


@pytest.mark.parametrize("src,dst,staged", [("fp32", "bf16", False), ("fp32", "fp16", True),
                                            ("bf16", "fp32", False)])
def test_execute_cast_program(src, dst, staged):
    from tests import programs as P
    s_dt = {"fp32": "f32", "fp16": "f16", "bf16": "bf16"}[src]
    d_dt = {"fp32": "f32", "fp16": "f16", "bf16": "bf16"}[dst]
    R, C = 256, 384
    bits = random_bits(s_dt, (R, C), seed=seed_of("cast", src, dst))
    y = torch.empty(R, C, dtype=TORCH[d_dt], device="cuda")
    _run(P.tiled_cast(R, C, BR=64, BC=128, src=src, dst=dst, staged=staged),
         [device_from_bits(s_dt, bits), y])
    assert_same_bits(d_dt, bits_of(d_dt, y).reshape(-1), T.convert(s_dt, d_dt, bits).reshape(-1))


def test_execute_fill_program():
    from tests import programs as P
    y = torch.zeros(64, 128, device="cuda")
    _run(P.tiled_fill(64, 128, -2.75), [y])
    assert torch.equal(y, torch.full_like(y, -2.75))


def test_execute_gemm_then_cast_sequence():
    """fill C; C += A . B^T (f32); D = bf16(C): the f32 GEMM followed by the
    converting copy equals the bf16-output GEMM bit for bit (both round the
    same f32 accumulator once, to nearest even)."""
    from tests import programs as P
    from tests.gpu_util import randn
    M = N = K = 256
    a = randn((M, K), 61).to(torch.bfloat16)
    b = randn((N, K), 62).to(torch.bfloat16)
    d = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _run(P.gemm_then_cast(M, N, K), [a, b, d])
    ref = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    rt.gemm(a, b, ref, trans_b=True)
    torch.cuda.synchronize()
    assert torch.equal(d.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("kind", ["sum", "max"])
@pytest.mark.parametrize("shape", [(256, 3), (300, 256), (4097, 1031), (20000, 64)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_reduce_axis0_two_pass_matches_single_pass_and_oracle(dtype, kind, shape):
    """The workspace path (row blocks over the whole GPU, then the block
    roots) is the same tree as the single pass and the oracle."""
    src = values(dtype, shape, seed=seed_of("twopass", dtype, kind, shape))
    x = device_from_bits(dtype, T.to_bits(dtype, src))
    rows, cols = shape
    desc = rt.ReduceDesc(rows, cols, rt.torch_dtype_code(TORCH[dtype]), rt.REDUCE_KINDS[kind], 0,
                         1, 16, cols, 16, 1)
    assert rt.load().frisk_reduce_workspace_size(desc) > 0
    two = Guarded((cols,), TORCH[dtype])
    one = torch.empty(cols, dtype=TORCH[dtype], device="cuda")
    rt.reduce(x, two.t, kind, axis=0)
    rt.reduce(x, one, kind, axis=0, workspace=False)
    torch.cuda.synchronize()
    want = T.to_bits(dtype, T.reduce(src, kind, 0, dtype))
    assert_same_bits(dtype, bits_of(dtype, two.t), want, "two-pass")
    assert_same_bits(dtype, bits_of(dtype, one), want, "single pass")
    assert two.guards_intact()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("kind", ["sum", "min"])
def test_reduce_axis0_two_pass_unaligned_view(dtype, kind):
    """x[:, 1:] of a row-major tensor: element-aligned but not aligned to
    four-element vectors, at >= 256 rows so the workspace (two-pass) path
    runs; its loads fall back to elements and the result is the canonical
    tree, bit for bit."""
    rows, cols = 1000, 331
    src = values(dtype, (rows, cols + 1), seed=seed_of("twopass-unaligned", dtype, kind))
    full = device_from_bits(dtype, T.to_bits(dtype, src))
    x = full[:, 1:]
    assert x.data_ptr() % 16 != 0
    assert rt.reduce_workspace_bytes(x, torch.empty(cols, dtype=TORCH[dtype], device="cuda"),
                                     kind, axis=0) > 0
    out = Guarded((cols,), TORCH[dtype])
    rt.reduce(x, out.t, kind, axis=0)
    torch.cuda.synchronize()
    want = T.to_bits(dtype, T.reduce(src[:, 1:], kind, 0, dtype))
    assert_same_bits(dtype, bits_of(dtype, out.t), want, "two-pass unaligned")
    assert out.guards_intact()
