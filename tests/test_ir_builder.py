"""CPU tests of the tile-IR builder (frisk_ffi.ir), the normalizer and the
CDNA4 layout target.

The first group re-runs the reference's own Python scripts
(test/python/bind_test.py, helper_test.py, map_expr_test.py) with `frisk`
replaced by `frisk_amd`, and the cases of legacy_normalization_test.py with
the gfx950 target; the rest pins contracts restated from
LegacyImportSemantics.cpp:11-46, FriskOps.cpp and FriskLayoutOps.cpp.
"""
import itertools
import math
import random

import pytest

import frisk_amd as F

from tests import programs as P


# ---------------------------------------------------------------------------
# The reference scripts
# ---------------------------------------------------------------------------
def _bind_test_module():
    """test/python/bind_test.py:3-60 verbatim apart from the module name."""
    context = F.context()
    F.frisk.load_dialects(context)
    builder = F.builder(context)
    module = builder.create_module()
    module.context = context
    shape, shape2 = [4096, 4096], [4096]
    dtype = builder.get_f16_ty()
    mem_type = builder.get_memref_ty(dtype, shape, F.AffineMap(), F.MemorySpace.GLOBAL)
    mem2_type = builder.get_memref_ty(dtype, shape2, F.AffineMap(), F.MemorySpace.GLOBAL)
    kernel_type = builder.get_kernel_ty([mem_type, mem_type, mem_type, mem2_type])
    kernel = builder.create_kernel_op(module, "test_gemm", kernel_type)
    module.push_back(kernel)
    entry1 = kernel.add_entry_block()
    builder.set_insertion_point_to_start(entry1)
    prarllel = builder.create_parallel_op([8, 8], 128)
    entry2 = prarllel.add_entry_block()
    builder.set_insertion_point_to_start(entry2)
    input_val = [entry1.get_argument(i) for i in range(4)]
    builder.create_alloc_buffer_op([128, 32], "fp16", F.MemorySpace.SHARED, 1024)
    builder.create_alloc_buffer_op([32, 128], "fp16", F.MemorySpace.SHARED, 1024)
    builder.create_alloc_buffer_op([128, 128], "fp16", F.MemorySpace.LOCAL)

    def for_body_test(b, iv):
        builder.create_fill_op(input_val[0], 0.0, "fp16")
        builder.create_reduce_op(input_val[0], input_val[3], "max", 1, True)
        builder.create_copy_op(input_val[0], input_val[1], [iv, iv], [iv, iv])

        def block_body_test(b, ivs):
            b.create_gemm_op(input_val[0], input_val[1], input_val[2])
        builder.create_block_op([128, 128], block_body_test)
    builder.create_for_op(0, 128, 1, for_body_test)
    return module


def test_bind_test_script(capsys):
    module = _bind_test_module()
    module.dump()
    out = capsys.readouterr().out
    assert out.startswith("module {\n  frisk.kernel @test_gemm(memref<4096x4096xf16, 1>")
    for needle in ("frisk.parallel (%arg4, %arg5) = (8, 8), threads = 128 {",
                   "frisk.alloc_buffer {alignment = 1024 : i64} -> memref<128x32xf16, 3>",
                   "-> memref<128x128xf16>",
                   "frisk.for %arg6 = 0 to 128 {",
                   "frisk.fill %arg0 {value = 0.000000e+00 : f16} : memref<4096x4096xf16, 1>",
                   'frisk.reduce %arg0, %arg3 {clear = true, dim = 1 : i64, kind = "max"}',
                   "frisk.copy %arg0[%arg6, %arg6], %arg1[%arg6, %arg6]",
                   "frisk.block (%arg7, %arg8) to (128, 128) {",
                   "frisk.gemm(%arg0, %arg1, %arg2) {K = 4096 : i64, M = 4096 : i64, N = 4096 : i64"):
        assert needle in out, needle
    assert module.verify()
    kernel = module.get_kernel("test_gemm")
    assert kernel.get_num_arguments() == 4 and str(kernel.type.param_types()[3]) == "memref<4096xf16, 1>"


def test_helper_test_script(capsys):
    """test/python/helper_test.py:4-24."""
    helper = F.create_session()
    f16 = helper.builder.get_f16_ty()
    a_ty = helper.memref_type((128, 64), f16, space=F.MemorySpace.SHARED)
    b_ty = helper.memref_type((64, 128), f16, space=F.MemorySpace.SHARED)
    c_ty = helper.memref_type((128, 128), f16, space=F.MemorySpace.LOCAL)
    kernel, entry = helper.new_kernel("helper_demo", [a_ty, b_ty, c_ty])
    args = [entry.get_argument(i) for i in range(3)]
    helper.create_gemm(args[0], args[1], args[2])
    scratch = helper.alloc_buffer((32, 32), "fp16", space=F.MemorySpace.SHARED, alignment=64)
    assert "memref" in str(scratch.get_type())
    assert kernel.verify()
    assert helper.module.verify()
    helper.module.dump("Helper utilities emitted the following module:")
    out = capsys.readouterr().out
    assert out.splitlines()[0] == "Helper utilities emitted the following module:"
    assert "memref<32x32xf16, 3>" in out


def test_map_expr_test_script(capsys):
    """test/python/map_expr_test.py:3-25, with the printed forms checked."""
    context = F.context()
    builder = F.builder(context)
    dim0 = builder.get_affine_dim_expr(0)
    symbol = builder.get_affine_symbol_expr(0)
    cst0 = builder.get_affine_constant_expr(0)
    cst5 = builder.get_affine_constant_expr(5)
    expr = dim0 * cst5 + symbol + cst0
    assert str(expr) == "d0 * 5 + s0"
    assert expr.get_kind() == F.AffineExprKind.Add
    expr = F.get_affine_binary_op_expr(expr.get_kind(), expr, expr)
    assert str(expr) == "d0 * 5 + s0 + d0 * 5 + s0"
    binary_expr = expr.as_binary()
    assert str(binary_expr.get_lhs()) == "d0 * 5 + s0"
    assert expr.as_dim() is None
    amap = F.AffineMap.get(1, 1, [expr], context)
    assert str(amap) == "(d0)[s0] -> (d0 * 5 + s0 + d0 * 5 + s0)"
    assert map(str, amap.get_results()).__next__() == str(amap.get_result(0))


# ---------------------------------------------------------------------------
# Affine algebra (checked against Python integer arithmetic)
# ---------------------------------------------------------------------------
def _random_expr(rng, ctx, depth):
    if depth == 0 or rng.random() < 0.25:
        r = rng.random()
        if r < 0.4:
            i = rng.randrange(3)
            return F.get_affine_dim_expr(i, ctx), (lambda d, s, i=i: d[i])
        if r < 0.6:
            return F.get_affine_symbol_expr(0, ctx), (lambda d, s: s[0])
        c = rng.randrange(-7, 8)
        return F.get_affine_constant_expr(c, ctx), (lambda d, s, c=c: c)
    a, fa = _random_expr(rng, ctx, depth - 1)
    kind = rng.randrange(5)
    if kind == 0:
        b, fb = _random_expr(rng, ctx, depth - 1)
        return a + b, (lambda d, s: fa(d, s) + fb(d, s))
    if kind == 1:
        c = rng.randrange(-4, 5)
        return a * c, (lambda d, s: fa(d, s) * c)
    c = rng.randrange(1, 6)
    if kind == 2:
        return a % c, (lambda d, s: fa(d, s) % c)
    if kind == 3:
        return a.floor_div(c), (lambda d, s: fa(d, s) // c)
    return a.ceil_div(c), (lambda d, s: -((-fa(d, s)) // c))


def test_affine_simplification_preserves_value():
    """Constructors fold/canonicalise; evaluation must still match Python's
    floor-division semantics on every random expression."""
    rng = random.Random(7)
    ctx = F.context()
    for _ in range(400):
        e, f = _random_expr(rng, ctx, 4)
        for _ in range(5):
            d = [rng.randrange(-20, 21) for _ in range(3)]
            s = [rng.randrange(-20, 21)]
            assert e.evaluate(d, s) == f(d, s), str(e)
        simp = F.simplify_affine_expr(e, 3, 1)
        d = [rng.randrange(-9, 10) for _ in range(3)]
        s = [rng.randrange(-9, 10)]
        assert simp.evaluate(d, s) == e.evaluate(d, s)


def test_affine_printing_and_folding():
    ctx = F.context()
    d0, d1 = F.get_affine_dim_expr(0, ctx), F.get_affine_dim_expr(1, ctx)
    assert str(d0 - d1) == "d0 - d1"
    assert str(d0 - 3) == "d0 - 3"
    assert str((d0 + d1) * 2) == "(d0 + d1) * 2"
    assert str(d0 * 4 * 8) == "d0 * 32"
    assert str((d0 * 8).floor_div(4)) == "d0 * 2"
    assert str((d0 * 8) % 4) == "0"
    assert str(d0.floor_div(4)) == "d0 floordiv 4" and str(d0 % 4) == "d0 mod 4"
    assert (d0 + 2 + 3) == d0 + 5  # uniqued
    m = F.AffineMap.get_permutation_map([1, 0], ctx)
    assert str(m) == "(d0, d1) -> (d1, d0)" and m.is_permutation() and not m.is_identity()
    assert F.AffineMap.get_multi_dim_identity_map(2, ctx).is_identity()
    assert str(F.AffineMap.get(ctx)) == "() -> ()"
    assert not F.AffineMap() and bool(F.AffineMap.get(ctx))
    assert F.get_affine_expr_from_flat_form([2, -1, 3, 5], 2, 1, [], ctx).evaluate([1, 2], [3]) == 14
    assert (d0 * 3 + d1).compose(F.AffineMap.get(1, 0, [d0 * 2, d0 + 1], ctx)).evaluate([4]) == 29


# ---------------------------------------------------------------------------
# Types, attributes, printing
# ---------------------------------------------------------------------------
def test_types_and_float_attrs():
    s = F.create_session()
    b = s.builder
    t = b.get_memref_ty(b.get_bf16_ty(), [4, 8], F.AffineMap(), F.MemorySpace.SHARED)
    assert isinstance(t, F.memref_buffer) and isinstance(t, F.type)
    assert str(t) == "memref<4x8xbf16, 3>" and t.get_shape() == [4, 8] and t.get_elem_width() == 16
    assert t.get_memory_space() == F.MemorySpace.SHARED
    assert str(b.get_memref_ty(b.get_f32_ty(), [2], F.AffineMap(), F.MemorySpace.LOCAL)) == "memref<2xf32>"
    assert str(b.get_e4m3fn_ty()) == "f8E4M3FN" and str(b.get_bool_ty()) == "i8"
    assert str(b.get_function_ty([b.get_f16_ty()], [b.get_f32_ty()])) == "(f16) -> f32"
    # FloatAttr values are rounded to their type (round to nearest even).
    assert str(b.get_float_attr(0.1, "fp16")) == "9.997559e-02 : f16"
    assert str(b.get_float_attr(0.1, "fp32")) == "1.000000e-01 : f32"
    assert str(b.get_float_attr(1000.0, "e4m3fn")) == "0x7F : f8E4M3FN"  # no inf: overflow is NaN
    assert str(b.get_float_attr(float("-inf"), "fp32")) == "0xFF800000 : f32"
    assert str(b.get_float_attr(448.0, "e4m3fn")) == "4.480000e+02 : f8E4M3FN"
    with pytest.raises(ValueError, match="invalid float type"):
        b.get_float_attr(1.0, "fp128")


def test_constants_and_value_names():
    s = F.create_session()
    b = s.builder
    kernel, entry = s.new_kernel("k", [])
    c1 = b.get_int64(7)
    c2 = b.get_f32(1.5)
    t = b.get_f32_tensor([1, 2, 3, 4], [2, 2])
    assert str(c1) == "%c7_i64" and str(c2) == "%cst" and str(t) == "%cst_0"
    text = str(s.module)
    assert "arith.constant dense<[[1.000000e+00, 2.000000e+00], [3.000000e+00, 4.000000e+00]]>" in text
    const = t.get_defining_op().to_constant_op()
    assert const is not None and const.get_splat_float_value() is None
    assert s.module.verify()


# ---------------------------------------------------------------------------
# GEMM contract (LegacyImportSemantics.cpp:11-46 widened for fp8 / int8)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("a,b,c,ok", [
    ("fp16", "fp16", "fp16", True), ("fp16", "fp16", "fp32", True), ("bf16", "bf16", "fp32", True),
    ("fp32", "fp32", "fp32", True), ("bf16", "fp16", "fp32", False), ("fp16", "fp16", "bf16", False),
    ("fp32", "fp32", "fp16", False), ("e4m3fn", "e4m3fn", "bf16", True),
    ("e4m3fn", "e4m3fn", "fp32", True), ("int8", "int8", "int32", True), ("int8", "int8", "fp32", False),
])
def test_gemm_type_contract(a, b, c, ok):
    s = F.create_session()
    _, e = s.new_kernel("g", [s.memref_type([16, 32], a), s.memref_type([32, 8], b),
                              s.memref_type([16, 8], c)])
    args = [e.get_argument(i) for i in range(3)]
    if ok:
        g = s.create_gemm(*args)
        assert g.verify()
        assert [g.get_matrix_A(), g.get_matrix_B(), g.get_matrix_C()] == args
    else:
        with pytest.raises(ValueError, match="^legacy-gemm-type:"):
            s.create_gemm(*args)


@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_gemm_shape_derivation(ta, tb):
    """m = A[transA?1:0], k = A[transA?0:1], n = B[transB?0:1] (ffi/ir.cpp:335-337)."""
    s = F.create_session()
    M, N, K = 16, 8, 32
    _, e = s.new_kernel("g", [s.memref_type([K, M] if ta else [M, K]),
                              s.memref_type([N, K] if tb else [K, N]),
                              s.memref_type([M, N], "fp32")])
    g = s.create_gemm(*(e.get_argument(i) for i in range(3)), trans_a=ta, trans_b=tb)
    op = g.get_operation()
    assert (op.get_attr("M"), op.get_attr("N"), op.get_attr("K")) == (M, N, K)
    assert op.get_attr("transA") == ta and op.get_attr("transB") == tb
    assert op.get_attr("policy") == F.GemmWarpPolicy.Square
    # The transposed-the-other-way operands are rejected.
    s2 = F.create_session()
    _, e2 = s2.new_kernel("g", [s2.memref_type([K, M] if not ta else [M, K]),
                                s2.memref_type([N, K] if tb else [K, N]),
                                s2.memref_type([M, N], "fp32")])
    with pytest.raises(ValueError, match="^legacy-gemm-shape:"):
        s2.create_gemm(*(e2.get_argument(i) for i in range(3)), trans_a=ta, trans_b=tb)


def test_gemm_rank_and_c_shape():
    s = F.create_session()
    _, e = s.new_kernel("g", [s.memref_type([16, 32]), s.memref_type([32, 8]),
                              s.memref_type([16, 9], "fp32"), s.memref_type([16])])
    a, b, c, v = (e.get_argument(i) for i in range(4))
    with pytest.raises(ValueError, match="legacy-gemm-shape: C shape must be MxN"):
        s.create_gemm(a, b, c)
    with pytest.raises(ValueError, match="legacy-gemm-shape: A and B must be static rank-2"):
        s.create_gemm(v, b, c)


# ---------------------------------------------------------------------------
# Builder errors and verifiers
# ---------------------------------------------------------------------------
def test_builder_errors():
    s = F.create_session()
    b = s.builder
    _, e = s.new_kernel("k", [s.memref_type([4, 4], "fp32")])
    with pytest.raises(ValueError, match="invalid float type"):
        b.create_alloc_buffer_op([4], "fp128", F.MemorySpace.LOCAL, 0)
    with pytest.raises(ValueError, match="alignment must be non-negative"):
        b.create_alloc_buffer_op([4], "fp32", F.MemorySpace.LOCAL, -1)
    b.create_alloc_buffer_op([4], "fp32", F.MemorySpace.LOCAL, 0)
    with pytest.raises(ValueError, match="invalid parallel create"):
        b.create_parallel_op([2], 128)  # the block already holds more than the terminator
    # A map/extent mix the reference aborts on is a ValueError here.
    with pytest.raises(ValueError, match="copy op map error"):
        b.create_copy_op(e.get_argument(0), e.get_argument(0), [], [], srcMap=b.get_empty_affine_map())
    with pytest.raises(IndexError):
        s.module.get_kernel("k").arg(5)


def test_python_exception_in_body_builder_propagates():
    s = F.create_session()
    s.new_kernel("k", [])

    def body(b, iv):
        raise RuntimeError("boom")
    with pytest.raises(RuntimeError, match="boom"):
        s.builder.create_for_op(0, 4, 1, body)
    assert s.module.verify()  # nothing half-built was inserted
    assert "frisk.for" not in str(s.module)


def _diag(op):
    return op.verify_diagnostic()


def test_op_verifiers():
    s = F.create_session()
    b = s.builder
    _, e = s.new_kernel("k", [s.memref_type([8, 4], "fp32"), s.memref_type([8], "fp32"),
                              s.memref_type([8], "fp16")])
    x, y, z = (e.get_argument(i) for i in range(3))
    r = b.create_reduce_op(x, z, "max", 1)
    assert "same element type" in _diag(r)
    r.get_operation().get_block()  # still attached
    r2 = b.create_reduce_op(x, y, "prod", 1)
    assert "unsupported reduce kind: prod" in _diag(r2)
    r3 = b.create_reduce_op(x, y, "add", 2)
    assert "out of range" in _diag(r3)
    r4 = b.create_reduce_op(x, y, "add", 1)
    assert _diag(r4) is None
    f = b.create_fill_op(x, 1.0, "fp16")
    assert "does not match memref element type" in _diag(f)
    a = b.create_alloc_buffer_op([4], "fp32", F.MemorySpace.LOCAL, 24)
    assert "power of 2" in _diag(a)
    assert not s.module.verify()


def test_parallel_thread_contract():
    s = F.create_session()
    s.new_kernel("k", [])
    p = s.builder.create_parallel_op([2, 2], 96)
    p.add_entry_block()
    assert "threads must be one of" in p.verify_diagnostic()


def test_dominance_is_checked():
    s = F.create_session()
    b = s.builder
    _, e = s.new_kernel("k", [s.memref_type([4], "fp32")])
    holder = {}

    def body(bb, iv):
        holder["iv"] = iv
    b.create_for_op(0, 4, 1, body)
    # Use the loop's induction variable outside the loop.
    amap = F.AffineMap.get_multi_dim_identity_map(1, s.context)
    b.create_copy_op(e.get_argument(0), e.get_argument(0), [holder["iv"]], [holder["iv"]], amap, amap)
    assert "does not dominate" in s.module.verify_diagnostic()


# ---------------------------------------------------------------------------
# Normalization (legacy_normalization_test.py with the gfx950 target)
# ---------------------------------------------------------------------------
def _gemm_session(dtype="fp16", trans_a=False, trans_b=False, accumulator="fp32",
                  semantics="tensor_v1"):
    session = F.create_session()
    a_shape = [16, 64] if trans_a else [64, 16]
    b_shape = [64, 16] if trans_b else [16, 64]
    _, entry = session.new_kernel("gemm", [
        session.memref_type(a_shape, dtype, space=F.MemorySpace.SHARED),
        session.memref_type(b_shape, dtype, space=F.MemorySpace.SHARED),
        session.memref_type([64, 64], accumulator)])
    c = session.alloc_buffer([64, 64], accumulator)
    session.create_gemm(entry.get_argument(0), entry.get_argument(1), c, trans_a=trans_a,
                        trans_b=trans_b, clear_accum=True, legacy_semantics=semantics)
    session.builder.create_copy_op(c, entry.get_argument(2), [], [])
    return session


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_normalize_all_transposes_and_dtypes(dtype, ta, tb):
    s = _gemm_session(dtype, ta, tb)
    F.frisk.normalize_layout_ir(s.module, "gfx950")
    out = str(s.module)
    assert "frisk.mma" in out and "frisk.tile_store" in out and "frisk.gemm" not in out
    assert "frisk.alloc_buffer" not in out
    assert s.module.verify()


def test_normalize_requires_explicit_semantics():
    s = _gemm_session(semantics=None)
    assert "frisk.legacy_semantics" not in str(s.module)
    with pytest.raises(ValueError, match="legacy-math-contract"):
        F.frisk.normalize_layout_ir(s.module, "gfx950")


def test_normalize_rejects_f16_accumulator():
    with pytest.raises(ValueError, match="legacy-gemm-accumulator"):
        F.frisk.normalize_layout_ir(_gemm_session(accumulator="fp16").module, "gfx950")


def test_normalize_requires_gfx950_target():
    with pytest.raises(ValueError, match="cdna4-mma-target"):
        F.frisk.normalize_layout_ir(_gemm_session().module, "sm_90a")


def test_builder_rejects_effective_shape_mismatch():
    session = F.create_session()
    _, entry = session.new_kernel("bad", [session.memref_type([64, 16]), session.memref_type([8, 64]),
                                          session.memref_type([64, 64], "fp32")])
    with pytest.raises(ValueError, match="legacy-gemm-shape"):
        session.create_gemm(*(entry.get_argument(i) for i in range(3)))


def test_reduce_clear_false_has_explicit_destination_merge():
    session = F.create_session()
    _, entry = session.new_kernel("reduce", [session.memref_type([4], "fp32")])
    src = session.alloc_buffer([4, 4], "fp32")
    dst = session.alloc_buffer([4], "fp32")
    session.builder.create_fill_op(src, 2.0, "fp32")
    session.builder.create_fill_op(dst, -0.0, "fp32")
    session.create_reduce(src, dst, "max", 1, clear=False, legacy_semantics="tensor_v1")
    session.builder.create_copy_op(dst, entry.get_argument(0), [], [])
    F.frisk.normalize_layout_ir(session.module, "gfx950")
    out = str(session.module)
    assert "frisk.reduce_tensor" in out and "arith.maximumf" in out and "frisk.tile_store" in out
    assert 'kind = "max"' in out and "dense<-0.000000e+00> : tensor<4xf32>" in out


def test_normalize_loop_carries_fragment():
    """A K loop accumulating into a Local tile becomes scf.for with the tile as
    an iter_arg (processLegacyFor / processFor)."""
    s = F.create_session()
    b = s.builder
    S = F.MemorySpace.SHARED
    _, e = s.new_kernel("k", [s.memref_type([64, 32], "bf16", space=S), s.memref_type([32, 64], "bf16", space=S),
                              s.memref_type([64, 64], "fp32")])
    acc = s.alloc_buffer([64, 64], "fp32")
    b.create_fill_op(acc, 0.0, "fp32")

    def body(bb, k):
        bb.create_gemm_op(e.get_argument(0), e.get_argument(1), acc, False, False, False, "tensor_v1")
    b.create_for_op(0, 4, 1, body)
    b.create_copy_op(acc, e.get_argument(2), [], [])
    F.frisk.normalize_layout_ir(s.module, "gfx950")
    out = str(s.module)
    assert "scf.for" in out and "iter_args(" in out and "scf.yield" in out
    assert "frisk.mma" in out and "frisk.for" not in out
    assert s.module.verify()


def test_normalize_rejects_uninitialized_accumulate():
    s = F.create_session()
    S = F.MemorySpace.SHARED
    _, e = s.new_kernel("k", [s.memref_type([64, 32], "bf16", space=S), s.memref_type([32, 64], "bf16", space=S)])
    acc = s.alloc_buffer([64, 64], "fp32")
    s.create_gemm(e.get_argument(0), e.get_argument(1), acc, legacy_semantics="tensor_v1")
    with pytest.raises(ValueError, match="legacy-fragment-uninitialized"):
        F.frisk.normalize_layout_ir(s.module, "gfx950")


def test_normalize_rejects_unsupported_thread_grouping():
    s = F.create_session()
    S = F.MemorySpace.SHARED
    _, e = s.new_kernel("k", [s.memref_type([24, 32], "bf16", space=S), s.memref_type([32, 64], "bf16", space=S)])
    acc = s.alloc_buffer([32, 64], "fp32")  # Local tiles must have power-of-two extents
    with pytest.raises(ValueError):
        s.create_gemm(e.get_argument(0), e.get_argument(1), acc, clear_accum=True, legacy_semantics="tensor_v1")


# ---------------------------------------------------------------------------
# CDNA4 MFMA geometry and fragment maps
# ---------------------------------------------------------------------------
def _geometry(m, n, k, dtype="bf16", threads=256, policy=None):
    s = F.create_session()
    b = s.builder
    ins = {"bf16": b.get_bf16_ty(), "fp16": b.get_f16_ty(), "e4m3fn": b.get_e4m3fn_ty(),
           "int8": b.get_int8_ty()}[dtype]
    acc = b.get_int32_ty() if dtype == "int8" else b.get_f32_ty()
    policy = F.GemmWarpPolicy.Square if policy is None else policy
    return F.frisk.mma_geometry(m, n, k, ins, acc, threads, policy)


def test_mfma_table():
    names = {i["name"] for i in F.frisk.mfma_instructions()}
    assert {"v_mfma_f32_32x32x16_bf16", "v_mfma_f32_16x16x32_bf16", "v_mfma_f32_32x32x64_f8f6f4",
            "v_mfma_i32_32x32x32_i8"} <= names
    for i in F.frisk.mfma_instructions():
        assert i["m"] * i["k"] % 64 == 0 and i["m"] * i["n"] % 64 == 0


def test_geometry_policies():
    g = _geometry(256, 256, 64, threads=512)  # the GEMM kernel's 256x256 tile, 8 waves
    assert (g.gM, g.gN) in ((2, 4), (4, 2)) and g.atom["name"] == "v_mfma_f32_32x32x16_bf16"
    assert g.mRepeat * 32 * g.gM == 256 and g.nRepeat * 32 * g.gN == 256 and g.kRepeat == 4
    assert _geometry(128, 128, 32, threads=256, policy=F.GemmWarpPolicy.FullRow).gM == 4
    assert _geometry(128, 128, 32, threads=256, policy=F.GemmWarpPolicy.FullCol).gN == 4
    assert _geometry(16, 64, 32, threads=64).atom["m"] == 16  # falls back to the 16x16 atom
    assert _geometry(256, 256, 64, "e4m3fn").atom["k"] == 64
    assert _geometry(24, 64, 32) is None
    assert _geometry(64, 64, 32, policy=F.GemmWarpPolicy.Auto) is None
    assert _geometry(64, 64, 32, threads=96) is None


@pytest.mark.parametrize("m,n,k,dtype,threads", [(64, 64, 16, "bf16", 128), (256, 256, 64, "bf16", 512),
                                                (64, 32, 64, "fp16", 64), (128, 128, 128, "e4m3fn", 256),
                                                (64, 64, 64, "int8", 256), (32, 64, 32, "bf16", 128)])
def test_fragment_maps_cover_tiles(m, n, k, dtype, threads):
    """Every C element is held by exactly one (reg, lane, wave); A/B elements
    by gN / gM waves (replication), each wave once."""
    g = _geometry(m, n, k, dtype, threads)
    assert g is not None
    seen = {}
    for w in range(g.waves):
        for lane in range(64):
            for r in range(g.registers("C")):
                rc = g.coordinate("C", r, lane, w)
                assert rc not in seen, (rc, seen.get(rc), (r, lane, w))
                seen[rc] = (r, lane, w)
    assert len(seen) == m * n
    for op, rows, cols, rep in (("A", m, k, g.gN), ("B", k, n, g.gM)):
        count = {}
        for w in range(g.waves):
            for lane in range(64):
                for r in range(g.registers(op)):
                    rc = g.coordinate(op, r, lane, w)
                    assert 0 <= rc[0] < rows and 0 <= rc[1] < cols
                    count[rc] = count.get(rc, 0) + 1
        assert len(count) == rows * cols and set(count.values()) == {rep}


def test_fragment_gf2_forms():
    g = _geometry(64, 64, 32, "bf16", 256)
    for op in "ABC":
        f = g.gf2(op)
        assert f is not None
        rows = 32 if op == "B" else 64
        row_bits = rows.bit_length() - 1
        for x in random.Random(3).sample(range(1 << f["in_bits"]), 200):
            y = 0
            for i, c in enumerate(f["cols"]):
                if (x >> i) & 1:
                    y ^= c
            regs = g.registers(op)
            rb = regs.bit_length() - 1
            r, lane, w = x & (regs - 1), (x >> rb) & 63, x >> (rb + 6)
            rr, cc = g.coordinate(op, r, lane, w)
            assert y == rr | (cc << row_bits)
        # C is a bijection: full rank; A and B lose one bit per replicated wave bit.
        expect = f["out_bits"]
        assert f["rank"] == expect
    # The 32x32 accumulator layout the kernels store from: element e of lane L
    # is row 8(e/4) + 4(L/32) + e%4, column L%32.
    g = _geometry(32, 32, 16, "bf16", 64)
    assert g.coordinate("C", 0, 33, 0) == (4, 1)
    assert g.coordinate("C", 5, 2, 0) == (9, 2)
    assert g.coordinate("A", 3, 40, 0) == (8, 11)


# ---------------------------------------------------------------------------
# LDS swizzles
# ---------------------------------------------------------------------------
def _read_addrs(row_bytes, swz, base_chunk=0):
    out = []
    for lane in range(64):
        r = lane & 31
        c = (base_chunk + (lane >> 5)) ^ swz(r)
        out.append(r * row_bytes + c * 16)
    return out


def test_lds_model_against_measured_conflicts():
    """Measured on MI355X with SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE for
    the GEMM fragment read of 64-B rows: no swizzle and r&3 4-way, (r>>1)&3
    2-way, (r>>2)&3 conflict-free; 128-B rows with (r&7)^((r>>3)&1)
    conflict-free.  (((r>>1)^(r>>3))&3 measured 2-way; the model says 1-way.)"""
    f = F.frisk.lds_read_b128_conflict
    assert f(_read_addrs(64, lambda r: 0)) == 4.0
    assert f(_read_addrs(64, lambda r: r & 3)) == 4.0
    assert f(_read_addrs(64, lambda r: (r >> 1) & 3)) == 2.0
    assert f(_read_addrs(64, lambda r: (r >> 2) & 3)) == 1.0
    assert f(_read_addrs(128, lambda r: (r & 7) ^ ((r >> 3) & 1))) == 1.0


@pytest.mark.parametrize("row_bytes", [64, 128, 256])
@pytest.mark.parametrize("atom", [16, 32])
def test_swizzle_proposals_are_conflict_free_bijections(row_bytes, atom):
    p = F.frisk.lds_swizzle(row_bytes, atom)
    assert p.read_conflict == 1.0, p
    chunks = row_bytes // 16
    for r in range(64):
        assert sorted(p.chunk(r, c) for c in range(chunks)) == list(range(chunks))
    if row_bytes == 64 and atom == 32:
        assert p.formula == "c ^ ((r >> 2) & 3)"  # the swizzle of the GEMM kernel


def test_sm90_swizzle_form():
    # off ^ (((off >> 7) & (sw/16 - 1)) << 4), attention_tile_mma.py:113-114
    assert F.frisk.sm90_swizzle(0x80, 128) == 0x90
    assert F.frisk.sm90_swizzle(0x3F0, 128) == 0x3F0 ^ (7 << 4)
    assert F.frisk.sm90_swizzle(0x180, 64) == 0x180 ^ (3 << 4)
    with pytest.raises(ValueError):
        F.frisk.sm90_swizzle(0, 48)


# ---------------------------------------------------------------------------
# execute(): program recognition (host side)
# ---------------------------------------------------------------------------
def test_plan_recognises_tiled_gemm():
    from frisk_amd.executor import GemmPlan, plan
    key = lambda p: (p.a, p.b, p.c, p.trans_a, p.trans_b, p.clear_accum, p.m, p.n, p.k)
    for ta, tb in itertools.product([False, True], repeat=2):
        s, _ = P.tiled_gemm(512, 256, 1024, trans_a=ta, trans_b=tb)
        p = plan(s.module, "matmul")
        assert key(p) == key(GemmPlan(0, 1, 2, ta, tb, True, 512, 256, 1024))
        # 128x128 tiles on 256 threads (the builder's Square policy): the
        # 2x2 wave grid of the 128x128 kernel executes the tile's contract,
        # in the K slices the launch contract gives that tile and grid
        # (8 tiles of 128x128 on 256 CUs: 2 slices).
        assert p.launch["tile"] == [128, 128] and p.launch["wave_grid"] == [2, 2]
        assert p.variant == (128, 2, 2, p.launch["slices"]) and p.launch["slices"] == 2
        assert p.layouts_match and p.mismatch == ""
        assert 'wave_grid = [2, 2]' in p.contract and 'policy = "Square"' in p.contract
    s, _ = P.tiled_gemm(256, 256, 256, k_scale=32)
    assert plan(s.module, "matmul").k == 256
    s, _ = P.whole_gemm(64, 32, 16, clear=False)
    p = plan(s.module, "gemm")
    assert key(p) == key(GemmPlan(0, 1, 2, False, False, False, 64, 32, 16))
    # A whole-matrix program takes the target's launch contract (here the
    # 128x128 kernel: B is stored [K, N], which the small-M kernel does not
    # read), and the solved contract of that workgroup tile selects the
    # variant execute() requests.
    assert p.launch["kernel"] == "gemm_128" and p.variant == (128, 2, 2) and p.layouts_match
    s, _ = P.whole_gemm(16, 4096, 4096, trans_b=True)
    p = plan(s.module, "gemm")
    assert p.launch["kernel"] == "gemm_skinny" and p.variant is None and p.layouts_match
    assert p.contract.startswith("#frisk.gemm_launch<{kernel = \"gemm_skinny\"")


@pytest.mark.parametrize("m,n,k,dt,out,ta,tb", [
    (4096, 4096, 4096, "bf16", "bf16", False, True), (4096, 4096, 4096, "bf16", "bf16", False, False),
    (4096, 4096, 4096, "bf16", "bf16", True, True), (4096, 4096, 4096, "bf16", "bf16", True, False),
    (4096, 4096, 4096, "fp16", "fp16", False, True), (4096, 8192, 8192, "e4m3fn", "bf16", False, True),
    (4096, 4096, 4096, "int8", "int32", False, True), (1024, 1024, 1024, "fp32", "fp32", False, False),
    (512, 512, 512, "fp32", "fp32", False, False)] + [
    (m, n, k, "bf16", "bf16", False, True) for n, k in ((4096, 4096), (14336, 4096), (4096, 14336))
    for m in (16, 128, 1024, 8192)])
def test_whole_gemm_launch_contract_equals_the_library_plan(m, n, k, dt, out, ta, tb):
    # Every bench GEMM (configs[1..3] and the fp32 rows), built as a
    # whole-matrix program: the kernel, tile, wave grid, stage depth and K
    # split of the target's launch contract equal what frisk_gemm_plan
    # reports for the same call, and the instruction contract inference
    # solves for that workgroup tile selects the same kernel variant.
    import ctypes
    from frisk_amd import runtime as rt
    from frisk_amd.executor import plan
    s, _ = P.whole_gemm(m, n, k, dtype=dt, out=out, trans_a=ta, trans_b=tb)
    p = plan(s.module, "gemm")
    codes = {"bf16": rt.BF16, "fp16": rt.F16, "fp32": rt.F32, "int8": rt.I8, "int32": rt.I32,
             "e4m3fn": rt.E4M3}
    d = rt.GemmDesc(m, n, k, int(ta), int(tb), codes[dt], codes[dt], codes[out], 1, 16,
                    m if ta else k, 16, k if tb else n, 16, n, 1.0, 1.0, None, 0, 0, 0, 0, 0, 0)
    d.workspace_bytes = rt.load().frisk_gemm_workspace_size(ctypes.byref(d))
    lib = rt.plan_of(d)
    L = p.launch
    assert (L["kernel"], L["slices"], L["workspace_bytes"]) == \
        (lib["kernel"], lib["slices"], lib["workspace_bytes"]), (L, lib)
    assert L["tile"] == [lib["tile_m"], lib["tile_n"]] and L["wave_grid"] == lib["waves"]
    assert L["slice_sum"] == lib["slice_sum"]
    if lib["kernel"] in ("gemm_w4", "gemm_128"):
        assert L["stage_bytes"] == lib["stage_bytes"]
        # The kernel's LDS swizzles, and for a K-major operand the layout
        # target's own storage proposal for its stage rows.
        assert (L["lds_swizzle_a"], L["lds_swizzle_b"]) == (lib["lds_swizzle_a"], lib["lds_swizzle_b"])
        assert p.swizzle_match is (True if (not ta or tb) else None)
        assert p.variant[:3] == (lib["tile_m"], *lib["waves"]) and p.layouts_match, p.mismatch
        # The solver's contract is the library kernel's contract.
        from frisk_amd import variants
        mine, theirs = variants.parse_contract(p.contract), variants.parse_contract(lib["mma_contract"])
        assert variants.logical_grid(mine) == variants.logical_grid(theirs)
        assert mine["atom"] == theirs["atom"]
    # Requested explicitly, the solved variant makes the same launch.
    if p.variant is not None:
        d.tile, d.wave_m, d.wave_n = p.variant[:3]
        d.slices = p.variant[3] if len(p.variant) > 3 else 0
        d.workspace_bytes = rt.load().frisk_gemm_workspace_size(ctypes.byref(d))
        req = rt.plan_of(d)
        assert req["requested"] and (req["kernel"], req["slices"], req["stage_bytes"]) == \
            (lib["kernel"], lib["slices"], lib["stage_bytes"]), (req, lib)


@pytest.mark.parametrize("policy,grid", [("FullRow", (4, 1)), ("FullCol", (1, 4)),
                                         ("Square", (2, 2))])
def test_warp_policy_selects_the_wave_grid(policy, grid):
    # The GEMM op's warp policy reaches the kernel: the solver binds the
    # policy's wave grid for the 128x128 workgroup tile, and execute()
    # requests that variant (the 4x1 / 1x4 grids run unsplit; the 2x2 grid
    # takes the launch contract's K slices).
    from frisk_amd.executor import plan
    for whole in (False, True):
        if whole:
            s, _ = P.whole_gemm(1024, 4096, 4096, dtype="bf16", out="bf16", trans_b=True)
            name = "gemm"
        else:
            s, _ = P.tiled_gemm(512, 256, 1024, BM=128, BN=128, BK=64)
            name = "matmul"
        gemms = []
        s.module.walk(lambda op: gemms.append(op) if op.get_name() == "frisk.gemm" else None)
        F.frisk.GemmOp.from_operation(gemms[0]).set_attr(
            "policy", s.builder.get_gemm_warp_policy_attr(getattr(F.GemmWarpPolicy, policy)))
        p = plan(s.module, name)
        assert p.variant is not None and p.variant[:3] == (128, *grid), (whole, p.variant, p.mismatch)
        assert p.layouts_match and f'policy = "{policy}"' in p.contract
        if grid != (2, 2):
            assert len(p.variant) == 3


def test_attention_launch_contract():
    # The target's attention launch contract: the waves per workgroup the
    # library would choose (8 for C5, 4 for the reference's D64 lengths and
    # below head_dim 128).
    fr = F.frisk
    assert fr.attention_launch_plan(128, 4096, 128, False)["waves"] == 8
    assert fr.attention_launch_plan(128, 4096, 128, True)["waves"] == 8
    assert fr.attention_launch_plan(64, 1025, 64, False)["waves"] == 4
    assert fr.attention_launch_plan(16, 2048, 128, False)["waves"] == 4
    with pytest.raises(ValueError, match="head_dim"):
        fr.attention_launch_plan(1, 64, 96, False)


@pytest.mark.parametrize("bm,threads,variant", [(256, 256, (256, 2, 2)), (128, 128, (128, 1, 2)),
                                                (64, 128, None)])
def test_plan_takes_the_kernel_variant_from_the_contract(bm, threads, variant):
    # The solver's contract for the program's workgroup tile product picks
    # the compiled kernel that executes it; a tile no kernel computes keeps
    # the library's own tiling and says why.
    from frisk_amd.executor import plan
    s, _ = P.tiled_gemm(512, 512, 256, BM=bm, BN=bm, BK=64, threads=threads)
    p = plan(s.module, "matmul")
    assert p.variant == variant and p.layouts_match == (variant is not None)
    if variant is None:
        assert "no kernel computes a 64x64 workgroup tile" in p.mismatch


def test_plan_recognises_attention():
    from frisk_amd.executor import AttnPlan, plan
    s, _ = P.attention(2, 4, 256, 128)
    assert plan(s.module, "attention") == AttnPlan(0, 1, 2, 3, False, 2, 4, 256, 128)
    s, _ = P.attention(1, 2, 128, 64, k_transposed=True, staged=False, with_sum=False)
    assert plan(s.module, "attention").k_transposed


def _mutated_gemm(mutation):
    """A tiled GEMM program with one deliberate error."""
    s = F.create_session()
    b = s.builder
    G, SH = F.MemorySpace.GLOBAL, F.MemorySpace.SHARED
    M = N = K = 256
    BM = BN = 128
    BK = 32
    _, e = s.new_kernel("matmul", [s.memref_type([M, K], "bf16", space=G), s.memref_type([K, N], "bf16", space=G),
                                   s.memref_type([M, N], "bf16", space=G)])
    A, B, C = (e.get_argument(i) for i in range(3))
    grid = [M // BM, N // BN] if mutation != "grid" else [M // BM, 1]
    par = b.create_parallel_op(grid, 256)
    b.set_insertion_point_to_start(par.add_entry_block())
    by, bx = par.get_ivs()
    a_t = s.alloc_buffer([BM, BK], "bf16", space=SH)
    b_t = s.alloc_buffer([BK, BN], "bf16", space=SH)
    c_l = s.alloc_buffer([BM, BN], "fp32")
    if mutation != "nofill":
        b.create_fill_op(c_l, 0.0, "fp32")
    d0, d1 = b.get_affine_dim_expr(0), b.get_affine_dim_expr(1)
    ctx = s.context
    kstride = BK if mutation != "kstride" else BK // 2

    def body(bb, k):
        amap = F.AffineMap.get(2, 0, [d0 * BM, d1 * kstride], ctx)
        bmap = F.AffineMap.get(2, 0, [d0 * BK, d1 * BN] if mutation != "bswap" else [d0 * BK, d0 * BN], ctx)
        empty = b.get_empty_affine_map()
        bb.create_copy_op(A, a_t, [by, k], [], amap, empty)
        bb.create_copy_op(B, b_t, [k, bx], [], bmap, empty)
        bb.create_gemm_op(a_t, b_t, c_l, False, False, mutation == "clear", None)
    b.create_for_op(0, K // BK, 1, body)
    cmap = F.AffineMap.get(2, 0, [d0 * BM, d1 * BN] if mutation != "cswap" else [d1 * BM, d0 * BN], ctx)
    b.create_copy_op(c_l, C, [], [by, bx], b.get_empty_affine_map(), cmap, [BM, BN], [BM, BN])
    return s


@pytest.mark.parametrize("mutation", ["grid", "nofill", "kstride", "bswap", "clear", "cswap"])
def test_plan_rejects_wrong_programs(mutation):
    from frisk_amd.executor import plan
    assert plan(_mutated_gemm("none").module, "matmul").m == 256
    with pytest.raises(ValueError, match="not a recognised GEMM, attention or tile-op program"):
        plan(_mutated_gemm(mutation).module, "matmul")
