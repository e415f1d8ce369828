"""Tile programs built with the frisk builder API, shared by the CPU plan
tests and the GPU execute() tests.

They follow the tile programs of the reference's tmp/ir.mlir (GEMM :2-16,
attention :89-157), written with the builder calls of ffi/ir.cpp.
"""
import frisk_amd as F

_DT = {"fp16": "fp16", "bf16": "bf16", "fp32": "fp32", "e4m3fn": "e4m3fn", "int8": "int8",
       "int32": "int32"}


def tiled_gemm(M, N, K, BM=128, BN=128, BK=32, dtype="bf16", out="bf16", acc="fp32",
               trans_a=False, trans_b=False, threads=256, k_scale=1, name="matmul"):
    """C[M, N] = op(A) . op(B) as a (M/BM, N/BN) grid of tiles with a K/BK loop.

    `k_scale` writes the loop as `for k in 0 .. K/BK*k_scale step k_scale`
    with tile offset (k floordiv ... ) avoided: offsets are k * (BK / k_scale).
    """
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    a_shape = [K, M] if trans_a else [M, K]
    b_shape = [N, K] if trans_b else [K, N]
    kernel, entry = s.new_kernel(name, [s.memref_type(a_shape, dtype, space=G),
                                        s.memref_type(b_shape, dtype, space=G),
                                        s.memref_type([M, N], out, space=G)])
    A, B, C = (entry.get_argument(i) for i in range(3))
    par = b.create_parallel_op([M // BM, N // BN], threads)
    pb = par.add_entry_block()
    b.set_insertion_point_to_start(pb)
    by, bx = par.get_ivs()
    a_t = s.alloc_buffer([BK, BM] if trans_a else [BM, BK], dtype, space=F.MemorySpace.SHARED)
    b_t = s.alloc_buffer([BN, BK] if trans_b else [BK, BN], dtype, space=F.MemorySpace.SHARED)
    c_l = s.alloc_buffer([BM, BN], acc)
    b.create_fill_op(c_l, 0.0, "fp32" if acc == "fp32" else "fp32")
    d0, d1 = b.get_affine_dim_expr(0), b.get_affine_dim_expr(1)
    ctx = s.context
    step = BK // k_scale

    def body(bb, k):
        # A tile at (by*BM, k*step) (or transposed), B tile at (k*step, bx*BN).
        amap = F.AffineMap.get(2, 0, [d1 * step, d0 * BM] if trans_a else [d0 * BM, d1 * step], ctx)
        bmap = F.AffineMap.get(2, 0, [d1 * BN, d0 * step] if trans_b else [d0 * step, d1 * BN], ctx)
        empty = b.get_empty_affine_map()
        bb.create_copy_op(A, a_t, [by, k], [], amap, empty)
        bb.create_copy_op(B, b_t, [k, bx], [], bmap, empty)
        bb.create_gemm_op(a_t, b_t, c_l, trans_a, trans_b, False, None)

    b.create_for_op(0, (K // BK) * k_scale, k_scale, body)
    cmap = F.AffineMap.get(2, 0, [d0 * BM, d1 * BN], ctx)
    b.create_copy_op(c_l, C, [], [by, bx], b.get_empty_affine_map(), cmap, [BM, BN], [BM, BN])
    return s, kernel


def whole_gemm(M, N, K, dtype="bf16", out="bf16", trans_a=False, trans_b=False, clear=True,
               name="gemm"):
    s = F.create_session()
    G = F.MemorySpace.GLOBAL
    a_shape = [K, M] if trans_a else [M, K]
    b_shape = [N, K] if trans_b else [K, N]
    kernel, entry = s.new_kernel(name, [s.memref_type(a_shape, dtype, space=G),
                                        s.memref_type(b_shape, dtype, space=G),
                                        s.memref_type([M, N], out, space=G)])
    s.create_gemm(*(entry.get_argument(i) for i in range(3)), trans_a=trans_a, trans_b=trans_b,
                  clear_accum=clear)
    return s, kernel


def attention(Bt, H, S, D, BM=64, BN=64, dtype="bf16", k_transposed=False, threads=256,
              with_sum=True, staged=True, name="attention"):
    """Online-softmax attention tile program (grid (B, H, S/BM), key loop S/BN)."""
    s = F.create_session()
    b = s.builder
    G, SH, L = F.MemorySpace.GLOBAL, F.MemorySpace.SHARED, F.MemorySpace.LOCAL
    qt = s.memref_type([Bt, H, S, D], dtype, space=G)
    kt = s.memref_type([Bt, H, D, S] if k_transposed else [Bt, H, S, D], dtype, space=G)
    kernel, entry = s.new_kernel(name, [qt, kt, qt, qt])
    Q, K, V, O = (entry.get_argument(i) for i in range(4))
    par = b.create_parallel_op([Bt, H, S // BM], threads)
    pb = par.add_entry_block()
    b.set_insertion_point_to_start(pb)
    bz, by, bx = par.get_ivs()
    q = s.alloc_buffer([BM, D], dtype, space=SH)
    k = s.alloc_buffer([D, BN] if k_transposed else [BN, D], dtype, space=SH)
    v = s.alloc_buffer([BN, D], dtype, space=SH)
    o = s.alloc_buffer([BM, D], dtype, space=SH)
    acc_s = s.alloc_buffer([BM, BN], "fp32", space=L)
    acc_p = s.alloc_buffer([BM, BN], dtype, space=L)
    acc_o = s.alloc_buffer([BM, D], "fp32", space=L)
    row_max = s.alloc_buffer([BM], "fp32", space=L)
    row_sum = s.alloc_buffer([BM], "fp32", space=L)
    ctx = s.context
    d = [b.get_affine_dim_expr(i) for i in range(4)]
    empty = b.get_empty_affine_map()
    qmap = F.AffineMap.get(3, 0, [d[0], d[1], d[2] * BM, b.get_affine_constant_expr(0)], ctx)
    b.create_copy_op(Q, q, [bz, by, bx], [], qmap, empty)
    b.create_fill_op(acc_o, 0.0, "fp32")
    b.create_fill_op(row_sum, 0.0, "fp32")
    b.create_fill_op(row_max, float("-inf"), "fp32")

    def body(bb, kv):
        zero = bb.get_affine_constant_expr(0)
        kmap = F.AffineMap.get(3, 0, [d[0], d[1], zero, d[2] * BN] if k_transposed
                               else [d[0], d[1], d[2] * BN, zero], ctx)
        vmap = F.AffineMap.get(3, 0, [d[0], d[1], d[2] * BN, zero], ctx)
        bb.create_copy_op(K, k, [bz, by, kv], [], kmap, empty)
        bb.create_gemm_op(q, k, acc_s, False, not k_transposed, True, None)
        bb.create_reduce_op(acc_s, row_max, "max", 1, False)
        bb.create_block_op([BM, BN], lambda b2, ivs: None)  # exp2 of scaled scores
        if with_sum:
            bb.create_reduce_op(acc_s, row_sum, "add", 1, False)
        bb.create_copy_op(acc_s, acc_p, [], [])
        bb.create_copy_op(V, v, [bz, by, kv], [], vmap, empty)
        bb.create_gemm_op(acc_p, v, acc_o, False, False, False, None)

    b.create_for_op(0, S // BN, 1, body)
    omap = F.AffineMap.get(3, 0, [d[0], d[1], d[2] * BM, b.get_affine_constant_expr(0)], ctx)
    if staged:
        b.create_copy_op(acc_o, o, [], [])
        b.create_copy_op(o, O, [], [bz, by, bx], empty, omap, [BM, D], [1, 1, BM, D])
    else:
        b.create_copy_op(acc_o, O, [], [bz, by, bx], empty, omap, [BM, D], [1, 1, BM, D])
    return s, kernel


def attention_tensor_form(M=64, N=64, D=16, dtype="fp16", threads=128, scale=0.25,
                          name="attention"):
    """The tensor-form (normalized) attention tile program that layout
    inference consumes: the structure of the reference's
    test/Transforms/attention-layout.mlir (Q.K^T, scale, row max, exp, row
    sum, divide, truncate, P.V, store), built with the generic op builder."""
    s = F.create_session()
    b = s.builder
    G, SH = F.MemorySpace.GLOBAL, F.MemorySpace.SHARED
    in_ty = {"fp16": b.get_f16_ty(), "bf16": b.get_bf16_ty()}[dtype]
    f32 = b.get_f32_ty()
    mq = s.memref_type([M, D], dtype, space=G)
    mk = s.memref_type([N, D], dtype, space=G)
    mo = s.memref_type([M, D], "fp32", space=G)
    kernel, entry = s.new_kernel(name, [mq, mk, mk, mo])
    q, k, v, o = (entry.get_argument(i) for i in range(4))
    i64 = lambda x: b.get_int64_attr(x)
    sq = s.memref_type([M, D], dtype, space=SH)
    sk = s.memref_type([N, D], dtype, space=SH)
    par = b.create_parallel_op([1], threads)
    pb = par.add_entry_block()
    b.set_insertion_point_to_start(pb)
    qs = b.create_op("memref.alloc", [], [sq], {"alignment": i64(1024)}).get_result(0)
    ks = b.create_op("memref.alloc", [], [sk], {"alignment": i64(1024)}).get_result(0)
    vs = b.create_op("memref.alloc", [], [sk], {"alignment": i64(1024)}).get_result(0)
    view = lambda x, t: b.create_op("frisk.layout_view", [x], [t]).get_result(0)
    qg, kg, vg = view(q, mq), view(k, mk), view(v, mk)
    qv, kv, vv = view(qs, sq), view(ks, sk), view(vs, sk)
    empty = b.get_empty_affine_map()
    for src, dst, rows in ((qg, qv, M), (kg, kv, N), (vg, vv, N)):
        b.create_copy_op(src, dst, [], [], empty, empty, [rows, D], [rows, D])
    t2 = lambda r, c, e: b.get_ranked_tensor_ty(e, [r, c])
    t1 = lambda r, e: b.get_ranked_tensor_ty(e, [r])
    const = lambda ty, x: b.create_op("arith.constant", [], [ty],
                                      {"value": b.get_dense_splat_attr(ty, x)}).get_result(0)
    op = lambda n, ins, ty, attrs=None: b.create_op(n, ins, [ty], attrs or {}).get_result(0)
    zero = const(t2(M, N, f32), 0.0)
    # Waves along the queries (FullRow): every wave owns whole query rows of
    # S and of O, the layout of the attention kernel (frisk_amd/csrc/attn.h).
    # Without the attribute frisk.mma's policy is Square.
    full_row = b.get_gemm_warp_policy_attr(F.GemmWarpPolicy.FullRow)
    scores = op("frisk.mma", [qv, kv, zero], t2(M, N, f32),
                {"m": i64(M), "n": i64(N), "k": i64(D), "trans_a": b.get_bool_attr(False),
                 "trans_b": b.get_bool_attr(True), "policy": full_row})
    scaled = op("arith.mulf", [scores, const(t2(M, N, f32), scale)], t2(M, N, f32))
    mx = op("frisk.reduce_tensor", [scaled], t1(M, f32), {"kind": b.get_str_attr("max"), "dim": i64(1)})
    e0 = op("tensor.empty", [], t2(M, N, f32))
    bm = op("linalg.broadcast", [mx, e0], t2(M, N, f32), {"dimensions": b.get_i64_array_attr([1])})
    centered = op("arith.subf", [scaled, bm], t2(M, N, f32))
    ex = op("math.exp", [centered], t2(M, N, f32))
    sm = op("frisk.reduce_tensor", [ex], t1(M, f32), {"kind": b.get_str_attr("sum"), "dim": i64(1)})
    e1 = op("tensor.empty", [], t2(M, N, f32))
    bs = op("linalg.broadcast", [sm, e1], t2(M, N, f32), {"dimensions": b.get_i64_array_attr([1])})
    normalized = op("arith.divf", [ex, bs], t2(M, N, f32))
    p = op("arith.truncf", [normalized], t2(M, N, in_ty))
    ozero = const(t2(M, D, f32), 0.0)
    result = op("frisk.mma", [p, vv, ozero], t2(M, D, f32),
                {"m": i64(M), "n": i64(D), "k": i64(N), "trans_a": b.get_bool_attr(False),
                 "trans_b": b.get_bool_attr(False), "policy": full_row})
    b.create_op("frisk.tile_store", [result, view(o, mo)], [])
    return s, kernel


def row_reduce(R, C, BR=64, kind="max", dtype="fp32", init=None, threads=128, name="row_reduce"):
    """Y[r] = reduce_c X[r, c] as a grid of R/BR row tiles: each tile is
    copied into a Local buffer, reduced along dim 1 into a Local vector
    (clear, or merged into a vector filled with `init`) and stored."""
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], dtype, space=G),
                                        s.memref_type([R], dtype, space=G)])
    X, Y = entry.get_argument(0), entry.get_argument(1)
    par = b.create_parallel_op([R // BR], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    (i,) = par.get_ivs()
    t = s.alloc_buffer([BR, C], dtype)
    r = s.alloc_buffer([BR], dtype)
    ctx = s.context
    d0, zero = b.get_affine_dim_expr(0), b.get_affine_constant_expr(0)
    empty = b.get_empty_affine_map()
    b.create_copy_op(X, t, [i], [], F.AffineMap.get(1, 0, [d0 * BR, zero], ctx), empty)
    if init is None:
        b.create_reduce_op(t, r, kind, 1, True)
    else:
        b.create_fill_op(r, init, "fp32" if dtype != "fp16" else "fp16")
        b.create_reduce_op(t, r, kind, 1, False)
    b.create_copy_op(r, Y, [], [i], empty, F.AffineMap.get(1, 0, [d0 * BR], ctx), [BR], [BR])
    return s, kernel


def col_reduce_tiles(R, C, BC=64, kind="add", dtype="fp32", threads=128, name="col_reduce"):
    """Y[c] = reduce_r X[r, c] over a grid of C/BC column strips (each tile
    spans every row)."""
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], dtype, space=G),
                                        s.memref_type([C], dtype, space=G)])
    X, Y = entry.get_argument(0), entry.get_argument(1)
    par = b.create_parallel_op([C // BC], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    (j,) = par.get_ivs()
    t = s.alloc_buffer([R, BC], dtype, space=F.MemorySpace.SHARED)
    r = s.alloc_buffer([BC], dtype)
    ctx = s.context
    d0, zero = b.get_affine_dim_expr(0), b.get_affine_constant_expr(0)
    empty = b.get_empty_affine_map()
    b.create_copy_op(X, t, [j], [], F.AffineMap.get(1, 0, [zero, d0 * BC], ctx), empty)
    b.create_reduce_op(t, r, kind, 0, True)
    b.create_copy_op(r, Y, [], [j], empty, F.AffineMap.get(1, 0, [d0 * BC], ctx), [BC], [BC])
    return s, kernel


def tiled_cast(R, C, BR=64, BC=128, src="fp32", dst="bf16", staged=False, threads=256,
               name="cast"):
    """Y = X converted to Y's element type, tile by tile: the conversion is the
    store copy of a Local tile into the narrower global tensor (the epilogue
    of tmp/ir.mlir:154), or a Local-to-Local copy first when `staged`."""
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], src, space=G),
                                        s.memref_type([R, C], dst, space=G)])
    X, Y = entry.get_argument(0), entry.get_argument(1)
    par = b.create_parallel_op([R // BR, C // BC], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    i, j = par.get_ivs()
    t = s.alloc_buffer([BR, BC], src)
    ctx = s.context
    d0, d1 = b.get_affine_dim_expr(0), b.get_affine_dim_expr(1)
    empty = b.get_empty_affine_map()
    tile = F.AffineMap.get(2, 0, [d0 * BR, d1 * BC], ctx)
    b.create_copy_op(X, t, [i, j], [], tile, empty)
    out = t
    if staged:
        out = s.alloc_buffer([BR, BC], dst)
        b.create_copy_op(t, out, [], [])
    b.create_copy_op(out, Y, [], [i, j], empty, tile, [BR, BC], [BR, BC])
    return s, kernel


def tiled_fill(R, C, value, BR=32, BC=64, dtype="fp32", threads=128, name="fill"):
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], dtype, space=G)])
    Y = entry.get_argument(0)
    par = b.create_parallel_op([R // BR, C // BC], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    i, j = par.get_ivs()
    t = s.alloc_buffer([BR, BC], dtype)
    b.create_fill_op(t, value, dtype)
    ctx = s.context
    d0, d1 = b.get_affine_dim_expr(0), b.get_affine_dim_expr(1)
    b.create_copy_op(t, Y, [], [i, j], b.get_empty_affine_map(),
                     F.AffineMap.get(2, 0, [d0 * BR, d1 * BC], ctx), [BR, BC], [BR, BC])
    return s, kernel


def gemm_then_cast(M, N, K, dtype="bf16", name="gemm_cast"):
    """Whole-tensor sequence: C (Global f32 buffer) = 0; C += A . B^T; D = C
    converted to `dtype`."""
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel(name, [s.memref_type([M, K], dtype, space=G),
                                        s.memref_type([N, K], dtype, space=G),
                                        s.memref_type([M, N], dtype, space=G)])
    A, B, D = (entry.get_argument(i) for i in range(3))
    c = s.alloc_buffer([M, N], "fp32", space=G)
    b.create_fill_op(c, 0.0, "fp32")
    b.create_gemm_op(A, B, c, False, True, False, None)
    b.create_copy_op(c, D, [], [])
    return s, kernel


def single_tile_reduce(R=64, C=64, kind="add", dtype="fp32", init=None, dim=1, threads=128,
                       name="tile_reduce"):
    """One tile in the reference's normalizable form (whole-tile copies, a
    tensor_v1 frisk.reduce): Y = reduce(X) along `dim`, merged into a vector
    filled with `init` when given (LegacyNormalizationNumericTest.cpp:74-118
    builds the same shape of program)."""
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    out = C if dim == 0 else R
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], dtype, space=G),
                                        s.memref_type([out], dtype, space=G)])
    X, Y = entry.get_argument(0), entry.get_argument(1)
    par = b.create_parallel_op([1], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    t = s.alloc_buffer([R, C], dtype)
    r = s.alloc_buffer([out], dtype)
    b.create_copy_op(X, t, [], [])
    if init is None:
        b.create_reduce_op(t, r, kind, dim, True, "tensor_v1")
    else:
        b.create_fill_op(r, init, dtype)
        b.create_reduce_op(t, r, kind, dim, False, "tensor_v1")
    b.create_copy_op(r, Y, [], [])
    return s, kernel


def single_tile_fill(R=64, C=64, value=1.5, dtype="fp32", threads=128, name="tile_fill"):
    s = F.create_session()
    b = s.builder
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], dtype, space=F.MemorySpace.GLOBAL)])
    par = b.create_parallel_op([1], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    t = s.alloc_buffer([R, C], dtype)
    b.create_fill_op(t, value, dtype)
    b.create_copy_op(t, entry.get_argument(0), [], [])
    return s, kernel


def single_tile_copy(R=64, C=64, dtype="fp32", threads=128, name="tile_copy"):
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel(name, [s.memref_type([R, C], dtype, space=G),
                                        s.memref_type([R, C], dtype, space=G)])
    par = b.create_parallel_op([1], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    t = s.alloc_buffer([R, C], dtype)
    b.create_copy_op(entry.get_argument(0), t, [], [])
    b.create_copy_op(t, entry.get_argument(1), [], [])
    return s, kernel


def exported_packet(built):
    """Normalize (tensor_v1, gfx950), infer layouts and export the packet."""
    import json
    s, _ = built
    s.module.set_attr("frisk.legacy_semantics", s.builder.get_str_attr("tensor_v1"))
    F.frisk.normalize_layout_ir(s.module, "gfx950")
    report = F.frisk.infer_layouts(s.module)
    assert report["status"] == "materialized", report
    return json.loads(F.frisk.export_execution(s.module))
