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
    scores = op("frisk.mma", [qv, kv, zero], t2(M, N, f32),
                {"m": i64(M), "n": i64(N), "k": i64(D), "trans_a": b.get_bool_attr(False),
                 "trans_b": b.get_bool_attr(True)})
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
                 "trans_b": b.get_bool_attr(False)})
    b.create_op("frisk.tile_store", [result, view(o, mo)], [])
    return s, kernel
