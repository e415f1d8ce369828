"""Session helpers over the `frisk_ffi.ir` builder.

Same interface as the reference's python/frisk/common/utils.py:1-170
(create_context, create_session, FriskHelper with memref_type, new_kernel,
alloc_buffer, create_gemm, create_reduce, ensure_insertion_block, dump).
The dtype names also cover the MI355X matrix-core inputs (bf16, e4m3fn,
e5m2, int8, int32) that the GEMM contract of this package accepts.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence, Tuple, Union

from .. import _ir

ir = _ir()

DTypeLike = Union[str, "ir.type"]
ShapeLike = Sequence[int]

__all__ = ["create_context", "create_session", "FriskHelper"]

_TYPE_GETTERS = {
    "fp16": "get_f16_ty", "bf16": "get_bf16_ty", "fp32": "get_f32_ty", "fp64": "get_f64_ty",
    "int64": "get_int64_ty", "int32": "get_int32_ty", "int8": "get_int8_ty",
    "e4m3fn": "get_e4m3fn_ty", "e5m2": "get_e5m2_ty",
}


def create_context(*, load_dialects: bool = True, disable_multithreading: bool = True) -> "ir.context":
    """A context with the frisk dialect registered."""
    ctx = ir.context()
    if disable_multithreading:
        ctx.disable_multithreading()
    if load_dialects:
        ir.frisk.load_dialects(ctx)
    return ctx


def create_session(*, load_dialects: bool = True, disable_multithreading: bool = True) -> "FriskHelper":
    """A ready FriskHelper (context + builder + empty module)."""
    return FriskHelper.create(load_dialects=load_dialects, disable_multithreading=disable_multithreading)


@dataclass
class FriskHelper:
    """Context, builder and module of one IR-building session."""

    context: "ir.context"
    builder: "ir.builder"
    module: "ir.module"

    @classmethod
    def create(cls, *, load_dialects: bool = True, disable_multithreading: bool = True) -> "FriskHelper":
        ctx = create_context(load_dialects=load_dialects, disable_multithreading=disable_multithreading)
        builder = ir.builder(ctx)
        module = builder.create_module()
        module.context = ctx  # the module keeps its context alive
        return cls(ctx, builder, module)

    # ---- types ------------------------------------------------------------------
    def memref_type(self, shape: ShapeLike, dtype: DTypeLike = "fp16", *,
                    space=None, layout=None):
        """memref<shape x dtype> in `space` (default GLOBAL) with an optional layout map."""
        space = ir.MemorySpace.GLOBAL if space is None else space
        layout = layout if layout is not None else ir.AffineMap()
        return self.builder.get_memref_ty(self._as_type(dtype), [int(d) for d in shape], layout, space)

    # ---- ops --------------------------------------------------------------------
    def new_kernel(self, name: str, arg_types: Sequence) -> Tuple["ir.frisk.KernelOp", "ir.block"]:
        """Add a kernel to the module; return it with its entry block (insertion point set there)."""
        kernel = self.builder.create_kernel_op(self.module, name, self.builder.get_kernel_ty(list(arg_types)))
        self.module.push_back(kernel)
        entry = kernel.add_entry_block()
        self.builder.set_insertion_point_to_start(entry)
        return kernel, entry

    def alloc_buffer(self, shape: ShapeLike, dtype: DTypeLike = "fp16", *, space=None,
                     alignment: int = 0) -> "ir.value":
        """Allocate a buffer (default LOCAL) and return its SSA value."""
        space = ir.MemorySpace.LOCAL if space is None else space
        op = self.builder.create_alloc_buffer_op(list(shape), self._as_dtype_str(dtype), space, alignment)
        return ir.OpState.get_result(op, 0)

    def create_gemm(self, A, B, C, *, trans_a: bool = False, trans_b: bool = False,
                    clear_accum: bool = False, legacy_semantics: str | None = None):
        return self.builder.create_gemm_op(A, B, C, trans_a, trans_b, clear_accum, legacy_semantics)

    def create_reduce(self, src, dst, kind: str, dim: int, *, clear: bool = True,
                      legacy_semantics: str | None = None):
        return self.builder.create_reduce_op(src, dst, kind, dim, clear, legacy_semantics)

    # ---- utilities --------------------------------------------------------------
    def ensure_insertion_block(self) -> "ir.block":
        """The current insertion block; the module body when none is set."""
        block = self.builder.get_insertion_block()
        if block is not None:
            return block
        body = self.module.get_region(0).front()
        self.builder.set_insertion_point_to_end(body)
        return body

    def dump(self, msg: str | None = None) -> None:
        if msg:
            print(msg)
        print(self.module)

    # ---- internals --------------------------------------------------------------
    def _as_type(self, dtype: DTypeLike):
        if isinstance(dtype, ir.type):
            return dtype
        getter = _TYPE_GETTERS.get(dtype.lower())
        if getter is None:
            raise ValueError(f"Unsupported dtype '{dtype}'.")
        return getattr(self.builder, getter)()

    def _as_dtype_str(self, dtype: DTypeLike) -> str:
        if isinstance(dtype, str):
            return dtype
        for name in ("fp16", "bf16", "fp32", "fp64", "int8", "int32", "e4m3fn", "e5m2"):
            if str(dtype) == str(self._as_type(name)):
                return name
        raise ValueError("Unsupported type for the allocation helper.")
