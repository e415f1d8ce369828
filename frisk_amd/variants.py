"""The GEMM kernel variants of the C-ABI and the instruction contracts they
execute.

Layout inference gives every MMA of a tile program an instruction contract
(`#frisk.mma_contract<{atom, wave_grid, repeats, policy, swapped}>`,
frisk_amd/ir/infer.cpp; the reference's counterpart is the SM90 target's
MMA binding, lib/Dialect/Frisk/Target/SM90/SM90LayoutTarget.cpp:171-481).
The C-ABI runs a GEMM on one of a fixed set of compiled kernels, which a
caller can name through `frisk_gemm_desc.tile / wave_m / wave_n`
(include/frisk_hip.h).  `variant_for` maps a contract, together with the
workgroup tile and thread count it was solved for, to the variant that
executes exactly that workgroup product, or says why none does:

  * tile 256x256, 256 threads, wave grid 2x2: `gemm_w4` (256, 2, 2);
  * tile 128x128, wave grid 2x2, 4x1 or 1x4 (256 threads) or 2x1, 1x2
    (128 threads): `gemm_128` (128, gm, gn);

each with the 32x32 MFMA atom of the input type.  The wave grid compared is
the logical one (over M x N of the tile product): a swapped contract runs
the MFMAs on the transposed product, so its hardware grid is turned around.
The operand orientation itself does not have to agree: the GEMM kernels
store C to memory, so the register placement of the C fragment does not
reach the caller."""
from __future__ import annotations

import re
from typing import Optional, Tuple

_CONTRACT = re.compile(
    r'atom = "(?P<atom>[^"]+)", wave_grid = \[(?P<gm>\d+), (?P<gn>\d+)\], '
    r'repeats = \[(?P<rm>\d+), (?P<rn>\d+), (?P<rk>\d+)\], policy = "(?P<policy>\w+)", '
    r'swapped = (?P<swapped>true|false)')

# The 32x32 MFMA atom of each input type (the solver's name; the fp8 kernel
# issues its block-scaled form with unit scales).
ATOMS_32 = {"v_mfma_f32_32x32x16_bf16", "v_mfma_f32_32x32x16_f16", "v_mfma_f32_32x32x64_f8f6f4",
            "v_mfma_i32_32x32x32_i8", "v_mfma_f32_32x32x2_f32"}

GRIDS_128 = ((2, 2), (4, 1), (1, 4), (2, 1), (1, 2))

Variant = Tuple[int, int, int]


def parse_contract(text: str) -> dict:
    """Fields of a `#frisk.mma_contract` (or of `frisk_gemm_plan`'s
    "mma_contract"): atom, wave_grid, repeats, policy, swapped."""
    m = _CONTRACT.search(text or "")
    if not m:
        raise ValueError(f"not an MMA contract: {text!r}")
    return {"atom": m["atom"].replace("v_mfma_scale_", "v_mfma_"),
            "wave_grid": (int(m["gm"]), int(m["gn"])),
            "repeats": (int(m["rm"]), int(m["rn"]), int(m["rk"])),
            "policy": m["policy"], "swapped": m["swapped"] == "true"}


def logical_grid(contract: dict) -> Tuple[int, int]:
    """The contract's wave grid over M x N of the logical product."""
    gm, gn = contract["wave_grid"]
    return (gn, gm) if contract["swapped"] else (gm, gn)


def variant_for(contract_text: str, m: int, n: int, threads: int) -> Tuple[Optional[Variant], str]:
    """(variant, "") when a compiled kernel executes the contract of an m x n
    workgroup product on `threads` lanes, else (None, reason)."""
    try:
        c = parse_contract(contract_text)
    except ValueError as e:
        return None, str(e)
    lm, ln = logical_grid(c)
    if c["atom"] not in ATOMS_32:
        return None, f"atom {c['atom']}: the GEMM kernels issue the 32x32 MFMA atoms"
    if threads != 64 * lm * ln:
        return None, f"{threads} threads do not form the {lm}x{ln} wave grid"
    if (m, n) == (256, 256) and (lm, ln) == (2, 2):
        return (256, 2, 2), ""
    if (m, n) == (128, 128) and (lm, ln) in GRIDS_128:
        return (128, lm, ln), ""
    return None, (f"no kernel computes a {m}x{n} workgroup tile with a {lm}x{ln} wave grid "
                  f"(256x256 with 2x2; 128x128 with 2x2, 4x1, 1x4, 2x1 or 1x2)")
