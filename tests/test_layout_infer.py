"""Layout inference (frisk-infer-layouts), its cost model and the execution
packet export, for the CDNA4 target.

Reference behaviour these tests follow: lib/Dialect/Frisk/Transforms/
LayoutInfer.cpp:187-282 (collect -> solve exactly up to 256 combinations or
by beam search -> verify -> materialize), Passes.td:33-42 (solver limits),
test/Transforms/infer-gemm-layout.mlir (ss-form MMA contract, idempotent
re-run), test/Transforms/attention-layout.mlir (the attention tile program:
MMA / reduce contracts, form "ss" then "rs"), ExportExecution.cpp:46-295
(packet: values with distributed enumerations, storage addresses, reduction
fibers).  The fragment maps the layouts are built from are the ones
tests/test_layout_gpu.py pins against the hardware (v_mfma probe)."""
import itertools
import json
import re

import pytest

import frisk_amd as F
from frisk_amd import variants as V
from tests import programs as P


def _gemm_module(m=64, n=64, k=16, dtype="bf16", threads=None):
    s = F.create_session()
    S = F.MemorySpace.SHARED
    _, entry = s.new_kernel("gemm", [s.memref_type([m, k], dtype, space=S),
                                     s.memref_type([k, n], dtype, space=S),
                                     s.memref_type([m, n], "fp32")])
    c = s.alloc_buffer([m, n], "fp32")
    g = s.create_gemm(entry.get_argument(0), entry.get_argument(1), c, clear_accum=True,
                      legacy_semantics="tensor_v1")
    if threads:
        g.set_attr("frisk.execution_threads", s.builder.get_int64_attr(threads))
    s.builder.create_copy_op(c, entry.get_argument(2), [], [])
    F.frisk.normalize_layout_ir(s.module, "gfx950")
    return s


def _attention(M, N, D, threads, dtype="bf16"):
    s, _ = P.attention_tensor_form(M=M, N=N, D=D, dtype=dtype, threads=threads)
    s.module.set_attr("frisk.target", s.builder.get_str_attr("gfx950"))
    return s


def _basis(enc, key):
    m = re.search(key + r" = \[(.*?)\]\](?=, |>)", enc) or re.search(key + r" = \[\]", enc)
    if not m or m.group(0).endswith("[]"):
        return []
    return [tuple(map(int, p)) for p in re.findall(r"\[(-?\d+), (-?\d+)", m.group(1) + "]")]


def _layout(enc):
    """(reg, lane, wave) basis lists of a #frisk.distributed encoding."""
    return _basis(enc, "reg"), _basis(enc, "lane"), _basis(enc, "wave")


def _at(layout, reg, lane, wave):
    regs, lanes, waves = layout
    r = c = 0
    for bits, basis in ((reg, regs), (lane, lanes), (wave, waves)):
        for i, (dr, dc) in enumerate(basis):
            if (bits >> i) & 1:
                r ^= dr
                c ^= dc
    return r, c


# ---- GEMM -------------------------------------------------------------------

def test_gemm_ss_contract_materialized():
    s = _gemm_module()
    r = F.frisk.infer_layouts(s.module)
    assert r["status"] == "materialized" and r["method"] == "exact"
    assert r["conversions"] == [] and r["conversions_inserted"] == 0
    assert any("hard instruction-contract" in g for g in r["graph"])
    out = str(s.module)
    assert 'form = "ss"' in out and "frisk.mma_contract = #frisk.mma_contract<{atom = " in out
    assert "frisk.execution_threads = 128 : i64" in out
    assert "frisk.layout = #frisk.distributed<tile = [64, 64], topology = [" in out
    assert s.module.verify()


def test_inference_is_idempotent():
    # The reference runs the pass twice and diffs the output
    # (infer-gemm-layout.mlir RUN lines 2-5).
    s = _gemm_module()
    F.frisk.infer_layouts(s.module)
    once = str(s.module)
    F.frisk.infer_layouts(s.module)
    assert str(s.module) == once


def test_beam_search_matches_exact_search():
    for build in (lambda: _gemm_module(128, 128, 32, threads=256),
                  lambda: _attention(128, 64, 64, 256)):
        a, b = build(), build()
        ra = F.frisk.infer_layouts(a.module, analysis_only=True)
        rb = F.frisk.infer_layouts(b.module, analysis_only=True, exact_combination_limit=0)
        assert rb["method"] == "beam" and ra["status"] == rb["status"] == "solved"
        if ra["method"] == "exact":
            assert rb["cost"] == pytest.approx(ra["cost"])
        else:
            assert rb["cost"] <= ra["cost"] + 1e-9


def test_exhaustive_beam_equals_exact_and_features_add_up():
    # A beam at least as wide as the whole domain product is exhaustive, so
    # it must return the exact search's assignment; the MFMA feature must
    # equal MFMAs per wave x cycles per MFMA of the chosen binding
    # (v_mfma_f32_32x32x16_bf16: 32768 flops at 1024 flops/clk = 32).
    a, b = _gemm_module(128, 128, 32, threads=256), _gemm_module(128, 128, 32, threads=256)
    ra = F.frisk.infer_layouts(a.module, analysis_only=True)
    assert ra["method"] == "exact" and ra["expanded"] == ra["combinations"] > 1
    rb = F.frisk.infer_layouts(b.module, analysis_only=True, exact_combination_limit=0,
                               beam_width=ra["combinations"])
    assert rb["assignments"] == ra["assignments"] and rb["cost"] == pytest.approx(ra["cost"])
    chosen = ra["assignments"][0]
    bb = F.create_session().builder
    binding = next(x for x in F.frisk.mma_bindings(128, 128, 32, bb.get_bf16_ty(), bb.get_f32_ty(), 256)
                   if x["contract"] in chosen)
    cycles = {"v_mfma_f32_32x32x16_bf16": 32, "v_mfma_f32_16x16x32_bf16": 16}[binding["atom"]]
    assert ra["features"]["mfma_cycles"] == binding["mfma_per_wave"] * cycles
    weights = F.frisk.cost_profile_defaults()["weights"]
    assert ra["cost"] == pytest.approx(sum(weights[f] * v for f, v in ra["features"].items()))


def test_search_budget_is_enforced():
    s = _attention(256, 64, 128, 512)
    with pytest.raises(ValueError, match="search-budget"):
        F.frisk.infer_layouts(s.module, exact_combination_limit=0, max_expanded_states=10)


def test_rejects_wrong_target_and_unnormalized_ir():
    s = _gemm_module()
    with pytest.raises(ValueError, match="cdna4-target"):
        F.frisk.infer_layouts(s.module, target="sm_90a")
    legacy = F.create_session()
    S = F.MemorySpace.SHARED
    _, e = legacy.new_kernel("g", [legacy.memref_type([64, 16], "bf16", space=S),
                                   legacy.memref_type([16, 64], "bf16", space=S),
                                   legacy.memref_type([64, 64], "fp32")])
    legacy.create_gemm(e.get_argument(0), e.get_argument(1), e.get_argument(2))
    with pytest.raises(ValueError, match="normalize_layout_ir"):
        F.frisk.infer_layouts(legacy.module, target="gfx950")


# ---- attention --------------------------------------------------------------

def test_attention_d128_needs_no_conversion_and_transposes_scores():
    """At head_dim 128 the solver finds the layout the hand-written kernel
    uses (frisk_amd/csrc/attn.h): S is computed transposed (S^T = K.Q^T,
    queries on lanes), every wave owns whole query rows, and P feeds the PV
    product's k side without a conversion; the row max / sum then need one
    cross-lane step (lane ^ 32)."""
    s = _attention(256, 64, 128, 512)
    r = F.frisk.infer_layouts(s.module)
    assert r["conversions"] == [] and r["conversions_inserted"] == 0
    mma0, mma1 = [a for a in r["assignments"] if a.startswith("mma#")]
    assert "32x32x16_bf16" in mma0 and "swapped = true" in mma0 and "wave_grid = [1, 8]" in mma0
    assert "swapped = false" in mma1 and "wave_grid = [8, 1]" in mma1
    out = str(s.module)
    assert out.count('form = "ss"') == 1 and out.count('form = "rs"') == 1
    assert out.count("lane_xor_masks = [32]") == 2 and "wave_xor_masks = []" in out
    assert "frisk.convert_layout" not in out
    assert s.module.verify()


def test_attention_reference_shape_inserts_one_conversion():
    """The reference's attention-layout.mlir shape (64x64 scores, head_dim
    16, 128 threads): head_dim 16 admits only 16x16 atoms for the PV
    product while the 16-deep QK product admits only 32x32 atoms, so no
    binding pair shares the query-on-lane layout and P is converted."""
    s = _attention(64, 64, 16, 128, dtype="fp16")
    r = F.frisk.infer_layouts(s.module)
    assert r["conversions_inserted"] == 1 and len(r["conversions"]) == 1
    out = str(s.module)
    assert out.count("frisk.convert_layout") == 1
    assert r["features"]["barriers"] >= 1 and r["features"]["conversion_bytes"] > 0


def test_lds_swizzle_selected_for_fragment_reads():
    s = _attention(256, 64, 128, 512)
    F.frisk.infer_layouts(s.module)
    out = str(s.module)
    # Q and K (row-major, k contiguous, 256-B rows) get the conflict-free XOR.
    assert out.count('swizzle = "c ^ ((r >> 0) & 15)"') >= 2


def test_cost_profile_weights_change_the_decision():
    base = F.frisk.infer_layouts(_attention(64, 64, 16, 128, dtype="fp16").module,
                                 analysis_only=True)
    assert base["cost_model"] == "cdna4-layout-v1"
    free_barriers = json.dumps({"id": "test", "weights": {"barriers": 0, "conversion_bytes": 0}})
    r = F.frisk.infer_layouts(_attention(64, 64, 16, 128, dtype="fp16").module,
                              analysis_only=True, cost_profile=free_barriers)
    assert r["cost_model"] == "test" and r["cost"] < base["cost"]
    with pytest.raises(ValueError, match="unknown feature"):
        F.frisk.infer_layouts(_gemm_module().module, cost_profile='{"weights": {"bogus": 1}}')
    d = F.frisk.cost_profile_defaults()
    assert set(d["weights"]) >= {"mfma_cycles", "lds_read_cycles", "barriers"}


# ---- bindings and fragment maps ---------------------------------------------

@pytest.mark.parametrize("m,n,k,threads", [(64, 64, 16, 128), (128, 64, 32, 256), (64, 128, 64, 256)])
def test_binding_layouts_match_the_probed_fragment_maps(m, n, k, threads):
    """Every non-swapped binding's C layout is the (reg, lane, wave) ->
    (row, col) map of frisk.mma_geometry(...).coordinate, which the GPU test
    pins against v_mfma; a swapped binding is its exact transpose."""
    b = F.create_session().builder
    bf16, f32 = b.get_bf16_ty(), b.get_f32_ty()
    bindings = F.frisk.mma_bindings(m, n, k, bf16, f32, threads)
    assert bindings and any(x["swapped"] for x in bindings)
    checked = []
    for x in bindings:
        lay = _layout(x["c"])
        regs = 1 << len(lay[0])
        waves = threads // 64
        if not x["swapped"]:
            for pol in (F.GemmWarpPolicy.Square, F.GemmWarpPolicy.FullRow, F.GemmWarpPolicy.FullCol):
                g = F.frisk.mma_geometry(m, n, k, bf16, f32, threads, pol)
                if g and [g.gM, g.gN] == list(x["wave_grid"]) and x["atom"] == g.atom["name"]:
                    checked.append(x["contract"])
                    for reg, lane, wave in itertools.product(range(regs), range(64), range(waves)):
                        assert _at(lay, reg, lane, wave) == tuple(g.coordinate("C", reg, lane, wave))
        else:
            mirror = next(y for y in bindings if not y["swapped"] and y["atom"] == x["atom"]
                          and y["wave_grid"] == x["wave_grid"]) if m == n else None
            if mirror:
                ml = _layout(mirror["c"])
                for reg, lane, wave in itertools.product(range(regs), range(64), range(waves)):
                    r0, c0 = _at(ml, reg, lane, wave)
                    assert _at(lay, reg, lane, wave) == (c0, r0)
        # Coverage: every element of the m x n tile has exactly one owner.
        owners = {}
        for reg, lane, wave in itertools.product(range(regs), range(64), range(waves)):
            owners.setdefault(_at(lay, reg, lane, wave), 0)
            owners[_at(lay, reg, lane, wave)] += 1
        assert len(owners) == m * n and set(owners.values()) == {1}
    assert checked  # at least one binding compared point by point with the probed map


# ---- execution packet -------------------------------------------------------

def test_export_execution_packet():
    s = _attention(256, 64, 128, 512)
    F.frisk.infer_layouts(s.module)
    pk = json.loads(F.frisk.export_execution(s.module))
    assert pk["schema_version"] == 1 and pk["target"] == "gfx950"
    names = [o["name"] for o in pk["operations"]]
    assert names.count("frisk.mma") == 2 and names.count("frisk.reduce_tensor") == 2
    vals = {v["id"]: v for v in pk["values"]}
    for v in vals.values():
        d = v.get("distributed")
        if not d:
            continue
        regs, lanes, waves = d["topology"]
        assert len(d["logical"]) == regs * lanes * waves
        n_elems = 1
        for e in d["shape"]:
            n_elems *= e
        assert len(d["first"]) == n_elems and min(d["first"]) >= 0
        for idx, c in enumerate(d["first"]):
            assert d["logical"][c] == idx
        assert len(d["logical"]) == n_elems * d["replication"]
    for op in pk["operations"]:
        if op["name"] == "frisk.reduce_tensor":
            src = vals[op["operands"][0]]["distributed"]
            assert len(op["fibers"]) == src["shape"][0]
            for o, fiber in enumerate(op["fibers"]):
                assert len(fiber) == src["shape"][1]
                cols = {src["logical"][c] % src["shape"][1] for c in fiber}
                rows = {src["logical"][c] // src["shape"][1] for c in fiber}
                assert rows == {o} and len(cols) == src["shape"][1]
    swizzled = [v for v in vals.values() if "storage" in v and "byte_offsets" in v["storage"]]
    assert swizzled
    for v in swizzled:
        offs = v["storage"]["byte_offsets"]
        eb = 2
        assert sorted(offs) == list(range(0, len(offs) * eb, eb))  # a bijection on the tile


def test_export_requires_materialized_layouts():
    s = _gemm_module()
    with pytest.raises(ValueError, match="not materialized"):
        F.frisk.export_execution(s.module)


# ---- packet consumer (plan on CPU) ------------------------------------------

def _packet(s):
    F.frisk.infer_layouts(s.module)
    return F.frisk.export_execution(s.module)


def test_plan_packet_attention_and_gemm():
    p = F.plan_packet(_packet(_attention(64, 64, 16, 128, dtype="fp16")))
    assert p["kind"] == "attention" and p["scale"] == 0.25 and p["head_dim"] == 16
    assert (p["q"], p["k"], p["v"], p["o"]) == (0, 1, 2, 3)
    assert p["layouts_match"] is False  # head_dim 16: the packet converts P, the kernel pads V
    p = F.plan_packet(_packet(_attention(256, 64, 128, 512)))
    assert p["kind"] == "attention" and p["layouts_match"] is True
    g = F.plan_packet(_packet(_gemm_module()))
    assert g["kind"] == "gemm" and (g["a"], g["b"], g["c"]) == (0, 1, 2)
    assert (g["m"], g["n"], g["k"]) == (64, 64, 16) and not g["trans_a"] and not g["trans_b"]
    # A 64x64 tile on the default 128 threads: no compiled kernel executes it.
    assert g["threads"] == 128 and g["variant"] is None and g["layouts_match"] is False
    assert "no kernel computes a 64x64 workgroup tile" in g["mismatch"]


@pytest.mark.parametrize("m,threads,variant", [(128, 256, (128, 2, 2)), (128, 128, (128, 1, 2)),
                                               (256, 256, (256, 2, 2))])
def test_plan_packet_gemm_variant_from_contract(m, threads, variant):
    g = F.plan_packet(_packet(_gemm_module(m, m, 64, threads=threads)))
    assert g["threads"] == threads and g["variant"] == variant and g["layouts_match"] is True
    assert g["mismatch"] == ""
    assert V.logical_grid(V.parse_contract(g["contract"])) == variant[1:]


def test_execute_packet_refuses_a_contract_no_kernel_executes_when_asked():
    # execute_packet follows execute()'s rule: a packet whose contract no
    # kernel executes runs the library's own kernel (reporting the
    # mismatch), unless require_layout_match, which refuses before running.
    with pytest.raises(ValueError, match="require_layout_match"):
        F.execute_packet(_packet(_gemm_module()), [None, None, None], require_layout_match=True)
    with pytest.raises(ValueError, match="head_dim >= 32"):
        F.execute_packet(_packet(_attention(64, 64, 16, 128, dtype="fp16")), [None] * 4,
                         require_layout_match=True)
    # The older spelling still refuses.
    with pytest.raises(ValueError, match="require_layout_match"):
        F.execute_packet(_packet(_gemm_module()), [None, None, None], allow_layout_mismatch=False)


def test_variant_for_reasons():
    c = ('atom = "v_mfma_f32_32x32x16_bf16", wave_grid = [2, 2], repeats = [2, 2, 4], '
         'policy = "Square", swapped = false')
    assert V.variant_for(c, 128, 128, 256) == ((128, 2, 2), "")
    assert V.variant_for(c, 256, 256, 256) == ((256, 2, 2), "")
    assert "threads do not form" in V.variant_for(c, 128, 128, 128)[1]
    assert "64x128" in V.variant_for(c, 64, 128, 256)[1]
    c16 = c.replace("32x32x16", "16x16x32")
    assert "32x32 MFMA atoms" in V.variant_for(c16, 128, 128, 256)[1]
    # A swapped contract runs the transposed product: hardware grid [1, 2]
    # is the logical 2x1 grid.
    cs = c.replace("wave_grid = [2, 2]", "wave_grid = [1, 2]").replace("false", "true")
    assert V.variant_for(cs, 128, 128, 128) == ((128, 2, 1), "")
    fp8 = c.replace("v_mfma_f32_32x32x16_bf16", "v_mfma_scale_f32_32x32x64_f8f6f4")
    assert V.variant_for(fp8, 128, 128, 256) == ((128, 2, 2), "")
    assert V.variant_for("", 128, 128, 256)[0] is None


def test_plan_packet_rejects_other_programs():
    pk = json.loads(_packet(_attention(64, 64, 16, 128, dtype="fp16")))
    ops = pk["operations"]
    ex = next(i for i, o in enumerate(ops) if o["name"] == "math.exp")
    ops[ex]["name"] = "math.exp2"
    with pytest.raises(ValueError, match="not a GEMM, attention, reduction, fill or copy"):
        F.plan_packet(pk)
    pk = json.loads(_packet(_attention(64, 64, 16, 128, dtype="fp16")))
    pk["target"] = "sm_90a"
    with pytest.raises(ValueError, match="schema_version 1 for target gfx950"):
        F.plan_packet(pk)
