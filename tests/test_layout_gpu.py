"""On-device check of the CDNA4 fragment maps (frisk_amd/ir/layout.cpp)
against the gfx950 matrix cores, through frisk_probe_mfma_layout.

The probe encodes each product element (i, j) as the value i + S j; decoding
the value every (k0, lane, register) holds must give exactly the coordinate
the layout target predicts, for every k0 (which also checks that A and B
k-slots pair up for every k)."""
import numpy as np
import pytest
import torch

import frisk_amd as F
from frisk_amd import runtime as rt

pytestmark = pytest.mark.gpu


def _geometry(atom):
    s = F.create_session()
    b = s.builder
    m = 32 if atom in (0, 2) else 16
    k = {0: 16, 1: 32, 2: 32}[atom]
    ins = b.get_int8_ty() if atom == 2 else b.get_bf16_ty()
    acc = b.get_int32_ty() if atom == 2 else b.get_f32_ty()
    return F.frisk.mma_geometry(m, m, k, ins, acc, 64, F.GemmWarpPolicy.Square)


@pytest.mark.parametrize("atom", [0, 1, 2])
def test_mfma_fragment_map_matches_hardware(atom):
    name, K, R, S = rt.PROBE_ATOMS[atom]
    print(f"mfma probe atom={atom} ({name})", flush=True)
    g = _geometry(atom)
    assert g.atom["name"] == name and g.registers("C") == R
    out = torch.full((K * 64 * R,), -1.0, dtype=torch.float32, device="cuda")
    rt.probe_mfma_layout(atom, out)
    torch.cuda.synchronize()
    vals = out.cpu().numpy().reshape(K, 64, R)
    assert np.all(vals == np.round(vals)) and vals.min() >= 0
    expect = np.array([[g.coordinate("C", r, lane, 0) for r in range(R)] for lane in range(64)])
    for k0 in range(K):
        v = vals[k0].astype(np.int64)
        got = np.stack([v % S, v // S], axis=-1)
        assert np.array_equal(got, expect), f"k0={k0}"


@pytest.mark.parametrize("bits", [16, 8])
def test_transposing_lds_reads_match_the_gemm_lane_map(bits):
    # The GEMM kernels read M/N-major operand tiles with ds_read_b64_tr_b16 /
    # _tr_b8 assuming: inside each 16-lane group G, lane j receives element
    # j % per of the 8 bytes that lane 16 G + (16 / per) e + j // per
    # addressed, as its element e (per = elements in 8 bytes).
    per = 4 if bits == 16 else 8
    print(f"lds transpose probe bits={bits}", flush=True)
    out = torch.full((64 * per,), -1, dtype=torch.int16, device="cuda")
    rt.probe_lds_transpose(bits, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16).reshape(64, per).astype(np.int64)
    expect = np.empty((64, per), np.int64)
    for lane in range(64):
        grp, j = divmod(lane, 16)
        for e in range(per):
            src = 16 * grp + (16 // per) * e + j // per
            expect[lane, e] = per * src + j % per
    assert np.array_equal(got, expect)


def test_lds_probe_rejects_bad_requests():
    out = torch.zeros(16, dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError, match="buffer holds"):
        rt.probe_lds_transpose(16, out)
    with pytest.raises(ValueError, match="bits must be"):
        rt.probe_lds_transpose(4, out)


def test_probe_rejects_bad_requests():
    out = torch.zeros(16, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="buffer holds"):
        rt.probe_mfma_layout(0, out)
    with pytest.raises(ValueError, match="unknown atom"):
        rt.probe_mfma_layout(7, out)
