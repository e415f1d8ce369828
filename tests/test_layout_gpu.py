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


def test_probe_rejects_bad_requests():
    out = torch.zeros(16, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="buffer holds"):
        rt.probe_mfma_layout(0, out)
    with pytest.raises(ValueError, match="unknown atom"):
        rt.probe_mfma_layout(7, out)
