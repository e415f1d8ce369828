"""Attention with K stored [batch, heads, head_dim, seq_k] (k_transposed):
the layout of the reference's FA tile program (K as memref<1x32x128x4096>,
tmp/ir.mlir:89-92).  The kernel reads it in place through transposing LDS
reads.  Parity against the fp64 oracle (max|err| <= 1e-2 * ||ref row||_inf,
LSE to the rounding of one probability), at every head_dim, ragged key
counts, row pitches wider than seq_k, and the C5 workload through execute()
with no copy of K."""
import math

import numpy as np
import pytest
import torch

import frisk_amd as F
from frisk_amd import runtime as rt
from oracle import attention as A
from oracle import gemm as G
from tests import programs as P
from tests.gpu_util import Guarded, gen, sample_rows

pytestmark = pytest.mark.gpu

LSE_TOL = {torch.bfloat16: 4e-3, torch.float16: 1e-3}


def transposed(k, pad=0):
    """K [b, h, s, d] stored as [b, h, d, s] with a row pitch of s + pad
    keys (rounded up to 8 elements)."""
    b, h, s, d = k.shape
    pitch = -(-(s + pad) // 8) * 8
    buf = torch.full((b, h, d, pitch), float("nan"), dtype=k.dtype, device="cuda")
    kt = buf[..., :s]
    kt.copy_(k.transpose(-1, -2))
    return kt


# Key counts that end inside a 64-key block and inside an 8-key chunk (the
# last chunk reads keys past seq_k, which are masked); seq_k is even, as
# the transposed layout requires.
CASES = [(1, 2, 128, 128), (2, 2, 200, 334), (1, 1, 65, 64), (1, 2, 1, 70), (1, 2, 300, 300),
         (2, 2, 512, 1026), (1, 1, 64, 130)]


@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_k_transposed_parity(d, dt, causal):
    for i, (b, h, sq, sk) in enumerate(CASES):
        print(f"case attn-kt d{d} {dt} causal={causal} b{b} h{h} sq{sq} sk{sk}", flush=True)
        g = gen(1000 * d + 10 * i + causal)
        q = torch.randn(b, h, sq, d, generator=g, device="cuda").to(dt)
        k = torch.randn(b, h, sk, d, generator=g, device="cuda").to(dt)
        v = torch.randn(b, h, sk, d, generator=g, device="cuda").to(dt)
        kt = transposed(k, pad=24 if i % 2 else 0)  # NaN in the padding keys
        o = torch.empty_like(q)
        lse = torch.empty(b, h, sq, device="cuda")
        scale = d ** -0.5
        rt.attn_fwd(q, kt, v, o, causal=causal, sm_scale=scale, lse=lse, k_transposed=True)
        torch.cuda.synchronize()
        ref, rlse = A.attention_fp64(q.double().cpu().numpy(), k.double().cpu().numpy(),
                                     v.double().cpu().numpy(), causal=causal, scale=scale)
        got = o.double().cpu().numpy()
        live = np.isfinite(rlse)
        assert G.row_scaled_error(got[live], ref[live]) <= 1e-2
        assert np.all(got[~live] == 0)
        l = lse.cpu().numpy()
        assert np.abs(l[live] - rlse[live]).max() <= LSE_TOL[dt]


def test_k_transposed_rejects_odd_seq_k():
    q = torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16, device="cuda")
    kt = torch.zeros(1, 1, 64, 72, dtype=torch.bfloat16, device="cuda")[..., :65]
    v = torch.zeros(1, 1, 65, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="transposed K needs an even seq_k"):
        rt.attn_fwd(q, kt, v, torch.empty_like(q), k_transposed=True)


def test_k_transposed_exact_fixtures():
    # The reference's analytic fixtures read through the transposed layout:
    # uniform weights over a power-of-two key count give V's column mean
    # exactly; a dominant last key gives V[last] bit for bit.
    d = 128
    for n in (64, 1024):
        q, k, v = (torch.from_numpy(x).to(torch.bfloat16).cuda()
                   for x in A.fixture_inputs((1, 2, n, d), "uniform-sparse-value", dtype=np.float32))
        o = torch.empty_like(q)
        rt.attn_fwd(q, transposed(k), v, o, sm_scale=d ** -0.5, k_transposed=True)
        torch.cuda.synchronize()
        expect = (v.double().sum(dim=2, keepdim=True) / n).expand_as(o).to(torch.bfloat16)
        assert torch.equal(o, expect)
    for n in (66, 514):
        q, k, v = (torch.from_numpy(x).to(torch.bfloat16).cuda()
                   for x in A.fixture_inputs((1, 2, n, d), "last-key-dominant", dtype=np.float32))
        o = torch.empty_like(q)
        rt.attn_fwd(q, transposed(k), v, o, sm_scale=d ** -0.5, k_transposed=True)
        torch.cuda.synchronize()
        assert torch.equal(o[..., :-1, :], v[..., -1:, :].expand_as(o[..., :-1, :]))


def test_k_transposed_guards_and_inputs_unchanged():
    b, h, s, d = 2, 3, 200, 128
    g = gen(5)
    q, k, v = (torch.randn(b, h, s, d, generator=g, device="cuda").to(torch.bfloat16)
               for _ in range(3))
    kt = transposed(k)
    q0, kt0, v0 = q.clone(), kt.clone(), v.clone()
    go = Guarded((b, h, s, d), torch.bfloat16)
    rt.attn_fwd(q, kt, v, go.t, causal=True, sm_scale=d ** -0.5, k_transposed=True)
    o_ref = torch.empty_like(q)
    rt.attn_fwd(q, k, v, o_ref, causal=True, sm_scale=d ** -0.5)
    torch.cuda.synchronize()
    assert go.guards_intact()
    assert torch.equal(q, q0) and torch.equal(kt, kt0) and torch.equal(v, v0)
    # Against the [.., seq, head_dim] layout: the same values up to the
    # order of the head_dim products inside an MFMA.
    diff = (go.t.double() - o_ref.double()).abs().amax(dim=-1)
    scale = o_ref.double().abs().amax(dim=-1).clamp_min(1e-30)
    assert float((diff / scale).max()) <= 1e-2


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_config_c5_k_transposed_through_execute(native_oracle, causal):
    # configs[4] with K stored [B, H, D, S] (b4 h32 s4096 d128 bf16), built
    # as the tile program with a transposed K tile and run by execute():
    # every (b, h) head on 32 sampled query rows against the fp64 C oracle,
    # and no device memory allocated beyond the output (a copy of K would be
    # 128 MiB).
    b, h, s, d = 4, 32, 4096, 128
    sess, _ = P.attention(b, h, s, d, k_transposed=True)
    g = gen(5)
    q = torch.randn(b, h, s, d, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(b, h, s, d, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(b, h, s, d, generator=g, device="cuda").to(torch.bfloat16)
    kt = k.transpose(-1, -2).contiguous()
    o = torch.empty_like(q)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    before = torch.cuda.memory_allocated()
    F.execute(sess.module, "attention", [q, kt, v, o], causal=causal, sm_scale=1 / math.sqrt(d))
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated() - before < (1 << 20)
    Q, K, V = (t.float().cpu().numpy() for t in (q, k, v))
    O = o.float().cpu().numpy()
    worst = 0.0
    for bi in range(b):
        for hi in range(h):
            rows = sample_rows(s, 32, seed=100 * bi + hi)
            ro, _ = native_oracle.attn_rows_f64(Q[bi, hi], K[bi, hi], V[bi, hi], rows,
                                                causal=causal, scale=1 / math.sqrt(d))
            err = G.row_scaled_error(O[bi, hi][rows].astype(np.float64), ro)
            assert err <= 1e-2, (bi, hi, err)
            worst = max(worst, err)
    print(f"c5 k_transposed causal={causal}: worst row-scaled error {worst:.3e}")
