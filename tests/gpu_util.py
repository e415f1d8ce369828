"""Helpers shared by the GPU parity tests (sentinel-guarded buffers, seeded
inputs, sampled oracle rows)."""
import numpy as np
import torch

GUARD = 0xA5  # the reference's sentinel byte (run_execution.py:75-87)
PAD = 272


class Guarded:
    """A device tensor placed inside a byte buffer filled with 0xA5, so
    writes outside it are detectable."""

    def __init__(self, shape, dtype):
        elem = torch.empty((), dtype=dtype).element_size()
        n = int(np.prod(shape)) * elem
        self.nbytes = n
        self.buf = torch.full((n + 2 * PAD,), GUARD, dtype=torch.uint8, device="cuda")
        self.t = self.buf[PAD: PAD + n].view(dtype).view(*shape)

    def guards_intact(self) -> bool:
        raw = self.buf.cpu().numpy()
        return bool(np.all(raw[:PAD] == GUARD) and np.all(raw[PAD + self.nbytes:] == GUARD))


def gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def randn(shape, seed, std=1.0):
    return torch.randn(shape, generator=gen(seed), device="cuda") * std


def fp8_per_tensor(x: torch.Tensor):
    """N(0,1) values scaled to amax = 448 and cast to e4m3fn; returns the fp8
    tensor and the fp32 dequantisation scale."""
    s = 448.0 / float(x.abs().max())
    return (x * s).to(torch.float8_e4m3fn), 1.0 / s


def decode(t: torch.Tensor) -> np.ndarray:
    """Exact float64 values of a device tensor (fp8 via the oracle table)."""
    from oracle import gemm as G
    if t.dtype == torch.float8_e4m3fn:
        return G.e4m3fn_decode(t.view(torch.uint8).cpu().numpy())
    if t.dtype in (torch.int8, torch.int32):
        return t.cpu().numpy().astype(np.int64)
    return t.double().cpu().numpy()


def sample_rows(m, count, seed):
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(m, size=min(count, m), replace=False))
    rows[0], rows[-1] = 0, m - 1  # always include the edges
    return np.unique(rows)
