"""GPU bit-exactness of the fp16 / fp8 outputs of stochastic_rounding and of
sgd_update on fp8 weights against the CPU oracle (shared_ffi/sr_triton.py:
18-25,43-46,109-168; the oracle's fp8 handling is pinned in
tests/test_oracle_fp8.py)."""
import numpy as np
import pytest
import torch

import oracle
from haste_amd.sr import sgd_update, stochastic_rounding

pytestmark = pytest.mark.gpu

OUT = {torch.float16: oracle.F16, torch.float8_e4m3fn: oracle.F8E4M3,
       torch.float8_e5m2: oracle.F8E5M2, torch.bfloat16: oracle.BF16}
F8 = {torch.float8_e4m3fn: oracle.F8E4M3, torch.float8_e5m2: oracle.F8E5M2}


def codes(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return (t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16)).numpy().copy()


def inputs(n: int, seed: int) -> np.ndarray:
    """Normal values over many scales, values beyond fp8's range, infinities,
    zeros, fp32 subnormals."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * rng.choice([1e-6, 1e-3, 0.02, 1.0, 40.0, 500.0, 1e5], n))
    x = x.astype(np.float32)
    k = max(1, n // 50)
    x[rng.integers(0, n, k)] = np.inf
    x[rng.integers(0, n, k)] = -np.inf
    x[rng.integers(0, n, k)] = 0.0
    x[rng.integers(0, n, k)] = np.float32(3e-40)
    return x


@pytest.mark.parametrize("odt", list(OUT))
@pytest.mark.parametrize("n,off,seed", [(1, 0, 123), (7, 1, 5), (1000, 0, 42),
                                        (65536 + 5, 3, 2**32 + 9)])
def test_stochastic_rounding_outputs(dev, odt, n, off, seed):
    """off > 0: the output starts `off` elements into its buffer (unaligned)."""
    x = inputs(n, n + off)
    xd = torch.from_numpy(x).to(dev)
    buf = torch.zeros(n + off, dtype=odt, device=dev)
    out = buf[off:]
    stochastic_rounding(xd, out, seed)
    torch.cuda.synchronize()
    want = oracle.sr_round(x, OUT[odt], seed)
    got = codes(out)
    assert np.array_equal(got.view(want.dtype), want)
    assert np.all(codes(buf[:off]) == 0)


@pytest.mark.parametrize("wdt", list(F8))
@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("use_mom,do_sr", [(False, True), (True, True), (True, False)])
@pytest.mark.parametrize("n", [5, 4099, 200_000])
def test_sgd_update_fp8_weights(dev, wdt, gdt, use_mom, do_sr, n):
    rng = np.random.default_rng(n)
    fmt = F8[wdt]
    w0 = torch.from_numpy((rng.standard_normal(n) * 0.5).astype(np.float32)).to(wdt)
    g = torch.from_numpy((rng.standard_normal(n) * 0.3).astype(np.float32)).to(gdt)
    m0 = torch.from_numpy((rng.standard_normal(n) * 0.01).astype(np.float32))
    lr, wd, mu, seed = 0.05, 1e-4, 0.9, 77
    W, G, M = w0.to(dev), g.to(dev), m0.to(dev)
    sgd_update(W, G, M if use_mom else None, lr, wd, mu, use_mom, do_sr, seed)
    torch.cuda.synchronize()
    g_np = (g.view(torch.int16).numpy().view(np.uint16) if gdt == torch.bfloat16
            else g.numpy())
    want_w, want_m = oracle.sgd_sr_step_f8w(codes(w0), fmt, g_np, m0.numpy() if use_mom else None,
                                            lr, wd, mu, use_mom, do_sr, seed)
    assert np.array_equal(codes(W), want_w)
    if use_mom:
        assert np.array_equal(M.cpu().numpy().view(np.uint32), want_m.view(np.uint32))

