"""The device's GEMV arithmetic against the oracle's device-rounding model
(tests/device_round.py): for every weight format, the device's outputs equal
W16 @ f16(X) -- weights rounded once to f16 by the format's formula,
activations rounded to f16, sums exact -- up to the order of the device's
f32 sums.

Tolerance (stated): rel_err = max|y - y_model| / max|y_model| <= 1e-5 per
launch.  A wrong rounding formula moves outputs by ~1e-4 (2^-11 on a
fraction of the weights); f32 summation order moves them by ~1e-7.
"""
import numpy as np
import pytest

from cwen_amd import synth
from util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5
CASES = [("rs", 5120, 0), ("rsi", 5120, 0), ("rsi", 5120, 1), ("q4_0", 5120, 0), ("q8_0", 5120, 0),
         ("q4_1", 5120, 0), ("q5_k", 6144, 0), ("q6_k", 5120, 0), ("rs", 17408, 0)]


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    yield torch, gpu, ctx
    torch.cuda.synchronize()


def _weight(gpu, kind, M, K):
    if kind == "rs":
        data, sc = synth.q4_rs(131, M, K); return gpu.T_Q4_0RS, data, sc
    if kind == "rsi":
        data, sc = synth.q4_rsi(131, M, K); return gpu.T_Q4_0RSI, data, sc
    if kind == "q4_0":
        return gpu.T_Q4_0, synth.q4_gguf(131, M, K), None
    if kind == "q8_0":
        return gpu.T_Q8_0, synth.q8_0(131, M, K), None
    if kind == "q4_1":
        return gpu.T_Q4_1, synth.q4_1(131, M, K), None
    if kind == "q6_k":
        return gpu.T_Q6_K, synth.q6_k(131, M, K), None
    return gpu.T_Q5_K, synth.q5_k(131, M, K), None


@pytest.mark.parametrize("kind,K,side", CASES)
def test_gemv_equals_device_rounding_model(env, kind, K, side):
    import device_round
    torch, gpu, ctx = env
    M = 256
    wtype, data, sc = _weight(gpu, kind, M, K)
    W = gpu.Weight(ctx, wtype, data, sc, K, M)
    W16 = device_round.weights(wtype, data, sc, K, M, side)
    X = synth.activations(132, 16, K)
    worst = 0.0
    for B in (1, 8, 16):    # B <= 4 converts while staging, B > 4 through act_to_f16
        Xd = torch.from_numpy(np.ascontiguousarray(X[:B])).cuda()
        Y = torch.full((B, M), float("nan"), device="cuda")
        gpu.gemvb(ctx, W, Xd, Y, B, side=side)
        torch.cuda.synchronize()
        got = Y.cpu().numpy()
        want = np.stack([device_round.gemv(W16, device_round.operand(X[b])) for b in range(B)])
        e = rel_err(got, want)
        worst = max(worst, e)
        assert e <= TOL, (kind, K, side, B, e)
    print(f"{kind} K={K} side={side}: rel_err vs the device-rounding model {worst:.2e}")
