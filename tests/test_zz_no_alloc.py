"""The allocation-free FFN entry point (cwen_mlp_block_noalloc) against the
context-scratch one (cwen_mlp_block), through the C ABI.

Both run the same kernels with the same launch decomposition, so the bar is
bit-identical f32 outputs.  Calls in a row share the library's static per-GPU
scratch: the second call takes a smaller block on the same weights (stale
columns of the larger first call stay in the scratch), the third a smaller
FFN shape at B <= 4 (the GEMV stages f32 activations itself), then the 27B
shape again.  Shapes beyond the scratch's limit are refused before any
launch.
"""
import numpy as np
import pytest

from cwen_amd import synth

pytestmark = pytest.mark.gpu
T_RS, T_RSI = 101, 102


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cwen_amd import gpu
    ctx = gpu.Context(0)
    yield torch, gpu, ctx
    torch.cuda.synchronize()


def _ffn(gpu, ctx, seed, H, I):
    gq, gs = synth.q4_rsi(seed, I, H)
    dq, ds = synth.q4_rs(seed, H, I, key=1)
    return gpu.Weight(ctx, T_RSI, gq, gs, H, I), gpu.Weight(ctx, T_RS, dq, ds, I, H)


def _both(torch, gpu, ctx, Wgu, Wd, B, seed):
    H = Wgu.K
    X = torch.from_numpy(synth.activations(seed, B, H, key=B)).cuda()
    Y0 = synth.activations(seed + 1, B, H, key=B)
    want = torch.from_numpy(Y0).cuda()
    gpu.mlp_block(ctx, Wgu, Wd, X, want, B)
    got = torch.from_numpy(Y0).cuda()
    gpu.mlp_block_noalloc(Wgu, Wd, X, got, B)
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


def test_noalloc_equals_mlp_block(env):
    torch, gpu, ctx = env
    Wgu, Wd = _ffn(gpu, ctx, 120, 5120, 17408)           # the 27B FFN
    Sgu, Sd = _ffn(gpu, ctx, 121, 1024, 2048)            # a smaller FFN
    for W1, W2, B, seed in ((Wgu, Wd, 16, 1), (Wgu, Wd, 5, 2), (Sgu, Sd, 3, 3), (Wgu, Wd, 8, 4)):
        print(f"noalloc vs mlp_block: H={W1.K} I={W1.M} B={B}", flush=True)
        got, want = _both(torch, gpu, ctx, W1, W2, B, seed)
        assert np.isfinite(want).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (W1.K, W1.M, B)


def test_noalloc_refuses_beyond_limit(env):
    torch, gpu, ctx = env
    H = 32768 + 512                                      # d_model past CWEN_STATIC_KMAX
    Wgu, Wd = _ffn(gpu, ctx, 122, H, 512)
    X = torch.zeros(2, H, device="cuda")
    Y = torch.zeros(2, H, device="cuda")
    with pytest.raises(gpu.CwenError) as e:
        gpu.mlp_block_noalloc(Wgu, Wd, X, Y, 2)
    assert e.value.rc == -5
    torch.cuda.synchronize()
    assert float(Y.abs().max()) == 0.0                   # nothing launched
