"""HiFT vocoder activations at the full upsample-stage shapes, against the
oracle: Snake (alpha per channel along ne0, the reference's (C, T) layout
hift_vocoder.cpp:61-73, and time innermost with alpha along ne1) and
LeakyReLU(0.1) (hift_vocoder.cpp:686) on [1,128,48000], [1,64,120000] and
the batched [16,64,120000] stress shape (983 MB moved per launch: the
largest element counts the kernels index).

Tolerances as the other activation tests: LeakyReLU bit-exact, Snake within
|d| <= 1e-5 |exp| + 2^-22 |x| (device sin against glibc sinf)."""
import os

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

NTH = max(1, min(16, os.cpu_count() or 1))
CHUNK = 1 << 23   # elements per host comparison slice


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def alphas(C, tensor):
    a = W.uniform_range(W.seed_of(4, tensor) + C, (C,), 0.5, 1.5)
    return a, (np.float32(1.0) / (a + np.float32(1e-9))).astype(np.float32)


@pytest.mark.parametrize("C,T", [(128, 48000), (64, 120000)])
def test_stage_shapes_channel_inner(cbx, oracle, C, T):
    """[1,C,T] laid out (C, T): ne0 = C."""
    x = W.normal(W.seed_of(4, 8) + C, (T, C))
    a, ai = alphas(C, 9)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    assert_close(got, oracle.snake(x, a, ai, nth=NTH), x=x, what=f"snake (C, T) {C}x{T}")
    assert_bitexact(host(cbx.leaky_relu(dev(x), 0.1)), oracle.leaky_relu(x, 0.1, nth=NTH), f"leaky {C}x{T}")


@pytest.mark.parametrize("C,T", [(128, 48000), (64, 120000)])
def test_stage_shapes_time_inner(cbx, oracle, C, T):
    """[1,C,T] laid out time innermost: ne = (T, C), alpha of ne (1, C)."""
    x = W.normal(W.seed_of(4, 10) + C, (C, T))
    a, ai = alphas(C, 11)
    a, ai = a.reshape(C, 1), ai.reshape(C, 1)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    assert_close(got, oracle.snake(x, a, ai, nth=NTH), x=x, what=f"snake (T, C) {C}x{T}")


def compare_chunked(got, exp, x, exact, what):
    got, exp, x = got.reshape(-1), exp.reshape(-1), x.reshape(-1)
    for s in range(0, got.size, CHUNK):
        sl = slice(s, min(s + CHUNK, got.size))
        if exact:
            assert_bitexact(got[sl], exp[sl], f"{what} [{sl.start}:{sl.stop})")
        else:
            assert_close(got[sl], exp[sl], x=x[sl], what=f"{what} [{sl.start}:{sl.stop})")


def test_stress_16x64x120000(cbx, oracle):
    """The batched stress shape, every element checked.  x ~ N(0,1) from
    torch's seeded device generator with zero frames planted at the start,
    the middle and the very end (the last elements of the 122,880,000):
    Snake must give exactly 0 there, and x + sin^2(ax)/a >= x everywhere."""
    B, C, T = 16, 64, 120000
    gen = torch.Generator(device="cuda")
    gen.manual_seed(W.seed_of(4, 12))
    xd = torch.empty((B, T, C), dtype=torch.float32, device="cuda").normal_(generator=gen)
    xd[0, :3] = 0.0
    xd[7, T // 2] = 0.0
    xd[B - 1, T - 2:] = 0.0
    x = host(xd)
    a, ai = alphas(C, 13)
    print(f"stress: snake (C, T) on {x.size} elements", flush=True)
    yd = cbx.snake(xd, dev(a), dev(ai))
    got = host(yd)
    del yd
    assert not got[0, :3].any() and not got[7, T // 2].any() and not got[B - 1, T - 2:].any()
    assert np.all(got >= x)
    compare_chunked(got, oracle.snake(x, a, ai, nth=NTH), x, False, "snake stress (C, T)")
    del got
    print("stress: snake time-inner", flush=True)
    xt = xd.view(B, C, T)
    at, ait = a.reshape(C, 1), ai.reshape(C, 1)
    got = host(cbx.snake(xt, dev(at), dev(ait)))
    compare_chunked(got, oracle.snake(x.reshape(B, C, T), at, ait, nth=NTH), x, False, "snake stress (T, C)")
    del got
    print("stress: leaky_relu", flush=True)
    got = host(cbx.leaky_relu(xd, 0.1))
    compare_chunked(got, oracle.leaky_relu(x, 0.1, nth=NTH), x, True, "leaky stress")
    assert not got[B - 1, T - 2:].any()
