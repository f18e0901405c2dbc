"""One HiFT vocoder decode's node list (hift_vocoder.cpp:613-749, the
graph between the host STFT and iSTFT) planned on the host: every node
claimed, the launches the reference's structure implies, and the stage
frame counts the reference's sizes give."""
import collections

import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.hift_decode import HiFTDecode


@pytest.mark.parametrize("T_mel", [1, 4, 7])
def test_plan_counts(T_mel):
    e = HiFTDecode(T_mel, device=False)
    plan = e.plan()
    names = {v: k for k, v in vars(C).items() if k.startswith("GL_") and isinstance(v, int)}
    got = collections.Counter(names[p[0]] for p in plan)
    assert dict(got) == {
        # conv_pre; per stage the source down conv, 6 source-resblock convs and
        # 3 x 6 resblock convs; conv_post -- 72 of them behind a snake
        "GL_CONV1D": 1 + 3 * (1 + 6 + 18) + 1,
        "GL_CONV_TRANSPOSE1D": 3,            # leaky_relu -> ups[i] + bias
        "GL_BINARY": 3,                      # per stage add(x, source)
        "GL_VIEW": 1, "GL_CPY": 1, "GL_CONCAT": 1,   # stage 2's reflection pad
    }
    assert sum(p[2] for p in plan) == len(e.graph.nodes)
    flags = [p[3] for p in plan if p[0] == C.GL_CONV1D]
    assert sum(1 for fl in flags if fl & 3 == C.GLF_SNAKE) == 72
    assert sum(1 for fl in flags if fl & C.GLF_RESIDUAL) == 36      # every layer's second conv
    assert all(fl & C.GLF_BIAS for fl in flags)
    # the resblock sums ride on the last conv of resblocks 1 and 2 of each
    # stage, the mean (scale 1/3) on resblock 2's
    assert sum(1 for fl in flags if fl & C.GLF_SUM) == 6
    assert sum(1 for fl in flags if fl & C.GLF_SCALE) == 3
    assert all(fl & C.GLF_RESIDUAL for fl in flags if fl & C.GLF_SUM)
    assert all(p[3] == C.GLF_LEAKY | C.GLF_BIAS for p in plan if p[0] == C.GL_CONV_TRANSPOSE1D)
    # every conv launch ends in a tensor whose chain was recorded
    nd = e.graph.nodes
    extra = lambda fl: (1 if fl & C.GLF_SUM else 0) + (1 if fl & C.GLF_SCALE else 0)  # noqa: E731
    ends = {nd[f + n - 1 - extra(fl)].dst for k, f, n, fl in plan if k in (C.GL_CONV1D, C.GL_CONV_TRANSPOSE1D)}
    assert ends == set(e.conv_ref)


def test_stage_frames():
    """8, 40, 120 T_mel (+1 after the pad) frames, the source STFT's down
    convs landing on the same counts, and 18 channels out."""
    e = HiFTDecode(5, device=False)
    assert e.stage_frames == [40, 200, 601]
    assert e.b.shape(e.out) == (1, 601, 18)
    assert e.b.shape(e.stft) == (601, 18)

def test_flops_closed_form():
    """flops() against the convs' multiply-adds counted by stage: conv_pre,
    per stage the upsampler (per input frame), the source down conv, the
    source resblock's 6 convs, the resblocks' 6 convs of each kernel size;
    conv_post."""
    T = 3
    e = HiFTDecode(T, device=False)
    frames = [8 * T, 40 * T, 120 * T + 1]
    t_in = [T, 8 * T, 40 * T]
    total = 2 * 512 * T * 80 * 7
    for i, (c, u, k, s, ks) in enumerate(zip((256, 128, 64), (8, 5, 3), (16, 11, 7), (15, 3, 1), (7, 7, 11))):
        f = frames[i]
        total += 2 * (2 * c) * c * k * t_in[i]
        total += 2 * c * f * 18 * (2 * s if s > 1 else 1)
        total += 6 * 2 * c * f * c * ks
        total += 6 * 2 * c * f * c * (3 + 7 + 11)
    total += 2 * 18 * frames[2] * 64 * 7
    assert e.flops() == total
