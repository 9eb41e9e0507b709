"""Oracle weight quantiser (tools/q38_artifact_compiler.py:193-253,
quantize_groupwise) pinned by the reference's packing known answer, the
quantiser's invariants and library routines (numpy float16 casts, float32
division and rint).

Pins:
- int4 packing [-7, -1, 0, 7] -> [0xF9, 0x70] (tests/test_artifact_compiler.py:66-71);
- per group: |q| <= qmax; the element of largest magnitude quantises to
  +-qmax with its sign; an all-zero group has scale 1 (fp16 0x3C00) and q = 0;
  every |w/s - q| <= 1/2 (round to nearest), except where clipping binds;
- the stored scale is numpy's float16 (or torch's bfloat16, the reference's
  f32_to_bf16_rne at :61-66, :232) of the float32 absmax / qmax;
- q equals numpy's float32 rint(w / s) clipped (an independent float32 evaluation).
"""
import numpy as np
import pytest

from conftest import load_oracle

orc = load_oracle()


def unpack_w4(data, cols):
    lo = (data & 0xF).astype(np.int8)
    hi = (data >> 4).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty((data.shape[0], cols), dtype=np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def test_reference_int4_packing_kat():
    # scale 7/7 = 1 exactly, so q equals the values and packs as the reference test
    w = orc.f32_to_bf16(np.array([[-7.0, -1.0, 0.0, 7.0]], np.float32))
    data, scales = orc.quantize_weights(w, 4, 4)
    assert data.tolist() == [[0xF9, 0x70]]
    assert scales.tolist() == [[0x3C00]]


def bf16_words(x32):
    """torch's round-to-nearest-even bfloat16 of float32 values, as words."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x32, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("scale_bf16", [False, True])
@pytest.mark.parametrize("bits,group,cols", [(4, 32, 256), (4, 64, 256), (4, 128, 512),
                                             (8, 0, 512), (8, 64, 256), (8, 128, 256)])
def test_quantiser_invariants(bits, group, cols, scale_bf16):
    rng = np.random.default_rng(bits * 1000 + group + cols)
    rows = 64
    w32 = (rng.standard_normal((rows, cols)) * rng.uniform(1e-3, 3.0, (rows, 1))).astype(np.float32)
    g = group or cols
    w32[5, :g] = 0.0  # one all-zero group
    w = orc.f32_to_bf16(w32)
    wf = orc.bf16_to_f32(w)
    data, scales = orc.quantize_weights(w, bits, group, scale_bf16)
    qmax = 7 if bits == 4 else 127
    q = unpack_w4(data, cols) if bits == 4 else data.view(np.int8)
    assert np.abs(q).max() <= qmax
    grouped = wf.reshape(rows, cols // g, g)
    qg = q.reshape(rows, cols // g, g).astype(np.int32)
    amax = np.abs(grouped).max(axis=2)
    s32 = amax / np.float32(qmax)
    s32 = np.where(s32 == 0, np.float32(1.0), s32).astype(np.float32)
    # stored scale: numpy's float16 (torch's bfloat16) of the float32 scale
    if scale_bf16:
        assert np.array_equal(scales, bf16_words(s32))
    else:
        assert np.array_equal(scales, s32.astype(np.float16).view(np.uint16))
    # zero group
    assert scales[5, 0] == (0x3F80 if scale_bf16 else 0x3C00) and not qg[5, 0].any()
    # the largest element maps to +-qmax with its sign
    idx = np.abs(grouped).argmax(axis=2)
    top_w = np.take_along_axis(grouped, idx[..., None], 2)[..., 0]
    top_q = np.take_along_axis(qg, idx[..., None], 2)[..., 0]
    nz = amax > 0
    assert np.array_equal(top_q[nz], (np.sign(top_w[nz]) * qmax).astype(np.int32))
    # round to nearest where no clipping happens
    ratio = grouped / s32[..., None]
    inside = np.abs(ratio) <= qmax
    assert np.all(np.abs(ratio - qg)[inside] <= 0.5)
    # an independent float32 evaluation of rint(w / s), clipped
    expect = np.clip(np.rint((grouped / s32[..., None]).astype(np.float32)), -qmax, qmax)
    assert np.array_equal(qg, expect.astype(np.int32))


def test_quantiser_rejects_bad_shapes():
    w = np.zeros((2, 96), np.uint16)
    with pytest.raises(ValueError):
        orc.quantize_weights(w, 4, 64)  # 96 % 64 != 0
    with pytest.raises(ValueError):
        orc.quantize_weights(w, 5, 32)
