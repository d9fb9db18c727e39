"""Layer-level parity through the C ABI vs the CPU oracle.

Bars (relative L2 over valid frames): F32 path 1e-4; F16 path (f16, q8_0 and
q4_K weights) 1e-2.  Ragged batches exercise the key/query masks and the
depthwise-conv pad mask; the reference's own batch invariants (batched ==
per-item, padding invariance; tests/test_relpos_attention_batch.cpp:98-146,
tests/test_conformer_batch.cpp:103-152) are checked on the GPU path too.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CASES = {
    # name: (config kwargs, weight type, precision)
    "f32_dk32": (dict(d_model=128, n_heads=4, ff_dim=256), "f32", 0),
    "q8_dk64": (dict(d_model=256, n_heads=4, ff_dim=512), "q8_0", 1),
    "q4k_dk128": (dict(d_model=256, n_heads=2, ff_dim=512), "q4_k", 1),
    "f16_dk64": (dict(d_model=128, n_heads=2, ff_dim=256, attn_bias=False, conv_bias=False), "f16", 1),
    "f16_dk32": (dict(d_model=128, n_heads=4, ff_dim=256), "f16", 1),
    # depthwise kernel 5: the f16 path runs GLU GEMM + separate depthwise pass
    # (kernel 9 takes the fused one-pass conv-module GEMM)
    "f16_k5": (dict(d_model=128, n_heads=2, ff_dim=256, conv_kernel=5), "f16", 1),
}
# d_model 512 (pointwise_conv1: K = 512, N = 1024): the conv module's
# item-tile kernel, one 128-row tile per item of T <= 128 frames (no halo),
# longer items in parts of at most 120 frames with 4-row halos (T = 129: two
# parts of 65; 240: two of 120; 375: four of 94)
CONV_CASES = {
    "q8_d512": (dict(d_model=512, n_heads=4, ff_dim=1024), "q8_0", 1),
    "f16_d512": (dict(d_model=512, n_heads=4, ff_dim=1024), "f16", 1),
    "q4k_d512": (dict(d_model=512, n_heads=4, ff_dim=1024, conv_bias=False), "q4_k", 1),
}


def _cfg(kw, n_layers=2):
    base = dict(n_layers=n_layers, conv_kernel=9, n_mels=32, sub_channels=32, vocab_size=63,
                joint_hidden=64, pred_hidden=64)
    base.update(kw)
    return pm.Config(**base)


_CACHE = {}


def _models(gpu, name):
    if name not in _CACHE:
        kw, wt, prec = CASES[name] if name in CASES else CONV_CASES[name]
        m = pm.synthesize(_cfg(kw), wt, bn_random=True)
        _CACHE[name] = (m, oracle.OracleModel(m), gpu.Model.from_tensors(m, prec), prec)
    return _CACHE[name]


def _tol(prec):
    return 1e-4 if prec == 0 else 1e-2


def _valid_mask(B, T, valid):
    return np.arange(T)[None, :] < np.asarray(valid)[:, None]


# (16, 375): more 64-query blocks than one round of the chip holds, so the f16
# kernel takes its 96-query single-key-group form (the 4-head cases: dk 64, 32)
@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("B,T,valid", [(1, 1, [1]), (2, 37, [37, 20]), (3, 70, [70, 64, 1]),
                                       (2, 130, [130, 99]),
                                       (16, 375, [375, 375, 300, 1, 129, 128, 64, 65, 200, 374, 96, 97, 250, 33,
                                                  375, 2])])
def test_relpos_attention(gpu, stream, name, B, T, valid):
    m, om, gm, prec = _models(gpu, name)
    D = m.cfg.d_model
    rng = np.random.default_rng(B * 1000 + T)
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[attn] {name} B={B} T={T} valid={valid}", flush=True)
    ref = om.relpos_attention(0, x, oracle.rel_pos_encoding(T, D), valid)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    gm.relpos_attention(0, dx, valid, dy, stream)
    got = dy.numpy(stream)
    mask = _valid_mask(B, T, valid)
    assert rel_l2(got[mask], ref[mask]) < _tol(prec)
    # padded query rows reduce to linear_out.bias (relpos_attention.cpp:291-305)
    assert rel_l2(got[~mask], ref[~mask]) < _tol(prec) if (~mask).any() else True


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("B,T,valid", [(1, 5, [5]), (2, 37, [37, 20]), (3, 129, [129, 100, 3])])
def test_conv_module(gpu, stream, name, B, T, valid):
    m, om, gm, prec = _models(gpu, name)
    D = m.cfg.d_model
    rng = np.random.default_rng(B * 7 + T)
    c = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[conv] {name} B={B} T={T} valid={valid}", flush=True)
    ref = om.conv_module(0, c, valid)
    dc = gpu.DeviceArray.from_numpy(c, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    gm.conv_module(0, dc, valid, dy, stream)
    got = dy.numpy(stream)
    mask = _valid_mask(B, T, valid)
    err = rel_l2(got[mask], ref[mask])
    print(f"  rel_l2 {err:.3e}")
    # f16 path: 2.1-3.1e-4 measured (the f16 roundings of the activations,
    # pointwise weights and stored GLU / depthwise values; deterministic), so
    # the bar is kept at 3e-3 rather than the layer-level 1e-2
    assert err < (3e-3 if prec else _tol(prec)), err


@pytest.mark.parametrize("name", list(CONV_CASES))
@pytest.mark.parametrize("B,T,valid", [(16, 125, [125, 125, 100, 1, 64, 65, 124, 125, 33, 2, 125, 90, 125, 7, 125, 50]),
                                       (3, 128, [128, 127, 1]), (4, 1, [1, 1, 1, 1]), (1, 37, [37]),
                                       (1, 129, [129]), (2, 200, [200, 150]), (3, 240, [240, 121, 5]),
                                       (2, 375, [375, 241])])
def test_conv_module_item_tiles(gpu, stream, name, B, T, valid):
    test_conv_module(gpu, stream, name, B, T, valid)


@pytest.mark.parametrize("name", list(CASES) + ["q8_d512", "f16_d512"])
@pytest.mark.parametrize("B,T,valid", [(1, 26, [26]), (2, 63, [63, 40])])
def test_conformer_layer(gpu, stream, name, B, T, valid):
    m, om, gm, prec = _models(gpu, name)
    D = m.cfg.d_model
    rng = np.random.default_rng(B + 3 * T)
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[layer] {name} B={B} T={T} valid={valid}", flush=True)
    ref, ref_conv = om.conformer_layer(1, x, oracle.rel_pos_encoding(T, D), valid, want_conv=True)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    dconv = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(1, dx, valid, dy, dconv, stream)
    got, got_conv = dy.numpy(stream), dconv.numpy(stream)
    mask = _valid_mask(B, T, valid)
    assert rel_l2(got[mask], ref[mask]) < _tol(prec)
    assert rel_l2(got_conv[mask], ref_conv[mask]) < _tol(prec)
    # sublayer delta, not only the residual-dominated output
    delta_ref = ref[mask] - x[mask]
    delta_got = got[mask] - x[mask]
    assert rel_l2(delta_got, delta_ref) < 3 * _tol(prec)


@pytest.mark.parametrize("name", list(CASES) + ["q8_d512", "f16_d512"])
@pytest.mark.parametrize("offset", [0.0, 4.0])
def test_conformer_layer_folded_layernorm(gpu, stream, name, offset):
    """The encoder's own path through a block (no conv-module capture): on the
    f16 path norm_self_att, norm_conv and norm_feed_forward2 are folded into
    the neighbouring GEMMs (statistics from the residual product, the
    normalisation in the next product's epilogue).  A per-row mean of 4 sigma
    in the residual stream checks that the folded form keeps its accuracy when
    the mean is large against the spread (d_model 512: the conv module's
    item-tile kernel with norm_conv folded in)."""
    m, om, gm, prec = _models(gpu, name)
    D, B, T = m.cfg.d_model, 3, 77
    valid = [77, 50, 9]
    rng = np.random.default_rng(int(31 + offset))
    x = (rng.normal(0, 1, (B, T, D)) + offset * (1 + rng.random((B, T, 1)))).astype(np.float32)
    print(f"[layer-fold] {name} offset={offset}", flush=True)
    ref = om.conformer_layer(1, x, oracle.rel_pos_encoding(T, D), valid)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(1, dx, valid, dy, None, stream)
    got = dy.numpy(stream)
    mask = _valid_mask(B, T, valid)
    err = rel_l2(got[mask], ref[mask])
    print(f"  rel_l2 {err:.3e}")
    assert err < _tol(prec), err


@pytest.mark.parametrize("name", ["f32_dk32", "q8_dk64"])
def test_batched_equals_per_item(gpu, stream, name):
    """tests/test_conformer_batch.cpp:103-152 on the GPU path: a full item is
    unchanged by a shorter neighbour; the short item's valid rows equal its
    standalone run."""
    m, om, gm, prec = _models(gpu, name)
    D, T = m.cfg.d_model, 48
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, (2, T, D)).astype(np.float32)
    x[1] = x[0]
    valid = [T, T // 2]
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((2, T, D), np.float32)
    gm.conformer_layer(0, dx, valid, dy, None, stream)
    both = dy.numpy(stream)
    d1 = gpu.DeviceArray.from_numpy(x[:1].copy(), stream)
    y1 = gpu.DeviceArray((1, T, D), np.float32)
    gm.conformer_layer(0, d1, [T], y1, None, stream)
    full = y1.numpy(stream)[0]
    gm.conformer_layer(0, d1, [T // 2], y1, None, stream)
    short = y1.numpy(stream)[0]
    assert rel_l2(both[0], full) < 1e-3
    assert rel_l2(both[1, :T // 2], short[:T // 2]) < 1e-3


@pytest.mark.parametrize("ragged", [False, True])
def test_conformer_layer_production_shape(gpu, stream, ragged):
    """One 0.6B-shape block (d=1024, 8 heads x 128, FFN 4096, q8_0 linears) at
    batch 16 x T'=125: the tile shapes and epilogues the encoder benchmark runs
    (128x128 SiLU/store, 128x64 residual, 64x64 positional projection, f16
    64x128 GLU) all checked against the oracle."""
    cfg = _cfg(dict(d_model=1024, n_heads=8, ff_dim=4096, attn_bias=False, ff_bias=False, conv_bias=False),
               n_layers=1)
    m = pm.synthesize(cfg, "q8_0", bn_random=True)
    om = oracle.OracleModel(m)
    gm = gpu.Model.from_tensors(m, 1)
    B, T, D = 16, 125, 1024
    rng = np.random.default_rng(2026 + ragged)
    valid = rng.integers(2, T + 1, B).tolist() if ragged else [T] * B
    valid[0] = T
    x = rng.normal(0, 1, (B, T, D)).astype(np.float32)
    print(f"[layer-0.6B] B={B} T={T} valid={valid}", flush=True)
    ref, ref_conv = om.conformer_layer(0, x, oracle.rel_pos_encoding(T, D), valid, want_conv=True)
    dx = gpu.DeviceArray.from_numpy(x, stream)
    dy = gpu.DeviceArray((B, T, D), np.float32)
    dconv = gpu.DeviceArray((B, T, D), np.float32)
    gm.conformer_layer(0, dx, valid, dy, dconv, stream)
    got, got_conv = dy.numpy(stream), dconv.numpy(stream)
    # the encoder's path (no capture): LayerNorms folded into the GEMMs
    gm.conformer_layer(0, dx, valid, dy, None, stream)
    got_fold = dy.numpy(stream)
    gm.close()
    mask = _valid_mask(B, T, valid)
    assert rel_l2(got[mask], ref[mask]) < 1e-2
    assert rel_l2(got_conv[mask], ref_conv[mask]) < 1e-2
    assert rel_l2(got[mask] - x[mask], ref[mask] - x[mask]) < 3e-2
    assert rel_l2(got_fold[mask], ref[mask]) < 1e-2
    assert rel_l2(got_fold[mask] - x[mask], ref[mask] - x[mask]) < 3e-2
