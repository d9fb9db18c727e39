"""Pins of the CPU oracle (no GPU).

Each function of oracle/pk_oracle.c is checked against something it does not
share code with: numpy/torch library routines (float64), closed forms,
hand-built known-answer blocks, brute force on tiny inputs, and an emulation
of the reference's ggml view/reshape sequence for rel_shift.  Planted-mistake
checks (a wrong shift, a dropped term) fail these pins; see
test_pins_detect_planted_mistakes.
"""
import numpy as np
import pytest

import oracle
import pk_model as pm
from conftest import rel_l2


def tiny_cfg(**kw):
    base = dict(d_model=64, n_layers=2, n_heads=4, ff_dim=128, conv_kernel=9, n_mels=24, sub_channels=16,
                vocab_size=31, joint_hidden=32, pred_hidden=32)
    base.update(kw)
    return pm.Config(**base)


# ---------------------------------------------------------------- binary16
def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 5000), rng.normal(0, 1e-5, 2000), rng.normal(0, 3e4, 2000),
                        [0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8,
                         6.1035156e-05, 6.103515e-05, np.inf, -np.inf]]).astype(np.float32)
    lib = oracle.lib()
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    back = np.array([lib.orc_f16_to_f32(int(h)) for h in range(0, 65536, 7)], dtype=np.float32)
    ref_back = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(ref_back)
    assert np.array_equal(back[fin].view(np.uint32), ref_back[fin].view(np.uint32))


# ---------------------------------------------------------------- block formats
def _q8_block(d_bits, qs):
    return np.concatenate([np.array([d_bits & 0xFF, d_bits >> 8], np.uint8), np.asarray(qs, np.int8).view(np.uint8)])


def test_q8_0_known_answer():
    # d = 0.5 (f16 0x3800), q = -127..? ; w = d*q exactly
    qs = np.array([-128, -127, -1, 0, 1, 2, 3, 127] * 4, dtype=np.int8)
    blk = _q8_block(0x3800, qs)
    blk2 = _q8_block(0xC000, np.arange(32, dtype=np.int8))          # d = -2
    got = oracle.dequantize(pm.GGML_Q8_0, np.concatenate([blk, blk2]), 64)
    assert np.array_equal(got[:32], qs.astype(np.float32) * 0.5)
    assert np.array_equal(got[32:], np.arange(32, dtype=np.float32) * -2.0)


def _pack_q4k_scales(sc, mn):
    """Own packing of eight 6-bit scales/mins into ggml's 12-byte block_q4_K field."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return s


def test_q4_k_known_answer():
    # d = 1, dmin = 0.25: element e of sub-block j is sc_j * q - 0.25 * m_j with the
    # 4-bit q of element e taken from the low (first 32 of each 64) or high nibble.
    sc = np.array([1, 2, 3, 63, 16, 33, 47, 62])
    mn = np.array([0, 5, 63, 7, 17, 48, 31, 60])
    q = (np.arange(256) * 7 + 3) % 16
    qs = np.zeros(128, np.uint8)
    for c in range(4):
        qs[32 * c:32 * c + 32] = q[64 * c:64 * c + 32] | (q[64 * c + 32:64 * c + 64] << 4)
    blk = np.concatenate([np.array([0x00, 0x3C, 0x00, 0x34], np.uint8), _pack_q4k_scales(sc, mn), qs])
    assert blk.size == 144
    got = oracle.dequantize(pm.GGML_Q4_K, blk, 256)
    j = np.arange(256) // 32
    ref = (sc[j] * q - 0.25 * mn[j]).astype(np.float32)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("gtype,tol", [(pm.GGML_Q8_0, 0.5 / 127), (pm.GGML_Q4_K, 0.6 / 15)])
def test_quantize_roundtrip_error_bound(gtype, tol):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 0.02, 256 * 8).astype(np.float32)
    back = oracle.dequantize(gtype, oracle.quantize(gtype, x), x.size)
    blk = 32
    err = np.abs(back - x).reshape(-1, blk).max(1)
    amp = (x.reshape(-1, blk).max(1) - np.minimum(x.reshape(-1, blk).min(1), 0)) + 1e-12
    if gtype == pm.GGML_Q8_0:
        amp = np.abs(x.reshape(-1, blk)).max(1)
    assert (err <= tol * amp * 1.3 + 1e-7).all()


# ---------------------------------------------------------------- pos-enc, LN, linear
@pytest.mark.parametrize("T,d", [(1, 8), (5, 16), (125, 512)])
def test_rel_pos_encoding_closed_form(T, d):
    pe = oracle.rel_pos_encoding(T, d)
    pos = np.arange(T - 1, -T, -1, dtype=np.float64)[:, None]
    div = np.exp(np.arange(0, d, 2) * -(np.log(10000.0) / d))
    ref = np.zeros((2 * T - 1, d))
    ref[:, 0::2] = np.sin(pos * div)
    ref[:, 1::2] = np.cos(pos * div)
    assert np.array_equal(pe, ref.astype(np.float32))
    mid = pe[T - 1]                                    # relative position 0
    assert np.all(mid[0::2] == 0.0) and np.all(mid[1::2] == 1.0)


def test_layer_norm_vs_numpy_and_invariants():
    rng = np.random.default_rng(2)
    x = (rng.normal(0, 3, (50, 96)) + 5).astype(np.float32)
    ones, zeros = np.ones(96, np.float32), np.zeros(96, np.float32)
    y = oracle.layer_norm(x, ones, zeros)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5)
    assert np.abs(y - ref).max() < 2e-6
    assert np.abs(y.mean(1)).max() < 1e-6 and np.abs(y.var(1) - 1).max() < 1e-4


def test_linear_vs_numpy():
    rng = np.random.default_rng(3)
    for M, K, N in [(1, 8, 1), (7, 13, 5), (33, 200, 47)]:
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        W = rng.normal(0, 1, (N, K)).astype(np.float32)
        b = rng.normal(0, 1, N).astype(np.float32)
        ref = x.astype(np.float64) @ W.astype(np.float64).T + b
        assert rel_l2(oracle.linear(x, W, b), ref) < 1e-6


# ---------------------------------------------------------------- rel_shift
def _ggml_rel_shift(bd, T):
    """Emulate relpos_attention.cpp:226-238 on raw memory: bd is [T][P] (row per
    query, P = 2T-1 positions) = ggml ne [P, T]."""
    P = 2 * T - 1
    padded = np.concatenate([np.zeros((T, 1)), bd], axis=1).reshape(-1)      # ggml_pad_ext lp0=1: ne [2T, T]
    # reshape_3d(T, 2T) keeps memory; view_3d(T, 2T-1, nb1, offset nb1) then cont
    view1 = np.lib.stride_tricks.as_strided(padded[T:], shape=(2 * T - 1, T), strides=(T * 8, 8)).copy().reshape(-1)
    # reshape_3d(2T-1, T): ne0 = 2T-1; view_3d(T, T, nb1, 0) then cont
    view2 = np.lib.stride_tricks.as_strided(view1, shape=(T, T), strides=((2 * T - 1) * 8, 8)).copy()
    return view2                                                                # [T_q][T_k]


@pytest.mark.parametrize("T", [1, 2, 3, 5, 26, 125])
def test_rel_shift_index_identity(T):
    rng = np.random.default_rng(T)
    bd = rng.normal(0, 1, (T, 2 * T - 1))
    got = _ggml_rel_shift(bd, T)
    i, j = np.meshgrid(np.arange(T), np.arange(T), indexing="ij")
    assert np.array_equal(got, bd[i, T - 1 - i + j])        # the identity the oracle and kernels use


# ---------------------------------------------------------------- model-level vs torch library routines
@pytest.fixture(scope="module")
def tiny():
    torch = pytest.importorskip("torch")
    import torch_ref
    m = pm.synthesize(tiny_cfg(), "f32", bn_random=True, std=0.1)
    om = oracle.OracleModel(m)
    return m, om, torch_ref.TorchModel(om), torch


def test_attention_vs_torch(tiny):
    m, om, tm, torch = tiny
    rng = np.random.default_rng(4)
    B, Tn, D = 3, 11, m.cfg.d_model
    x = rng.normal(0, 1, (B, Tn, D)).astype(np.float32)
    pe = oracle.rel_pos_encoding(Tn, D)
    valid = [11, 6, 1]
    got = om.relpos_attention(0, x, pe, valid)
    ref = tm.attention(0, torch.as_tensor(x, dtype=torch.float64), pe, valid).numpy()
    assert rel_l2(got, ref) < 1e-5


def test_attention_reduces_to_sdpa_without_position_terms(tiny):
    """With linear_pos = 0 and pos_bias_u = pos_bias_v = 0 the module is plain
    multi-head attention: compare with torch's scaled_dot_product_attention."""
    m, om, tm, torch = tiny
    import torch.nn.functional as F
    w = dict(om.w)
    p = "encoder.layers.0.self_attn."
    saved = {k: w[k].copy() for k in (p + "linear_pos.weight", p + "pos_bias_u", p + "pos_bias_v")}
    try:
        for k in saved:
            om.w[k][...] = 0
        rng = np.random.default_rng(5)
        B, Tn, D, H = 2, 9, m.cfg.d_model, m.cfg.n_heads
        x = rng.normal(0, 1, (B, Tn, D)).astype(np.float32)
        got = om.relpos_attention(0, x, oracle.rel_pos_encoding(Tn, D), [Tn, Tn])
        X = torch.as_tensor(x, dtype=torch.float64)

        def lin(n):
            return F.linear(X, torch.as_tensor(om.w[p + n + ".weight"], dtype=torch.float64),
                            torch.as_tensor(om.w[p + n + ".bias"], dtype=torch.float64))
        q, k, v = (lin(n).view(B, Tn, H, D // H).transpose(1, 2) for n in ("linear_q", "linear_k", "linear_v"))
        ctx = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(B, Tn, D)
        ref = F.linear(ctx, torch.as_tensor(om.w[p + "linear_out.weight"], dtype=torch.float64),
                       torch.as_tensor(om.w[p + "linear_out.bias"], dtype=torch.float64)).numpy()
        assert rel_l2(got, ref) < 1e-5
    finally:
        for k, v in saved.items():
            om.w[k][...] = v


def test_conv_module_vs_torch(tiny):
    m, om, tm, torch = tiny
    rng = np.random.default_rng(6)
    c = rng.normal(0, 1, (2, 17, m.cfg.d_model)).astype(np.float32)
    valid = [17, 9]
    got = om.conv_module(0, c, valid)
    ref = tm.conv_module(0, torch.as_tensor(c, dtype=torch.float64), valid).numpy()
    assert rel_l2(got, ref) < 1e-5


def test_depthwise_impulse_response(tiny):
    """A single impulse at t0 reproduces the depthwise taps: with identity-like
    pointwise convs this is checked through the torch pin above; here the oracle
    alone: shifting the input by one frame shifts the output by one frame."""
    m, om, tm, torch = tiny
    rng = np.random.default_rng(7)
    c = rng.normal(0, 1, (1, 40, m.cfg.d_model)).astype(np.float32)
    c2 = np.zeros_like(c)
    c2[:, 1:] = c[:, :-1]
    a = om.conv_module(0, c, None)
    b = om.conv_module(0, c2, None)
    assert rel_l2(b[:, 10:30], a[:, 9:29]) < 1e-6


def test_conformer_layer_vs_torch(tiny):
    m, om, tm, torch = tiny
    rng = np.random.default_rng(8)
    x = rng.normal(0, 1, (2, 13, m.cfg.d_model)).astype(np.float32)
    pe = oracle.rel_pos_encoding(13, m.cfg.d_model)
    valid = [13, 8]
    got, conv = om.conformer_layer(1, x, pe, valid, want_conv=True)
    ref = tm.layer(1, torch.as_tensor(x, dtype=torch.float64), torch.as_tensor(pe, dtype=torch.float64), valid)
    assert rel_l2(got, ref.numpy()) < 1e-5


@pytest.mark.parametrize("T,valid_T", [(64, [64]), (70, [70, 33])])
def test_subsampling_and_encoder_vs_torch(tiny, T, valid_T):
    m, om, tm, torch = tiny
    rng = np.random.default_rng(T)
    B = len(valid_T)
    mel = rng.normal(0, 1, (B, m.cfg.n_mels, T)).astype(np.float32)
    vin = np.array(valid_T) - 1
    sub, vo = om.subsampling(mel, vin, stage_masks=True)
    ref_sub, v_ref = tm.subsampling(mel, vin)
    assert list(vo) == list(v_ref)
    assert rel_l2(sub, ref_sub.numpy()) < 1e-5
    out, vo2, cap = om.encoder(mel, vin, capture=True)
    ref, _, outs = tm.encoder(mel, vin)
    for l in range(m.cfg.n_layers):
        mask = np.arange(out.shape[1])[None, :] < vo2[:, None]
        assert rel_l2(cap[l][mask], outs[l].numpy()[mask]) < 1e-5


def test_scalar_subsampling_masks_only_the_output(tiny):
    """subsampling.cpp:281-300: with a full-length clip the scalar path differs
    from the batched one only through the zeroed last mel frame."""
    m, om, tm, torch = tiny
    rng = np.random.default_rng(9)
    mel = rng.normal(0, 1, (1, m.cfg.n_mels, 48)).astype(np.float32)
    a, _ = om.subsampling(mel, None, stage_masks=False)
    mel2 = mel.copy()
    mel2[:, :, 47] = 0.0
    b, _ = om.subsampling(mel2, None, stage_masks=False)
    c, _ = om.subsampling(mel, None, stage_masks=True)
    assert np.array_equal(b, c)            # batched = scalar after zeroing frame T-1 here
    assert not np.array_equal(a, c)


def test_ctc_head_and_greedy(tiny):
    m, om, tm, torch = tiny
    rng = np.random.default_rng(10)
    enc = rng.normal(0, 1, (20, m.cfg.d_model)).astype(np.float32)
    lp, am = om.ctc(enc)
    W = om.w["ctc_decoder.decoder_layers.0.weight"].reshape(-1, m.cfg.d_model)
    b = om.w["ctc_decoder.decoder_layers.0.bias"]
    ref = torch.log_softmax(torch.as_tensor(enc, dtype=torch.float64) @ torch.as_tensor(W, dtype=torch.float64).T
                            + torch.as_tensor(b, dtype=torch.float64), dim=-1).numpy()
    assert np.abs(lp - ref).max() < 1e-5
    assert np.array_equal(am, ref.argmax(1))
    blank = 5
    seq = np.array([5, 1, 1, 5, 1, 2, 2, 2, 5, 5, 3, 1, 5], np.int32)   # search.cpp:63 collapse rule
    assert list(oracle.ctc_greedy(seq, blank)) == [1, 1, 2, 3, 1]


def test_tdt_joint_vs_torch(tiny):
    m, om, tm, torch = tiny
    rng = np.random.default_rng(11)
    enc = rng.normal(0, 1, (15, m.cfg.d_model)).astype(np.float32)
    g = rng.normal(0, 1, m.cfg.pred_hidden).astype(np.float32)
    lg, tok, dur = om.tdt_joint(enc, g)
    t = lambda n: torch.as_tensor(om.w[n], dtype=torch.float64)
    f = torch.relu(torch.as_tensor(enc, dtype=torch.float64) @ t("joint.enc.weight").T + t("joint.enc.bias")
                   + (torch.as_tensor(g, dtype=torch.float64) @ t("joint.pred.weight").T + t("joint.pred.bias")))
    ref = (f @ t("joint.joint_net.2.weight").T + t("joint.joint_net.2.bias")).numpy()
    assert rel_l2(lg, ref) < 1e-5
    n_tok = ref.shape[1] - len(m.cfg.tdt_durations)
    assert np.array_equal(tok, ref[:, :n_tok].argmax(1))
    assert np.array_equal(dur, ref[:, n_tok:].argmax(1))


def test_pins_detect_planted_mistakes(tiny):
    """A mistake planted in a copy of the oracle's inputs is caught by the pins:
    transposing the position table (a wrong shift direction) and dropping the
    pos_bias_v term both move the attention output far outside tolerance."""
    m, om, tm, torch = tiny
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, (1, 9, m.cfg.d_model)).astype(np.float32)
    pe = oracle.rel_pos_encoding(9, m.cfg.d_model)
    ref = tm.attention(0, torch.as_tensor(x, dtype=torch.float64), pe, [9]).numpy()
    wrong_shift = om.relpos_attention(0, x, pe[::-1].copy(), [9])
    assert rel_l2(wrong_shift, ref) > 1e-3
    p = "encoder.layers.0.self_attn.pos_bias_v"
    keep = om.w[p].copy()
    try:
        om.w[p][...] = 0
        dropped = om.relpos_attention(0, x, pe, [9])
    finally:
        om.w[p][...] = keep
    assert rel_l2(dropped, ref) > 1e-4


def test_pins_detect_more_planted_mistakes(tiny):
    """Three more slips, each planted in the oracle's own weights (on the CPU):
    a dropped 1/2 on the macaron FFN residual, depthwise taps applied as a
    convolution instead of a cross-correlation, and a transposed query
    projection.  Each moves the oracle far outside the torch pin's tolerance,
    while the unmodified oracle sits within 1e-5 of it."""
    m, om, tm, torch = tiny
    rng = np.random.default_rng(13)
    D = m.cfg.d_model
    x = rng.normal(0, 1, (1, 11, D)).astype(np.float32)
    pe = oracle.rel_pos_encoding(11, D)
    xt, pet = torch.as_tensor(x, dtype=torch.float64), torch.as_tensor(pe, dtype=torch.float64)
    ref_layer = tm.layer(0, xt, pet, [11]).numpy()
    assert rel_l2(om.conformer_layer(0, x, pe, [11]), ref_layer) < 1e-5

    def with_plant(name, fn, run):
        keep = om.w[name].copy()
        try:
            om.w[name][...] = fn(keep)
            return run()
        finally:
            om.w[name][...] = keep

    # dropped 1/2: FFN1's output doubled
    got = with_plant("encoder.layers.0.feed_forward1.linear2.weight", lambda w: 2 * w,
                     lambda: om.conformer_layer(0, x, pe, [11]))
    assert rel_l2(got, ref_layer) > 1e-3
    # convolution instead of cross-correlation: taps reversed in time
    ref_conv = tm.conv_module(0, xt, [11]).numpy()
    got = with_plant("encoder.layers.0.conv.depthwise_conv.weight", lambda w: w[..., ::-1].copy(),
                     lambda: om.conv_module(0, x, [11]))
    assert rel_l2(got, ref_conv) > 1e-3
    # transposed operand: W_q^T in place of W_q
    ref_attn = tm.attention(0, xt, pe, [11]).numpy()
    got = with_plant("encoder.layers.0.self_attn.linear_q.weight", lambda w: w.T.copy(),
                     lambda: om.relpos_attention(0, x, pe, [11]))
    assert rel_l2(got, ref_attn) > 1e-3


# ---------------------------------------------------------------- length arithmetic
def test_valid_length_arithmetic():
    # subsampling.cpp:25-46 with the offline T-1 entry convention
    assert oracle.subsampled_len(1000) == 125 and oracle.valid_out_len(1000) == 125
    assert oracle.subsampled_len(1001) == 126 and oracle.valid_out_len(1001) == 125
    assert oracle.subsampled_len(3000) == 375
    assert oracle.valid_out_len(1, -1) == 1 and oracle.subsampled_len(1) == 1
    for T in range(1, 400):
        v = T - 1
        for _ in range(3):
            v = (v + 2 - 3) // 2 + 1 if v >= 1 else 1
        assert oracle.valid_out_len(T) == v
