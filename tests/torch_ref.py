"""Independent float64 restatement of the encoder path in torch (CPU) library
routines, NeMo-style, used only to pin the C oracle in CPU tests.

It is written from the model definition, not from the oracle's code:
convolutions go through F.conv2d / F.conv1d, norms through F.layer_norm /
F.batch_norm, the GLU through F.glu, and the relative shift through NeMo's
pad-and-view formulation (RelPositionMultiHeadAttention.rel_shift) rather
than the oracle's index identity.  Masking follows the reference graphs
(key mask -inf, padded query rows zeroed, relpos_attention.cpp:252-302;
per-stage time masks in batched subsampling, subsampling.cpp:95-147).

Import torch only inside test functions (GPU processes never load it).
"""
import numpy as np
import torch
import torch.nn.functional as F

DT = torch.float64


def T(a):
    return torch.as_tensor(np.asarray(a), dtype=DT)


class TorchModel:
    def __init__(self, om):
        """om: oracle.OracleModel (its dequantised f32 weights are the shared inputs)."""
        self.cfg = om.cfg
        self.w = {k: T(v) for k, v in om.w.items()}

    def g(self, name):
        return self.w.get(name)

    # ---- pieces ----------------------------------------------------------
    @staticmethod
    def rel_shift(x):
        b, h, qlen, pos_len = x.size()
        x = F.pad(x, pad=(1, 0))
        x = x.view(b, h, -1, qlen)
        x = x[:, :, 1:].view(b, h, qlen, pos_len)
        return x

    def linear(self, x, w, b):
        return F.linear(x, self.g(w), self.g(b) if b and self.g(b) is not None else None)

    def attention(self, i, x, pe, valid):
        c = self.cfg
        p = f"encoder.layers.{i}.self_attn."
        B, Tn, D = x.shape
        H, dk = c.n_heads, D // c.n_heads
        q = self.linear(x, p + "linear_q.weight", p + "linear_q.bias").view(B, Tn, H, dk).transpose(1, 2)
        k = self.linear(x, p + "linear_k.weight", p + "linear_k.bias").view(B, Tn, H, dk).transpose(1, 2)
        v = self.linear(x, p + "linear_v.weight", p + "linear_v.bias").view(B, Tn, H, dk).transpose(1, 2)
        pp = F.linear(T(pe), self.g(p + "linear_pos.weight")).view(1, -1, H, dk).transpose(1, 2)
        qu = q + self.g(p + "pos_bias_u").view(1, H, 1, dk)
        qv = q + self.g(p + "pos_bias_v").view(1, H, 1, dk)
        ac = torch.matmul(qu, k.transpose(-2, -1))
        bd = self.rel_shift(torch.matmul(qv, pp.transpose(-2, -1)))[:, :, :, :Tn]
        scores = (ac + bd) / np.sqrt(dk)
        keymask = torch.arange(Tn)[None, :] >= torch.as_tensor(valid)[:, None]      # [B, T]
        scores = scores.masked_fill(keymask[:, None, None, :], float("-inf"))
        attn = torch.softmax(scores, dim=-1)
        ctx = torch.matmul(attn, v).transpose(1, 2).reshape(B, Tn, D)
        ctx = ctx.masked_fill(keymask[:, :, None], 0.0)                              # padded queries
        return self.linear(ctx, p + "linear_out.weight", p + "linear_out.bias")

    def conv_module(self, i, cin, valid):
        c = self.cfg
        p = f"encoder.layers.{i}.conv."
        B, Tn, D = cin.shape
        x = cin.transpose(1, 2)                                                      # [B, D, T]
        x = F.conv1d(x, self.g(p + "pointwise_conv1.weight"), self.g(p + "pointwise_conv1.bias"))
        x = F.glu(x, dim=1)
        pad = torch.arange(Tn)[None, :] >= torch.as_tensor(valid)[:, None]
        x = x.masked_fill(pad[:, None, :], 0.0)
        x = F.conv1d(x, self.g(p + "depthwise_conv.weight"), self.g(p + "depthwise_conv.bias"),
                     padding=(c.conv_kernel - 1) // 2, groups=D)
        x = F.batch_norm(x, self.g(p + "batch_norm.running_mean"), self.g(p + "batch_norm.running_var"),
                         self.g(p + "batch_norm.weight"), self.g(p + "batch_norm.bias"), training=False,
                         eps=1e-5)
        x = F.silu(x)
        x = F.conv1d(x, self.g(p + "pointwise_conv2.weight"), self.g(p + "pointwise_conv2.bias"))
        return x.transpose(1, 2)

    def ln(self, x, name):
        return F.layer_norm(x, (x.shape[-1],), self.g(name + ".weight"), self.g(name + ".bias"), eps=1e-5)

    def ffn(self, x, name):
        h = F.silu(self.linear(x, name + ".linear1.weight", name + ".linear1.bias"))
        return self.linear(h, name + ".linear2.weight", name + ".linear2.bias")

    def layer(self, i, x, pe, valid):
        p = f"encoder.layers.{i}."
        r = x + 0.5 * self.ffn(self.ln(x, p + "norm_feed_forward1"), p + "feed_forward1")
        r = r + self.attention(i, self.ln(r, p + "norm_self_att"), pe, valid)
        r = r + self.conv_module(i, self.ln(r, p + "norm_conv"), valid)
        r = r + 0.5 * self.ffn(self.ln(r, p + "norm_feed_forward2"), p + "feed_forward2")
        return self.ln(r, p + "norm_out")

    def subsampling(self, mel, valid_in):
        """Batched semantics: zero frames t >= v before every conv stage."""
        p = "encoder.pre_encode."
        x = T(mel).transpose(1, 2)[:, None]                        # [B, 1, T, F]
        v = list(valid_in)

        def mask(x, v):
            t = torch.arange(x.shape[2])[None, :] >= torch.as_tensor(v)[:, None]
            return x.masked_fill(t[:, None, :, None], 0.0)

        def nxt(v):
            return [(a + 2 - 3) // 2 + 1 if a + 2 - 3 >= 0 else 1 for a in v]

        x = F.relu(F.conv2d(mask(x, v), self.g(p + "conv.0.weight"), self.g(p + "conv.0.bias"), stride=2, padding=1))
        v = nxt(v)
        C = x.shape[1]
        x = F.conv2d(mask(x, v), self.g(p + "conv.2.weight"), self.g(p + "conv.2.bias"), stride=2, padding=1, groups=C)
        x = F.relu(F.conv2d(x, self.g(p + "conv.3.weight"), self.g(p + "conv.3.bias")))
        v = nxt(v)
        x = F.conv2d(mask(x, v), self.g(p + "conv.5.weight"), self.g(p + "conv.5.bias"), stride=2, padding=1, groups=C)
        x = F.relu(F.conv2d(x, self.g(p + "conv.6.weight"), self.g(p + "conv.6.bias")))
        v = nxt(v)
        B, C, Tp, Fp = x.shape
        x = x.transpose(1, 2).reshape(B, Tp, C * Fp)
        x = mask(x[:, None], v)[:, 0]
        return self.linear(x, p + "out.weight", p + "out.bias"), v

    def rel_pos(self, Tn, D):
        pos = torch.arange(Tn - 1, -Tn, -1, dtype=DT)[:, None]
        div = torch.exp(torch.arange(0, D, 2, dtype=DT) * (-np.log(10000.0) / D))
        pe = torch.zeros(2 * Tn - 1, D, dtype=DT)
        pe[:, 0::2] = torch.sin(pos * div)
        pe[:, 1::2] = torch.cos(pos * div)
        return pe

    def encoder(self, mel, valid_in):
        x, v = self.subsampling(mel, valid_in)
        if self.cfg.xscaling:
            x = x * np.sqrt(self.cfg.d_model)
        pe = self.rel_pos(x.shape[1], self.cfg.d_model).float().double()   # table is stored as f32
        outs = []
        for i in range(self.cfg.n_layers):
            x = self.layer(i, x, pe, v)
            outs.append(x)
        return x, v, outs
