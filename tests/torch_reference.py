"""Float64 re-derivation of a KataGo forward pass with torch library routines.

Walks the layer program a backend receives (kgn_model_flatten) and evaluates
it with torch.nn.functional.conv2d (direct convolution, NCHW), dense matmuls,
scaled_dot_product_attention and silu, in float64, following the semantics
of Model::apply (/root/reference/cpp/neuralnet/eigenbackend.cpp:1091-2205):
pre-activation blocks, BN output zeroed where mask != 1, conv outputs and
residual adds unmasked, transformer residuals masked, gpool max from -1 with
the +mask-1 offset. It shares no code with the oracle (no Winograd, no NHWC
indexing, no GEMM kernel), so agreement pins the oracle's composition and
layouts; agreement after scale8 also pins that transform.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

LAYER_DTYPE = np.dtype([("op", "<i4"), ("i", "<i4", 7), ("f", "<f4", 2), ("w", "<i8", 2), ("wn", "<i8", 2)])
assert LAYER_DTYPE.itemsize == 72

OP_CONV, OP_BN, OP_ACT, OP_MATMUL, OP_MATBIAS, OP_RMSNORM, OP_TRMSNORM = 1, 2, 3, 4, 5, 6, 7
OP_ORD, OP_GPOOL, OP_NBT, OP_ATTN, OP_FFN = 10, 11, 12, 13, 14
OP_TRUNK, OP_POLICY, OP_VALUE = 20, 21, 22


def flatten(loaded_model):
    """(layers structured array, weights float32 array) for a nn.LoadedModel."""
    from katago_amd import nn
    return nn.flatten_model(loaded_model)


def act(x, kind):
    if kind == 0:
        return x
    if kind == 1:
        return torch.relu(x)
    if kind == 2:
        return x * torch.tanh(F.softplus(x))
    if kind == 3:
        return F.silu(x)
    if kind == 12:
        return x * torch.tanh(F.softplus(8.0 * x))
    raise ValueError(kind)


class Program:
    def __init__(self, layers, weights):
        self.L = layers
        self.W = weights.astype(np.float64)
        self.pos = 0

    def take(self, op):
        rec = self.L[self.pos]
        assert rec["op"] == op, (self.pos, rec["op"], op)
        self.pos += 1
        return rec

    def peek(self):
        return int(self.L[self.pos]["op"]) if self.pos < len(self.L) else -1

    def w(self, rec, k):
        o, n = int(rec["w"][k]), int(rec["wn"][k])
        return torch.from_numpy(self.W[o:o + n].copy())

    def conv(self):
        r = self.take(OP_CONV)
        ky, kx, ci, co = (int(v) for v in r["i"][:4])
        return ("conv", self.w(r, 0).reshape(co, ci, ky, kx))

    def bnact(self):
        r = self.take(OP_BN)
        s, b = self.w(r, 0), self.w(r, 1)
        a = int(self.take(OP_ACT)["i"][0])
        return ("bn", s, b, a)

    def matmul(self):
        r = self.take(OP_MATMUL)
        return self.w(r, 0).reshape(int(r["i"][0]), int(r["i"][1]))

    def matbias(self):
        return self.w(self.take(OP_MATBIAS), 0)

    def act(self):
        return int(self.take(OP_ACT)["i"][0])

    def trms(self):
        r = self.take(OP_TRMSNORM)
        return (float(r["f"][0]), self.w(r, 0))

    def block(self):
        op = self.peek()
        if op == OP_ORD:
            self.take(op)
            return ("ord", self.bnact(), self.conv(), self.bnact(), self.conv())
        if op == OP_GPOOL:
            self.take(op)
            return ("gpool", self.bnact(), self.conv(), self.conv(), self.bnact(), self.matmul(), self.bnact(), self.conv())
        if op == OP_NBT:
            r = self.take(op)
            pre, pc = self.bnact(), self.conv()
            inner = [self.block() for _ in range(int(r["i"][0]))]
            return ("nbt", pre, pc, inner, self.bnact(), self.conv())
        if op == OP_ATTN:
            r = self.take(op)
            info = tuple(int(v) for v in r["i"][:6])
            freqs = self.w(r, 0) if int(r["wn"][0]) > 0 else None
            theta = float(r["f"][0])
            return ("attn", info, freqs, theta, self.trms(), self.matmul(), self.matmul(), self.matmul(), self.matmul())
        if op == OP_FFN:
            r = self.take(op)
            swiglu = int(r["i"][2])
            norm, l1 = self.trms(), self.matmul()
            gate = self.matmul() if swiglu else None
            return ("ffn", norm, l1, gate, self.matmul())
        raise ValueError(op)


def _conv(x, c):
    w = c[1]
    return F.conv2d(x, w, padding=(w.shape[2] // 2, w.shape[3] // 2))


def _bn(x, b, mask):
    _, s, bias, a = b
    y = act(x * s.view(1, -1, 1, 1) + bias.view(1, -1, 1, 1), a)
    return torch.where(mask == 1.0, y, torch.zeros_like(y))


def _gpool(x, mask, mask_sum):
    s = x.sum(dim=(2, 3))
    mean = s / mask_sum[:, None]
    sq = torch.sqrt(mask_sum)[:, None] - 14.0
    mx = torch.clamp((x + (mask - 1.0)).amax(dim=(2, 3)), min=-1.0)
    return torch.cat([mean, mean * sq * 0.1, mx], dim=1)


def _vpool(x, mask_sum):
    mean = x.sum(dim=(2, 3)) / mask_sum[:, None]
    sq = torch.sqrt(mask_sum)[:, None] - 14.0
    return torch.cat([mean, mean * sq * 0.1, mean * (sq * sq * 0.01 - 0.1)], dim=1)


def _trms(x, norm, mask):
    eps, w = norm
    y = x * torch.rsqrt((x * x).mean(dim=1, keepdim=True) + eps) * w.view(1, -1, 1, 1)
    return torch.where(mask == 1.0, y, torch.zeros_like(y)) * mask


def _rope_tables(info, freqs, theta, H, W):
    heads, kv, dq, dv, use, learn = info
    pairs = dq // 2
    ys, xs = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    ys = ys.reshape(-1).astype(np.float32)
    xs = xs.reshape(-1).astype(np.float32)
    if learn:
        f = freqs.numpy().reshape(kv, pairs, 2).astype(np.float32)
        ang = xs[None, None, :] * f[:, :, 0:1] + ys[None, None, :] * f[:, :, 1:2]
    else:
        half = pairs // 2
        ang = np.zeros((1, pairs, H * W), np.float32)
        for p in range(pairs):
            q = p if p < half else p - half
            freq = 1.0 / np.float32(theta) ** (np.float32(2 * q) / np.float32(dq // 2))
            ang[0, p] = (ys if p < half else xs) * freq
    return torch.from_numpy(np.cos(ang).astype(np.float64)), torch.from_numpy(np.sin(ang).astype(np.float64))


def _rope(t, cos, sin, nheads, kv, learn):
    # t: [N, S, nheads, d]; rotate (2p, 2p+1)
    N, S, h, d = t.shape
    x0 = t[..., 0::2]
    x1 = t[..., 1::2]
    if learn:
        idx = torch.tensor([hh * kv // nheads for hh in range(nheads)])
        c = cos[idx].permute(2, 0, 1)[None]
        s = sin[idx].permute(2, 0, 1)[None]
    else:
        c = cos[0].permute(1, 0)[None, :, None, :]
        s = sin[0].permute(1, 0)[None, :, None, :]
    out = torch.empty_like(t)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def _run_block(b, x, mask, mask_sum):
    kind = b[0]
    if kind == "ord":
        _, pre, c1, mid, c2 = b
        return x + _conv(_bn(_conv(_bn(x, pre, mask), c1), mid, mask), c2)
    if kind == "gpool":
        _, pre, reg, gp, gbn, mul, mid, fin = b
        a = _bn(x, pre, mask)
        r = _conv(a, reg)
        g = _bn(_conv(a, gp), gbn, mask)
        bias = _gpool(g, mask, mask_sum) @ mul
        r = r + bias[:, :, None, None]
        return x + _conv(_bn(r, mid, mask), fin)
    if kind == "nbt":
        _, pre, pc, inner, post, qc = b
        m = _conv(_bn(x, pre, mask), pc)
        for ib in inner:
            m = _run_block(ib, m, mask, mask_sum)
        return x + _conv(_bn(m, post, mask), qc)
    if kind == "attn":
        _, info, freqs, theta, norm, qw, kw, vw, ow = b
        heads, kv, dq, dv, use_rope, learn = info
        N, C, H, W = x.shape
        S = H * W
        xn = _trms(x, norm, mask).permute(0, 2, 3, 1).reshape(N, S, C)
        q = (xn @ qw).reshape(N, S, heads, dq)
        k = (xn @ kw).reshape(N, S, kv, dq)
        v = (xn @ vw).reshape(N, S, kv, dv)
        if use_rope:
            cos, sin = _rope_tables(info, freqs, theta, H, W)
            q = _rope(q, cos, sin, heads, kv, learn)
            k = _rope(k, cos, sin, kv, kv, learn)
        rep = heads // kv
        k = k.repeat_interleave(rep, dim=2)
        v = v.repeat_interleave(rep, dim=2)
        keymask = mask.reshape(N, 1, 1, S) == 1.0
        o = F.scaled_dot_product_attention(q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3),
                                           attn_mask=keymask)
        o = o.permute(0, 2, 1, 3).reshape(N, S, heads * dv)
        o = o * mask.reshape(N, S, 1)
        out = (o @ ow).reshape(N, H, W, C).permute(0, 3, 1, 2)
        return x + out * mask
    if kind == "ffn":
        _, norm, l1, gate, l2 = b
        N, C, H, W = x.shape
        xn = _trms(x, norm, mask).permute(0, 2, 3, 1).reshape(N, H * W, C)
        h = F.silu(xn @ l1) * (xn @ gate)
        out = (h @ l2).reshape(N, H, W, C).permute(0, 3, 1, 2)
        return x + out * mask
    raise ValueError(kind)


def forward(layers, weights, spatial_nhwc, global_in, nn_x, nn_y, policy_optimism=None, output_scale=1.0):
    """Returns raw outputs (times output_scale) like NeuralNet::getOutput with
    symmetry 0: policy [N, HW+1], value [N, 3], score [N, k], ownership [N, HW]."""
    P = Program(layers, weights)
    N = global_in.shape[0]
    H, W = nn_y, nn_x
    x = torch.from_numpy(np.asarray(spatial_nhwc, np.float64).reshape(N, H, W, -1)).permute(0, 3, 1, 2).contiguous()
    g = torch.from_numpy(np.asarray(global_in, np.float64).reshape(N, -1))
    mask = x[:, 0:1]
    mask_sum = mask.sum(dim=(1, 2, 3))

    t = P.take(OP_TRUNK)
    nblocks, trunk_c, norm_kind = (int(v) for v in t["i"][:3])
    stem = P.conv()
    gmul = P.matmul()
    trunk = _conv(x, stem) + (g @ gmul)[:, :, None, None]
    blocks = [P.block() for _ in range(nblocks)]
    for b in blocks:
        trunk = _run_block(b, trunk, mask, mask_sum)
    if norm_kind == 0:
        tip = _bn(trunk, P.bnact(), mask)
    else:
        r = P.take(OP_RMSNORM)
        C, spatial = int(r["i"][0]), int(r["i"][1])
        eps = float(r["f"][0])
        gamma, beta = P.w(r, 0), P.w(r, 1)
        a = P.act()
        if spatial:
            cnt = mask_sum * C
            ss = (trunk * trunk * mask).sum(dim=(1, 2, 3))
            inv = torch.rsqrt(ss / cnt + eps)[:, None, None, None]
        else:
            inv = torch.rsqrt((trunk * trunk).mean(dim=1, keepdim=True) + eps)
        y = trunk * inv * gamma.view(1, -1, 1, 1) + beta.view(1, -1, 1, 1)
        if a == 3:
            y = F.silu(y)
        tip = torch.where(mask == 1.0, y, torch.zeros_like(y))

    ph = P.take(OP_POLICY)
    pc, version = int(ph["i"][0]), int(ph["i"][1])
    p1c, g1c = P.conv(), P.conv()
    g1bn = P.bnact()
    to_bias = P.matmul()
    p1bn = P.bnact()
    p2c = P.conv()
    pass_mul = P.matmul()
    p1 = _conv(tip, p1c)
    g1 = _bn(_conv(tip, g1c), g1bn, mask)
    gp = _gpool(g1, mask, mask_sum)
    p1 = p1 + (gp @ to_bias)[:, :, None, None]
    policy = _conv(_bn(p1, p1bn, mask), p2c)
    if P.peek() == OP_MATBIAS:
        pb = P.matbias()
        pa = P.act()
        pm2 = P.matmul()
        passv = act(gp @ pass_mul + pb, pa) @ pm2
    else:
        passv = gp @ pass_mul

    P.take(OP_VALUE)
    v1c = P.conv()
    v1bn = P.bnact()
    v2m, v2b, v2a = P.matmul(), P.matbias(), P.act()
    v3m, v3b = P.matmul(), P.matbias()
    s3m, s3b = P.matmul(), P.matbias()
    oc = P.conv()
    v1 = _bn(_conv(tip, v1c), v1bn, mask)
    v2 = act(_vpool(v1, mask_sum) @ v2m + v2b, v2a)
    value = v2 @ v3m + v3b
    score = v2 @ s3m + s3b
    own = _conv(v1, oc)

    opt = torch.zeros(N, dtype=torch.float64) if policy_optimism is None else torch.as_tensor(policy_optimism, dtype=torch.float64)
    pol = policy.reshape(N, pc, H * W)
    mix = pc == 2 or (pc == 4 and version >= 16)
    if mix:
        pmain = pol[:, 0] + (pol[:, 1] - pol[:, 0]) * opt[:, None]
        pss = passv[:, 0] + (passv[:, 1] - passv[:, 0]) * opt
    else:
        pmain = pol[:, 0]
        pss = passv[:, 0]
    out_policy = torch.cat([pmain, pss[:, None]], dim=1)
    s = float(output_scale)
    return {"policy": (out_policy * s).numpy(), "value": (value * s).numpy(), "score": (score * s).numpy(),
            "ownership": (own.reshape(N, H * W) * s).numpy()}
