"""fp64 pure-Python loop restatements for tiny sizes.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function takes plain nested lists / numpy arrays and the module's
parameters (as numpy fp64) and evaluates the upstream formula with explicit
loops over every index.  They exist to pin ``oracle.boltz_ref`` (vectorised,
einsum/matmul/transpose based) at sizes where loops finish in well under a
second; they are not used at benchmark sizes.
"""

from __future__ import annotations

import math

import numpy as np


def _p(module, name):
    t = module
    for part in name.split("."):
        t = getattr(t, part)
    return t.detach().double().numpy()


def layer_norm_vec(v, w=None, b=None, eps=1e-5):
    n = len(v)
    mean = sum(v) / n
    var = sum((x - mean) ** 2 for x in v) / n
    inv = 1.0 / math.sqrt(var + eps)
    out = []
    for c in range(n):
        y = (v[c] - mean) * inv
        if w is not None:
            y *= w[c]
        if b is not None:
            y += b[c]
        out.append(y)
    return out


def linear_vec(v, w, b=None):
    out = []
    for o in range(w.shape[0]):
        acc = 0.0 if b is None else float(b[o])
        for i in range(w.shape[1]):
            acc += w[o, i] * v[i]
        out.append(acc)
    return out


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def silu(x):
    return x * sigmoid(x)


def softmax_list(xs):
    m = max(xs)
    e = [math.exp(x - m) for x in xs]
    s = sum(e)
    return [v / s for v in e]


def triangle_multiplication(module, x, mask, outgoing):
    """x: [N, N, C] fp64 array, mask: [N, N]; returns [N, N, C]."""
    n, _, c = x.shape
    wi, bi = _p(module, "norm_in.weight"), _p(module, "norm_in.bias")
    wo, bo = _p(module, "norm_out.weight"), _p(module, "norm_out.bias")
    p_in, g_in = _p(module, "p_in.weight"), _p(module, "g_in.weight")
    p_out, g_out = _p(module, "p_out.weight"), _p(module, "g_out.weight")
    xn = [[layer_norm_vec(list(x[i, j]), wi, bi, module.norm_in.eps) for j in range(n)] for i in range(n)]
    a = np.zeros((n, n, c))
    b = np.zeros((n, n, c))
    for i in range(n):
        for j in range(n):
            p = linear_vec(xn[i][j], p_in)
            g = linear_vec(xn[i][j], g_in)
            for ch in range(c):
                a[i, j, ch] = p[ch] * sigmoid(g[ch]) * mask[i, j]
                b[i, j, ch] = p[c + ch] * sigmoid(g[c + ch]) * mask[i, j]
    out = np.zeros((n, n, c))
    for i in range(n):
        for j in range(n):
            o = []
            for ch in range(c):
                acc = 0.0
                for k in range(n):
                    if outgoing:
                        acc += a[i, k, ch] * b[j, k, ch]
                    else:
                        acc += a[k, i, ch] * b[k, j, ch]
                o.append(acc)
            on = layer_norm_vec(o, wo, bo, module.norm_out.eps)
            y = linear_vec(on, p_out)
            gate = linear_vec(xn[i][j], g_out)
            for ch in range(c):
                out[i, j, ch] = y[ch] * sigmoid(gate[ch])
    return out


def triangle_attention(module, x, mask, starting):
    """Explicit loops over row i, query q, key k and head h."""
    n, _, c = x.shape
    if not starting:
        x = x.transpose(1, 0, 2)
        mask = mask.T
    h_count, d = module.no_heads, module.c_hidden
    w_ln, b_ln = _p(module, "layer_norm.weight"), _p(module, "layer_norm.bias")
    w_tb = _p(module, "linear.weight")
    wq, wk, wv = (_p(module, f"mha.linear_{t}.weight") for t in "qkv")
    wg, bg = _p(module, "mha.linear_g.weight"), _p(module, "mha.linear_g.bias")
    wo, bo = _p(module, "mha.linear_o.weight"), _p(module, "mha.linear_o.bias")
    xn = [[layer_norm_vec(list(x[i, j]), w_ln, b_ln, module.layer_norm.eps) for j in range(n)] for i in range(n)]
    tb = [[linear_vec(xn[i][j], w_tb) for j in range(n)] for i in range(n)]  # [q][k][h]
    q = [[linear_vec(xn[i][j], wq) for j in range(n)] for i in range(n)]
    k = [[linear_vec(xn[i][j], wk) for j in range(n)] for i in range(n)]
    v = [[linear_vec(xn[i][j], wv) for j in range(n)] for i in range(n)]
    out = np.zeros((n, n, c))
    scale = 1.0 / math.sqrt(d)
    for i in range(n):
        for qi in range(n):
            gate = [sigmoid(t) for t in linear_vec(xn[i][qi], wg, bg)]
            o = [0.0] * (h_count * d)
            for h in range(h_count):
                logits = []
                for kj in range(n):
                    dot = sum(q[i][qi][h * d + e] * k[i][kj][h * d + e] for e in range(d)) * scale
                    logits.append(dot + module.inf * (mask[i, kj] - 1.0) + tb[qi][kj][h])
                probs = softmax_list(logits)
                for e in range(d):
                    o[h * d + e] = sum(probs[kj] * v[i][kj][h * d + e] for kj in range(n)) * gate[h * d + e]
            y = linear_vec(o, wo, bo)
            out[i, qi] = y
    if not starting:
        out = out.transpose(1, 0, 2)
    return out


def transition(module, x):
    """x: [..., C] flattened to rows."""
    rows = x.reshape(-1, x.shape[-1])
    w, b = _p(module, "norm.weight"), _p(module, "norm.bias")
    f1, f2, f3 = _p(module, "fc1.weight"), _p(module, "fc2.weight"), _p(module, "fc3.weight")
    out = []
    for r in rows:
        xn = layer_norm_vec(list(r), w, b, module.norm.eps)
        h1, h2 = linear_vec(xn, f1), linear_vec(xn, f2)
        hid = [silu(u) * t for u, t in zip(h1, h2)]
        out.append(linear_vec(hid, f3))
    return np.array(out).reshape(x.shape[:-1] + (f3.shape[0],))


def adaln(module, a, s):
    ws = _p(module, "s_norm.weight")
    wsc, bsc = _p(module, "s_scale.weight"), _p(module, "s_scale.bias")
    wsb = _p(module, "s_bias.weight")
    ar, sr = a.reshape(-1, a.shape[-1]), s.reshape(-1, s.shape[-1])
    out = []
    for av, sv in zip(ar, sr):
        an = layer_norm_vec(list(av), None, None, module.a_norm.eps)
        sn = layer_norm_vec(list(sv), ws, None, module.s_norm.eps)
        sc = linear_vec(sn, wsc, bsc)
        sb = linear_vec(sn, wsb)
        out.append([sigmoid(sc[c]) * an[c] + sb[c] for c in range(len(an))])
    return np.array(out).reshape(a.shape)


def conditioned_transition(module, a, s):
    ad = adaln(module.adaln, a, s)
    wsw = _p(module, "swish_gate.0.weight")
    wab, wba = _p(module, "a_to_b.weight"), _p(module, "b_to_a.weight")
    wop, bop = _p(module, "output_projection.0.weight"), _p(module, "output_projection.0.bias")
    di = wab.shape[0]
    ar, sr = ad.reshape(-1, ad.shape[-1]), s.reshape(-1, s.shape[-1])
    out = []
    for av, sv in zip(ar, sr):
        u = linear_vec(list(av), wsw)
        t = linear_vec(list(av), wab)
        bvec = [silu(u[di + c]) * u[c] * t[c] for c in range(di)]
        y = linear_vec(bvec, wba)
        g = linear_vec(list(sv), wop, bop)
        out.append([sigmoid(g[c]) * y[c] for c in range(len(y))])
    return np.array(out).reshape(a.shape[:-1] + (wba.shape[0],))


def attention_pair_bias(module, s, z, mask, k_in):
    """Loops for ``AttentionPairBias`` (compute_pair_bias=True), batch 1."""
    s0, k0, z0, m0 = s[0], k_in[0], z[0], mask[0]
    n = s0.shape[0]
    h_count, d = module.num_heads, module.head_dim
    wq, bq = _p(module, "proj_q.weight"), _p(module, "proj_q.bias")
    wk, wv, wg, wo = (_p(module, f"proj_{t}.weight") for t in "kvgo")
    wz_ln, bz_ln = _p(module, "proj_z.0.weight"), _p(module, "proj_z.0.bias")
    wz = _p(module, "proj_z.1.weight")
    q = [linear_vec(list(s0[i]), wq, bq) for i in range(n)]
    k = [linear_vec(list(k0[i]), wk) for i in range(n)]
    v = [linear_vec(list(k0[i]), wv) for i in range(n)]
    g = [[sigmoid(t) for t in linear_vec(list(s0[i]), wg)] for i in range(n)]
    bias = [[linear_vec(layer_norm_vec(list(z0[i, j]), wz_ln, bz_ln, module.proj_z[0].eps), wz)
             for j in range(n)] for i in range(n)]
    out = []
    for i in range(n):
        o = [0.0] * (h_count * d)
        for h in range(h_count):
            logits = []
            for j in range(n):
                dot = sum(q[i][h * d + e] * k[j][h * d + e] for e in range(d)) / math.sqrt(d)
                logits.append(dot + bias[i][j][h] - (1.0 - m0[j]) * module.inf)
            p = softmax_list(logits)
            for e in range(d):
                o[h * d + e] = sum(p[j] * v[j][h * d + e] for j in range(n))
        out.append(linear_vec([g[i][c] * o[c] for c in range(h_count * d)], wo))
    return np.array(out)[None]


def attention_pair_bias_keys(module, s, k_in, bias, mask, multiplicity=1):
    """Loops for ``AttentionPairBias`` with the bias given directly
    (compute_pair_bias=False, as in the diffusion transformers): s [B, Q, D],
    k_in [B, K, D], bias [B / multiplicity, Q, K, H] (the layout before
    proj_z's Rearrange), mask [B, K]; batch element b uses bias
    b // multiplicity (upstream ``repeat_interleave``)."""
    h_count, d = module.num_heads, module.head_dim
    wq, bq = _p(module, "proj_q.weight"), _p(module, "proj_q.bias")
    wk, wv, wg, wo = (_p(module, f"proj_{t}.weight") for t in "kvgo")
    out = np.zeros(s.shape[:2] + (wo.shape[0],))
    for b in range(s.shape[0]):
        nq, nk = s.shape[1], k_in.shape[1]
        q = [linear_vec(list(s[b, i]), wq, bq) for i in range(nq)]
        k = [linear_vec(list(k_in[b, j]), wk) for j in range(nk)]
        v = [linear_vec(list(k_in[b, j]), wv) for j in range(nk)]
        for i in range(nq):
            g = [sigmoid(t) for t in linear_vec(list(s[b, i]), wg)]
            o = [0.0] * (h_count * d)
            for h in range(h_count):
                logits = []
                for j in range(nk):
                    dot = sum(q[i][h * d + e] * k[j][h * d + e] for e in range(d)) / math.sqrt(d)
                    logits.append(dot + bias[b // multiplicity, i, j, h] - (1.0 - mask[b, j]) * module.inf)
                p = softmax_list(logits)
                for e in range(d):
                    o[h * d + e] = sum(p[j] * v[j][h * d + e] for j in range(nk))
            out[b, i] = linear_vec([g[c] * o[c] for c in range(h_count * d)], wo)
    return out
