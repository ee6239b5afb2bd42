"""Pure-Python loop restatements for tiny shapes (test infrastructure only).

These pin ``oracle.restatement`` without going through ATen's kernels: plain Python
floats (double precision), explicit index loops written from the mathematics of the
reference's operators. They are meant for N <= 6 and a handful of channels.
"""

from __future__ import annotations

import math


def layer_norm(rows, weight=None, bias=None, eps=1e-5):
    """Row LayerNorm: (x - mean) / sqrt(var + eps) * w + b, biased variance
    (``xfold/fastnn/layer_norm.py:56-59`` = ``F.layer_norm``)."""
    out = []
    for row in rows:
        n = len(row)
        mean = sum(row) / n
        var = sum((x - mean) ** 2 for x in row) / n
        inv = 1.0 / math.sqrt(var + eps)
        normed = [(x - mean) * inv for x in row]
        if weight is not None:
            normed = [y * w for y, w in zip(normed, weight)]
        if bias is not None:
            normed = [y + b for y, b in zip(normed, bias)]
        out.append(normed)
    return out


def _sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def attention(q, k, v, key_valid=None, bias=None):
    """Single (batch, head) attention with the reference's semantics
    (``xfold/fastnn/attention.py:45-66``): logits = (q*d^-0.5).k + bias; a key with
    ``key_valid[j] == False`` gets logit exactly -1e9; softmax over keys; @v.

    q: [Q][D], k: [K][D], v: [K][Dv], bias: [Q][K] or None, key_valid: [K] or None.
    """
    d = len(q[0])
    scale = d ** -0.5
    out = []
    for i, qi in enumerate(q):
        logits = []
        for j, kj in enumerate(k):
            s = sum(qi[t] * scale * kj[t] for t in range(d))
            if bias is not None:
                s += bias[i][j]
            if key_valid is not None and not key_valid[j]:
                s = -1e9
            logits.append(s)
        m = max(logits)
        e = [math.exp(s - m) for s in logits]
        total = sum(e)
        p = [x / total for x in e]
        out.append([sum(p[j] * v[j][c] for j in range(len(k))) for c in range(len(v[0]))])
    return out


def triangle_multiplication(pair, mask, params, outgoing):
    """Triangle multiplication update for a tiny pair tensor.

    pair: [N][N][C] nested lists; mask: [N][N]; params: dict of nested lists with keys
    ``left_w, left_b, proj [2C][C], gate [2C][C], center_w, center_b, out [C][C],
    gating [C][C]`` (nn.Linear layout [out][in]). Follows
    ``xfold/nn/triangle_multiplication.py:71-105``: a_c = channel 2c, b_c = channel 2c+1 of
    mask * proj * sigmoid(gate); outgoing out[c,i,j] = sum_k a[c,i,k] b[c,j,k], incoming
    out[c,i,j] = sum_k a[c,k,j] b[c,k,i]; then LN over c, output projection, gate.
    """
    n = len(pair)
    c = len(pair[0][0])

    def linear(x, w):
        return [sum(w[o][t] * x[t] for t in range(len(x))) for o in range(len(w))]

    normed = [[layer_norm([pair[i][j]], params["left_w"], params["left_b"])[0] for j in range(n)]
              for i in range(n)]
    a = [[[0.0] * n for _ in range(n)] for _ in range(c)]
    b = [[[0.0] * n for _ in range(n)] for _ in range(c)]
    for i in range(n):
        for j in range(n):
            p = linear(normed[i][j], params["proj"])
            g = linear(normed[i][j], params["gate"])
            for ch in range(c):
                a[ch][i][j] = p[2 * ch] * mask[i][j] * _sigmoid(g[2 * ch])
                b[ch][i][j] = p[2 * ch + 1] * mask[i][j] * _sigmoid(g[2 * ch + 1])
    out = [[None] * n for _ in range(n)]
    for i in range(n):
        for j in range(n):
            vec = []
            for ch in range(c):
                if outgoing:
                    vec.append(sum(a[ch][i][t] * b[ch][j][t] for t in range(n)))
                else:
                    vec.append(sum(a[ch][t][j] * b[ch][t][i] for t in range(n)))
            centred = layer_norm([vec], params["center_w"], params["center_b"])[0]
            projected = linear(centred, params["out"])
            gate = linear(normed[i][j], params["gating"])
            out[i][j] = [projected[o] * _sigmoid(gate[o]) for o in range(c)]
    return out


def outer_product_mean(msa, mask, params, eps=1e-3):
    """OuterProductMean (``xfold/nn/primitives.py:40-72``) by loops: per row (s, i), LN then
    left/right = mask[s][i] * (W x); out[i][j][f] = (sum over c, e of (sum over s of
    left[s][i][c] right[s][j][e]) w[c][e][f] + b[f]) / (eps + sum over s of mask[s][i]
    mask[s][j]). msa: [S][N][C]; params: ln_w, ln_b, left [c][C], right [c][C],
    w [c][c][F], b [F]."""
    rows, n = len(msa), len(msa[0])
    cc = len(params["left"])

    def linear(x, w):
        return [sum(w[o][t] * x[t] for t in range(len(x))) for o in range(len(w))]

    left = [[None] * n for _ in range(rows)]
    right = [[None] * n for _ in range(rows)]
    for s in range(rows):
        for i in range(n):
            x = layer_norm([msa[s][i]], params["ln_w"], params["ln_b"])[0]
            left[s][i] = [mask[s][i] * v for v in linear(x, params["left"])]
            right[s][i] = [mask[s][i] * v for v in linear(x, params["right"])]
    f_out = len(params["b"])
    out = [[None] * n for _ in range(n)]
    for i in range(n):
        for j in range(n):
            norm = sum(mask[s][i] * mask[s][j] for s in range(rows))
            vec = []
            for f in range(f_out):
                acc = params["b"][f]
                for c in range(cc):
                    for e in range(cc):
                        outer = sum(left[s][i][c] * right[s][j][e] for s in range(rows))
                        acc += outer * params["w"][c][e][f]
                vec.append(acc / (eps + norm))
            out[i][j] = vec
    return out


def msa_attention(msa, mask, pair, params, heads):
    """MSAAttention (``xfold/nn/attention.py:108-144``) by loops: weights[h][q][k] =
    softmax over k of (W_pair LN(pair[q][k]))[h] + 1e9 (max over s of mask[s][k] - 1);
    out[s][q] = W_out((sum over k of weights[h][q][k] v[s][k][h, :]) * sigmoid(W_gate x))
    with x = LN(msa[s][q]) and v = W_v x. msa: [S][N][C]; pair: [N][N][P]."""
    rows, n, c = len(msa), len(msa[0]), len(msa[0][0])
    dv = c // heads

    def linear(x, w):
        return [sum(w[o][t] * x[t] for t in range(len(x))) for o in range(len(w))]

    key_bias = [1e9 * (max(mask[s][k] for s in range(rows)) - 1.0) for k in range(n)]
    weights = [[None] * n for _ in range(heads)]
    for q in range(n):
        logits = [linear(layer_norm([pair[q][k]], params["pair_ln_w"], params["pair_ln_b"])[0], params["logits"])
                  for k in range(n)]
        for h in range(heads):
            row = [logits[k][h] + key_bias[k] for k in range(n)]
            top = max(row)
            ex = [math.exp(x - top) for x in row]
            total = sum(ex)
            weights[h][q] = [e / total for e in ex]
    out = [[None] * n for _ in range(rows)]
    for s in range(rows):
        xs = [layer_norm([msa[s][k]], params["ln_w"], params["ln_b"])[0] for k in range(n)]
        vs = [linear(xs[k], params["v"]) for k in range(n)]
        for q in range(n):
            avg = [sum(weights[ch // dv][q][k] * vs[k][ch] for k in range(n)) for ch in range(c)]
            gate = linear(xs[q], params["gate"])
            gated = [avg[ch] * _sigmoid(gate[ch]) for ch in range(c)]
            out[s][q] = linear(gated, params["out"])
    return out


def cross_attention(x_q, x_k, mask_q, mask_k, pair_logits, cond_q, cond_k, params, heads):
    """CrossAttention (``xfold/nn/diffusion_transformer.py:275-350``) for one subset by
    loops. x_q: [Q][C], x_k: [K][C], masks [Q] / [K], pair_logits [H][Q][K] or None,
    cond_q [Q][S], cond_k [K][S]. AdaLN(x, c) = sigmoid(W_s LN_w(c) + b_s) * LN(x) + W_b LN_w(c);
    logit = d^-0.5 q.k + 1e9 [both masked] + pair; out = sigmoid(W_z c_q + b_z) * W_t(avg * sigmoid(W_g x_q'))."""
    c = len(x_q[0])
    d = c // heads

    def linear(x, w, b=None):
        return [sum(w[o][t] * x[t] for t in range(len(x))) + (b[o] if b is not None else 0.0)
                for o in range(len(w))]

    def ada(x, cond, pre):
        xn = layer_norm([x])[0]
        cn = layer_norm([cond], params[pre + "cond_ln_w"])[0]
        scale = linear(cn, params[pre + "scale_w"], params[pre + "scale_b"])
        shift = linear(cn, params[pre + "shift_w"])
        return [_sigmoid(scale[i]) * xn[i] + shift[i] for i in range(c)]

    xq = [ada(x_q[i], cond_q[i], "q_") for i in range(len(x_q))]
    xk = [ada(x_k[j], cond_k[j], "k_") for j in range(len(x_k))]
    qs = [linear(x, params["q_w"], params["q_b"]) for x in xq]
    ks = [linear(x, params["k_w"]) for x in xk]
    vs = [linear(x, params["v_w"]) for x in xk]
    out = []
    for i in range(len(x_q)):
        avg = [0.0] * c
        for h in range(heads):
            logits = []
            for j in range(len(x_k)):
                s = sum(qs[i][h * d + t] * d ** -0.5 * ks[j][h * d + t] for t in range(d))
                if mask_q[i] == 0 and mask_k[j] == 0:
                    s += 1e9
                if pair_logits is not None:
                    s += pair_logits[h][i][j]
                logits.append(s)
            top = max(logits)
            ex = [math.exp(s - top) for s in logits]
            total = sum(ex)
            for j in range(len(x_k)):
                for t in range(d):
                    avg[h * d + t] += ex[j] / total * vs[j][h * d + t]
        gate = linear(xq[i], params["gate_w"])
        gated = [avg[ch] * _sigmoid(gate[ch]) for ch in range(c)]
        zero = linear(cond_q[i], params["zero_w"], params["zero_b"])
        upd = linear(gated, params["t2_w"])
        out.append([_sigmoid(zero[ch]) * upd[ch] for ch in range(c)])
    return out
