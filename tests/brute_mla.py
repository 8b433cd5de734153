"""Brute-force scalar-loop restatement of the absorbed MLA layer, for tiny shapes only.

Independent of ``oracle/mla_ref.py`` (no torch ops, no shared helpers): plain Python floats
(IEEE double) and ``math`` functions, written straight from the mathematics of
exhaustive_benchmark_suite.py:210-304.  Used to pin the oracle.
"""

from __future__ import annotations

import math


def rope_angles(pos, rope_dim, base=10000.0):
    return [pos / (base ** ((2 * i) / rope_dim)) for i in range(rope_dim // 2)]


def layer(x, W_q_a, gain, W_q_b, wkv_b, c_kv, pe, positions, H, nope, rope, v,
          eps=1e-6, causal=False, scale=None):
    """All arguments are nested Python lists (fp64 values).  Returns out[b][s][h][d]."""
    B, Sq, hidden = len(x), len(x[0]), len(x[0][0])
    q_lora = len(gain)
    R = len(c_kv[0][0])
    Sk = len(c_kv[0])
    qk = nope + rope
    if scale is None:
        scale = math.sqrt(qk)
    out = [[[[0.0] * v for _ in range(H)] for _ in range(Sq)] for _ in range(B)]
    for b in range(B):
        for s in range(Sq):
            lat = [sum(x[b][s][c] * W_q_a[c][j] for c in range(hidden)) for j in range(q_lora)]
            ms = sum(t * t for t in lat) / q_lora
            inv = 1.0 / math.sqrt(ms + eps)
            lat = [lat[j] * inv * gain[j] for j in range(q_lora)]
            q = [sum(lat[j] * W_q_b[j][n] for j in range(q_lora)) for n in range(H * qk)]
            ang = rope_angles(float(positions[s]), rope)
            for h in range(H):
                qh = q[h * qk:(h + 1) * qk]
                qn, qp = qh[:nope], qh[nope:]
                # RoPE on interleaved pairs
                qr = [0.0] * rope
                for i in range(rope // 2):
                    e, o = qp[2 * i], qp[2 * i + 1]
                    c_, s_ = math.cos(ang[i]), math.sin(ang[i])
                    qr[2 * i] = e * c_ - o * s_
                    qr[2 * i + 1] = e * s_ + o * c_
                # absorption with W_uk = wkv_b[h][:nope]
                qa = [sum(qn[i] * wkv_b[h][i][r] for i in range(nope)) for r in range(R)]
                # scores over visible keys
                lim = Sk - Sq + s if causal else Sk - 1
                sc = []
                for k in range(lim + 1):
                    dot = sum(qa[r] * c_kv[b][k][r] for r in range(R))
                    dot += sum(qr[d] * pe[b][k][d] for d in range(rope))
                    sc.append(dot / scale)
                mx = max(sc)
                ex = [math.exp(t - mx) for t in sc]
                den = sum(ex)
                ctx = [sum(ex[k] / den * c_kv[b][k][r] for k in range(len(ex)))
                       for r in range(R)]
                for d in range(v):
                    out[b][s][h][d] = sum(ctx[r] * wkv_b[h][nope + d][r] for r in range(R))
    return out


def kv_append(x, W_kv_a, gain, positions, R, eps=1e-6):
    """New cache rows for x[b][s]: (c_kv_row [R], pe_row [D]) per (b, s), from the
    mathematics: kv = x W_kv_a; c = kv[:R] / sqrt(mean(kv[:R]^2) + eps) * gain;
    pe pair i of kv[R:] rotated by positions[s] / 10000^(2i/D)."""
    B, Sq, hidden = len(x), len(x[0]), len(x[0][0])
    N = len(W_kv_a[0])
    D = N - R
    rows = {}
    for b in range(B):
        for s in range(Sq):
            kv = [sum(x[b][s][c] * W_kv_a[c][j] for c in range(hidden)) for j in range(N)]
            lat = kv[:R]
            inv = 1.0 / math.sqrt(sum(t * t for t in lat) / R + eps)
            crow = [lat[j] * inv * gain[j] for j in range(R)]
            ang = rope_angles(positions[s], D)
            prow = [0.0] * D
            for i in range(D // 2):
                e, o = kv[R + 2 * i], kv[R + 2 * i + 1]
                prow[2 * i] = e * math.cos(ang[i]) - o * math.sin(ang[i])
                prow[2 * i + 1] = e * math.sin(ang[i]) + o * math.cos(ang[i])
            rows[(b, s)] = (crow, prow)
    return rows


def o_proj(attn, W_o):
    """out[b][s][n] = sum over (h, d) of attn[b][s][h][d] * W_o[h*v + d][n]."""
    B, Sq, H, v = len(attn), len(attn[0]), len(attn[0][0]), len(attn[0][0][0])
    N = len(W_o[0])
    return [[[sum(attn[b][s][h][d] * W_o[h * v + d][n] for h in range(H) for d in range(v))
              for n in range(N)] for s in range(Sq)] for b in range(B)]



def q_rows(x, W_q_a, gain, W_q_b, wkv_b, positions, H, nope, rope, eps=1e-6):
    """The Q path alone, with per-sequence positions: positions[b][s] is query (b, s)'s
    position.  Returns (q_absorbed[b][s][h][r], q_rope[b][s][h][d]) from the mathematics:
    q = RMSNorm(x W_q_a) * gain . W_q_b; q_rope = interleaved-pair rotation of each head's
    rope part; q_absorbed = each head's nope part times W_uk = wkv_b[h][:nope]."""
    B, Sq, hidden = len(x), len(x[0]), len(x[0][0])
    q_lora = len(gain)
    R = len(wkv_b[0][0])
    qk = nope + rope
    qa_all = [[[None] * H for _ in range(Sq)] for _ in range(B)]
    qr_all = [[[None] * H for _ in range(Sq)] for _ in range(B)]
    for b in range(B):
        for s in range(Sq):
            lat = [sum(x[b][s][c] * W_q_a[c][j] for c in range(hidden)) for j in range(q_lora)]
            inv = 1.0 / math.sqrt(sum(t * t for t in lat) / q_lora + eps)
            lat = [lat[j] * inv * gain[j] for j in range(q_lora)]
            q = [sum(lat[j] * W_q_b[j][n] for j in range(q_lora)) for n in range(H * qk)]
            ang = rope_angles(float(positions[b][s]), rope)
            for h in range(H):
                qn, qp = q[h * qk:h * qk + nope], q[h * qk + nope:(h + 1) * qk]
                qr = [0.0] * rope
                for i in range(rope // 2):
                    e, o = qp[2 * i], qp[2 * i + 1]
                    qr[2 * i] = e * math.cos(ang[i]) - o * math.sin(ang[i])
                    qr[2 * i + 1] = e * math.sin(ang[i]) + o * math.cos(ang[i])
                qa_all[b][s][h] = [sum(qn[i] * wkv_b[h][i][r] for i in range(nope))
                                   for r in range(R)]
                qr_all[b][s][h] = qr
    return qa_all, qr_all
