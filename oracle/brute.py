"""Pure-Python loop restatements for tiny inputs, used to pin the vectorised
oracle (no numpy linear algebra, no vectorised masking)."""
import math


def attention(q, k, v, scale, causal):
    """q[b][i][h][r], k[b][n][hk][r], v[b][n][hk][rv] nested lists -> out, lse."""
    B, Q, H = len(q), len(q[0]), len(q[0][0])
    N, Hk = len(k[0]), len(k[0][0])
    g = H // Hk
    out = [[[None] * H for _ in range(Q)] for _ in range(B)]
    lse = [[[None] * Q for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for i in range(Q):
            for h in range(H):
                kv = h // g
                visible = [n for n in range(N) if not causal or n <= i + N - Q]
                scores = [scale * sum(a * c for a, c in zip(q[b][i][h], k[b][n][kv])) for n in visible]
                if not scores:
                    out[b][i][h] = [0.0] * len(v[0][0][0])
                    lse[b][h][i] = -math.inf
                    continue
                m = max(scores)
                z = sum(math.exp(s - m) for s in scores)
                lse[b][h][i] = m + math.log(z)
                weights = [math.exp(s - m) / z for s in scores]
                width = len(v[0][0][0])
                out[b][i][h] = [sum(w * v[b][n][kv][c] for w, n in zip(weights, visible)) for c in range(width)]
    return out, lse
