"""Writes the golden fixtures of tests/test_oracle.py with the Python standard library only (no torch, no numpy).

Every value is evaluated with scalar loops straight from the definitions, independently of the oracle's tensor code:

attn_tiny.json   SISA attention on B=1, H=2, L=6, d_head=4, d_state=2 (README.md:33-72 of tlstngud/sisa):
                   s_tj = q_t.k_j / sqrt(d_head) + lam_h exp(g_t - g_j) (c_t.b_j) + (F_t - F_j),  j <= t
                   o_t  = sum_j softmax_j(s_t.) v_j
                 the objective sum(o * do) and its gradient w.r.t. every input by central finite differences
                 (step 1e-6, error ~1e-9); head 0 has lam = 0.7, head 1 lam = 0 and a zero forget gate.
glue_tiny.json   the layer glue on B=1, L=5, H=2 (src/sisa/modeling.py:185-197):
                   g = cumsum(-softplus(a)), F = cumsum(log sigmoid(z)), Phi = cumsum(theta),
                   c~ = pairwise rotation of c by Phi (z_{2i}, z_{2i+1}) -> (z_{2i} cos - z_{2i+1} sin,
                   z_{2i} sin + z_{2i+1} cos), and rowf / colf over 2-row blocks.
lmce_tiny.json   linear cross-entropy on N=5, D=3, V=7 with one ignored row (src/sisa/kernels/linear_ce.py:3-6):
                 mean loss over the valid rows, dL/dx and dL/dW from the closed form (softmax - onehot) / N_valid.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import os
import random

HERE = os.path.dirname(os.path.abspath(__file__))


def _mat(rng, r, c, scale=1.0):
    return [[rng.gauss(0.0, scale) for _ in range(c)] for _ in range(r)]


# ------------------------------------------------------------------------------------------------ attention
def attn_head(q, k, v, c, b, g, F, lam):
    L, D = len(q), len(q[0])
    sc = 1.0 / math.sqrt(D)
    out = []
    for t in range(L):
        s = []
        for j in range(t + 1):
            qk = sum(q[t][d] * k[j][d] for d in range(D)) * sc
            cb = sum(c[t][e] * b[j][e] for e in range(len(c[0])))
            s.append(qk + lam * math.exp(g[t] - g[j]) * cb + (F[t] - F[j]))
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        out.append([sum(e[j] / z * v[j][d] for j in range(t + 1)) for d in range(len(v[0]))])
    return out


def attn_objective(X, do):
    tot = 0.0
    for h in range(len(X["q"])):
        o = attn_head(X["q"][h], X["k"][h], X["v"][h], X["c"][h], X["b"][h], X["g"][h], X["F"][h], X["lam"][h])
        tot += sum(o[t][d] * do[h][t][d] for t in range(len(o)) for d in range(len(o[0])))
    return tot


def _leaves(X):
    """(name, path) of every scalar input."""
    for name in ("q", "k", "v", "c", "b"):
        for h, M in enumerate(X[name]):
            for t, row in enumerate(M):
                for d in range(len(row)):
                    yield name, (h, t, d)
    for name in ("g", "F"):
        for h, row in enumerate(X[name]):
            for t in range(len(row)):
                yield name, (h, t)
    for h in range(len(X["lam"])):
        yield "lam", (h,)


def _get(X, name, path):
    x = X[name]
    for i in path[:-1]:
        x = x[i]
    return x, path[-1]


def make_attn():
    rng = random.Random(20251201)
    H, L, D, S = 2, 6, 4, 2
    X = {n: [_mat(rng, L, D) for _ in range(H)] for n in ("q", "k", "v")}
    X["c"] = [_mat(rng, L, S, 0.8) for _ in range(H)]
    X["b"] = [_mat(rng, L, S, 0.8) for _ in range(H)]
    g, F = [], []
    for h in range(H):
        acc, gr = 0.0, []
        for _ in range(L):
            acc -= math.log1p(math.exp(rng.gauss(-1.0, 0.7)))
            gr.append(acc)
        g.append(gr)
        acc, fr = 0.0, []
        for _ in range(L):
            zz = rng.gauss(1.0, 1.0)
            acc += -math.log1p(math.exp(-zz)) if h == 0 else 0.0
            fr.append(acc)
        F.append(fr)
    X["g"], X["F"] = g, F
    X["lam"] = [0.7, 0.0]
    do = [_mat(rng, L, D) for _ in range(H)]
    o = [attn_head(X["q"][h], X["k"][h], X["v"][h], X["c"][h], X["b"][h], X["g"][h], X["F"][h], X["lam"][h])
         for h in range(H)]
    grads = {n: json.loads(json.dumps(X[n])) for n in X}
    step = 1e-6
    for name, path in _leaves(X):
        cont, i = _get(X, name, path)
        x0 = cont[i]
        cont[i] = x0 + step
        fp = attn_objective(X, do)
        cont[i] = x0 - step
        fm = attn_objective(X, do)
        cont[i] = x0
        gc, gi = _get(grads, name, path)
        gc[gi] = (fp - fm) / (2 * step)
    return {"inputs": X, "do": do, "o": o, "grads": grads,
            "note": "heads (H, L, .); gradients of sum(o * do) by central differences, step 1e-6"}


# ------------------------------------------------------------------------------------------------ glue
def make_glue():
    rng = random.Random(7)
    L, H, S, T = 5, 2, 4, 2
    a = [[rng.gauss(-2.0, 1.5) for _ in range(H)] for _ in range(L)]
    a[1][0] = 25.0                                       # above the softplus threshold (20): softplus(a) = a
    z = [[rng.gauss(1.0, 2.0) for _ in range(H)] for _ in range(L)]
    z[2][1] = -30.0
    theta = [[[rng.gauss(0.1, 0.3) for _ in range(S // 2)] for _ in range(H)] for _ in range(L)]
    cvec = [[[rng.gauss(0.0, 1.0) for _ in range(S)] for _ in range(H)] for _ in range(L)]

    def softplus(x):
        return x if x > 20.0 else math.log1p(math.exp(x))

    def logsigmoid(x):
        return min(x, 0.0) - math.log1p(math.exp(-abs(x)))
    g = [[0.0] * L for _ in range(H)]
    Fg = [[0.0] * L for _ in range(H)]
    phi = [[[0.0] * (S // 2) for _ in range(L)] for _ in range(H)]
    crot = [[[0.0] * S for _ in range(L)] for _ in range(H)]
    for h in range(H):
        ga = fa = 0.0
        pa = [0.0] * (S // 2)
        for t in range(L):
            ga -= softplus(a[t][h])
            fa += logsigmoid(z[t][h])
            g[h][t], Fg[h][t] = ga, fa
            for i in range(S // 2):
                pa[i] += theta[t][h][i]
                phi[h][t][i] = pa[i]
                ce, co = cvec[t][h][2 * i], cvec[t][h][2 * i + 1]
                cs, sn = math.cos(pa[i]), math.sin(pa[i])
                crot[h][t][2 * i] = ce * cs - co * sn
                crot[h][t][2 * i + 1] = ce * sn + co * cs
    rowf = [[0.0] * L for _ in range(H)]
    colf = [[0.0] * L for _ in range(H)]
    for h in range(H):
        for t in range(L):
            st = (t // T) * T
            en = min(st + T - 1, L - 1)
            rowf[h][t] = math.exp(min(g[h][t] - g[h][st], 0.0))
            colf[h][t] = math.exp(min(g[h][en] - g[h][t], 0.0))
    return {"inputs": {"a": a, "z": z, "theta": theta, "c": cvec, "T": T},
            "g": g, "F": Fg, "Phi": phi, "c_rot": crot, "rowf": rowf, "colf": colf,
            "note": "a, z (L, H); theta (L, H, S/2); c (L, H, S); outputs (H, L, .)"}


# ------------------------------------------------------------------------------------------------ linear CE
def make_lmce():
    rng = random.Random(11)
    N, D, V, ign = 5, 3, 7, -100
    x = _mat(rng, N, D)
    W = _mat(rng, V, D, 0.8)
    y = [rng.randrange(V) for _ in range(N)]
    y[2] = ign
    logits = [[sum(x[n][d] * W[v][d] for d in range(D)) for v in range(V)] for n in range(N)]
    valid = [yy != ign for yy in y]
    nv = sum(valid)
    loss = 0.0
    G = [[0.0] * V for _ in range(N)]
    for n in range(N):
        if not valid[n]:
            continue
        m = max(logits[n])
        lse = m + math.log(sum(math.exp(l - m) for l in logits[n]))
        loss += lse - logits[n][y[n]]
        for v in range(V):
            G[n][v] = (math.exp(logits[n][v] - lse) - (1.0 if v == y[n] else 0.0)) / nv
    dx = [[sum(G[n][v] * W[v][d] for v in range(V)) for d in range(D)] for n in range(N)]
    dW = [[sum(G[n][v] * x[n][d] for n in range(N)) for d in range(D)] for v in range(V)]
    return {"inputs": {"x": x, "W": W, "labels": y, "ignore_index": ign}, "loss": loss / nv, "dx": dx, "dW": dW}


def main():
    for name, fn in (("attn_tiny.json", make_attn), ("glue_tiny.json", make_glue), ("lmce_tiny.json", make_lmce)):
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(fn(), f, indent=None, separators=(",", ":"))
            f.write("\n")
        print("wrote", name)


if __name__ == "__main__":
    main()
