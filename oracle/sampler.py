"""Oracle: temperature softmax and chain/tree rejection sampling (fp32).

Reference neighbour: nanovllm/layers/sampler.py:9-11 -- ``logits.float() /
temperature``, ``softmax(dim=-1)``, then a categorical draw.  The reference has no
rejection sampler and cannot take injected uniforms (its draw uses device RNG), so
the contract below is restated from the published algorithms:

* chain: Leviathan et al. 2023, Algorithm 1 (arXiv:2211.17192) -- accept draft
  token x with probability min(1, p(x)/q(x)); on rejection draw from
  norm(max(p - q, 0)); if every draft token is accepted draw a bonus token from p.
* tree: SpecInfer multi-step speculative sampling -- at the current node, test its
  children in ascending node order against the current distribution; each
  rejection replaces it by norm(max(cur - q, 0)); an accepted child becomes the
  current node with distribution P[child].

Exact fp32 contract (shared with the HIP kernel so integer outputs are bit-exact).
At the current node the distribution is tracked in closed form:

* stochastic mode: ``cur[y] = max(p[y] - c*q[y], 0) / Z`` with scalars (c, Z),
  starting at (0, 1).  Rejecting a child replaces cur by norm(max(cur - q, 0)),
  which in exact arithmetic is the same form with ``c <- c + Z`` and
  ``Z <- canonical_sum_y(max(p[y] - c*q[y], 0))`` (products and differences are
  separately rounded fp32 operations).  If the new Z is not > 0 the distribution
  falls back to P[cur] (c, Z = 0, 1).
* delta mode (children are deterministic proposals, q is a point mass on the
  child's token): ``cur[y] = (y in R ? 0 : p[y]) / Z``; rejecting a token x not
  yet in R adds it to R and sets ``Z <- Z - p[x]`` (fp32, starting at 1); if Z
  is not > 0 the distribution falls back to P[cur] (R empty, Z = 1).
* acceptance of child c with token x: ``U[c] * q[x] <= cur[x] and cur[x] > 0``
  (``q[x]`` is 1 in delta mode); a token outside [0, V) is rejected;
* the final token is ``cdf_pick`` of the unnormalised current values with
  U_final (below);
* greedy rows (temperature 0): child accepted iff its token equals the first
  index of the maximum of the row; otherwise the next token is that index.

``canonical_sum`` and ``cdf_pick`` fix the fp32 association order, shared with
the kernel's walk whether it runs one workgroup or several per sequence.  The row,
padded with zeros, is cut into subtiles of 512 elements; 64 logical waves own
contiguous runs of R = ceil(nsub / 64) subtiles (logical wave w: subtiles
[w*R, (w+1)*R)), and lane l of a logical wave holds elements 8l..8l+7 of each of
them.
* lane sum L_l: the lane's values added in order (its subtiles ascending, the 8
  elements of each ascending);
* wave chain: E_l = E_{l-1} + L_l over the 64 lanes in order (E_{-1} = 0); the wave
  total is T_w = E_63;
* row chain: W_0 = 0, W_{w+1} = W_w + T_w over the 64 logical waves; the sum is W_64.
The inverse CDF runs over the elements in that order (logical waves, then lanes,
then the lane's elements): lane l of wave w ends at W_w + E_l and starts at
W_w + E_{l-1} (W_w for l = 0).  The pick with uniform u: tau = u * sum; the chosen
lane is the first whose end exceeds tau (it always holds mass: a lane with L_l = 0
ends where the previous one does); inside it F(y) = start + the lane's values up to
y, added in order, and the pick is the first y with F(y) > tau and v(y) > 0, else
the lane's last y with v(y) > 0.  When no lane ends above tau (u * sum rounds to the
sum) the largest y with v(y) > 0 is picked (-1 for an all-zero row).  Any fixed
order of the elements gives an exact inverse-CDF sampler; this one needs no
cross-lane traffic while a row streams, and splits into 1, 2, 4, 8 or 16 workgroups
per sequence (16 waves each up to 4 workgroups, then 64 / workgroups; each real wave
holds 64 / (workgroups x waves) logical waves) without changing a bit.  The pick works on the unnormalised
residual max(p - c*q, 0) (stochastic) or p with rejected tokens zeroed (delta): the
kernel picks from the lane sums of the pass that computed the last normaliser.

Pinned by (tests/test_oracle_sampler.py): Q=P always accepts; disjoint supports
always reject; the output distribution enumerated over uniform grids on tiny
vocabularies equals P; chain sampling agrees in distribution with transformers'
``_speculative_sampling`` (generation/utils.py:3992); canonical_sum agrees with
math.fsum; cdf_pick agrees with a float64 searchsorted away from CDF steps;
committed golden fixtures under tests/golden/.
"""
import numpy as np

WAVE = 64
NWAVES = 64        # logical waves of the canonical order
F32 = np.float32


# --------------------------------------------------------------------------- softmax
def temperature_softmax(logits, temperatures):
    """softmax(logits.float() / T) per row (reference sampler.py:9-10).

    Rows with temperature 0 (greedy) return the fp32 logits unchanged: only their
    argmax is used.  Computed in float64 and rounded, so it is the correctly
    rounded target the fp32 kernel is compared against (1e-5 relative).
    """
    x32 = np.asarray(logits, dtype=F32)
    t32 = np.asarray(temperatures, dtype=F32).reshape(-1, 1)
    greedy = t32[:, 0] == 0
    # logits.float().div_(T) is one correctly rounded fp32 division (sampler.py:9);
    # exp and the normalisation are then done in float64.
    xs = (x32 / np.where(greedy[:, None], F32(1), t32)).astype(np.float64)
    m = xs.max(axis=1, keepdims=True)
    e = np.exp(xs - m)
    p = e / e.sum(axis=1, keepdims=True)
    out = p.astype(F32)
    out[greedy] = x32[greedy]
    return out


# ------------------------------------------------------------ canonical reductions
SUB = 512          # elements per subtile (64 lanes x 8)
LANE_ELEMS = 8


def _cdiv(a, b):
    return -(-a // b)


def _lane_major(row):
    """Row padded with zeros and laid out in the canonical order:
    [64 logical waves, 64 lanes, R*8 values] fp32 (R subtiles of 512 per wave)."""
    row = np.asarray(row, dtype=F32)
    nsub = max(1, _cdiv(row.shape[0], SUB))
    R = _cdiv(nsub, NWAVES)
    pad = np.zeros(NWAVES * R * SUB, dtype=F32)
    pad[:row.shape[0]] = row
    X = pad.reshape(NWAVES, R, WAVE, LANE_ELEMS).transpose(0, 2, 1, 3)
    return X.reshape(NWAVES, WAVE, R * LANE_ELEMS)


def _index_layout(V):
    nsub = max(1, _cdiv(V, SUB))
    R = _cdiv(nsub, NWAVES)
    idx = np.arange(NWAVES * R * SUB).reshape(NWAVES, R, WAVE, LANE_ELEMS).transpose(0, 2, 1, 3)
    return idx.reshape(NWAVES, WAVE, R * LANE_ELEMS)


def _chains(X):
    """Lane sums, wave chains and row chain: (lane ends E [64, 64], W [65]).
    Every sum is sequential fp32 (add.accumulate adds in order, unlike np.sum)."""
    L = np.add.accumulate(X, axis=2, dtype=F32)[:, :, -1]
    E = np.add.accumulate(L, axis=1, dtype=F32)
    W = np.zeros(NWAVES + 1, dtype=F32)
    W[1:] = np.add.accumulate(E[:, -1], dtype=F32)
    return E, W


def canonical_order(V):
    """Element indices in the order the inverse CDF runs over them (padding dropped)."""
    idx = _index_layout(V).reshape(-1)
    return idx[idx < V]


def canonical_sum(row):
    return _chains(_lane_major(row))[1][-1]


def cdf_pick(row, u):
    """Inverse-CDF pick in the canonical order (module docstring); row holds the
    unnormalised non-negative values v(y)."""
    row = np.asarray(row, dtype=F32)
    X = _lane_major(row)
    E, W = _chains(X)
    total = W[-1]
    tau = F32(F32(u) * total)
    ends = (W[:-1, None] + E).astype(F32)       # [64 waves, 64 lanes]
    hits = np.argwhere(ends > tau)
    if hits.size == 0:
        pos = np.nonzero(row > 0)[0]
        return int(pos[-1]) if pos.size else -1
    w, lane = (int(t) for t in hits[0])        # first in (wave, lane) order
    start = F32(W[w] + E[w, lane - 1]) if lane > 0 else W[w]
    v = X[w, lane]
    F = np.add.accumulate(np.concatenate([[start], v]).astype(F32), dtype=F32)[1:]
    ys = _index_layout(row.shape[0])[w, lane]
    hit = np.nonzero((F > tau) & (v > 0))[0]
    if hit.size:
        return int(ys[hit[0]])
    pos = np.nonzero(v > 0)[0]
    return int(ys[pos[-1]]) if pos.size else -1


def first_argmax(row):
    return int(np.argmax(np.asarray(row, dtype=F32)))


# ------------------------------------------------------------------- tree sampling
class _Residual:
    """Current distribution at a node, in the closed form of the contract above."""

    def __init__(self, p, q, delta):
        self.p, self.q, self.delta = p, q, delta
        self.c, self.Z = F32(0), F32(1)
        self.R = []

    def residual(self, ys=None):
        """Unnormalised current values: max(p - c*q, 0) or p with R zeroed."""
        p = self.p if ys is None else self.p[ys]
        if self.delta:
            yy = np.arange(self.p.shape[0]) if ys is None else np.asarray(ys)
            out = np.where(np.isin(yy, self.R), F32(0), p)
        else:
            q = self.q if ys is None else self.q[ys]
            out = np.maximum(p - self.c * q, F32(0))
        return out.astype(F32)

    def eval(self, ys=None):
        return (self.residual(ys) / self.Z).astype(F32)

    def reject(self, x):
        V = self.p.shape[0]
        if self.delta:
            if 0 <= x < V and x not in self.R:
                self.R.append(x)
                self.Z = F32(self.Z - self.p[x])
            if not self.Z > 0:
                self.R, self.Z = [], F32(1)
        else:
            c = F32(self.c + self.Z)
            Z = canonical_sum(np.maximum(self.p - c * self.q, F32(0)))
            if Z > 0:
                self.c, self.Z = c, Z
            else:
                self.c, self.Z = F32(0), F32(1)


def sample_tree_one(P, Q, tokens, parents, U, u_final, greedy, delta=False):
    """One sequence.  P: [T, V] fp32 target rows, Q: [T, V] fp32 draft rows (ignored
    in delta and greedy modes), tokens/parents/U: [T].  Returns
    (path list of node ids starting at 0, next token)."""
    T = len(parents)
    children = [[] for _ in range(T)]
    for j in range(1, T):
        children[int(parents[j])].append(j)
    cur, path = 0, [0]
    while True:
        kids = children[cur]
        if greedy:
            a = first_argmax(P[cur])
            nxt = next((c for c in kids if int(tokens[c]) == a), None)
            if nxt is None:
                return path, a
            cur = nxt
            path.append(cur)
            continue
        p = np.asarray(P[cur], dtype=F32)
        q = None if delta else np.asarray(Q[cur], dtype=F32)
        chain = _Residual(p, q, delta)
        accepted = None
        V = p.shape[0]
        for c in kids:
            x = int(tokens[c])
            if 0 <= x < V:  # a token outside the vocabulary is rejected
                cx = chain.eval(np.array([x]))[0]
                qx = F32(1) if delta else q[x]
                if F32(F32(U[c]) * qx) <= cx and cx > 0:
                    accepted = c
                    break
            chain.reject(x)
        if accepted is None:
            return path, cdf_pick(chain.residual(), u_final)
        cur = accepted
        path.append(cur)


def rejection_sample_tree(P, Q, tokens, parents, U, U_final, greedy, num_nodes=None,
                          delta=False):
    """Batched oracle.  P, Q: [B, T, V]; tokens, parents, U: [B, T]; U_final, greedy: [B].

    Returns (path [B, T] int32 padded -1, accepted_len [B], out_tokens [B, T] int32
    (accepted tokens then the next token, padded -1), next_token [B])."""
    P = np.asarray(P, dtype=F32)
    B, T = np.asarray(parents).shape
    path_o = np.full((B, T), -1, np.int32)
    acc_o = np.zeros(B, np.int32)
    tok_o = np.full((B, T), -1, np.int32)
    nxt_o = np.zeros(B, np.int32)
    for b in range(B):
        n = T if num_nodes is None else int(num_nodes[b])
        path, nxt = sample_tree_one(P[b, :n], None if Q is None else Q[b, :n],
                                    tokens[b, :n], parents[b, :n], U[b, :n], U_final[b],
                                    bool(greedy[b]), delta)
        path_o[b, :len(path)] = path
        acc_o[b] = len(path) - 1
        toks = [int(tokens[b, i]) for i in path[1:]] + [nxt]
        tok_o[b, :len(toks)] = toks
        nxt_o[b] = nxt
    return path_o, acc_o, tok_o, nxt_o


def rejection_sample_chain(P, Q, draft_tokens, U, U_final, greedy):
    """Chain special case (parents[i] = i-1).  P: [B, k+1, V], Q: [B, k, V],
    draft_tokens / U: [B, k].  Returns (accepted_len [B], recovered [B] (-1 if every
    draft token was accepted), bonus [B] (-1 otherwise), tokens [B, k+1])."""
    P = np.asarray(P, dtype=F32)
    B, k1, V = P.shape
    k = k1 - 1
    Qp = np.zeros((B, k1, V), F32)
    Qp[:, :k] = Q
    tok = np.zeros((B, k1), np.int32)
    tok[:, 1:] = draft_tokens
    Up = np.zeros((B, k1), F32)
    Up[:, 1:] = U
    parents = np.tile(np.arange(-1, k, dtype=np.int32), (B, 1))
    _, acc, toks, nxt = rejection_sample_tree(P, Qp, tok, parents, Up, U_final, greedy)
    recovered = np.where(acc < k, nxt, -1).astype(np.int32)
    bonus = np.where(acc == k, nxt, -1).astype(np.int32)
    return acc, recovered, bonus, toks
