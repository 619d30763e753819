"""Float64 restatement of a mixture of experts with low-rank adapters on every
layer, forward and backward, in numpy.

TEST INFRASTRUCTURE ONLY (the parity oracle): only tests/ import this
module; the product never does.

Follows, step for step in what it computes:
* Layer.Forward with an adapter (perceptron/layer.go:133-162,
  perceptron/adapter.go:66-76): pre = (x W^T + s (x Down^T) Up^T) + b,
  s = alpha / rank, then the activation;
* Layer.Backward with the base frozen (layer.go:164-210, adapter.go:78-99):
  g = out_grad * act'(pre); UpGrad += s g^T u; t = s g Up; DownGrad += t^T x;
  in_grad = g W + t Down (g W row by row is Rows.AddScaledRowTo,
  lowprecision/rows.go:285-324);
* GatedFeedForward.Forward / Backward (feedforward/gatedfeedforward.go:
  49-67), SiLU / ClampedSiLU / ClampedLinear and their derivatives
  (activationfunction/activationfunction.go:102-115,
  moreactivationfunctions.go:207-244);
* MixtureOfExperts.Forward routing and combine (mixtureofexperts.go:122-216)
  and Backward (:227-285), with the affinity derivative of :84-86.
Weights are the decoded float64 values of the compressed rows (Rows.Row), so
sums are numpy's, not the reference's sequential order; the checks here are
to fp32-device tolerance and to finite differences.

Adapters are a dict keyed by (kind, index, which) for the experts' layers
(kind "shared"/"routed", which "gate"/"up"/"down") and ("router", 0, None),
each value a namespace with down (rank x inputs), up (outputs x rank) and
alpha.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np

from oracle import decode_rows, hash_route, route_from_logits


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _gate_act(x, limit):
    if limit > 0:
        x = np.minimum(x, limit)  # ClampedSiLU: silu(limit) above the limit
    return x * _sigmoid(x)


def _gate_deriv(x, limit):
    s = _sigmoid(x)
    d = s + x * s * (1 - s)
    return np.where(x > limit, 0.0, d) if limit > 0 else d


def _up_act(x, limit):
    return np.clip(x, -limit, limit) if limit > 0 else x


def _up_deriv(x, limit):
    if limit > 0:
        return np.where((x > limit) | (x < -limit), 0.0, 1.0)
    return np.ones_like(x)


def _layer_forward(W, b, ad, x):
    """pre = (x W^T + s (x Down^T) Up^T) + b; returns (pre, u)."""
    pre = x @ W.T
    u = None
    if ad is not None:
        u = x @ ad.down.T
        pre = pre + (ad.alpha / ad.down.shape[0]) * (u @ ad.up.T)
    return pre + b, u


def _layer_backward(W, ad, x, u, pre_grad, grads, key):
    """Frozen-base Layer.Backward from the pre-activation gradient."""
    dx = pre_grad @ W
    if ad is not None:
        s = ad.alpha / ad.down.shape[0]
        dA, dB = grads[key]
        dB += s * (pre_grad.T @ u)
        t = s * (pre_grad @ ad.up)
        dA += t.T @ x
        dx = dx + t @ ad.down
    return dx


def _expert_weights(e):
    return {w: (decode_rows(getattr(e, w).weights), np.asarray(getattr(e, w).biases, np.float64))
            for w in ("gate", "up", "down")}


def _expert_forward(e, key, adapters, x, limit):
    W = _expert_weights(e)
    ad = {w: adapters.get(key + (w,)) for w in ("gate", "up", "down")}
    gpre, ug = _layer_forward(*W["gate"], ad["gate"], x)
    upre, uu = _layer_forward(*W["up"], ad["up"], x)
    gout, uout = _gate_act(gpre, limit), _up_act(upre, limit)
    hidden = gout * uout
    out, ud = _layer_forward(*W["down"], ad["down"], hidden)
    return out, SimpleNamespace(W=W, ad=ad, x=x, gpre=gpre, upre=upre, gout=gout, uout=uout, hidden=hidden,
                                u={"gate": ug, "up": uu, "down": ud})


def _expert_backward(st, key, out_grad, grads, limit):
    hg = _layer_backward(st.W["down"][0], st.ad["down"], st.hidden, st.u["down"], out_grad, grads, key + ("down",))
    gg = hg * st.uout * _gate_deriv(st.gpre, limit)
    ug = hg * st.gout * _up_deriv(st.upre, limit)
    dx = _layer_backward(st.W["gate"][0], st.ad["gate"], st.x, st.u["gate"], gg, grads, key + ("gate",))
    return dx + _layer_backward(st.W["up"][0], st.ad["up"], st.x, st.u["up"], ug, grads, key + ("up",))


def _affinity(logits):
    sp = np.where(logits > 20, logits, np.where(logits < -20, np.exp(logits), np.log1p(np.exp(logits))))
    return np.sqrt(sp)


def forward(moe, adapters, x, token_ids=None, chosen=None):
    """MixtureOfExperts.Forward with adapters.  `chosen` (T x k, ascending per
    row) replaces the top-k choice when given (to follow another
    implementation's routing at near-ties); the gates always come from this
    forward's own logits.  Returns (outputs, state for backward)."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    T = x.shape[0]
    E, k = len(moe.routed), moe.experts_per_token
    limit = float(getattr(moe, "clamp_limit", 0.0) or 0.0)
    logits = u_router = None
    if moe.use_hash_routing:
        r = hash_route(token_ids, E, k)
        ch, gates = r.chosen, r.gates
    else:
        Wr = decode_rows(moe.router.weights)
        logits, u_router = _layer_forward(Wr, np.asarray(moe.router.biases, np.float64),
                                          adapters.get(("router", 0, None)), x)
        r = route_from_logits(logits, k, moe.balance_biases)
        ch = r.chosen if chosen is None else np.asarray(chosen, np.int32)
        aff = _affinity(logits)
        a = np.take_along_axis(aff, ch.astype(np.int64), axis=1)
        gates = a / a.sum(axis=1, keepdims=True)
    out = np.zeros((T, moe.vector_size))
    shared_states = []
    for s, e in enumerate(moe.shared):
        y, st = _expert_forward(e, ("shared", s), adapters, x, limit)
        out = out + y
        shared_states.append(st)
    routed_states, rows_for = {}, {}
    expert_out = {}
    for e in range(E):
        rows = [t for t in range(T) if e in ch[t]]
        rows_for[e] = rows
        if rows:
            y, st = _expert_forward(moe.routed[e], ("routed", e), adapters, x[rows], limit)
            routed_states[e] = st
            expert_out[e] = y
    for t in range(T):
        for i in range(k):
            e = int(ch[t, i])
            out[t] += gates[t, i] * expert_out[e][rows_for[e].index(t)]
    state = SimpleNamespace(x=x, chosen=ch, gates=gates, logits=logits, u_router=u_router, shared=shared_states,
                            routed=routed_states, rows_for=rows_for, expert_out=expert_out, limit=limit)
    return out, state


def zero_grads(moe, adapters):
    return {key: [np.zeros_like(ad.down), np.zeros_like(ad.up)] for key, ad in adapters.items()}


def backward(moe, adapters, state, out_grad, grads):
    """MixtureOfExperts.Backward; adds to grads[key] = [DownGrad, UpGrad] and
    returns the input gradients."""
    G = np.atleast_2d(np.asarray(out_grad, np.float64))
    T = G.shape[0]
    dx = np.zeros_like(state.x)
    for s, st in enumerate(state.shared):
        dx = dx + _expert_backward(st, ("shared", s), G, grads, state.limit)
    ch, gates = state.chosen, state.gates
    for e, rows in state.rows_for.items():
        if not rows:
            continue
        eg = np.stack([G[t] * gates[t, list(ch[t]).index(e)] for t in rows])
        dxe = _expert_backward(state.routed[e], ("routed", e), eg, grads, state.limit)
        for i, t in enumerate(rows):
            dx[t] += dxe[i]
    if moe.use_hash_routing:
        return dx
    E = len(moe.routed)
    aff = _affinity(state.logits)
    lg = np.zeros((T, E))
    for t in range(T):
        gg = np.array([G[t] @ state.expert_out[int(e)][state.rows_for[int(e)].index(t)] for e in ch[t]])
        wsum = float(np.sum(gg * gates[t]))
        atot = float(np.sum(aff[t, ch[t]]))
        for i, e in enumerate(ch[t]):
            ag = (gg[i] - wsum) / atot
            lg[t, e] = ag * (_sigmoid(state.logits[t, e]) / (2 * aff[t, e]))
    Wr = decode_rows(moe.router.weights)
    return dx + _layer_backward(Wr, adapters.get(("router", 0, None)), state.x, state.u_router, lg, grads,
                                ("router", 0, None))


def gradient_check(moe, adapters, x, token_ids=None, seed=0, step=1e-6, allowed=1e-5):
    """gradientcheck.Compare (gradientcheck/gradientcheck.go:17-61) on the
    adapters and the inputs: loss = sum(outputs * G) with G uniform in
    [-1, 1); central differences of step 1e-6 must agree with the backward to
    1e-5 * max(1, |numerical|).  Returns the list of problems."""
    rng = np.random.default_rng(seed)
    x = np.array(x, np.float64)
    out, _ = forward(moe, adapters, x, token_ids)
    G = rng.uniform(-1, 1, out.shape)

    def loss():
        return float(np.sum(forward(moe, adapters, x, token_ids)[0] * G))

    grads = zero_grads(moe, adapters)
    _, st = forward(moe, adapters, x, token_ids)
    dx = backward(moe, adapters, st, G, grads)
    problems = []

    def check(name, arr, analytic):
        flat, an = arr.reshape(-1), analytic.reshape(-1)
        for i in range(flat.size):
            orig = flat[i]
            flat[i] = orig + step
            hi = loss()
            flat[i] = orig - step
            lo = loss()
            flat[i] = orig
            num = (hi - lo) / (2 * step)
            if abs(num - an[i]) > allowed * max(1.0, abs(num)):
                problems.append(f"{name}[{i}]: backward gave {an[i]}, finite difference gave {num}")

    for key, ad in adapters.items():
        check(f"{key}.lora.down", ad.down, grads[key][0])
        check(f"{key}.lora.up", ad.up, grads[key][1])
    check("input", x, dx)
    return problems


def make_adapters(moe, rank, alpha, rng, up_scale=0.5):
    """Adapters on every layer as Model.AddLowRankAdapters gives them
    (rank min(rank, inputs, outputs), Down uniform in +-1/sqrt(inputs)), with
    Up uniform in [-up_scale, up_scale) as a trained adapter has it
    (perceptron_test.go:210-216)."""
    d, h, E = moe.vector_size, moe.hidden_size, len(moe.routed)
    ads = {}

    def one(inputs, outputs):
        r = min(rank, inputs, outputs)
        lim = 1 / np.sqrt(inputs)
        return SimpleNamespace(down=rng.uniform(-lim, lim, (r, inputs)),
                               up=rng.uniform(-up_scale, up_scale, (outputs, r)), alpha=alpha)

    for kind, experts in (("shared", moe.shared), ("routed", moe.routed)):
        for i in range(len(experts)):
            ads[(kind, i, "gate")] = one(d, h)
            ads[(kind, i, "up")] = one(d, h)
            ads[(kind, i, "down")] = one(h, d)
    ads[("router", 0, None)] = one(d, E)
    return ads
