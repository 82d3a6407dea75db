"""A float64 torch statement of the training step's forward (the reference's Ava-0.4 block, written for
autograd), so that autograd gives the reference gradients the GPU step is compared with.

The pieces follow the reference's formulas, the same ones oracle/forward64.py states in numpy (and
tests/test_oracle_forward64.py pins against the f32 oracle):
  - spiking: cur = rms(x, lif_norm) Win (1 - sigmoid(beta_p)); the LIF with lif_ref's straight-through
    spikes, soft + (hard - soft).detach() (gpu/arch.rs:964-1071), the hard spikes FORCED from a trace
    so that both sides take the same decisions; theta detached; x += s Wout;
  - memory: unit q, k, e = unit(k + h We), value residual, log alpha = logsigmoid(h Wa + ba + off +
    (h Wa1) Wa2), b = 2 sigmoid(h Wb + bb + (h Wb1) Wb2), delta_rec with the bound (gpu/arch.rs:1091-1136),
    head_norm(y) silu(h Wg) Wo;
  - engram: causal softmax attention per head (gpu/memory.rs:610-700);
  - MLP: relu(u mask)^2 W2 with the kWTA mask FORCED; the dense mix; the final norm and the tied head;
  - loss: the mean cross-entropy over the targets in [0, V).
"""
import numpy as np
import torch

from test_oracle_backward import delta_rec_t

f64 = torch.float64
BLOCK_KEYS = ["lif_norm", "win", "beta_p", "theta", "arho", "again", "wout", "mem_norm", "wq", "wk", "wv", "we",
              "wg", "wo", "wa", "ba", "wb", "bb", "off", "wa1", "wa2", "wb1", "wb2", "vres", "eng_norm", "ewq",
              "ewk", "ewv", "ewo", "mlp_norm", "w1", "w2", "dense"]


def leaves(params):
    """float64 torch leaves of a parameter dict of numpy arrays; every one is trained (requires_grad)
    except the gate offsets, constants of the fixed timescales (gpu/arch.rs:656-666)."""
    t = lambda a, g=True: torch.tensor(np.asarray(a, np.float64), requires_grad=g)
    out = {"tok_emb": t(params["tok_emb"]), "final_norm": t(params["final_norm"]), "blocks": []}
    for b in params["blocks"]:
        out["blocks"].append({k: t(v, k != "off") for k, v in b.items() if k in BLOCK_KEYS and v is not None})
    return out


def _rms(x, g):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5) * g


def _unit(x, hs):
    sh = x.shape
    z = x.reshape(sh[:-1] + (sh[-1] // hs, hs))
    return (z / torch.sqrt((z * z).sum(-1, keepdim=True) + 1e-6)).reshape(sh)


def _head_norm(y, hs):
    sh = y.shape
    z = y.reshape(sh[:-1] + (sh[-1] // hs, hs))
    return (z / torch.sqrt((z * z).mean(-1, keepdim=True) + 1e-5)).reshape(sh)


def _lif_forced(cur, beta, theta, rho, gain, forced, levels, alif, slope):
    """lif_ref (gpu/arch.rs:964-1071) from a zero state, no reset gradient, the hard spikes forced.
    cur [B, T, D]; forced [B, T, D]. Returns the spikes [B, T, D] (value = forced, gradient = soft's)."""
    B, T, D = cur.shape
    th = theta.detach()
    v = torch.zeros(B, D, dtype=f64)
    sp = torch.zeros(B, D, dtype=f64)
    a = torch.zeros(B, D, dtype=f64)
    th_prev = th.expand(B, D) + a * gain if alif else th.expand(B, D)

    def soft(u):
        return u / (u.abs() * slope + 1.0)

    outs = []
    for t in range(T):
        if alif:
            a = a * rho + sp.abs().detach() * (1.0 - rho)
            th_t = th + a * gain
        else:
            th_t = th.expand(B, D)
        v = v * beta + cur[:, t] - (sp * th_prev).detach()
        sf = 0.0
        for k in range(1, levels + 1):
            sf = sf + (soft(v - th_t * k) - soft(-v - th_t * k))
        s = sf + (forced[:, t] - sf).detach()
        outs.append(s)
        sp = s.detach()
        th_prev = th_t
    return torch.stack(outs, 1)


def forward_t(cfg, P, ids, targets, spikes, keep, slope=4.0):
    """The loss (and logits) of ids, targets [B, T] (numpy int) under the forced decisions spikes
    [L, B*T, d] and keep [L, B*T, H] (numpy), every value float64 and differentiable in P (leaves())."""
    B, T = ids.shape
    N = B * T
    L, d, H, hs = cfg["layers"], cfg["d"], cfg["hidden"], cfg["head_size"]
    nh = d // hs
    M, cap = float(cfg["momentum"]), float(cfg["cap"])
    E = P["tok_emb"]
    x = E[torch.as_tensor(ids.reshape(-1), dtype=torch.long)]
    streams = [x]
    vfirst = None
    for i in range(L):
        b = P["blocks"][i]
        beta = torch.sigmoid(b["beta_p"])
        cur = _rms(x, b["lif_norm"]) @ b["win"]
        if cfg["lif_scale"]:
            cur = cur * (1.0 - beta)
        forced = torch.as_tensor(np.asarray(spikes[i], np.float64)).reshape(B, T, d)
        s = _lif_forced(cur.reshape(B, T, d), beta, b["theta"], torch.sigmoid(b["arho"]), b["again"], forced,
                        cfg["levels"], cfg["alif"], slope).reshape(N, d)
        x = x + s @ b["wout"]
        h = _rms(x, b["mem_norm"])
        q = _unit(h @ b["wq"], hs)
        kr = h @ b["wk"]
        k = _unit(kr, hs)
        v = h @ b["wv"]
        if cfg["value_residual"]:
            if i == 0:
                vfirst = v
            else:
                v = v * (1.0 + b["vres"][0]) + vfirst * b["vres"][1]
        e = _unit(kr + h @ b["we"], hs)
        g = h @ b["wg"]
        za = (h @ b["wa"] + b["ba"]).repeat_interleave(hs, dim=1) + b["off"] + (h @ b["wa1"]) @ b["wa2"]
        zb = (h @ b["wb"] + b["bb"]).repeat_interleave(hs, dim=1) + (h @ b["wb1"]) @ b["wb2"]
        la = torch.nn.functional.logsigmoid(za)
        bw = 2.0 * torch.sigmoid(zb)

        def heads(z):
            return z.reshape(B, T, nh, hs).permute(0, 2, 1, 3).reshape(B * nh, T, hs)

        zero = torch.zeros(B * nh, hs, hs, dtype=f64)
        y, _, _ = delta_rec_t(heads(q), heads(k), heads(e), heads(v), heads(la), heads(bw), M, cap, zero, zero)
        y = y.reshape(B, nh, T, hs).permute(0, 2, 1, 3).reshape(N, d)
        x = x + (_head_norm(y, hs) * (g * torch.sigmoid(g))) @ b["wo"]
        if i == cfg["eng_block"]:
            he = _rms(x, b["eng_norm"])
            eq, ek, ev = he @ b["ewq"], he @ b["ewk"], he @ b["ewv"]
            de = cfg["eng_dim"]
            enh = max(1, int(cfg.get("eng_heads", 1) or 1))
            hd = de // enh
            causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
            rows = []
            for r in range(B):
                sl = slice(r * T, (r + 1) * T)
                hs_ = []
                for hh in range(enh):
                    c = slice(hh * hd, (hh + 1) * hd)
                    sc = eq[sl, c] @ ek[sl, c].T / np.sqrt(hd)
                    sc = sc.masked_fill(~causal, float("-inf"))
                    hs_.append(torch.softmax(sc, dim=1) @ ev[sl, c])
                rows.append(torch.cat(hs_, dim=1))
            x = x + torch.cat(rows, dim=0) @ b["ewo"]
        u = _rms(x, b["mlp_norm"]) @ b["w1"]
        kp = torch.as_tensor(np.asarray(keep[i], np.float64)).reshape(N, H)
        act = torch.relu(u * kp)
        act = act * act
        x = x + act @ b["w2"]
        if cfg["dense"]:
            streams.append(x)
            mixed = x
            for j, sj in enumerate(streams):
                mixed = mixed + b["dense"][j] * sj
            x = mixed
    logits = _rms(x, P["final_norm"]) @ E.T
    tg = torch.as_tensor(np.asarray(targets).reshape(-1), dtype=torch.long)
    ok = (tg >= 0) & (tg < cfg["vocab"])
    lp = torch.log_softmax(logits, dim=1)
    loss = -(lp[ok.nonzero().squeeze(1), tg[ok]]).sum() / max(int(ok.sum()), 1)
    return loss, logits


def grads_t(cfg, params, ids, targets, spikes, keep, slope=4.0):
    """(loss, logits, gradient dict of numpy arrays keyed as params) by autograd."""
    P = leaves(params)
    loss, logits = forward_t(cfg, P, ids, targets, spikes, keep, slope)
    loss.backward()
    g = {"tok_emb": P["tok_emb"].grad.numpy(), "final_norm": P["final_norm"].grad.numpy(), "blocks": []}
    for b in P["blocks"]:
        g["blocks"].append({k: (v.grad.numpy() if v.grad is not None else np.zeros(v.shape)) for k, v in b.items()})
    return float(loss.detach()), logits.detach().numpy(), g
