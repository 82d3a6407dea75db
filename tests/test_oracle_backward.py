"""The oracle's backward functions pinned against automatic differentiation (CPU, float64 torch).

The oracle's backward passes (orc_lif_bwd, orc_mem_rec_bwd, kwta_relu2_bwd, dense_back) are
hand-derived. Here each is compared with torch.autograd of a float64 statement of the reference's
FORWARD as the reference writes it for autograd:
  - the LIF: lif_ref's straight-through spikes, soft + (hard - soft).detach(), with the detached
    threshold and trace spikes and, under the reset gradient, the capped reset carry
    (gpu/arch.rs:942-1071);
  - the memory: delta_rec's token loop (gpu/arch.rs:1091-1136) with the state bound;
  - relu² after kWTA: relu(u * mask)² with the mask a constant (gpu/model.rs:504-528, arch.rs:1833-1835);
  - the dense mix: out = raw + sum_j w_j S_j (gpu/arch.rs:1492-1500) chained over blocks.
Autograd differentiates the forward, so a wrong sign, a dropped term, an index off by one step or a
missing cap in the hand-derived backward fails here.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

# every tensor here is made float64 explicitly (no global default: the GPU tests share the process)


# --------------------------------------------------------------------------- LIF

def lif_ref_t(cur, beta, theta, rho, gain, v0, s0, a0, levels, signed, alif, slope, rg, capped=None):
    """gpu/arch.rs:964-1071 in float64 torch ops (autograd gives its gradient). capped (a list):
    gets the number of units whose reset carry was capped, per step."""
    B, T, D = cur.shape
    th = theta.detach()
    v, sp = v0, s0.detach()
    a = a0 if alif else None
    th_prev = th.expand(B, D)
    if alif:
        th_prev = th_prev + a0 * gain

    def soft(u):
        return u / (u.abs() * slope + 1.0)

    def sur(x):
        return 1.0 / (x.abs() * slope + 1.0) ** 2

    outs = []
    for t in range(T):
        if alif:
            a = a * rho + sp.abs().detach() * (1.0 - rho)
            th_t = th + a * gain
        else:
            th_t = th.expand(B, D)
        reset = sp * th_prev
        v = v * beta + cur[:, t] - (reset if rg else reset.detach())
        if not signed:
            u = v - th_t
            sg = soft(u)
            s = sg + ((u >= 0).double() - sg).detach()
        else:
            sf, hd = 0.0, 0.0
            for k in range(1, levels + 1):
                up, dn = v - th_t * k, -v - th_t * k
                sf = sf + (soft(up) - soft(dn))
                hd = hd + ((up >= 0).double() - (dn >= 0).double())
            s = sf + (hd - sf).detach()
        outs.append(s)
        if rg:
            vd, thd = v.detach(), th_t.detach()
            if not signed:
                dv = sur(vd - thd)
            else:
                dv = sum(sur(vd - thd * k) + sur(-vd - thd * k) for k in range(1, levels + 1))
            cap = (beta.detach() * 2.0).expand(B, D)
            q = thd * dv
            sc = torch.where(q > cap, cap / q, torch.ones_like(q))
            if capped is not None:
                capped.append(int((q > cap).sum()))
            sd = s.detach()
            sp = sd + (s - sd) * sc
        else:
            sp = s.detach()
        th_prev = th_t
    return torch.stack(outs, 1), v, a


def lif_case(seed, B=2, T=37, D=6):
    rng = np.random.default_rng(seed)
    cur = (rng.normal(size=(B, T, D)) * 1.2).astype(np.float32)
    ps = np.concatenate([rng.uniform(0.15, 0.95, D), rng.uniform(0.6, 1.4, D), rng.uniform(0.8, 0.99, D),
                         rng.uniform(0.02, 0.5, D)]).astype(np.float32)
    v0 = rng.normal(size=(B, D)).astype(np.float32)
    s0 = rng.integers(-2, 3, (B, D)).astype(np.float32)
    a0 = rng.uniform(0, 1, (B, D)).astype(np.float32)
    g = rng.normal(size=(B, T, D)).astype(np.float32)
    gv = rng.normal(size=(B, D)).astype(np.float32)
    ga = rng.normal(size=(B, D)).astype(np.float32)
    return cur, ps, v0, s0, a0, g, gv, ga


LIF_KINDS = [(2, True), (1, True), (1, False)]


@pytest.mark.parametrize("levels,signed", LIF_KINDS)
@pytest.mark.parametrize("alif", [True, False])
@pytest.mark.parametrize("rg", [False, True])
def test_lif_bwd_matches_autograd(levels, signed, alif, rg):
    """Every spike kind, with and without the trace and the reset gradient. With the reset gradient
    the slope is 0.5, wide enough that th ds/dv > 2 beta on many steps (the cap is counted)."""
    slope = 0.5 if rg else 2.0
    cur, ps, v0, s0, a0, g, gv, ga = lif_case(11 + 7 * levels + 3 * signed + alif + 5 * rg)
    if not signed:
        s0 = (s0 > 0).astype(np.float32)
    elif levels == 1:
        s0 = np.clip(s0, -1, 1)
    D = cur.shape[2]
    T_ = lambda x, grad=False: torch.tensor(np.asarray(x, np.float64), requires_grad=grad)
    tc, tb, tth, tr, tg = T_(cur, True), T_(ps[:D], True), T_(ps[D:2 * D]), T_(ps[2 * D:3 * D], True), T_(ps[3 * D:], True)
    tv0, ts0, ta0 = T_(v0, True), T_(s0), T_(a0, True)
    capped = []
    spk, vT, aT = lif_ref_t(tc, tb, tth, tr, tg, tv0, ts0, ta0, levels, signed, alif, slope, rg, capped)
    if rg:
        assert sum(capped) >= 10, sum(capped)
    # the float32 forward takes the same decisions (no near-tie at these seeds)
    spk32, _, _, _ = O.lif_scan(cur, ps, v0, s0, a0, levels=levels, signed=signed, alif=alif)
    assert np.array_equal(spk.detach().numpy(), spk32.astype(np.float64))
    loss = (spk * T_(g)).sum() + (vT * T_(gv)).sum()
    if alif:
        loss = loss + (aT * T_(ga)).sum()
    loss.backward()
    o = O.lif_bwd(cur, ps, g, v0, s0, a0, gv, ga if alif else None, levels=levels, signed=signed, alif=alif,
                  slope=slope, reset_grad=rg)

    def close(mine, ref, name):
        ref = ref.detach().numpy()
        err = np.max(np.abs(mine - ref)) / max(np.max(np.abs(ref)), 1e-12)
        assert err < 2e-5, (name, err)

    close(o["dI"], tc.grad, "dI")
    close(o["dv0"], tv0.grad, "dv0")
    close(o["dbeta"].sum(0), tb.grad, "dbeta")
    if alif:
        close(o["da0"], ta0.grad, "da0")
        close(o["drho"].sum(0), tr.grad, "drho")
        close(o["dgain"].sum(0), tg.grad, "dgain")
    else:
        assert not np.any(o["da0"]) and not np.any(o["drho"]) and not np.any(o["dgain"])


def test_lif_bwd_known_answer_by_hand():
    """One channel, beta = 0.5, theta = 1, binary spikes, no ALIF, no reset gradient, slope 1:
    currents [0.8, 0.9, 0.3] give membranes 0.8, 1.3, -0.05 (grad/tests/lif.rs:1-60's forward) and
    spikes [0, 1, 0]. With dL/ds = [1, 1, 1]: G_2 = sur(-1.05) = 1/2.05^2; G_1 = sur(0.3) + 0.5 G_2;
    G_0 = sur(-0.2) + 0.5 G_1, sur(x) = 1/(1+|x|)^2 (worked by hand)."""
    cur = np.array([0.8, 0.9, 0.3], np.float32).reshape(1, 3, 1)
    ps = np.array([0.5, 1.0, 0.0, 0.0], np.float32)
    o = O.lif_bwd(cur, ps, np.ones((1, 3, 1), np.float32), levels=1, signed=False, alif=False, slope=1.0)
    sur = lambda x: 1.0 / (1.0 + abs(x)) ** 2
    g2 = sur(-0.05 - 1.0)
    g1 = sur(1.3 - 1.0) + 0.5 * g2
    g0 = sur(0.8 - 1.0) + 0.5 * g1
    np.testing.assert_allclose(o["dI"].ravel(), [g0, g1, g2], rtol=1e-6)
    # dbeta = sum_t G_t v_{t-1} (v_{-1} = 0): G_1 0.8 + G_2 1.3
    np.testing.assert_allclose(o["dbeta"].ravel(), [g1 * 0.8 + g2 * 1.3], rtol=1e-6)
    np.testing.assert_allclose(o["dv0"].ravel(), [0.5 * g0], rtol=1e-6)


# --------------------------------------------------------------------------- memory

def delta_rec_t(q, k, e, v, la, b, m, cap, F0, S0):
    """gpu/arch.rs:1091-1136 in float64 torch ops."""
    BH, T, hs = q.shape
    alpha = la.exp()
    F, S = F0, S0
    ys = []
    for t in range(T):
        ai = alpha[:, t, :, None]                   # [BH, g, 1]: one rate per key row
        bi = b[:, t, None, :]                       # [BH, 1, g]
        kb = (k[:, t, None, :] * bi).transpose(1, 2)
        eb = (e[:, t, None, :] * bi).transpose(1, 2)
        pred = e[:, t, None, :] @ F                 # [BH, 1, hs]
        upd = kb @ v[:, t, None, :] - (eb @ pred) * ai
        fa = F * ai
        if m > 0:
            S = S * m + upd
            F = fa + S
        else:
            F = fa + upd
        F = F.clamp(-cap, cap)
        ys.append(q[:, t, None, :] @ F)
    return torch.cat(ys, 1), F, S


def mem_case(seed, BH=3, T=23, hs=64, g=64):
    rng = np.random.default_rng(seed)

    def unit(x):
        return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)

    q, k, e = (unit(rng.normal(size=(BH, T, hs))) for _ in range(3))
    v = rng.normal(size=(BH, T, hs)).astype(np.float32)
    la = np.log(rng.uniform(0.85, 0.999, (BH, T, g))).astype(np.float32)
    b = rng.uniform(0.1, 1.9, (BH, T, g)).astype(np.float32)
    F0 = (rng.normal(size=(BH, hs, hs)) * 0.3).astype(np.float32)
    S0 = (rng.normal(size=(BH, hs, hs)) * 0.1).astype(np.float32)
    dy = rng.normal(size=(BH, T, hs)).astype(np.float32)
    dF = (rng.normal(size=(BH, hs, hs)) * 0.2).astype(np.float32)
    dS = (rng.normal(size=(BH, hs, hs)) * 0.2).astype(np.float32)
    return q, k, e, v, la, b, F0, S0, dy, dF, dS


@pytest.mark.parametrize("g", [64, 1])
@pytest.mark.parametrize("m", [0.0, 0.5])
@pytest.mark.parametrize("cap", [1e5, 0.6])
def test_mem_rec_bwd_matches_autograd(g, m, cap):
    q, k, e, v, la, b, F0, S0, dy, dF, dS = mem_case(3 + g + int(10 * m) + int(cap < 1), g=g)
    T_ = lambda x: torch.tensor(np.asarray(x, np.float64), requires_grad=True)
    t = {n: T_(x) for n, x in dict(q=q, k=k, e=e, v=v, la=la, b=b, F0=F0, S0=S0).items()}
    y, FT, ST = delta_rec_t(t["q"], t["k"], t["e"], t["v"], t["la"], t["b"], m, cap, t["F0"], t["S0"] if m else None)
    if cap < 1:
        frac = float((FT.detach().abs() >= cap).double().mean())
        assert frac > 0.01, frac  # the bound is met, so its mask is exercised
    loss = (y * torch.tensor(dy, dtype=torch.float64)).sum() + (FT * torch.tensor(dF, dtype=torch.float64)).sum()
    if m:
        loss = loss + (ST * torch.tensor(dS, dtype=torch.float64)).sum()
    loss.backward()
    o = O.mem_rec_bwd(q, k, e, v, la, b, dy, m=m, cap=cap, F0=F0, S0=S0 if m else None, dF_T=dF,
                      dS_T=dS if m else None)
    for name, ref in (("dq", "q"), ("dk", "k"), ("de", "e"), ("dv", "v"), ("dla", "la"), ("db", "b"),
                      ("dF0", "F0")) + ((("dS0", "S0"),) if m else ()):
        r = t[ref].grad.numpy()
        err = np.max(np.abs(o[name] - r)) / max(np.max(np.abs(r)), 1e-12)
        assert err < 1e-5, (name, err)


def test_mem_rec_bwd_zero_initial_state():
    """F0 = S0 = 0 and no final-state gradient (the start of a text): the NULL paths."""
    q, k, e, v, la, b, F0, S0, dy, dF, dS = mem_case(99, BH=2, T=9, g=64)
    T_ = lambda x: torch.tensor(np.asarray(x, np.float64), requires_grad=True)
    t = {n: T_(x) for n, x in dict(q=q, k=k, e=e, v=v, la=la, b=b).items()}
    z = torch.zeros(2, 64, 64, dtype=torch.float64)
    y, _, _ = delta_rec_t(t["q"], t["k"], t["e"], t["v"], t["la"], t["b"], 0.5, 1e5, z, z)
    (y * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    o = O.mem_rec_bwd(q, k, e, v, la, b, dy, m=0.5)
    for name, ref in (("dq", "q"), ("dk", "k"), ("de", "e"), ("dv", "v"), ("dla", "la"), ("db", "b")):
        r = t[ref].grad.numpy()
        assert np.max(np.abs(o[name] - r)) / np.max(np.abs(r)) < 1e-5, name


# --------------------------------------------------------------------------- relu² and the dense mix

def test_kwta_relu2_bwd_matches_autograd():
    rng = np.random.default_rng(5)
    n, h, kk = 7, 48, 12
    u = rng.normal(size=(n, h)).astype(np.float32)
    u[:, :3] = u[:, 3:6]  # ties at the boundary are kept
    a, kth = O.kwta(u, kk, relu2=True)
    ga = rng.normal(size=(n, h)).astype(np.float32)
    tu = torch.tensor(u.astype(np.float64), requires_grad=True)
    mask = torch.tensor((u - kth[:, None] >= 0).astype(np.float64))
    out = torch.relu(tu * mask) ** 2
    np.testing.assert_allclose(out.detach().numpy(), a, rtol=1e-6)
    (out * torch.tensor(ga.astype(np.float64))).sum().backward()
    gu = O.kwta_relu2_bwd(u, kth, ga)
    np.testing.assert_allclose(gu, tu.grad.numpy(), rtol=1e-6, atol=0)


def test_dense_back_matches_autograd():
    """Three blocks of a dense stack, S_0 = x0, raw_i the block outputs: autograd of the chained mix
    against dense_back's dL/dS_c and dL/dw_i (block i's base is G_i = dL/d(mix_i))."""
    rng = np.random.default_rng(8)
    L, M = 3, 40
    wf = rng.normal(size=L * (L + 3) // 2).astype(np.float32)
    x0 = torch.tensor(rng.normal(size=M), requires_grad=True)
    raws = [torch.tensor(rng.normal(size=M), requires_grad=True) for _ in range(L)]
    tw = torch.tensor(wf.astype(np.float64), requires_grad=True)
    S = [x0]
    mixes = []
    for i in range(L):
        # block i's input is the previous mix; its raw output is raws[i] plus that input (a residual
        # block), so dL/draw flows into the earlier mixes too
        inp = mixes[-1] if mixes else x0
        raw = raws[i] + inp
        S.append(raw)
        w = tw[i * (i + 3) // 2: i * (i + 3) // 2 + i + 2]
        out = raw
        for j in range(i + 2):
            out = out + w[j] * S[j]
        mixes.append(out)
        mixes[-1].retain_grad()
    for z in S:
        z.retain_grad()
    gL = torch.tensor(rng.normal(size=M))
    (mixes[-1] * gL).sum().backward()
    Gs = np.stack([m.grad.numpy() for m in mixes]).astype(np.float32)
    Sn = np.stack([z.detach().numpy() for z in S]).astype(np.float32)
    for i in range(L):
        # dL/draw_{i+1} (stream i + 1) = G_i + sum_{k >= i} w_k[i + 1] G_k; dL/dw_i = G_i . S_j
        out, dw = O.dense_back(Sn, Gs, wf, Gs[i], col=i + 1, i0=i, L=L, nd=i + 2)
        np.testing.assert_allclose(out, S[i + 1].grad.numpy(), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(dw, tw.grad.numpy()[i * (i + 3) // 2: i * (i + 3) // 2 + i + 2], rtol=1e-5)
    # the embedding: base = dL/dx0 through the first block's input path, col 0 over every block
    out, _ = O.dense_back(Sn, Gs, wf, np.zeros(M, np.float32), col=0, i0=0, L=L, nd=0)
    direct = x0.grad.numpy() - S[1].grad.numpy()  # x0 also feeds raw_0 (the residual), which is S_1
    np.testing.assert_allclose(out, direct, rtol=1e-5, atol=1e-5)
