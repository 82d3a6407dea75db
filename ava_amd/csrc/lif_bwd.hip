// The backward of the general LIF scan for gfx950 (the surrogate gradient of the straight-through
// spikes: gpu/arch.rs:964-1071 lif_ref's autograd; the CUDA form lifg_bwd, gpu/lif.cu:3228-3290).
//
// One lane per (b, c), channel-contiguous as the forward, walking T twice:
//   1. the forward replayed from (v0, s0, a0), nothing kept but the state at the start of every
//      segment of K steps (segments are cut from the end, so only the first may be short). That
//      state (v, s, a) is parked in the segment's own first three rows of dI, which the reverse
//      pass overwrites last: no workspace and 12 bytes per segment of traffic.
//   2. segment by segment from the last: the K steps replayed from the parked state with v_t and
//      a_t in registers, then walked back. The next (earlier) segment's currents, incoming
//      gradients and parked state are loaded while this one is processed.
// HBM per element: the currents twice, the incoming gradient once and dI once, 16 bytes (a
// backward that stores the membrane and trace instead moves 28).
//
// Per step, backwards (G = dL/dv_t, carried: cv = beta G_{t+1}, ca = dL/da_{t+1} rho):
//   ds/dv, ds/dth from the surrogate 1 / (1 + S |x|)^2 of each spike edge x = v - k th, -v - k th;
//   gs = dL/ds_t (minus te G_{t+1} when the reset carries gradient, te = th_t or 2 beta / (ds/dv)
//   where th_t ds/dv > 2 beta);  G = gs ds/dv + cv;  dbeta += G v_{t-1};
//   ALIF: gth = gs ds/dth (- s_t G_{t+1}), ga = gth gain + ca, dgain += gth a_t,
//   drho += ga (a_{t-1} - |s_{t-1}|), ca = rho ga.
// Every operation is rounded on its own (-ffp-contract=off), in the order of the CPU statement.
#include "common.h"

namespace {

template <int LEVELS, bool SIGNED>
__device__ __forceinline__ float spike_of(float v, float th) {
    if (!SIGNED) return (v - th >= 0.0f) ? 1.0f : 0.0f;
    float h = 0.0f;
#pragma unroll
    for (int k = 1; k <= LEVELS; k++) {
        const float kth = th * (float)k;
        h += ((v - kth >= 0.0f) ? 1.0f : 0.0f) - ((-v - kth >= 0.0f) ? 1.0f : 0.0f);
    }
    return h;
}

__device__ __forceinline__ float surrogate(float x, float slope) {
    const float a = 1.0f + slope * fabsf(x);
    return 1.0f / (a * a);
}

// d s / d v and d s / d th of one step's surrogate spike.
template <int LEVELS, bool SIGNED>
__device__ __forceinline__ void dspike(float v, float th, float slope, float &dv, float &dth) {
    if (!SIGNED) {
        const float g = surrogate(v - th, slope);
        dv = g;
        dth = -g;
        return;
    }
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int k = 1; k <= LEVELS; k++) {
        const float kth = th * (float)k;
        const float gu = surrogate(v - kth, slope), gd = surrogate(-v - kth, slope);
        a += gu + gd;
        b += (float)k * (gd - gu);
    }
    dv = a;
    dth = b;
}

struct LifBwdArgs {
    const float *cur, *ps, *v0, *s0, *a0, *gs, *gv, *ga;
    float *dI, *dv0, *da0, *dbeta, *drho, *dgain;
    int B, T, D;
    float slope;
    int rg;
};

template <int K, int LEVELS, bool SIGNED, bool ALIF>
__global__ __launch_bounds__(256, 2) void lif_bwd_kernel(LifBwdArgs p) {
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const int D = p.D, T = p.T;
    if (gid >= p.B * D) return;
    const int b = gid / D, c = gid - b * D;
    const float bt = p.ps[c], th0 = p.ps[D + c], rho = p.ps[2 * D + c], gain = p.ps[3 * D + c];
    const float omr = 1.0f - rho;
    const size_t col = (size_t)b * T * D + c;
    const float *x = p.cur + col, *g = p.gs + col;
    float *o = p.dI + col;
    const float v0 = p.v0[gid], s0 = p.s0[gid], a0 = ALIF ? p.a0[gid] : 0.0f;
    const int nseg = (T + K - 1) / K;
    // segment q (0 = the last) covers [max(0, T - (q + 1) K), T - q K)
    auto seg0 = [&](int q) { return max(0, T - (q + 1) * K); };

    float buf[K] = {}, nxt[K] = {};  // (entries past a short segment are never read)
    auto load_cur = [&](int q, float (&dst)[K]) {
        const int t0 = seg0(q), n = T - q * K - t0;
#pragma unroll
        for (int i = 0; i < K; i++)
            if (i < n) dst[i] = __builtin_nontemporal_load(x + (size_t)(t0 + i) * D);
    };

    // 1. the forward, parking the state at each segment's start (segments after the first)
    {
        float v = v0, sp = s0, a = a0, thp = ALIF ? th0 + a0 * gain : th0;
        load_cur(nseg - 1, buf);
        for (int q = nseg - 1; q >= 0; q--) {
            if (q > 0) load_cur(q - 1, nxt);
            const int t0 = seg0(q), n = T - q * K - t0;
            if (t0 > 0) {
                o[(size_t)t0 * D] = v;
                o[(size_t)(t0 + 1) * D] = sp;
                if (ALIF) o[(size_t)(t0 + 2) * D] = a;
            }
#pragma unroll
            for (int i = 0; i < K; i++) {
                if (i < n) {
                    float tht = th0;
                    if (ALIF) {
                        a = a * rho + fabsf(sp) * omr;
                        tht = th0 + a * gain;
                    }
                    v = (v * bt + buf[i]) - sp * thp;
                    sp = spike_of<LEVELS, SIGNED>(v, tht);
                    thp = tht;
                }
            }
#pragma unroll
            for (int i = 0; i < K; i++) buf[i] = nxt[i];
        }
    }

    // 2. backwards, segment by segment
    float cv = p.gv ? p.gv[gid] : 0.0f, ca = (ALIF && p.ga) ? p.ga[gid] : 0.0f;
    float gb = 0.0f, gr = 0.0f, gg = 0.0f, Gn = 0.0f;  // Gn = dL/dv_{t+1}
    float gbuf[K] = {}, gnxt[K] = {};
    auto load_g = [&](int q, float (&dst)[K]) {
        const int t0 = seg0(q), n = T - q * K - t0;
#pragma unroll
        for (int i = 0; i < K; i++)
            if (i < n) dst[i] = g[(size_t)(t0 + i) * D];
    };
    float ckv, cks, cka, nkv = 0.0f, nks = 0.0f, nka = 0.0f;
    auto load_ck = [&](int q, float &kv, float &ks, float &ka) {
        const int t0 = seg0(q);
        if (t0 > 0) {
            kv = o[(size_t)t0 * D];
            ks = o[(size_t)(t0 + 1) * D];
            ka = ALIF ? o[(size_t)(t0 + 2) * D] : 0.0f;
        } else {
            kv = v0;
            ks = s0;
            ka = a0;
        }
    };
    load_cur(0, buf);
    load_g(0, gbuf);
    load_ck(0, ckv, cks, cka);
    for (int q = 0; q < nseg; q++) {
        if (q + 1 < nseg) {
            load_cur(q + 1, nxt);
            load_g(q + 1, gnxt);
            load_ck(q + 1, nkv, nks, nka);
        }
        const int t0 = seg0(q), n = T - q * K - t0;
        float vs[K] = {}, as[K] = {};
        {
            float v = ckv, sp = cks, a = cka, thp = ALIF ? th0 + cka * gain : th0;
#pragma unroll
            for (int i = 0; i < K; i++) {
                if (i < n) {
                    float tht = th0;
                    if (ALIF) {
                        a = a * rho + fabsf(sp) * omr;
                        tht = th0 + a * gain;
                    }
                    v = (v * bt + buf[i]) - sp * thp;
                    sp = spike_of<LEVELS, SIGNED>(v, tht);
                    thp = tht;
                    vs[i] = v;
                    as[i] = a;
                }
            }
        }
#pragma unroll
        for (int i = K - 1; i >= 0; i--) {
            if (i < n) {
                const float vt = vs[i], at = ALIF ? as[i] : 0.0f;
                const float tht = ALIF ? th0 + at * gain : th0;
                float dv, dth;
                dspike<LEVELS, SIGNED>(vt, tht, p.slope, dv, dth);
                float gst = gbuf[i];
                if (p.rg) {
                    const float qq = tht * dv, cap = 2.0f * bt;
                    gst -= (qq > cap ? cap / dv : tht) * Gn;
                }
                const float G = gst * dv + cv;
                gb += G * (i > 0 ? vs[i - 1] : ckv);
                if (ALIF) {
                    // the spikes are re-formed from the kept membranes and thresholds
                    float gth = gst * dth;
                    if (p.rg) gth -= spike_of<LEVELS, SIGNED>(vt, tht) * Gn;
                    const float gaa = gth * gain + ca;
                    gg += gth * at;
                    const float ap = i > 0 ? as[i - 1] : cka;
                    const float sprev = i > 0 ? spike_of<LEVELS, SIGNED>(vs[i - 1], th0 + as[i - 1] * gain) : cks;
                    gr += gaa * (ap - fabsf(sprev));
                    ca = rho * gaa;
                }
                o[(size_t)(t0 + i) * D] = G;
                Gn = G;
                cv = bt * G;
            }
        }
#pragma unroll
        for (int i = 0; i < K; i++) {
            buf[i] = nxt[i];
            gbuf[i] = gnxt[i];
        }
        ckv = nkv;
        cks = nks;
        cka = nka;
    }
    if (ALIF && p.rg) {  // the first step's reset used the initial threshold theta + a0 gain
        const float g0 = -s0 * Gn;
        gg += g0 * a0;
        ca += g0 * gain;
    }
    p.dv0[gid] = cv;
    if (p.da0) p.da0[gid] = ALIF ? ca : 0.0f;
    p.dbeta[gid] = gb;
    if (p.drho) p.drho[gid] = ALIF ? gr : 0.0f;
    if (p.dgain) p.dgain[gid] = ALIF ? gg : 0.0f;
}

// Steps per segment: 5 x 16 registers of currents, gradients and replayed state. 32-step segments
// (226 VGPRs, the same two waves per SIMD) measured 7% slower at config[1]'s shape.
constexpr int SEG = 16;

// ------------------------------------------------------------------ the backward in parallel segments
//
// With few (stream, channel) chains (the training step's B = 4: 4,096 lanes, a sixteenth of the SIMDs)
// the walk above is a long dependent chain per lane. Given the forward trajectory, though, the walk
// is linear in what it carries between steps, X = (Gn, cv, ca): per step
//   gst = g - te Gn;  G = gst dv + cv;  ALIF: gth = gst dth - s Gn (reset gradient), gaa = gth gain + ca;
//   then (Gn, cv, ca) <- (G, beta G, rho gaa), and dbeta, dgain, drho gather G v_prev, gth a, gaa (a_prev -
//   |s_prev|),
// so a segment of SK steps maps the X entering it (from the later steps) to the X leaving it, and its
// parameter gradients, by affine functions of X. Four passes:
//   A (one lane per chain): the forward replayed, the state (v, s, a) parked at every segment start
//      (skipped when the caller's forward parked them: ava::lif_scan's park);
//   B (one lane per (chain, segment)): the segment's forward replayed from its parked state, then walked
//      back with every carried and gathered quantity held as its 4 coefficients (1, X) — the affine
//      functions, written to the workspace;
//   C (one lane per chain): the segments' functions applied from the last to the first, from X = (0, dL/dv_T,
//      dL/da_T): each segment's entering X is kept, and the parameter gradients are summed;
//   D (one lane per (chain, segment)): the segment replayed and walked back with its entering X, as the
//      walk above, writing dI.
// The forward arithmetic is the scan's own (the same spikes and states); the backward sums associate
// differently from the one-lane walk (rounding only). Per (chain, segment): 3 parked state floats and
// 27 workspace floats (24 coefficients, the entering X).
constexpr int SK = ava::LIF_SEG_STEPS;
constexpr int SW = 27;  // workspace floats per (chain, segment): 24 coefficients, the entering X

struct LifSegArgs {
    LifBwdArgs p;
    float *ws;    // [nseg][SW][chains]
    float *park;  // [nseg][3][chains]: the state at each segment's start
    int nseg;
};

// field f of (segment sg, chain ch): 0..23 the coefficients, 24..26 the entering X
__device__ __forceinline__ float *ws_at(const LifSegArgs &a, int sg, int f, int ch) {
    return a.ws + ((size_t)sg * SW + f) * (size_t)(a.p.B * a.p.D) + ch;
}
__device__ __forceinline__ float *park_at(const LifSegArgs &a, int sg, int f, int ch) {
    return a.park + ((size_t)sg * 3 + f) * (size_t)(a.p.B * a.p.D) + ch;
}

// one forward step of the scan (lif_scan_kernel's loop body)
template <int LEVELS, bool SIGNED, bool ALIF>
__device__ __forceinline__ void fwd1(float x, float bt, float th0, float rho, float omr, float gain, float &v,
                                     float &sp, float &a, float &thp) {
    float tht = th0;
    if (ALIF) {
        a = a * rho + fabsf(sp) * omr;
        tht = th0 + a * gain;
    }
    v = (v * bt + x) - sp * thp;
    sp = spike_of<LEVELS, SIGNED>(v, tht);
    thp = tht;
}

template <int LEVELS, bool SIGNED, bool ALIF>
__global__ __launch_bounds__(256) void lif_seg_park_kernel(LifSegArgs A) {
    const LifBwdArgs &p = A.p;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const int D = p.D, T = p.T;
    if (gid >= p.B * D) return;
    const int b = gid / D, c = gid - b * D;
    const float bt = p.ps[c], th0 = p.ps[D + c], rho = p.ps[2 * D + c], gain = p.ps[3 * D + c], omr = 1.0f - rho;
    const float *x = p.cur + (size_t)b * T * D + c;
    float v = p.v0[gid], sp = p.s0[gid], a = ALIF ? p.a0[gid] : 0.0f;
    float thp = ALIF ? th0 + a * gain : th0;
    *park_at(A, 0, 0, gid) = v;
    *park_at(A, 0, 1, gid) = sp;
    *park_at(A, 0, 2, gid) = a;
    constexpr int PF = 16;
    float buf[PF];
    for (int t0 = 0; t0 < T; t0 += PF) {
#pragma unroll
        for (int i = 0; i < PF; i++) buf[i] = t0 + i < T ? __builtin_nontemporal_load(x + (size_t)(t0 + i) * D) : 0.0f;
#pragma unroll
        for (int i = 0; i < PF; i++) {
            const int t = t0 + i;
            if (t < T) {
                fwd1<LEVELS, SIGNED, ALIF>(buf[i], bt, th0, rho, omr, gain, v, sp, a, thp);
                if ((t + 1) % SK == 0 && t + 1 < T) {
                    const int sg = (t + 1) / SK;
                    *park_at(A, sg, 0, gid) = v;
                    *park_at(A, sg, 1, gid) = sp;
                    *park_at(A, sg, 2, gid) = a;
                }
            }
        }
    }
}

// The segment's forward from its parked state: vs, as after each of its n steps (and the state before)
template <int LEVELS, bool SIGNED, bool ALIF>
__device__ __forceinline__ void seg_replay(const float *x, int D, int t0, int n, float bt, float th0, float rho,
                                           float omr, float gain, float v, float sp, float a, float (&vs)[SK],
                                           float (&as)[SK]) {
    float thp = ALIF ? th0 + a * gain : th0;
#pragma unroll
    for (int i = 0; i < SK; i++) {
        if (i < n) {
            fwd1<LEVELS, SIGNED, ALIF>(x[(size_t)(t0 + i) * D], bt, th0, rho, omr, gain, v, sp, a, thp);
            vs[i] = v;
            as[i] = a;
        }
    }
}

// an affine function of X = (Gn, cv, ca): c[0] + c[1] Gn + c[2] cv + c[3] ca
struct Aff {
    float c[4];
};
__device__ __forceinline__ Aff aff(float k) { return Aff{{k, 0.0f, 0.0f, 0.0f}}; }
__device__ __forceinline__ Aff axpy(float s, const Aff &x, const Aff &y) {  // s x + y
    Aff r;
#pragma unroll
    for (int i = 0; i < 4; i++) r.c[i] = fmaf(s, x.c[i], y.c[i]);
    return r;
}
__device__ __forceinline__ Aff scal(float s, const Aff &x) {
    Aff r;
#pragma unroll
    for (int i = 0; i < 4; i++) r.c[i] = s * x.c[i];
    return r;
}

template <int LEVELS, bool SIGNED, bool ALIF>
__global__ __launch_bounds__(256) void lif_seg_affine_kernel(LifSegArgs A) {
    const LifBwdArgs &p = A.p;
    const int chains = p.B * p.D;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;  // chain fastest
    if (gid >= chains * A.nseg) return;
    const int sg = gid / chains, ch = gid - sg * chains;
    const int D = p.D, T = p.T, b = ch / D, c = ch - b * D;
    const float bt = p.ps[c], th0 = p.ps[D + c], rho = p.ps[2 * D + c], gain = p.ps[3 * D + c], omr = 1.0f - rho;
    const int t0 = sg * SK, n = min(SK, T - t0);
    const float *x = p.cur + (size_t)b * T * D + c, *g = p.gs + (size_t)b * T * D + c;
    const float pv = *park_at(A, sg, 0, ch), ps_ = *park_at(A, sg, 1, ch), pa = *park_at(A, sg, 2, ch);
    float vs[SK] = {}, as[SK] = {};
    seg_replay<LEVELS, SIGNED, ALIF>(x, D, t0, n, bt, th0, rho, omr, gain, pv, ps_, pa, vs, as);
    Aff Gn{{0.0f, 1.0f, 0.0f, 0.0f}}, cv{{0.0f, 0.0f, 1.0f, 0.0f}}, ca{{0.0f, 0.0f, 0.0f, 1.0f}};
    Aff gb = aff(0.0f), gg = aff(0.0f), gr = aff(0.0f);
#pragma unroll
    for (int i = SK - 1; i >= 0; i--) {
        if (i < n) {
            const float vt = vs[i], at = ALIF ? as[i] : 0.0f;
            const float tht = ALIF ? th0 + at * gain : th0;
            float dv, dth;
            dspike<LEVELS, SIGNED>(vt, tht, p.slope, dv, dth);
            const float gt = g[(size_t)(t0 + i) * D];
            float te = 0.0f;
            if (p.rg) {
                const float qq = tht * dv, cap = 2.0f * bt;
                te = qq > cap ? cap / dv : tht;
            }
            const Aff gst = axpy(-te, Gn, aff(gt));   // g - te Gn
            const Aff G = axpy(dv, gst, cv);          // gst dv + cv
            gb = axpy(i > 0 ? vs[i - 1] : pv, G, gb);
            if (ALIF) {
                Aff gth = scal(dth, gst);
                if (p.rg) gth = axpy(-spike_of<LEVELS, SIGNED>(vt, tht), Gn, gth);
                const Aff gaa = axpy(gain, gth, ca);
                gg = axpy(at, gth, gg);
                const float ap = i > 0 ? as[i - 1] : pa;
                const float sprev = i > 0 ? spike_of<LEVELS, SIGNED>(vs[i - 1], th0 + as[i - 1] * gain) : ps_;
                gr = axpy(ap - fabsf(sprev), gaa, gr);
                ca = scal(rho, gaa);
            }
            Gn = G;
            cv = scal(bt, G);
        }
    }
    const Aff *out[6] = {&Gn, &cv, &ca, &gb, &gg, &gr};
#pragma unroll
    for (int f = 0; f < 6; f++)
#pragma unroll
        for (int i = 0; i < 4; i++) *ws_at(A, sg, 4 * f + i, ch) = out[f]->c[i];
}

__device__ __forceinline__ float apply_aff(const LifSegArgs &A, int sg, int f, int ch, float Gn, float cv, float ca) {
    const float *w = ws_at(A, sg, 4 * f, ch);
    const size_t st = (size_t)A.p.B * A.p.D;
    return fmaf(w[3 * st], ca, fmaf(w[2 * st], cv, fmaf(w[st], Gn, w[0])));
}

template <bool ALIF>
__global__ __launch_bounds__(256) void lif_seg_carry_kernel(LifSegArgs A) {
    const LifBwdArgs &p = A.p;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= p.B * p.D) return;
    const int c = gid % p.D;
    const float gain = p.ps[3 * p.D + c];
    float Gn = 0.0f, cv = p.gv ? p.gv[gid] : 0.0f, ca = (ALIF && p.ga) ? p.ga[gid] : 0.0f;
    float gb = 0.0f, gg = 0.0f, gr = 0.0f;
    for (int sg = A.nseg - 1; sg >= 0; sg--) {
        *ws_at(A, sg, 24, gid) = Gn;
        *ws_at(A, sg, 25, gid) = cv;
        *ws_at(A, sg, 26, gid) = ca;
        gb += apply_aff(A, sg, 3, gid, Gn, cv, ca);
        if (ALIF) {
            gg += apply_aff(A, sg, 4, gid, Gn, cv, ca);
            gr += apply_aff(A, sg, 5, gid, Gn, cv, ca);
        }
        const float nG = apply_aff(A, sg, 0, gid, Gn, cv, ca), ncv = apply_aff(A, sg, 1, gid, Gn, cv, ca);
        const float nca = ALIF ? apply_aff(A, sg, 2, gid, Gn, cv, ca) : 0.0f;
        Gn = nG;
        cv = ncv;
        ca = nca;
    }
    if (ALIF && p.rg) {  // the first step's reset used the initial threshold theta + a0 gain
        const float g0 = -p.s0[gid] * Gn;
        gg += g0 * p.a0[gid];
        ca += g0 * gain;
    }
    p.dv0[gid] = cv;
    if (p.da0) p.da0[gid] = ALIF ? ca : 0.0f;
    p.dbeta[gid] = gb;
    if (p.drho) p.drho[gid] = ALIF ? gr : 0.0f;
    if (p.dgain) p.dgain[gid] = ALIF ? gg : 0.0f;
}

template <int LEVELS, bool SIGNED, bool ALIF>
__global__ __launch_bounds__(256) void lif_seg_walk_kernel(LifSegArgs A) {
    const LifBwdArgs &p = A.p;
    const int chains = p.B * p.D;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= chains * A.nseg) return;
    const int sg = gid / chains, ch = gid - sg * chains;
    const int D = p.D, T = p.T, b = ch / D, c = ch - b * D;
    const float bt = p.ps[c], th0 = p.ps[D + c], rho = p.ps[2 * D + c], gain = p.ps[3 * D + c], omr = 1.0f - rho;
    const int t0 = sg * SK, n = min(SK, T - t0);
    const float *x = p.cur + (size_t)b * T * D + c, *g = p.gs + (size_t)b * T * D + c;
    float *o = p.dI + (size_t)b * T * D + c;
    const float pv = *park_at(A, sg, 0, ch), ps_ = *park_at(A, sg, 1, ch), pa = *park_at(A, sg, 2, ch);
    float Gn = *ws_at(A, sg, 24, ch), cv = *ws_at(A, sg, 25, ch), ca = *ws_at(A, sg, 26, ch);
    float vs[SK] = {}, as[SK] = {};
    seg_replay<LEVELS, SIGNED, ALIF>(x, D, t0, n, bt, th0, rho, omr, gain, pv, ps_, pa, vs, as);
#pragma unroll
    for (int i = SK - 1; i >= 0; i--) {
        if (i < n) {
            const float vt = vs[i], at = ALIF ? as[i] : 0.0f;
            const float tht = ALIF ? th0 + at * gain : th0;
            float dv, dth;
            dspike<LEVELS, SIGNED>(vt, tht, p.slope, dv, dth);
            float gst = g[(size_t)(t0 + i) * D];
            if (p.rg) {
                const float qq = tht * dv, cap = 2.0f * bt;
                gst -= (qq > cap ? cap / dv : tht) * Gn;
            }
            const float G = gst * dv + cv;
            if (ALIF) {
                float gth = gst * dth;
                if (p.rg) gth -= spike_of<LEVELS, SIGNED>(vt, tht) * Gn;
                ca = rho * (gth * gain + ca);
            }
            o[(size_t)(t0 + i) * D] = G;
            Gn = G;
            cv = bt * G;
        }
    }
}

template <int LEVELS, bool SIGNED, bool ALIF>
int launch_seg(const LifSegArgs &A, bool parked, hipStream_t st) {
    const long chains = (long)A.p.B * A.p.D, lanes = chains * A.nseg;
    if (!parked) lif_seg_park_kernel<LEVELS, SIGNED, ALIF><<<ava::ceil_div(chains, 256), 256, 0, st>>>(A);
    lif_seg_affine_kernel<LEVELS, SIGNED, ALIF><<<ava::ceil_div(lanes, 256), 256, 0, st>>>(A);
    lif_seg_carry_kernel<ALIF><<<ava::ceil_div(chains, 256), 256, 0, st>>>(A);
    lif_seg_walk_kernel<LEVELS, SIGNED, ALIF><<<ava::ceil_div(lanes, 256), 256, 0, st>>>(A);
    AVA_LAUNCHED("lif_scan_bwd segments");
    return AVA_OK;
}

}  // namespace

// The LIF scan's backward. Outputs per (b, c): dI [B][T][D], dv0, da0 and this stream's shares of
// dbeta, drho, dgain ([B][D] each; the parameter gradients are their sums over b).
extern "C" int ava_lif_scan_bwd(const float *cur, int B, int T, int D, const float *ps, const float *v0,
                                const float *s0, const float *a0, int levels, int is_signed, int alif, float slope,
                                int reset_grad, const float *g_spk, const float *g_vT, const float *g_aT, float *dI,
                                float *dv0, float *da0, float *dbeta, float *drho, float *dgain, ava_stream stream) {
    AVA_REQUIRE(cur && ps && v0 && s0 && g_spk && dI && dv0 && dbeta, AVA_ERR_ARG, "lif_scan_bwd: NULL buffer");
    AVA_REQUIRE(!alif || (a0 && da0 && drho && dgain), AVA_ERR_ARG, "lif_scan_bwd: ALIF needs a0, da0, drho, dgain");
    AVA_REQUIRE(B > 0 && T > 0 && D > 0 && (long)B * D <= (1L << 30), AVA_ERR_SHAPE, "lif_scan_bwd: B=%d T=%d D=%d",
                B, T, D);
    AVA_REQUIRE(levels == 1 || levels == 2, AVA_ERR_ARG, "lif_scan_bwd: levels %d (1 or 2)", levels);
    AVA_REQUIRE(slope >= 0.0f, AVA_ERR_ARG, "lif_scan_bwd: slope %g (the reset gradient is reset_grad)", slope);
    LifBwdArgs p{cur, ps, v0, s0, a0, g_spk, g_vT, alif ? g_aT : nullptr, dI, dv0, da0, dbeta, drho, dgain,
                 B, T, D, slope, reset_grad ? 1 : 0};
    const hipStream_t st = (hipStream_t)stream;
    dim3 grid(ava::ceil_div((long)B * D, 256)), block(256);
#define AVA_LB(L, S, A) lif_bwd_kernel<SEG, L, S, A><<<grid, block, 0, st>>>(p)
    if (!is_signed) {
        if (alif) AVA_LB(1, false, true);
        else AVA_LB(1, false, false);
    } else if (levels == 1) {
        if (alif) AVA_LB(1, true, true);
        else AVA_LB(1, true, false);
    } else {
        if (alif) AVA_LB(2, true, true);
        else AVA_LB(2, true, false);
    }
#undef AVA_LB
    AVA_LAUNCHED("lif_scan_bwd");
    return AVA_OK;
}

namespace ava {

size_t lif_bwd_seg_floats(int B, int T, int D) {
    return (size_t)((T + SK - 1) / SK) * (SW + 3) * (size_t)B * D;
}

// ava_lif_scan_bwd in parallel segments (the training step's form for few chains): the same outputs
// up to the association of the backward sums; ws holds lif_bwd_seg_floats(B, T, D) floats (the parked
// states at its end unless park, the forward's, is given).
int lif_scan_bwd_seg(const float *cur, int B, int T, int D, const float *ps, const float *v0, const float *s0,
                     const float *a0, int levels, int is_signed, int alif, float slope, int reset_grad,
                     const float *g_spk, const float *g_vT, const float *g_aT, float *dI, float *dv0, float *da0,
                     float *dbeta, float *drho, float *dgain, float *ws, size_t ws_floats, const float *park,
                     hipStream_t st) {
    AVA_REQUIRE(cur && ps && v0 && s0 && g_spk && dI && dv0 && dbeta && ws, AVA_ERR_ARG,
                "lif_scan_bwd_seg: NULL buffer");
    AVA_REQUIRE(!alif || (a0 && da0 && drho && dgain), AVA_ERR_ARG, "lif_scan_bwd_seg: ALIF needs a0, da0, drho, dgain");
    AVA_REQUIRE(B > 0 && T > 0 && D > 0 && (long)B * D * ((T + SK - 1) / SK) <= (1L << 30), AVA_ERR_SHAPE,
                "lif_scan_bwd_seg: B=%d T=%d D=%d", B, T, D);
    AVA_REQUIRE(ws_floats >= lif_bwd_seg_floats(B, T, D), AVA_ERR_SHAPE, "lif_scan_bwd_seg: workspace of %zu floats",
                ws_floats);
    AVA_REQUIRE(levels == 1 || levels == 2, AVA_ERR_ARG, "lif_scan_bwd_seg: levels %d (1 or 2)", levels);
    const int nseg = (T + SK - 1) / SK;
    float *own_park = ws + (size_t)nseg * SW * B * D;
    LifSegArgs A{LifBwdArgs{cur, ps, v0, s0, a0, g_spk, g_vT, alif ? g_aT : nullptr, dI, dv0, da0, dbeta, drho,
                            dgain, B, T, D, slope, reset_grad ? 1 : 0},
                 ws, park ? const_cast<float *>(park) : own_park, nseg};
    const bool parked = park != nullptr;
    if (!is_signed) return alif ? launch_seg<1, false, true>(A, parked, st) : launch_seg<1, false, false>(A, parked, st);
    if (levels == 1) return alif ? launch_seg<1, true, true>(A, parked, st) : launch_seg<1, true, false>(A, parked, st);
    return alif ? launch_seg<2, true, true>(A, parked, st) : launch_seg<2, true, false>(A, parked, st);
}

}  // namespace ava

extern "C" size_t ava_lif_scan_bwd_segments_workspace(int B, int T, int D) {
    return B > 0 && T > 0 && D > 0 ? ava::lif_bwd_seg_floats(B, T, D) * sizeof(float) : 0;
}

extern "C" int ava_lif_scan_bwd_segments(const float *cur, int B, int T, int D, const float *ps, const float *v0,
                                         const float *s0, const float *a0, int levels, int is_signed, int alif,
                                         float slope, int reset_grad, const float *g_spk, const float *g_vT,
                                         const float *g_aT, float *dI, float *dv0, float *da0, float *dbeta,
                                         float *drho, float *dgain, void *ws, size_t ws_bytes, ava_stream stream) {
    AVA_REQUIRE(slope >= 0.0f, AVA_ERR_ARG, "lif_scan_bwd_segments: slope %g (the reset gradient is reset_grad)",
                slope);
    return ava::lif_scan_bwd_seg(cur, B, T, D, ps, v0, s0, a0, levels, is_signed, alif, slope, reset_grad, g_spk, g_vT,
                                 g_aT, dI, dv0, da0, dbeta, drho, dgain, static_cast<float *>(ws),
                                 ws_bytes / sizeof(float), nullptr, (hipStream_t)stream);
}
