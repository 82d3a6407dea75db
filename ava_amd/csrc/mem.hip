// The general fast-weight (delta-rule) memory recurrence for gfx950, one workgroup per head.
//
// Per head, F [64][64] (row i = key channel, column j = value channel) and the momentum S live in
// registers for the whole scan: 4 waves, wave w owns columns 16w..16w+15; lane l of a wave owns
// column 16w + (l & 15) and the 16 rows 16(l >> 4)..+15, so the column reductions
// r_j = sum_i e_i F_ij and y_j = sum_i q_i F_ij are 16 register FMAs plus two lane exchanges inside
// the wave (no LDS, no barrier per step). Per step and element:
//   u_ij = (b_i k_i) v_j - (a_i b_i e_i) r_j;  S <- M S + u;  F <- clamp(a_i F + S, +-cap)  (M = 0: F <- clamp(a_i F + u))
// then y_j = sum_i q_i F_ij (the read after the write), as gpu/mem_gen.rs:220-246 / gpu/arch.rs:1091-1136.
//
// Inputs are staged through LDS 16 time steps at a time: one cooperative, coalesced load of
// q, k, e, v and the gates per chunk (the next chunk's loads are in flight while this chunk is
// scanned), with the per-row factors a_i = exp(la_i), b_i k_i and a_i b_i e_i formed once per
// (step, row) at staging. The read-outs y are gathered in LDS and written once per chunk.
//
// Layout: head bh = (b, h) with b = bh / nh, h = bh % nh reads row (b T + t) of a [B T][ld] matrix at
// columns 64h..64h+63 (ld = 64, nh = 1 is the [BH][T][64] layout of the C ABI; ld = d, nh = d / 64 is
// the block stack's [B T][d] projection output, read in place). Per-head gates (G1) are one value
// per (row, head) at column h of a [B T][ldg] matrix.
#include <stdlib.h>

#include "common.h"

namespace {

constexpr int HS = 64, TS = 16;

struct MemArgs {
    const float *q, *k, *e, *v, *la, *b;
    int T, nh, ld, ldg, ldy;
    float m, cap;
    float *F, *S, *y;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// The sum of v over the 8 lanes l & ~7 .. l | 7, in each of them: DPP quad_perm [1,0,3,2] and
// [2,3,0,1], then row_half_mirror (lane i <-> 7 - i of each 8). Each stage adds the same two partial
// sums in every lane (in either order), so the 8 lanes hold the same bits.
__device__ __forceinline__ float sum8(float v) {
    v += dppf<0xB1>(v);
    v += dppf<0x4E>(v);
    return v + dppf<0x141>(v);
}
// v[l] + v[l ^ 16] and v[l] + v[l ^ 32] in every lane l, through the VALU lane swaps of gfx950
// (v_permlane16_swap / v_permlane32_swap: no LDS round trip). With both operands v, the swap leaves
// v[l] in one result and v[l ^ 16] (v[l ^ 32]) in the other.
__device__ __forceinline__ float xsum16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xsum32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
// The sum of v over the wave, in every lane: DPP within each row of 16 lanes (sum8, then
// row_mirror, lane i <-> 15 - i), then the lane swaps across rows.
__device__ __forceinline__ float wsum(float v) {
    v = sum8(v);
    v += dppf<0x140>(v);
    return xsum32(xsum16(v));
}

// State layout per head: 4 waves, wave w holds columns 16w..16w+15; lane l holds rows
// i0 = 8 (l & 7) .. i0 + 7 of the two columns j0 = 16 w + 2 (l >> 3), j0 + 1, as Fr[2 r + c] (S alike).
// A column's 64 rows are then 8 lanes: a column sum is 8 FMAs per lane and 3 DPP adds, and a step
// reads 10 + 1 16-byte LDS vectors per lane (the row group's e, q, a, bk, abe and the two v_j).
__device__ __forceinline__ void lane_origin(int lane, int wave, int &i0, int &j0) {
    i0 = (lane & 7) * 8;
    j0 = wave * 16 + (lane >> 3) * 2;
}

// One step of the recurrence on this lane's 8 x 2 block, with the step's staged inputs e, q, a,
// bk = b k, abe = a b e at rows i0.. and v at column j0: F (and S) updated in place; y0, y1 get
// y_j = sum_i q_i F_ij of the two columns over all 64 rows (the read after the write).
template <bool MOM>
__device__ __forceinline__ void scan_step(float (&Fr)[16], float (&Sr)[16], const float *e, const float *q,
                                          const float *a, const float *bk, const float *abe, const float *v,
                                          float M, float cap, float &y0, float &y1) {
    // r_j = sum_i e_i F_ij
    const f32x4 e0 = *reinterpret_cast<const f32x4 *>(e), e1 = *reinterpret_cast<const f32x4 *>(e + 4);
    float r0 = 0.0f, r1 = 0.0f;
#pragma unroll
    for (int rr = 0; rr < 8; rr++) {
        const float er = rr < 4 ? e0[rr] : e1[rr - 4];
        r0 = fmaf(er, Fr[2 * rr], r0);
        r1 = fmaf(er, Fr[2 * rr + 1], r1);
    }
    r0 = sum8(r0);
    r1 = sum8(r1);
    const float v0 = v[0], v1 = v[1];
    float ya = 0.0f, yb = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const f32x4 q4 = *reinterpret_cast<const f32x4 *>(q + 4 * h);
        const f32x4 a4 = *reinterpret_cast<const f32x4 *>(a + 4 * h);
        const f32x4 k4 = *reinterpret_cast<const f32x4 *>(bk + 4 * h);
        const f32x4 x4 = *reinterpret_cast<const f32x4 *>(abe + 4 * h);
#pragma unroll
        for (int z = 0; z < 4; z++) {
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int mm = 2 * (4 * h + z) + c;
                const float u = fmaf(-x4[z], c ? r1 : r0, k4[z] * (c ? v1 : v0));  // b_i k_i v_j - a_i b_i e_i r_j
                float f;
                if (MOM) {
                    Sr[mm] = fmaf(M, Sr[mm], u);
                    f = fmaf(a4[z], Fr[mm], Sr[mm]);
                } else {
                    f = fmaf(a4[z], Fr[mm], u);
                }
                f = __builtin_amdgcn_fmed3f(f, -cap, cap);  // clamp to +-cap
                Fr[mm] = f;
                if (c) yb = fmaf(q4[z], f, yb);
                else ya = fmaf(q4[z], f, ya);
            }
        }
    }
    y0 = sum8(ya);
    y1 = sum8(yb);
}

template <bool G1, bool MOM>
__global__ __launch_bounds__(256) void mem_scan_kernel(MemArgs p) {
    __shared__ __attribute__((aligned(16))) float s_q[TS][HS], s_e[TS][HS], s_v[TS][HS];
    __shared__ __attribute__((aligned(16))) float s_a[TS][HS], s_bk[TS][HS], s_abe[TS][HS];
    __shared__ __attribute__((aligned(16))) float s_y[TS][HS];

    const int bh = blockIdx.x;
    const int bi = bh / p.nh, hh = bh - bi * p.nh;
    const size_t base = (size_t)bi * p.T * p.ld + (size_t)hh * HS;
    const size_t gbase = G1 ? (size_t)bi * p.T * p.ldg + hh : (size_t)bi * p.T * p.ldg + (size_t)hh * HS;
    const size_t ybase = (size_t)bi * p.T * p.ldy + (size_t)hh * HS;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int i0, j0;
    lane_origin(lane, wave, i0, j0);

    float Fr[16], Sr[16];
    float *Fh = p.F + (size_t)bh * HS * HS, *Sh = MOM ? p.S + (size_t)bh * HS * HS : nullptr;
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int o = (i0 + (m >> 1)) * HS + j0 + (m & 1);
        Fr[m] = Fh[o];
        Sr[m] = MOM ? Sh[o] : 0.0f;
    }

    // staging: thread -> (step st, rows si..si+3)
    const int st = tid >> 4, si = (tid & 15) * 4;
    f32x4 rq, rk, re, rv, rla, rb;
    auto load = [&](int t0) {
        const int t = t0 + st;
        if (t < p.T) {
            const size_t o = base + (size_t)t * p.ld + si;
            rq = *reinterpret_cast<const f32x4 *>(p.q + o);
            rk = *reinterpret_cast<const f32x4 *>(p.k + o);
            re = *reinterpret_cast<const f32x4 *>(p.e + o);
            rv = *reinterpret_cast<const f32x4 *>(p.v + o);
            if (G1) {
                const float l = p.la[gbase + (size_t)t * p.ldg], b = p.b[gbase + (size_t)t * p.ldg];
                rla = f32x4{l, l, l, l};
                rb = f32x4{b, b, b, b};
            } else {
                const size_t og = gbase + (size_t)t * p.ldg + si;
                rla = *reinterpret_cast<const f32x4 *>(p.la + og);
                rb = *reinterpret_cast<const f32x4 *>(p.b + og);
            }
        } else {
            rq = rk = re = rv = rla = rb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    auto stage = [&]() {
        f32x4 a, bk, abe;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            a[c] = expf(rla[c]);
            bk[c] = rb[c] * rk[c];
            abe[c] = (a[c] * rb[c]) * re[c];
        }
        *reinterpret_cast<f32x4 *>(&s_q[st][si]) = rq;
        *reinterpret_cast<f32x4 *>(&s_e[st][si]) = re;
        *reinterpret_cast<f32x4 *>(&s_v[st][si]) = rv;
        *reinterpret_cast<f32x4 *>(&s_a[st][si]) = a;
        *reinterpret_cast<f32x4 *>(&s_bk[st][si]) = bk;
        *reinterpret_cast<f32x4 *>(&s_abe[st][si]) = abe;
    };

    const float M = p.m, cap = p.cap;
    load(0);
    for (int t0 = 0; t0 < p.T; t0 += TS) {
        __syncthreads();  // the previous chunk's LDS reads (and y writes-out) are done
        stage();
        __syncthreads();
        if (t0 + TS < p.T) load(t0 + TS);  // in flight during this chunk's scan
        const int n = min(TS, p.T - t0);
        for (int s = 0; s < n; s++) {
            float y0, y1;
            scan_step<MOM>(Fr, Sr, &s_e[s][i0], &s_q[s][i0], &s_a[s][i0], &s_bk[s][i0], &s_abe[s][i0], &s_v[s][j0], M,
                           cap, y0, y1);
            if ((lane & 7) < 2) s_y[s][j0 + (lane & 1)] = (lane & 1) ? y1 : y0;
        }
        __syncthreads();
        // write the chunk's read-outs: thread -> (step st, columns si..si+3)
        if (st < n) *reinterpret_cast<f32x4 *>(p.y + ybase + (size_t)(t0 + st) * p.ldy + si) =
            *reinterpret_cast<const f32x4 *>(&s_y[st][si]);
    }

#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int o = (i0 + (m >> 1)) * HS + j0 + (m & 1);
        Fh[o] = Fr[m];
        if (MOM) Sh[o] = Sr[m];
    }
}

// The same scan for few heads: each head's 64 value columns in four workgroups (the recurrence never
// mixes columns), so B nh < 512 heads still fill the GPU. Workgroup (head, cg) owns columns 16 cg ..;
// wave w four of them, lane l rows 4 (l & 15) .. + 3 of column 16 cg + 4 w + l / 16: a column sum is 4
// FMAs and a sum over the 16 lanes of a DPP row. The staging is mem_scan_kernel's (every workgroup
// stages all 64 rows of its head's inputs).
__device__ __forceinline__ float sum16r(float v) {
    v = sum8(v);
    return v + dppf<0x140>(v);
}

template <bool G1, bool MOM>
__global__ __launch_bounds__(256) void mem_scan_cols_kernel(MemArgs p) {
    __shared__ __attribute__((aligned(16))) float s_q[TS][HS], s_e[TS][HS], s_v[TS][HS];
    __shared__ __attribute__((aligned(16))) float s_a[TS][HS], s_bk[TS][HS], s_abe[TS][HS];
    __shared__ __attribute__((aligned(16))) float s_y[TS][16];

    const int bh = blockIdx.x >> 2, cg = blockIdx.x & 3;
    const int bi = bh / p.nh, hh = bh - bi * p.nh;
    const size_t base = (size_t)bi * p.T * p.ld + (size_t)hh * HS;
    const size_t gbase = G1 ? (size_t)bi * p.T * p.ldg + hh : (size_t)bi * p.T * p.ldg + (size_t)hh * HS;
    const size_t ybase = (size_t)bi * p.T * p.ldy + (size_t)hh * HS + 16 * cg;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i0 = 4 * (lane & 15), jl = 4 * wave + (lane >> 4), j = 16 * cg + jl;

    float Fr[4], Sr[4];
    float *Fh = p.F + (size_t)bh * HS * HS, *Sh = MOM ? p.S + (size_t)bh * HS * HS : nullptr;
#pragma unroll
    for (int ri = 0; ri < 4; ri++) {
        const int o = (i0 + ri) * HS + j;
        Fr[ri] = Fh[o];
        Sr[ri] = MOM ? Sh[o] : 0.0f;
    }

    const int st = tid >> 4, si = (tid & 15) * 4;
    f32x4 rq, rk, re, rv, rla, rb;
    auto load = [&](int t0) {
        const int t = t0 + st;
        if (t < p.T) {
            const size_t o = base + (size_t)t * p.ld + si;
            rq = *reinterpret_cast<const f32x4 *>(p.q + o);
            rk = *reinterpret_cast<const f32x4 *>(p.k + o);
            re = *reinterpret_cast<const f32x4 *>(p.e + o);
            rv = *reinterpret_cast<const f32x4 *>(p.v + o);
            if (G1) {
                const float l = p.la[gbase + (size_t)t * p.ldg], b = p.b[gbase + (size_t)t * p.ldg];
                rla = f32x4{l, l, l, l};
                rb = f32x4{b, b, b, b};
            } else {
                const size_t og = gbase + (size_t)t * p.ldg + si;
                rla = *reinterpret_cast<const f32x4 *>(p.la + og);
                rb = *reinterpret_cast<const f32x4 *>(p.b + og);
            }
        } else {
            rq = rk = re = rv = rla = rb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    auto stage = [&]() {
        f32x4 a, bk, abe;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            a[c] = expf(rla[c]);
            bk[c] = rb[c] * rk[c];
            abe[c] = (a[c] * rb[c]) * re[c];
        }
        *reinterpret_cast<f32x4 *>(&s_q[st][si]) = rq;
        *reinterpret_cast<f32x4 *>(&s_e[st][si]) = re;
        *reinterpret_cast<f32x4 *>(&s_v[st][si]) = rv;
        *reinterpret_cast<f32x4 *>(&s_a[st][si]) = a;
        *reinterpret_cast<f32x4 *>(&s_bk[st][si]) = bk;
        *reinterpret_cast<f32x4 *>(&s_abe[st][si]) = abe;
    };

    const float M = p.m, cap = p.cap;
    load(0);
    for (int t0 = 0; t0 < p.T; t0 += TS) {
        __syncthreads();
        stage();
        __syncthreads();
        if (t0 + TS < p.T) load(t0 + TS);
        const int n = min(TS, p.T - t0);
        for (int s = 0; s < n; s++) {
            const f32x4 e4 = *reinterpret_cast<const f32x4 *>(&s_e[s][i0]);
            float r = e4[0] * Fr[0];
            r = fmaf(e4[1], Fr[1], r);
            r = fmaf(e4[2], Fr[2], r);
            r = fmaf(e4[3], Fr[3], r);
            r = sum16r(r);
            const float vj = s_v[s][j];
            const f32x4 q4 = *reinterpret_cast<const f32x4 *>(&s_q[s][i0]);
            const f32x4 a4 = *reinterpret_cast<const f32x4 *>(&s_a[s][i0]);
            const f32x4 k4 = *reinterpret_cast<const f32x4 *>(&s_bk[s][i0]);
            const f32x4 x4 = *reinterpret_cast<const f32x4 *>(&s_abe[s][i0]);
            float ya = 0.0f;
#pragma unroll
            for (int ri = 0; ri < 4; ri++) {
                const float u = fmaf(-x4[ri], r, k4[ri] * vj);
                float f;
                if (MOM) {
                    Sr[ri] = fmaf(M, Sr[ri], u);
                    f = fmaf(a4[ri], Fr[ri], Sr[ri]);
                } else {
                    f = fmaf(a4[ri], Fr[ri], u);
                }
                f = __builtin_amdgcn_fmed3f(f, -cap, cap);
                Fr[ri] = f;
                ya = fmaf(q4[ri], f, ya);
            }
            ya = sum16r(ya);
            if ((lane & 15) == 0) s_y[s][jl] = ya;
        }
        __syncthreads();
        // the chunk's read-outs of the workgroup's 16 columns: thread -> (step, 4 columns)
        if (tid < 4 * n) {
            const int sy = tid >> 2, c4 = (tid & 3) * 4;
            *reinterpret_cast<f32x4 *>(p.y + ybase + (size_t)(t0 + sy) * p.ldy + c4) =
                *reinterpret_cast<const f32x4 *>(&s_y[sy][c4]);
        }
    }
#pragma unroll
    for (int ri = 0; ri < 4; ri++) {
        const int o = (i0 + ri) * HS + j;
        Fh[o] = Fr[ri];
        if (MOM) Sh[o] = Sr[ri];
    }
}

// ------------------------------------------------------------------ the block's memory, prep fused

// The memory of one Ava-0.4 block in one kernel: the preparation of gpu/arch.rs:1873-1941 (unit q, k
// and erase key, value residual, per-channel log alpha and write strength from the f32 gate
// projections) is computed while each 16-step chunk is staged, then the same register-resident scan
// as mem_scan_kernel runs on it. Staging: wave w prepares steps t0 + 4w .. t0 + 4w + 3 with lane =
// channel, so every norm is a wave reduction and the rank-r gate read-outs are r FMAs per lane with
// the row's z1 values broadcast by readlane. Nothing of the preparation goes through HBM.
struct FusedArgs {
    const float *P;    // [B T][5d]: q | k | v | we | g (raw projections)
    const float *G;    // [B T][2 nh + 2 r]: za | zb | z1a | z1b
    const float *ba, *bb, *off, *wa2, *wb2;  // [nh], [nh], [d], [r][d], [r][d]
    const float *vres;                       // [2] (value residual, blocks after the first) or NULL
    const float *v0;                         // [B T][d]: the first block's raw v (read) or NULL
    float *v0_out;                           // [B T][d]: write the raw v (first block) or NULL
    int T, nh, r;
    float m, cap;
    float *F, *S, *y;  // F, S [B nh][64][64]; y [B T][d]
    int *bad;          // [B] or NULL: streams that met a non-finite memory input
};

// The fused step's guard (gpu/model/fstep/arch.rs:780-783, 861-864): a non-finite gate, key, query or
// value refuses the token before anything is committed. Here a head that stages one leaves its F and
// S as they were (the scan keeps them in registers until the end) and marks its stream in bad.
__device__ __forceinline__ bool finite6(float a, float b, float c, float d, float e, float f) {
    return isfinite(a) && isfinite(b) && isfinite(c) && isfinite(d) && isfinite(e) && isfinite(f);
}

// The gates as the reference forms them, with the correctly rounded-to-an-ulp expf/logf and an IEEE
// divide: a bias of a few ulp in alpha would move the fast weights by that bias over (1 - alpha), ~256x
// for the slowest head (alpha ~ 1 - 2^-8). alpha = exp(logsigmoid(z)), logsigmoid(z) =
// -(relu(-z) + ln(exp(-|z|) + 1)) (gpu/model.rs:618-622); b = 2 sigmoid(z), sigmoid(z) =
// 1 / (exp(-z) + 1) (gpu/model.rs:465-467).
__device__ __forceinline__ float gate_alpha(float z) {
    const float soft = logf(expf(-fabsf(z)) * 1.0f + 1.0f);
    return expf(-(fmaxf(-z, 0.0f) + soft));
}
__device__ __forceinline__ float gate_sig(float z) { return 1.0f / (expf(-z) * 1.0f + 1.0f); }


template <bool MOM, bool PF>
__global__ __launch_bounds__(256, 4) void mem_fused_kernel(FusedArgs p) {
    // 40 KB of LDS and at most 128 VGPRs, so all four heads' blocks of a CU are resident at once
    // (1024 heads of config[3] on 256 CUs run as one round, not two)
    __shared__ __attribute__((aligned(16))) float s_q[TS][HS], s_e[TS][HS], s_v[TS][HS];
    __shared__ __attribute__((aligned(16))) float s_a[TS][HS], s_bk[TS][HS], s_abe[TS][HS];
    __shared__ float s_wa2[32][HS], s_wb2[32][HS];

    const int bh = blockIdx.x;
    const int d = p.nh * HS, ldp = 5 * d, ldg = 2 * p.nh + 2 * p.r;
    const int bi = bh / p.nh, hh = bh - bi * p.nh;
    const size_t row0 = (size_t)bi * p.T;  // the stream's first row
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);     // wave-uniform, so per-step rows are scalar
    int i0, j0;  // scan: this lane's first row and column
    lane_origin(lane, wave, i0, j0);
    const int c = hh * HS + lane;                                   // staging: this lane's channel

    for (int x = tid; x < p.r * HS; x += 256) {
        const int rr = x >> 6, cc = x & 63;
        s_wa2[rr][cc] = p.wa2[(size_t)rr * d + hh * HS + cc];
        s_wb2[rr][cc] = p.wb2[(size_t)rr * d + hh * HS + cc];
    }
    const float offc = p.off[c], bah = p.ba[hh], bbh = p.bb[hh];
    float p0 = 0.0f, p1 = 0.0f;
    if (p.vres) {
        p0 = p.vres[0] * 1.0f + 1.0f;
        p1 = p.vres[1];
    }

    float Fr[16], Sr[16];
    float *Fh = p.F + (size_t)bh * HS * HS, *Sh = MOM ? p.S + (size_t)bh * HS * HS : nullptr;
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int o = (i0 + (m >> 1)) * HS + j0 + (m & 1);
        Fr[m] = Fh[o];
        Sr[m] = MOM ? Sh[o] : 0.0f;
    }

    // the raw inputs of this wave's 4 steps of a chunk, prefetched one chunk ahead
    float rq[4], rk[4], rv[4], rw[4], rv0[4], rz[4], rza[4], rzb[4];
    int nf = 0;  // this lane staged a non-finite value
    auto load = [&](int t0) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int t = min(t0 + wave * 4 + s, p.T - 1);  // past the end: the last step, never used
            const size_t rw_ = row0 + t;
            const float *Pr = p.P + rw_ * ldp, *Gr = p.G + rw_ * ldg;
            rq[s] = Pr[c];
            rk[s] = Pr[d + c];
            rv[s] = Pr[2 * d + c];
            rw[s] = Pr[3 * d + c];
            rv0[s] = p.v0 ? p.v0[rw_ * d + c] : 0.0f;
            rz[s] = (lane & 31) < p.r ? Gr[2 * p.nh + (lane < 32 ? lane : lane - 32 + p.r)] : 0.0f;
            rza[s] = Gr[hh];
            rzb[s] = Gr[p.nh + hh];
        }
    };
    auto stage = [&](int t0) {
        // the rank-r gate read-outs of the wave's 4 steps on the matrix cores (v_mfma_f32_4x4x1, 16
        // blocks): lane l gives A = z(step l & 3, jj) and B = w2(jj, channel l), and register s of the
        // accumulator then holds sum_jj z(s, jj) w2(jj, l). The z rows pass through LDS rows of s_abe
        // that only this wave uses and rewrites below.
        float *zs = &s_abe[wave * 4][0];
#pragma unroll
        for (int s = 0; s < 4; s++) zs[s * HS + lane] = rz[s];
        f32x4 lra = {0.0f, 0.0f, 0.0f, 0.0f}, lrb = {0.0f, 0.0f, 0.0f, 0.0f};
        const float *za = zs + (lane & 3) * HS;
        for (int jj = 0; jj < p.r; jj++) {
            lra = __builtin_amdgcn_mfma_f32_4x4x1f32(za[jj], s_wa2[jj][lane], lra, 0, 0, 0);
            lrb = __builtin_amdgcn_mfma_f32_4x4x1f32(za[32 + jj], s_wb2[jj][lane], lrb, 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int st = wave * 4 + s, t = t0 + st;
            const float ek = rk[s] + rw[s];
            const float sq = wsum(rq[s] * rq[s]), sk = wsum(rk[s] * rk[s]), se = wsum(ek * ek);
            const float qn = rq[s] * rsqrtf(sq + 1e-6f);
            const float kn = rk[s] * rsqrtf(sk + 1e-6f);
            const float en = ek * rsqrtf(se + 1e-6f);
            float v = rv[s];
            if (p.v0_out && t < p.T) p.v0_out[(row0 + t) * d + c] = v;
            if (p.v0) v = v * p0 + rv0[s] * p1;
            const float a = gate_alpha(((rza[s] + bah) + offc) + lra[s]);
            const float bw = gate_sig((rzb[s] + bbh) + lrb[s]) * 2.0f;
            const float bk = bw * kn, abe = (a * bw) * en;
            if (t < p.T && !finite6(qn, en, v, a, bk, abe)) nf = 1;
            s_q[st][lane] = qn;
            s_e[st][lane] = en;
            s_v[st][lane] = v;
            s_a[st][lane] = a;
            s_bk[st][lane] = bk;
            s_abe[st][lane] = abe;
        }
    };

    const float M = p.m, cap = p.cap;
    // y_j is stored by lanes 8g and 8g + 1 (columns j0, j0 + 1); the step's row offset is wave-uniform
    const unsigned ycol = hh * HS + j0 + (lane & 1);
    const BufRes yres = buf_res(p.y + row0 * d, (unsigned)(p.T * d) * 4u);  // this stream's rows of y
    if (PF) load(0);
    for (int t0 = 0; t0 < p.T; t0 += TS) {
        if (!PF) load(t0);
        __syncthreads();  // the previous chunk's LDS reads are done
        stage(t0);
        __syncthreads();
        if (PF && t0 + TS < p.T) load(t0 + TS);  // in flight during this chunk's scan
        const int n = min(TS, p.T - t0);
        auto step = [&](int s) {
            float y0, y1;
            scan_step<MOM>(Fr, Sr, &s_e[s][i0], &s_q[s][i0], &s_a[s][i0], &s_bk[s][i0], &s_abe[s][i0], &s_v[s][j0],
                           M, cap, y0, y1);
            if ((lane & 7) < 2) store_f32(yres, ycol * 4u, (unsigned)((t0 + s) * d) * 4u, (lane & 1) ? y1 : y0);
        };
        if (n == TS) {
            // a whole chunk unrolled: F and S stay in fixed registers (a rolled loop rotates them)
#pragma unroll
            for (int s = 0; s < TS; s++) step(s);
        } else {
            for (int s = 0; s < n; s++) step(s);
        }
    }

    // the workgroup's vote on nf, through LDS the scan no longer reads (a row of s_q): a block-wide
    // vote primitive would add LDS of its own, and 4 x 40 KB is what lets four heads share a CU
    __syncthreads();  // every wave is past its last read of s_q
    const bool wave_nf = __any(nf);
    if (lane == 0) s_q[0][wave] = wave_nf ? 1.0f : 0.0f;
    __syncthreads();
    if (s_q[0][0] + s_q[0][1] + s_q[0][2] + s_q[0][3] != 0.0f) {
        if (tid == 0 && p.bad) p.bad[bi] = 1;
        return;  // nothing committed
    }
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int o = (i0 + (m >> 1)) * HS + j0 + (m & 1);
        Fh[o] = Fr[m];
        if (MOM) Sh[o] = Sr[m];
    }
}

// ------------------------------------------------------------------ the chunked form

// The same recurrence in chunks of CK = 16 tokens with the state contractions on the fp32 matrix
// cores: the algebra of delta_chunk / chunk_core (gpu/arch.rs:1138-1164, 1243-1327). Inside a chunk
// (positions 0..n-1; everything per key channel): Gamma_i = prod_{t<=i} alpha_t; D_im =
// prod_{t=m+1..i} alpha_t, a ratio <= 1 formed pair by pair (no division by Gamma, so strong
// forgetting cannot overflow); the momentum kernel K_ij = sum_{m=j..i} M^(m-j) D_im, i.e. K_ii = 1,
// K_ij = D_ij + M K_i,j+1 (M = 0: K = D). With the write key w = b k and the erase key ah = alpha b e:
//   recalls    (I + Ae) R = (e Gamma_{i-1}) F0 + (e M K_{i-1,0}) S0 + Ke V
//   read-outs  Y = (q Gamma) F0 + (q M K_0) S0 + Qw V - Qa R
//   state      F' = Gamma_{n-1} F0 + M K_{n-1,0} S0 + sum_j K_{n-1,j} (w_j v_j^T - ah_j r_j^T)
//              S' = M^n S0 + sum_j M^(n-1-j) (w_j v_j^T - ah_j r_j^T)
// where Qw_ij = sum_ch q_i K_ij w_j (j <= i), Qa the same with ah, and Ke, Ae the same with e_i and
// K_{i-1,j} (j < i). A closed form per chunk cannot hold the bound clamp(F, +-cap) per token (the
// reference's chunked CPU path has none, arch.rs:1138-1141), so the bounded rule is kept this way: a
// wave whose columns of F start a chunk above cap / 8 runs that chunk token by token with the bound at
// every step (the runaway heads that approach the bound grow by a few per cent per chunk), and the
// closed form's result is bounded at the chunk's end.
//
// One workgroup of 4 waves per head. Wave w owns the value columns 16w..16w+15 of F and S, in the
// accumulator layout of v_mfma_f32_16x16x4f32 (tile mt: key rows 16mt + 4(lane/16) + r, column
// 16w + lane%16, register r). The same registers are the B operand of a product over the key rows
// (k-step r covers rows 16mt + 4(lane/16) + r, the A operand's columns permuted alike), so both
// contractions read the state from the wave's own registers and the chunk needs no state in LDS:
//   [Z_R ; Z_Y] = [e Gamma_{i-1} | e M K_{i-1,0} ; q Gamma_i | q M K_{i,0}] [F0 ; S0]   (32 x 128 x 16)
//   [F' ; S']  += [K_{n-1,j} w_j | -K_{n-1,j} ah_j ; M^(n-1-j) w_j | -M^(n-1-j) ah_j] [V ; R] (128 x 32 x 16)
// The recalls are solved per column inside the wave: lane group g = lane/16 holds rows 4g..4g+3 of a
// column, solves its 4 x 4 block and passes the block's R to the later groups (ds_bpermute).
// The pair matrices Qw, Qa, Ke, Ae are VALU work: lane (row i, channels 4c..4c+3) walks j = 15..0 with
// D and K in registers, and the 16 lanes of a row add their partials by a DPP reduce-scatter.
// The rows of q, e, Gamma and M K_0, which the first contraction reads down a column (16 rows at once),
// are XOR-swizzled in 16-byte chunks (chunk ^ row); the others in 16-column blocks. 40 KB of LDS.
constexpr int CK = 16;

struct ChunkLds {
    float q[CK * HS], e[CK * HS], v[CK * HS], a[CK * HS], w[CK * HS], ah[CK * HS];
    float G[CK * HS];    // row i: Gamma_i
    float MK0[CK * HS];  // row i: M K_{i,0}
    float KL[CK * HS];   // row j: K_{n-1,j}
    float pm[4][CK][CK];  // Qw, Qa, Ke, Ae (row i, column j)
};

// Unrolled steps keep their LDS reads next to their uses: the scheduler would otherwise issue the reads
// of every step at once and spill them.
#define CK_FENCE() __builtin_amdgcn_sched_barrier(0)

__device__ __forceinline__ int swz(int r, int c) { return r * HS + (c ^ ((r & 15) << 2)); }
// The arrays read along rows (v, alpha, w, ah, K_last): 16-column blocks XOR-ed with (row / 4) % 4, so
// the four lane groups, which read rows 4g + r at the same columns, fall on different banks.
__device__ __forceinline__ int rsw(int r, int c) { return r * HS + (c ^ (((r >> 2) & 3) << 4)); }
__device__ __forceinline__ f32x4 ld4s(const float *A, int r, int c) {
    return *reinterpret_cast<const f32x4 *>(A + swz(r, c));
}
__device__ __forceinline__ void st4s(float *A, int r, int c, f32x4 x) { *reinterpret_cast<f32x4 *>(A + swz(r, c)) = x; }
__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }

// One stage of a reduce-scatter over the DPP pairing CTRL (the partner differs in the lane bit that
// `up` tests): lanes with `up` keep x[N..2N) plus the partner's, the others x[0..N) plus the partner's;
// the kept half lands in x[0..N).
template <int CTRL, int N>
__device__ __forceinline__ void rs_stage(float *x, bool up) {
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float lo = x[i], hi = x[i + N];
        x[i] = (up ? hi : lo) + dppf<CTRL>(up ? lo : hi);
    }
}

// M^p in double, rounded once (the reference's m.powi(p) as f32, arch.rs:1289, 1299).
__device__ __forceinline__ float mpow(float M, int p) {
    double r = 1.0;
    for (int i = 0; i < p; i++) r *= (double)M;
    return (float)r;
}

// The pair matrices and the per-channel decay rows of one chunk of n valid positions, from the staged
// alpha, w, ah, q, e (see the comment above). Lane group g of wave w takes row i = w, 7 - w, 8 + w,
// 15 - w (g = 0..3: every wave walks the same 16 steps and the lanes of a group the same row).
template <bool MOM>
__device__ __forceinline__ void chunk_pairs(ChunkLds &s, int wave, int lane, int n, float M) {
    const int g = lane >> 4, cl = lane & 15, c0 = 4 * cl;
    const int i = g == 0 ? wave : g == 1 ? 7 - wave : g == 2 ? 8 + wave : 15 - wave;
    const f32x4 qi = ld4s(s.q, i, c0);
    const f32x4 ei = i + 1 < CK ? ld4s(s.e, i + 1, c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float D[4] = {0.0f, 0.0f, 0.0f, 0.0f}, K[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int half = 1; half >= 0; half--) {
        float x[32];
#pragma unroll
        for (int z = 0; z < 32; z++) x[z] = 0.0f;
#pragma unroll
        for (int jj = 7; jj >= 0; jj--) {
            const int j = 8 * half + jj;
            CK_FENCE();  // one step's loads at a time (the unrolled walk would hoist them all)
            const f32x4 al = ld4(&s.a[rsw(j < CK - 1 ? j + 1 : CK - 1, c0)]);  // alpha_{j+1} (j = 15: unused)
            const f32x4 wj = ld4(&s.w[rsw(j, c0)]), aj = ld4(&s.ah[rsw(j, c0)]);
            const float dl = j == i ? 1.0f : 0.0f;  // D_ii = 1; rows j > i keep D = K = 0
#pragma unroll
            for (int c = 0; c < 4; c++) {
                D[c] = fmaf(D[c], al[c], dl);
                K[c] = MOM ? fmaf(M, K[c], D[c]) : D[c];
                const float kw = K[c] * wj[c], ka = K[c] * aj[c];
                x[jj] = fmaf(qi[c], kw, x[jj]);
                x[8 + jj] = fmaf(qi[c], ka, x[8 + jj]);
                x[16 + jj] = fmaf(ei[c], kw, x[16 + jj]);
                x[24 + jj] = fmaf(ei[c], ka, x[24 + jj]);
            }
            if (i == n - 1) *reinterpret_cast<f32x4 *>(&s.KL[rsw(j, c0)]) = f32x4{K[0], K[1], K[2], K[3]};
        }
        // x[8 m + jj]: matrix m (Qw, Qa, Ke, Ae) at j = 8 half + jj. After the four stages lane cl holds
        // matrix cl >> 2 at j = 8 half + 2 (cl & 3) + {0, 1}, summed over the row's 16 lanes.
        rs_stage<0x140, 16>(x, cl & 8);  // row_mirror: lane cl <-> 15 - cl
        rs_stage<0x141, 8>(x, cl & 4);   // row_half_mirror: cl <-> 7 - cl within each 8
        rs_stage<0x1B, 4>(x, cl & 2);    // quad_perm [3,2,1,0]
        rs_stage<0xB1, 2>(x, cl & 1);    // quad_perm [1,0,3,2]
        const int mm = cl >> 2, row = mm < 2 ? i : (i + 1) & (CK - 1);  // Ke, Ae: row i + 1 (row 0: zeros)
        s.pm[mm][row][8 * half + 2 * (cl & 3)] = x[0];
        s.pm[mm][row][8 * half + 2 * (cl & 3) + 1] = x[1];
    }
    const f32x4 a0 = ld4(&s.a[rsw(0, c0)]);
    f32x4 gm, mk;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        gm[c] = D[c] * a0[c];  // Gamma_i = D_i0 alpha_0
        mk[c] = M * K[c];
    }
    st4s(s.G, i, c0, gm);
    if (MOM) st4s(s.MK0, i, c0, mk);
}

// The state contractions, the recalls and the read-outs of one chunk for wave `wave`'s 16 value
// columns: F and S (in the accumulator layout) advance by the chunk; Y[r] = the read-out at position
// 4 (lane / 16) + r of column 16 wave + lane % 16. The intra-chunk products Ke V, Qw V and Qa R run on
// the matrix cores too: their K dimension is the chunk position, with k-step r covering positions
// 4g + r, so the B operand is the lane's own value or recall at row 4g + r.
template <bool MOM>
__device__ __forceinline__ void chunk_state(const ChunkLds &s, int wave, int lane, int n, float Mn, const float (&mu)[4],
                                            float M, float cap, f32x4 (&Fr)[4], f32x4 (&Sr)[4], float (&Y)[4]) {
    const int g = lane >> 4, cl = lane & 15, col = 16 * wave + cl;
    // A wave whose columns start the chunk above cap / 8 runs it token by token with the bound applied
    // at every step (the closed form cannot bound a head inside the chunk). In this layout a column's 64
    // rows are the wave's four lane groups, so the loop needs no other wave.
    float fmax = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) fmax = fmaxf(fmax, fabsf(Fr[mt][r]));
    fmax = ava::wave_max(fmax);
    if (__builtin_amdgcn_readfirstlane(__float_as_int(fmax)) > __float_as_int(0.125f * cap)) {
#pragma unroll
        for (int r = 0; r < 4; r++) Y[r] = 0.0f;
        for (int t = 0; t < n; t++) {
            float rp = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; mt++) {
                const f32x4 e4 = ld4s(s.e, t, 16 * mt + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; r++) rp = fmaf(e4[r], Fr[mt][r], rp);
            }
            const float rj = xsum32(xsum16(rp)), vj = s.v[rsw(t, col)];
            float yp = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; mt++) {
                const int k0 = 16 * mt + 4 * g;
                const f32x4 a4 = ld4(&s.a[rsw(t, k0)]), w4 = ld4(&s.w[rsw(t, k0)]), x4 = ld4(&s.ah[rsw(t, k0)]);
                const f32x4 q4 = ld4s(s.q, t, k0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float u = fmaf(-x4[r], rj, w4[r] * vj);  // b_i k_i v_j - a_i b_i e_i r_j
                    float f;
                    if (MOM) {
                        Sr[mt][r] = fmaf(M, Sr[mt][r], u);
                        f = fmaf(a4[r], Fr[mt][r], Sr[mt][r]);
                    } else {
                        f = fmaf(a4[r], Fr[mt][r], u);
                    }
                    f = __builtin_amdgcn_fmed3f(f, -cap, cap);
                    Fr[mt][r] = f;
                    yp = fmaf(q4[r], f, yp);
                }
            }
            const float yj = xsum32(xsum16(yp));
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (t == 4 * g + r) Y[r] = yj;
        }
        return;
    }
    // [Z_R ; Z_Y]: A rows are chunk positions (cl), the K dimension the key rows of F and S
    f32x4 zr = {0.0f, 0.0f, 0.0f, 0.0f}, zy = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool first = cl == 0;  // Gamma_{-1} = 1, K_{-1,0} = 0
    const int im1 = first ? 0 : cl - 1;
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        CK_FENCE();
        const int k0 = 16 * mt + 4 * g;
        const f32x4 e4 = ld4s(s.e, cl, k0), q4 = ld4s(s.q, cl, k0);
        const f32x4 gp = ld4s(s.G, im1, k0), gc = ld4s(s.G, cl, k0);
        f32x4 kp = {0.0f, 0.0f, 0.0f, 0.0f}, kc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (MOM) {
            kp = ld4s(s.MK0, im1, k0);
            kc = ld4s(s.MK0, cl, k0);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            zr = __builtin_amdgcn_mfma_f32_16x16x4f32(first ? e4[r] : e4[r] * gp[r], Fr[mt][r], zr, 0, 0, 0);
            zy = __builtin_amdgcn_mfma_f32_16x16x4f32(q4[r] * gc[r], Fr[mt][r], zy, 0, 0, 0);
            if (MOM) {
                zr = __builtin_amdgcn_mfma_f32_16x16x4f32(first ? 0.0f : e4[r] * kp[r], Sr[mt][r], zr, 0, 0, 0);
                zy = __builtin_amdgcn_mfma_f32_16x16x4f32(q4[r] * kc[r], Sr[mt][r], zy, 0, 0, 0);
            }
        }
    }
    CK_FENCE();
    // this column's values at the lane's rows 4g + r; Z_R + Ke V and Z_Y + Qw V
    float Vb[4];
#pragma unroll
    for (int r = 0; r < 4; r++) Vb[r] = s.v[rsw(4 * g + r, col)];
    {
        const f32x4 ke = ld4(&s.pm[2][cl][4 * g]), qw = ld4(&s.pm[0][cl][4 * g]);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            zr = __builtin_amdgcn_mfma_f32_16x16x4f32(ke[r], Vb[r], zr, 0, 0, 0);
            zy = __builtin_amdgcn_mfma_f32_16x16x4f32(qw[r], Vb[r], zy, 0, 0, 0);
        }
    }
    // (I + Ae) R = Z_R + Ke V by 4 x 4 blocks: group blk solves its block, the later groups take the
    // block's R from its lanes and subtract its share
    float R[4] = {0.0f, 0.0f, 0.0f, 0.0f}, rhs[4] = {zr[0], zr[1], zr[2], zr[3]};
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
        CK_FENCE();
        if (g == blk) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const f32x4 ae = ld4(&s.pm[3][4 * blk + r][4 * blk]);
                float x = rhs[r];
#pragma unroll
                for (int rr = 0; rr < r; rr++) x = fmaf(-ae[rr], R[rr], x);
                R[r] = x;
            }
        }
        if (blk < 3) {
            float Rb[4];
#pragma unroll
            for (int r = 0; r < 4; r++) Rb[r] = __shfl(R[r], 16 * blk + cl, 64);
            if (g > blk) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const f32x4 ae = ld4(&s.pm[3][4 * g + r][4 * blk]);
#pragma unroll
                    for (int rr = 0; rr < 4; rr++) rhs[r] = fmaf(-ae[rr], Rb[rr], rhs[r]);
                }
            }
        }
    }
    CK_FENCE();
    // read-outs Y = Z_Y + Qw V - Qa R
    {
        const f32x4 qa = ld4(&s.pm[1][cl][4 * g]);
#pragma unroll
        for (int r = 0; r < 4; r++) zy = __builtin_amdgcn_mfma_f32_16x16x4f32(-qa[r], R[r], zy, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) Y[r] = zy[r];
    }
    // the state: F' = Gamma_{n-1} F0 + M K_{n-1,0} S0 + ..., S' = M^n S0 + ...; A rows are key rows,
    // the K dimension the chunk positions j = 4g + r (V, then R), B the lane's own Vb and R
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        CK_FENCE();
        const int k0 = 16 * mt + 4 * g, ch = 16 * mt + cl;
        const f32x4 gl = ld4s(s.G, n - 1, k0);
        f32x4 F2, S2 = {0.0f, 0.0f, 0.0f, 0.0f};
        if (MOM) {
            const f32x4 mk = ld4s(s.MK0, n - 1, k0);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                F2[r] = fmaf(mk[r], Sr[mt][r], gl[r] * Fr[mt][r]);
                S2[r] = Mn * Sr[mt][r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) F2[r] = gl[r] * Fr[mt][r];
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int o = rsw(4 * g + r, ch);
            const float wv = s.w[o], av = s.ah[o], kl = s.KL[o];
            // F and S alternate, so no product waits on the one just issued
            F2 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv * kl, Vb[r], F2, 0, 0, 0);
            if (MOM) S2 = __builtin_amdgcn_mfma_f32_16x16x4f32(wv * mu[r], Vb[r], S2, 0, 0, 0);
            F2 = __builtin_amdgcn_mfma_f32_16x16x4f32(-(av * kl), R[r], F2, 0, 0, 0);
            if (MOM) S2 = __builtin_amdgcn_mfma_f32_16x16x4f32(-(av * mu[r]), R[r], S2, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) Fr[mt][r] = __builtin_amdgcn_fmed3f(F2[r], -cap, cap);
        if (MOM) Sr[mt] = S2;
    }
}

// The chunked memory over the inputs of ava_mem_scan's layout (G1: one gate per row and head).
template <bool G1, bool MOM>
__global__ __launch_bounds__(256, 2) void mem_chunk_kernel(MemArgs p) {
    __shared__ __attribute__((aligned(16))) ChunkLds s;
    const int T = p.T, nh = p.nh;
    const float M = p.m, cap = p.cap;
    const int bh = blockIdx.x, bi = bh / nh, hh = bh - bi * nh;
    const int tid = threadIdx.x, lane_ = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    f32x4 Fr[4], Sr[4];
    float *Fh = p.F + (size_t)bh * HS * HS;
    float *Sh = MOM ? p.S + (size_t)bh * HS * HS : nullptr;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int o = (16 * mt + 4 * (lane_ >> 4) + r) * HS + 16 * wave + (lane_ & 15);
            Fr[mt][r] = Fh[o];
            Sr[mt][r] = MOM ? Sh[o] : 0.0f;
        }

    const size_t base = (size_t)bi * T * p.ld + (size_t)hh * HS;
    const size_t gbase = G1 ? (size_t)bi * T * p.ldg + hh : (size_t)bi * T * p.ldg + (size_t)hh * HS;
    const size_t ybase = (size_t)bi * T * p.ldy + (size_t)hh * HS;
    // the raw inputs of a chunk, loaded one chunk ahead: thread -> (position tid / 16, channels
    // 4 (tid % 16)..+3)
    const int sp = tid >> 4, si = (tid & 15) * 4;
    f32x4 dq, dk, de, dv, dl, db;
    auto load = [&](int t0) {
        const int t = min(t0 + sp, T - 1);  // past the end: the last position, never used
        const size_t o = base + (size_t)t * p.ld + si;
        dq = ld4(p.q + o);
        dk = ld4(p.k + o);
        de = ld4(p.e + o);
        dv = ld4(p.v + o);
        if (G1) {
            const float l = p.la[gbase + (size_t)t * p.ldg], b = p.b[gbase + (size_t)t * p.ldg];
            dl = f32x4{l, l, l, l};
            db = f32x4{b, b, b, b};
        } else {
            const size_t og = gbase + (size_t)t * p.ldg + si;
            dl = ld4(p.la + og);
            db = ld4(p.b + og);
        }
    };
    load(0);

    float mu[4], Mn = 0.0f;  // M^(n-1-j) at j = 4g + r (0 past n), M^n
    int nprev = -1;
    for (int t0 = 0; t0 < T; t0 += CK) {
        const int n = min(CK, T - t0);
        // the lane index passes through an empty asm each chunk, so the many lane-dependent LDS addresses
        // are formed where they are used instead of being hoisted out of the loop and held in registers
        int lane = lane_;
        asm volatile("" : "+v"(lane));
        const int g = lane >> 4, cl = lane & 15, col = 16 * wave + cl;
        if (n != nprev) {
#pragma unroll
            for (int r = 0; r < 4; r++) mu[r] = 4 * g + r < n ? mpow(M, n - 1 - (4 * g + r)) : 0.0f;
            Mn = mpow(M, n);
            nprev = n;
        }
        f32x4 a4 = {1.0f, 1.0f, 1.0f, 1.0f}, w4 = {0.0f, 0.0f, 0.0f, 0.0f}, x4 = w4;
        if (t0 + sp < T) {
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                a4[cc] = expf(dl[cc]);
                w4[cc] = db[cc] * dk[cc];
                x4[cc] = (a4[cc] * db[cc]) * de[cc];
            }
        } else {
            dq = de = dv = w4;  // positions past the end change nothing
        }
        __syncthreads();  // the previous chunk's LDS reads are done
        st4s(s.q, sp, si, dq);
        st4s(s.e, sp, si, de);
        *reinterpret_cast<f32x4 *>(&s.v[rsw(sp, si)]) = dv;
        *reinterpret_cast<f32x4 *>(&s.a[rsw(sp, si)]) = a4;
        *reinterpret_cast<f32x4 *>(&s.w[rsw(sp, si)]) = w4;
        *reinterpret_cast<f32x4 *>(&s.ah[rsw(sp, si)]) = x4;
        if (t0 + CK < T) load(t0 + CK);  // in flight during this chunk's work
        __syncthreads();
        chunk_pairs<MOM>(s, wave, lane, n, M);
        __syncthreads();
        float Y[4];
        chunk_state<MOM>(s, wave, lane, n, Mn, mu, M, cap, Fr, Sr, Y);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (4 * g + r < n) p.y[ybase + (size_t)(t0 + 4 * g + r) * p.ldy + col] = Y[r];
    }
    // the store addresses from a laundered lane index, so they are not the loads' addresses kept alive
    // across the scan
    int ls = lane_;
    asm volatile("" : "+v"(ls));
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int o = (16 * mt + 4 * (ls >> 4) + r) * HS + 16 * wave + (ls & 15);
            Fh[o] = Fr[mt][r];
            if (MOM) Sh[o] = Sr[mt][r];
        }
}

// ------------------------------------------------------------------ the chunked form on bf16 matrix cores
//
// mem_chunk_kernel's algebra (chunks of CK = 16) with its two state contractions as bf16 products on
// v_mfma_f32_16x16x32_bf16, every operand split in three terms (x = t0 + t1 + t2, each term the bf16
// rounding of what the terms before it leave), of which the six products t_i s_j with i + j < 3 are
// formed: the dropped ones are below 2^-24 of the product, so the contractions keep f32's precision.
//   [Z_R ; Z_Y]  = Lhs [F0 ; S0]        32 x 128 by 128 x 64 (per wave: 2 row tiles x 4 K blocks)
//   [F' ; S']   += Wm [V ; R]           128 x 32 by 32 x 64  (per wave: 8 row tiles x 1 K block)
// Lhs (rows e Gamma_{i-1} | e M K_{i-1,0}, then q Gamma_i | q M K_{i,0}) and Wm (rows K_{n-1,j} w_j |
// -K_{n-1,j} ah_j, then M^(n-1-j) w_j | -M^(n-1-j) ah_j) are the same for the four waves, so they are
// formed once per chunk, split, and stored in LDS already in the A-operand layout of the instruction
// (lane l of a tile: row l % 16, K slots 8 (l / 16) .. + 7; one 16-byte read per term). Each wave splits
// its own right operands, and the K order is chosen so that they are the lane's own registers: K block
// kb of the first product takes state tiles 2 kb and 2 kb + 1 of [F0 tiles 0..3 | S0 tiles 0..3], slot s
// of lane group g being row 4 g + s of the first tile (s < 4) or 4 g + s - 4 of the second, exactly the
// rows the accumulator layout leaves in the lane; in the second product slot s of group g is position
// 4 g + s of V (s < 4) or of R (the recalls, in the same accumulator layout). The pair walk writes Lhs
// directly (a lane ends its row's walk with Gamma_i and M K_i0 for its four channels); Wm is formed after
// it from the last row's K_{n-1,j}, in the LDS the walk's q, e and alpha leave. The intra-chunk products
// (Ke V, Qw V, Qa R) and the recalls' solve stay f32 (v_mfma_f32_16x16x4f32), as in mem_chunk_kernel.
// The bound: when any wave's columns of F start a chunk above cap / 8, the whole workgroup runs that
// chunk token by token with the bound at every step. 69 KB of LDS: two heads per CU.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int SP = HS + 4;  // row stride of the staged rows (column reads of four rows 4 apart miss each other's banks)

struct ChunkBfLds {
    float v[CK * SP], w[CK * SP], ah[CK * SP], KL[CK * SP];
    float pm[4][CK][CK];  // Qw, Qa, Ke, Ae
    float gl[HS];         // Gamma_{n-1}
    int fb[4];            // per wave: its columns of F start the chunk above cap / 8
    bf16x8 lhs[3][2][4][64];  // term, (recall rows, read rows), K block, lane
    union {
        struct {
            float q[CK * SP], e[CK * SP], a[CK * SP];
        } in;
        bf16x8 wm[3][8][64];  // term, state row tile (F 0..3, S 4..7), lane
    } x;
};

__device__ __forceinline__ void split3(float x, __bf16 &t0, __bf16 &t1, __bf16 &t2) {
    t0 = (__bf16)x;
    x = x - (float)t0;
    t1 = (__bf16)x;
    x = x - (float)t1;
    t2 = (__bf16)x;
}
struct Terms {
    bf16x8 t[3];
};
__device__ __forceinline__ Terms split8(const float (&x)[8]) {
    Terms r;
#pragma unroll
    for (int z = 0; z < 8; z++) {
        __bf16 a, b, c;
        split3(x[z], a, b, c);
        r.t[0][z] = a;
        r.t[1][z] = b;
        r.t[2][z] = c;
    }
    return r;
}
// acc m (+)= a0 b0, x (+)= a0 b1 + a1 b0, y (+)= a0 b2 + a1 b1 + a2 b0 (three chains, so consecutive
// instructions rarely wait on each other); the total is m + (x + y)
struct Acc4 {
    f32x4 m, x, y;
};
__device__ __forceinline__ void mfma3(Acc4 &c, const bf16x8 *a, const Terms &b) {
    c.m = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b.t[0], c.m, 0, 0, 0);
    c.x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b.t[1], c.x, 0, 0, 0);
    c.y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b.t[2], c.y, 0, 0, 0);
    c.x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b.t[0], c.x, 0, 0, 0);
    c.y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b.t[1], c.y, 0, 0, 0);
    c.y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b.t[0], c.y, 0, 0, 0);
}
__device__ __forceinline__ f32x4 total4(const Acc4 &c) { return c.m + (c.x + c.y); }

// The LDS slot of lane ln's A operand in K block kb of Lhs: the slot index's low bits XOR-ed with the lane
// group and kb's parity, so that the pair walk's 8-byte writes (16 lanes of one row, four lane groups,
// two K blocks, two halves) fall on distinct banks; any 16 consecutive lanes still read 16 distinct
// bank groups.
__device__ __forceinline__ int lhs_slot(int ln, int kb) { return ln ^ (((ln >> 4) & 3) << 2) ^ ((kb & 1) << 1); }

// Four consecutive K rows kr0 .. kr0 + 3 (kr0 = 64 part + 4 cl: F channels, then S channels) of Lhs row
// `row` of tile ot, split, into their A-operand slots.
__device__ __forceinline__ void lhs_put(ChunkBfLds &s, int ot, int row, int part, int cl, const f32x4 &x) {
    const int kb = 2 * part + (cl >> 3), ln = lhs_slot(row + 16 * (cl & 3), kb), s0 = 4 * ((cl >> 2) & 1);
    bf16x4 t0, t1, t2;
#pragma unroll
    for (int z = 0; z < 4; z++) {
        __bf16 a, b, c;
        split3(x[z], a, b, c);
        t0[z] = a;
        t1[z] = b;
        t2[z] = c;
    }
    *reinterpret_cast<bf16x4 *>(reinterpret_cast<__bf16 *>(&s.lhs[0][ot][kb][ln]) + s0) = t0;
    *reinterpret_cast<bf16x4 *>(reinterpret_cast<__bf16 *>(&s.lhs[1][ot][kb][ln]) + s0) = t1;
    *reinterpret_cast<bf16x4 *>(reinterpret_cast<__bf16 *>(&s.lhs[2][ot][kb][ln]) + s0) = t2;
}

// The pair walk of chunk_pairs (same rows per lane, same order of operations) over the padded rows,
// ending in the lane's Lhs entries: read row i (q_i Gamma_i, q_i M K_i0) and recall row i + 1
// (e_{i+1} Gamma_i, e_{i+1} M K_i0); the lanes of row 15 write recall row 0 (e_0, 0).
template <bool MOM>
__device__ __forceinline__ void chunk_walk_bf(ChunkBfLds &s, int wave, int lane, int n, float M) {
    const int g = lane >> 4, cl = lane & 15, c0 = 4 * cl;
    const int i = g == 0 ? wave : g == 1 ? 7 - wave : g == 2 ? 8 + wave : 15 - wave;
    const f32x4 qi = ld4(&s.x.in.q[i * SP + c0]);
    const f32x4 ei = i + 1 < CK ? ld4(&s.x.in.e[(i + 1) * SP + c0]) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float D[4] = {0.0f, 0.0f, 0.0f, 0.0f}, K[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int half = 1; half >= 0; half--) {
        float x[32];
#pragma unroll
        for (int z = 0; z < 32; z++) x[z] = 0.0f;
#pragma unroll
        for (int jj = 7; jj >= 0; jj--) {
            const int j = 8 * half + jj;
            CK_FENCE();
            const f32x4 al = ld4(&s.x.in.a[(j < CK - 1 ? j + 1 : CK - 1) * SP + c0]);
            const f32x4 wj = ld4(&s.w[j * SP + c0]), aj = ld4(&s.ah[j * SP + c0]);
            const float dl = j == i ? 1.0f : 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                D[c] = fmaf(D[c], al[c], dl);
                K[c] = MOM ? fmaf(M, K[c], D[c]) : D[c];
                const float kw = K[c] * wj[c], ka = K[c] * aj[c];
                x[jj] = fmaf(qi[c], kw, x[jj]);
                x[8 + jj] = fmaf(qi[c], ka, x[8 + jj]);
                x[16 + jj] = fmaf(ei[c], kw, x[16 + jj]);
                x[24 + jj] = fmaf(ei[c], ka, x[24 + jj]);
            }
            if (i == n - 1) *reinterpret_cast<f32x4 *>(&s.KL[j * SP + c0]) = f32x4{K[0], K[1], K[2], K[3]};
        }
        rs_stage<0x140, 16>(x, cl & 8);
        rs_stage<0x141, 8>(x, cl & 4);
        rs_stage<0x1B, 4>(x, cl & 2);
        rs_stage<0xB1, 2>(x, cl & 1);
        const int mm = cl >> 2, row = mm < 2 ? i : (i + 1) & (CK - 1);
        s.pm[mm][row][8 * half + 2 * (cl & 3)] = x[0];
        s.pm[mm][row][8 * half + 2 * (cl & 3) + 1] = x[1];
    }
    const f32x4 a0 = ld4(&s.x.in.a[c0]);
    f32x4 gm, mk;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        gm[c] = D[c] * a0[c];
        mk[c] = M * K[c];
    }
    if (i == n - 1) *reinterpret_cast<f32x4 *>(&s.gl[c0]) = gm;
    f32x4 y0, y1;
#pragma unroll
    for (int c = 0; c < 4; c++) y0[c] = qi[c] * gm[c];
    lhs_put(s, 1, i, 0, cl, y0);
    if (MOM) {
#pragma unroll
        for (int c = 0; c < 4; c++) y1[c] = qi[c] * mk[c];
        lhs_put(s, 1, i, 1, cl, y1);
    }
    if (i + 1 < CK) {
#pragma unroll
        for (int c = 0; c < 4; c++) y0[c] = ei[c] * gm[c];
        lhs_put(s, 0, i + 1, 0, cl, y0);
        if (MOM) {
#pragma unroll
            for (int c = 0; c < 4; c++) y1[c] = ei[c] * mk[c];
            lhs_put(s, 0, i + 1, 1, cl, y1);
        }
    } else {
        lhs_put(s, 0, 0, 0, cl, ld4(&s.x.in.e[c0]));  // Gamma_{-1} = 1
        if (MOM) lhs_put(s, 0, 0, 1, cl, f32x4{0.0f, 0.0f, 0.0f, 0.0f});  // K_{-1,0} = 0
    }
}

// Wm's A operands: thread tid forms lane tid % 64 of state tile tid / 64 (and, with momentum, of tile
// 4 + tid / 64): slots 0..3 the V positions 4 g .., 4..7 the R positions, g = (tid % 64) / 16.
template <bool MOM>
__device__ __forceinline__ void chunk_wm_bf(ChunkBfLds &s, int tid, const float (&mu)[4]) {
    const int lane = tid & 63, g = lane >> 4, ch = 16 * (tid >> 6) + (lane & 15);
    float wv[4], av[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        wv[r] = s.w[(4 * g + r) * SP + ch];
        av[r] = s.ah[(4 * g + r) * SP + ch];
    }
    {
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float kl = s.KL[(4 * g + r) * SP + ch];
            x[r] = wv[r] * kl;
            x[4 + r] = -(av[r] * kl);
        }
        const Terms t = split8(x);
#pragma unroll
        for (int z = 0; z < 3; z++) s.x.wm[z][tid >> 6][lane] = t.t[z];
    }
    if (MOM) {
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            x[r] = wv[r] * mu[r];
            x[4 + r] = -(av[r] * mu[r]);
        }
        const Terms t = split8(x);
#pragma unroll
        for (int z = 0; z < 3; z++) s.x.wm[z][4 + (tid >> 6)][lane] = t.t[z];
    }
}

// One chunk of wave `wave`'s 16 columns by the closed form (chunk_state's algebra, the contractions on
// the bf16 matrix cores).
template <bool MOM>
__device__ __forceinline__ void chunk_state_bf(const ChunkBfLds &s, int wave, int lane, float Mn, float M, float cap,
                                               f32x4 (&Fr)[4], f32x4 (&Sr)[4], float (&Y)[4]) {
    const int g = lane >> 4, cl = lane & 15, col = 16 * wave + cl;
    // [Z_R ; Z_Y] = Lhs [F0 ; S0]
    Acc4 cr{{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}}, cy = cr;
#pragma unroll
    for (int kb = 0; kb < (MOM ? 4 : 2); kb++) {
        CK_FENCE();
        float xb[8];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            xb[r] = kb < 2 ? Fr[2 * kb][r] : Sr[2 * kb - 4][r];
            xb[4 + r] = kb < 2 ? Fr[2 * kb + 1][r] : Sr[2 * kb - 3][r];
        }
        const Terms b = split8(xb);
        const int sl = lhs_slot(lane, kb);
        const bf16x8 ar[3] = {s.lhs[0][0][kb][sl], s.lhs[1][0][kb][sl], s.lhs[2][0][kb][sl]};
        const bf16x8 ay[3] = {s.lhs[0][1][kb][sl], s.lhs[1][1][kb][sl], s.lhs[2][1][kb][sl]};
        mfma3(cr, ar, b);
        mfma3(cy, ay, b);
    }
    f32x4 zr = total4(cr), zy = total4(cy);
    CK_FENCE();
    float Vb[4];
#pragma unroll
    for (int r = 0; r < 4; r++) Vb[r] = s.v[(4 * g + r) * SP + col];
    {
        const f32x4 ke = ld4(&s.pm[2][cl][4 * g]), qw = ld4(&s.pm[0][cl][4 * g]);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            zr = __builtin_amdgcn_mfma_f32_16x16x4f32(ke[r], Vb[r], zr, 0, 0, 0);
            zy = __builtin_amdgcn_mfma_f32_16x16x4f32(qw[r], Vb[r], zy, 0, 0, 0);
        }
    }
    // (I + Ae) R = Z_R + Ke V (mem_chunk_kernel's blocked solve)
    float R[4] = {0.0f, 0.0f, 0.0f, 0.0f}, rhs[4] = {zr[0], zr[1], zr[2], zr[3]};
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
        CK_FENCE();
        if (g == blk) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const f32x4 ae = ld4(&s.pm[3][4 * blk + r][4 * blk]);
                float x = rhs[r];
#pragma unroll
                for (int rr = 0; rr < r; rr++) x = fmaf(-ae[rr], R[rr], x);
                R[r] = x;
            }
        }
        if (blk < 3) {
            float Rb[4];
#pragma unroll
            for (int r = 0; r < 4; r++) Rb[r] = __shfl(R[r], 16 * blk + cl, 64);
            if (g > blk) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const f32x4 ae = ld4(&s.pm[3][4 * g + r][4 * blk]);
#pragma unroll
                    for (int rr = 0; rr < 4; rr++) rhs[r] = fmaf(-ae[rr], Rb[rr], rhs[r]);
                }
            }
        }
    }
    CK_FENCE();
    {
        const f32x4 qa = ld4(&s.pm[1][cl][4 * g]);
#pragma unroll
        for (int r = 0; r < 4; r++) zy = __builtin_amdgcn_mfma_f32_16x16x4f32(-qa[r], R[r], zy, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) Y[r] = zy[r];
    }
    // [F' ; S'] = prefill + Wm [V ; R]; the F tiles first (their prefill reads the old S)
    float xb[8];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        xb[r] = Vb[r];
        xb[4 + r] = R[r];
    }
    const Terms b = split8(xb);
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        CK_FENCE();
        const int k0 = 16 * mt + 4 * g;
        const f32x4 gl = ld4(&s.gl[k0]);
        Acc4 c{{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        if (MOM) {
            const f32x4 k0r = ld4(&s.KL[k0]);  // K_{n-1,0}
#pragma unroll
            for (int r = 0; r < 4; r++) c.m[r] = fmaf(M * k0r[r], Sr[mt][r], gl[r] * Fr[mt][r]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) c.m[r] = gl[r] * Fr[mt][r];
        }
        const bf16x8 a[3] = {s.x.wm[0][mt][lane], s.x.wm[1][mt][lane], s.x.wm[2][mt][lane]};
        mfma3(c, a, b);
        const f32x4 f = total4(c);
#pragma unroll
        for (int r = 0; r < 4; r++) Fr[mt][r] = __builtin_amdgcn_fmed3f(f[r], -cap, cap);
    }
    if (MOM) {
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            CK_FENCE();
            Acc4 c{{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
            for (int r = 0; r < 4; r++) c.m[r] = Mn * Sr[mt][r];
            const bf16x8 a[3] = {s.x.wm[0][4 + mt][lane], s.x.wm[1][4 + mt][lane], s.x.wm[2][4 + mt][lane]};
            mfma3(c, a, b);
            Sr[mt] = total4(c);
        }
    }
}

// One chunk of wave `wave`'s columns token by token with the bound at every step (mem_chunk_kernel's
// fallback over the padded rows).
template <bool MOM>
__device__ __forceinline__ void chunk_tokens_bf(const ChunkBfLds &s, int wave, int lane, int n, float M, float cap,
                                                f32x4 (&Fr)[4], f32x4 (&Sr)[4], float (&Y)[4]) {
    const int g = lane >> 4, cl = lane & 15, col = 16 * wave + cl;
#pragma unroll
    for (int r = 0; r < 4; r++) Y[r] = 0.0f;
    for (int t = 0; t < n; t++) {
        float rp = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const f32x4 e4 = ld4(&s.x.in.e[t * SP + 16 * mt + 4 * g]);
#pragma unroll
            for (int r = 0; r < 4; r++) rp = fmaf(e4[r], Fr[mt][r], rp);
        }
        const float rj = xsum32(xsum16(rp)), vj = s.v[t * SP + col];
        float yp = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const int k0 = 16 * mt + 4 * g;
            const f32x4 a4 = ld4(&s.x.in.a[t * SP + k0]), w4 = ld4(&s.w[t * SP + k0]), x4 = ld4(&s.ah[t * SP + k0]);
            const f32x4 q4 = ld4(&s.x.in.q[t * SP + k0]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float u = fmaf(-x4[r], rj, w4[r] * vj);
                float f;
                if (MOM) {
                    Sr[mt][r] = fmaf(M, Sr[mt][r], u);
                    f = fmaf(a4[r], Fr[mt][r], Sr[mt][r]);
                } else {
                    f = fmaf(a4[r], Fr[mt][r], u);
                }
                f = __builtin_amdgcn_fmed3f(f, -cap, cap);
                Fr[mt][r] = f;
                yp = fmaf(q4[r], f, yp);
            }
        }
        const float yj = xsum32(xsum16(yp));
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (t == 4 * g + r) Y[r] = yj;
    }
}

template <bool G1, bool MOM>
__global__ __launch_bounds__(256, 2) void mem_chunk_bf_kernel(MemArgs p) {
    __shared__ __attribute__((aligned(16))) ChunkBfLds s;
    const int T = p.T, nh = p.nh;
    const float M = p.m, cap = p.cap;
    const int bh = blockIdx.x, bi = bh / nh, hh = bh - bi * nh;
    const int tid = threadIdx.x, lane_ = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    f32x4 Fr[4], Sr[4];
    float *Fh = p.F + (size_t)bh * HS * HS;
    float *Sh = MOM ? p.S + (size_t)bh * HS * HS : nullptr;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int o = (16 * mt + 4 * (lane_ >> 4) + r) * HS + 16 * wave + (lane_ & 15);
            Fr[mt][r] = Fh[o];
            Sr[mt][r] = MOM ? Sh[o] : 0.0f;
        }

    const size_t base = (size_t)bi * T * p.ld + (size_t)hh * HS;
    const size_t gbase = G1 ? (size_t)bi * T * p.ldg + hh : (size_t)bi * T * p.ldg + (size_t)hh * HS;
    const size_t ybase = (size_t)bi * T * p.ldy + (size_t)hh * HS;
    const int sp = tid >> 4, si = (tid & 15) * 4;
    f32x4 dq, dk, de, dv, dl, db;
    auto load = [&](int t0) {
        const int t = min(t0 + sp, T - 1);
        const size_t o = base + (size_t)t * p.ld + si;
        dq = ld4(p.q + o);
        dk = ld4(p.k + o);
        de = ld4(p.e + o);
        dv = ld4(p.v + o);
        if (G1) {
            const float l = p.la[gbase + (size_t)t * p.ldg], b = p.b[gbase + (size_t)t * p.ldg];
            dl = f32x4{l, l, l, l};
            db = f32x4{b, b, b, b};
        } else {
            const size_t og = gbase + (size_t)t * p.ldg + si;
            dl = ld4(p.la + og);
            db = ld4(p.b + og);
        }
    };
    load(0);

    float mu[4], Mn = 0.0f;
    int nprev = -1;
    for (int t0 = 0; t0 < T; t0 += CK) {
        const int n = min(CK, T - t0);
        int lane = lane_;
        asm volatile("" : "+v"(lane));
        const int g = lane >> 4, cl = lane & 15, col = 16 * wave + cl;
        if (n != nprev) {
#pragma unroll
            for (int r = 0; r < 4; r++) mu[r] = 4 * g + r < n ? mpow(M, n - 1 - (4 * g + r)) : 0.0f;
            Mn = mpow(M, n);
            nprev = n;
        }
        f32x4 a4 = {1.0f, 1.0f, 1.0f, 1.0f}, w4 = {0.0f, 0.0f, 0.0f, 0.0f}, x4 = w4;
        if (t0 + sp < T) {
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                a4[cc] = expf(dl[cc]);
                w4[cc] = db[cc] * dk[cc];
                x4[cc] = (a4[cc] * db[cc]) * de[cc];
            }
        } else {
            dq = de = dv = w4;
        }
        float fmax = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) fmax = fmaxf(fmax, fabsf(Fr[mt][r]));
        fmax = ava::wave_max(fmax);
        __syncthreads();  // the previous chunk's LDS reads are done
        *reinterpret_cast<f32x4 *>(&s.x.in.q[sp * SP + si]) = dq;
        *reinterpret_cast<f32x4 *>(&s.x.in.e[sp * SP + si]) = de;
        *reinterpret_cast<f32x4 *>(&s.x.in.a[sp * SP + si]) = a4;
        *reinterpret_cast<f32x4 *>(&s.v[sp * SP + si]) = dv;
        *reinterpret_cast<f32x4 *>(&s.w[sp * SP + si]) = w4;
        *reinterpret_cast<f32x4 *>(&s.ah[sp * SP + si]) = x4;
        if (lane == 0) s.fb[wave] = fmax > 0.125f * cap ? 1 : 0;
        if (t0 + CK < T) load(t0 + CK);
        __syncthreads();
        float Y[4];
        if (s.fb[0] | s.fb[1] | s.fb[2] | s.fb[3]) {
            chunk_tokens_bf<MOM>(s, wave, lane, n, M, cap, Fr, Sr, Y);
        } else {
            chunk_walk_bf<MOM>(s, wave, lane, n, M);
            __syncthreads();  // KL, pm, Lhs written; q, e, alpha no longer read
            chunk_wm_bf<MOM>(s, tid, mu);
            __syncthreads();
            chunk_state_bf<MOM>(s, wave, lane, Mn, M, cap, Fr, Sr, Y);
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (4 * g + r < n) p.y[ybase + (size_t)(t0 + 4 * g + r) * p.ldy + col] = Y[r];
    }
    int ls = lane_;
    asm volatile("" : "+v"(ls));
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int o = (16 * mt + 4 * (ls >> 4) + r) * HS + 16 * wave + (ls & 15);
            Fh[o] = Fr[mt][r];
            if (MOM) Sh[o] = Sr[mt][r];
        }
}

// One token per stream (decode, T == 1): the same recurrence step as mem_fused_kernel, laid out for
// streaming the state rather than for a long scan. Wave w holds rows 16w..16w+15 of F and S and lane
// j column j, so each of the lane's 16 + 16 state loads and stores is one 256-byte row per wave
// (coalesced). Wave 0 stages the step's factors (the same formulas as mem_fused_kernel's staging, the
// rank-r gate read-outs as fma chains in jj order) while the other waves' state loads are in flight;
// the column sums r_j and y_j add four per-wave partials in LDS.
template <bool MOM>
__global__ __launch_bounds__(256) void mem_step_kernel(FusedArgs p) {
    __shared__ float s_q[HS], s_e[HS], s_v[HS], s_a[HS], s_bk[HS], s_abe[HS];
    __shared__ float s_part[4][HS], s_lr[2][4][HS];
    const int bh = blockIdx.x;
    const int d = p.nh * HS, ldp = 5 * d, ldg = 2 * p.nh + 2 * p.r;
    const int bi = bh / p.nh, hh = bh - bi * p.nh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t row = (size_t)bi;  // T == 1: stream bi's only row
    float *Fh = p.F + (size_t)bh * HS * HS, *Sh = MOM ? p.S + (size_t)bh * HS * HS : nullptr;
    const int i0 = wave * 16;
    // the state is streamed once each way: non-temporal loads and stores
    float Fr[16], Sr[16];
#pragma unroll
    for (int m = 0; m < 16; m++) {
        Fr[m] = __builtin_nontemporal_load(Fh + (i0 + m) * HS + lane);
        Sr[m] = MOM ? __builtin_nontemporal_load(Sh + (i0 + m) * HS + lane) : 0.0f;
    }
    const int c = hh * HS + lane;
    const float *Gr = p.G + row * ldg;
    int nf = 0;
    {
        // the rank-r gate read-outs, a quarter of the rank per wave (fma chains in jj order)
        const int q = (p.r + 3) / 4, j0 = wave * q, j1 = min(p.r, j0 + q);
        float la = 0.0f, lb = 0.0f;
#pragma unroll 8
        for (int jj = j0; jj < j1; jj++) {
            la = fmaf(Gr[2 * p.nh + jj], p.wa2[(size_t)jj * d + c], la);
            lb = fmaf(Gr[2 * p.nh + p.r + jj], p.wb2[(size_t)jj * d + c], lb);
        }
        s_lr[0][wave][lane] = la;
        s_lr[1][wave][lane] = lb;
    }
    __syncthreads();
    if (wave == 0) {
        const float *Pr = p.P + row * ldp;
        const float rq = Pr[c], rk = Pr[d + c], rv = Pr[2 * d + c], rw = Pr[3 * d + c];
        const float lra = ((s_lr[0][0][lane] + s_lr[0][1][lane]) + s_lr[0][2][lane]) + s_lr[0][3][lane];
        const float lrb = ((s_lr[1][0][lane] + s_lr[1][1][lane]) + s_lr[1][2][lane]) + s_lr[1][3][lane];
        const float ek = rk + rw;
        const float sq = wsum(rq * rq), sk = wsum(rk * rk), se = wsum(ek * ek);
        const float qn = rq * rsqrtf(sq + 1e-6f);
        const float kn = rk * rsqrtf(sk + 1e-6f);
        const float en = ek * rsqrtf(se + 1e-6f);
        float v = rv;
        if (p.v0_out) p.v0_out[row * d + c] = v;
        if (p.v0) {
            const float p0 = p.vres ? p.vres[0] * 1.0f + 1.0f : 0.0f, p1 = p.vres ? p.vres[1] : 0.0f;
            v = v * p0 + p.v0[row * d + c] * p1;
        }
        const float a = gate_alpha(((Gr[hh] + p.ba[hh]) + p.off[c]) + lra);
        const float bw = gate_sig((Gr[p.nh + hh] + p.bb[hh]) + lrb) * 2.0f;
        const float bk = bw * kn, abe = (a * bw) * en;
        nf = !finite6(qn, en, v, a, bk, abe);
        s_q[lane] = qn;
        s_e[lane] = en;
        s_v[lane] = v;
        s_a[lane] = a;
        s_bk[lane] = bk;
        s_abe[lane] = abe;
    }
    const bool refuse = __syncthreads_or(nf) != 0;  // every thread: a non-finite staged value
    if (refuse && tid == 0 && p.bad) p.bad[bi] = 1;
    // r_j = sum_i e_i F_ij
    float r = 0.0f;
#pragma unroll
    for (int m = 0; m < 16; m++) r = fmaf(s_e[i0 + m], Fr[m], r);
    s_part[wave][lane] = r;
    __syncthreads();
    r = ((s_part[0][lane] + s_part[1][lane]) + s_part[2][lane]) + s_part[3][lane];
    const float vj = s_v[lane], M = p.m, cap = p.cap;
    float y = 0.0f;
#pragma unroll
    for (int m = 0; m < 16; m++) {
        const int i = i0 + m;
        const float u = fmaf(-s_abe[i], r, s_bk[i] * vj);
        float f;
        if (MOM) {
            Sr[m] = fmaf(M, Sr[m], u);
            f = fmaf(s_a[i], Fr[m], Sr[m]);
        } else {
            f = fmaf(s_a[i], Fr[m], u);
        }
        f = __builtin_amdgcn_fmed3f(f, -cap, cap);
        Fr[m] = f;
        y = fmaf(s_q[i], f, y);
        if (!refuse) {
            __builtin_nontemporal_store(f, Fh + i * HS + lane);
            if (MOM) __builtin_nontemporal_store(Sr[m], Sh + i * HS + lane);
        }
    }
    __syncthreads();  // every wave has read s_part
    s_part[wave][lane] = y;
    __syncthreads();
    if (wave == 0)
        p.y[row * d + hh * HS + lane] = ((s_part[0][lane] + s_part[1][lane]) + s_part[2][lane]) + s_part[3][lane];
}

}  // namespace

namespace ava {

// The scan over heads laid out in a [B T][ld] matrix (see the file comment). g = 1 or 64 gate columns.
int mem_scan_strided(const float *q, const float *k, const float *e, const float *v, const float *la, const float *b,
                     int B, int T, int nh, int ld, int g, int ldg, float m, float cap, float *F, float *S, float *y,
                     int ldy, hipStream_t st) {
    AVA_REQUIRE(q && k && e && v && la && b && F && y, AVA_ERR_ARG, "mem_scan: NULL buffer");
    AVA_REQUIRE(m == 0.0f || S, AVA_ERR_ARG, "mem_scan: momentum %g needs S", (double)m);
    AVA_REQUIRE(g == 1 || g == HS, AVA_ERR_ARG, "mem_scan: gate width %d (1 or 64)", g);
    AVA_REQUIRE(B >= 0 && T >= 0 && nh > 0 && ld % 4 == 0 && ldy % 4 == 0 && (g == 1 || ldg % 4 == 0), AVA_ERR_SHAPE,
                "mem_scan: B=%d T=%d nh=%d ld=%d ldg=%d ldy=%d", B, T, nh, ld, ldg, ldy);
    if (B == 0 || T == 0) return AVA_OK;
    MemArgs a{q, k, e, v, la, b, T, nh, ld, ldg, ldy, m, cap, F, S, y};
    dim3 block(256);
    // fewer than 512 heads: four workgroups per head (AVA_MEM_SCAN_GROUPS=1 or 4 chooses)
    static const int forced = getenv("AVA_MEM_SCAN_GROUPS") ? atoi(getenv("AVA_MEM_SCAN_GROUPS")) : 0;
    const bool cols = forced == 4 || (forced != 1 && B * nh < 512);
    if (cols) {
        dim3 grid(B * nh * 4);
        if (g == 1) {
            if (m != 0.0f) mem_scan_cols_kernel<true, true><<<grid, block, 0, st>>>(a);
            else mem_scan_cols_kernel<true, false><<<grid, block, 0, st>>>(a);
        } else {
            if (m != 0.0f) mem_scan_cols_kernel<false, true><<<grid, block, 0, st>>>(a);
            else mem_scan_cols_kernel<false, false><<<grid, block, 0, st>>>(a);
        }
    } else {
        dim3 grid(B * nh);
        if (g == 1) {
            if (m != 0.0f) mem_scan_kernel<true, true><<<grid, block, 0, st>>>(a);
            else mem_scan_kernel<true, false><<<grid, block, 0, st>>>(a);
        } else {
            if (m != 0.0f) mem_scan_kernel<false, true><<<grid, block, 0, st>>>(a);
            else mem_scan_kernel<false, false><<<grid, block, 0, st>>>(a);
        }
    }
    AVA_LAUNCHED("mem_scan");
    return AVA_OK;
}

// The block's memory from the raw projections P and gate projections G (see mem_fused_kernel).
int mem_block(const float *P, const float *G, int B, int T, int nh, int r, const float *ba, const float *bb,
              const float *off, const float *wa2, const float *wb2, const float *vres, const float *v0, float *v0_out,
              float m, float cap, float *F, float *S, float *y, int *bad, hipStream_t st) {
    AVA_REQUIRE(P && G && ba && bb && off && wa2 && wb2 && F && y, AVA_ERR_ARG, "mem_block: NULL buffer");
    AVA_REQUIRE(m == 0.0f || S, AVA_ERR_ARG, "mem_block: momentum needs S");
    AVA_REQUIRE(B > 0 && T > 0 && nh > 0 && r > 0 && r <= 32, AVA_ERR_SHAPE, "mem_block: B=%d T=%d nh=%d r=%d", B, T,
                nh, r);
    FusedArgs a{P, G, ba, bb, off, wa2, wb2, vres, v0, v0_out, T, nh, r, m, cap, F, S, y, bad};
    if (T == 1) {
        if (m != 0.0f) mem_step_kernel<true><<<B * nh, 256, 0, st>>>(a);
        else mem_step_kernel<false><<<B * nh, 256, 0, st>>>(a);
        AVA_LAUNCHED("mem_step");
        return AVA_OK;
    }
    // the token loop (the chunk's inputs are staged by the scan's own waves); the chunked form
    // (mem_chunk_strided) measures slower on this shape
    if (m != 0.0f) mem_fused_kernel<true, false><<<B * nh, 256, 0, st>>>(a);
    else mem_fused_kernel<false, false><<<B * nh, 256, 0, st>>>(a);
    AVA_LAUNCHED("mem_block");
    return AVA_OK;
}

// The scan of mem_scan_strided in the chunked form.
int mem_chunk_strided(const float *q, const float *k, const float *e, const float *v, const float *la, const float *b,
                      int B, int T, int nh, int ld, int g, int ldg, float m, float cap, float *F, float *S, float *y,
                      int ldy, hipStream_t st) {
    AVA_REQUIRE(q && k && e && v && la && b && F && y, AVA_ERR_ARG, "mem_chunk: NULL buffer");
    AVA_REQUIRE(m == 0.0f || S, AVA_ERR_ARG, "mem_chunk: momentum %g needs S", (double)m);
    AVA_REQUIRE(g == 1 || g == HS, AVA_ERR_ARG, "mem_chunk: gate width %d (1 or 64)", g);
    AVA_REQUIRE(B >= 0 && T >= 0 && nh > 0 && ld % 4 == 0 && ldy % 4 == 0 && (g == 1 || ldg % 4 == 0), AVA_ERR_SHAPE,
                "mem_chunk: B=%d T=%d nh=%d ld=%d ldg=%d ldy=%d", B, T, nh, ld, ldg, ldy);
    if (B == 0 || T == 0) return AVA_OK;
    MemArgs a{q, k, e, v, la, b, T, nh, ld, ldg, ldy, m, cap, F, S, y};
    dim3 grid(B * nh), block(256);
    // the contractions on the bf16 matrix cores; AVA_MEM_CHUNK_FP32=1 runs them on the f32 ones
    static const bool f32 = getenv("AVA_MEM_CHUNK_FP32") && atoi(getenv("AVA_MEM_CHUNK_FP32")) == 1;
    if (f32) {
        if (g == 1) {
            if (m != 0.0f) mem_chunk_kernel<true, true><<<grid, block, 0, st>>>(a);
            else mem_chunk_kernel<true, false><<<grid, block, 0, st>>>(a);
        } else {
            if (m != 0.0f) mem_chunk_kernel<false, true><<<grid, block, 0, st>>>(a);
            else mem_chunk_kernel<false, false><<<grid, block, 0, st>>>(a);
        }
    } else if (g == 1) {
        if (m != 0.0f) mem_chunk_bf_kernel<true, true><<<grid, block, 0, st>>>(a);
        else mem_chunk_bf_kernel<true, false><<<grid, block, 0, st>>>(a);
    } else {
        if (m != 0.0f) mem_chunk_bf_kernel<false, true><<<grid, block, 0, st>>>(a);
        else mem_chunk_bf_kernel<false, false><<<grid, block, 0, st>>>(a);
    }
    AVA_LAUNCHED("mem_chunk");
    return AVA_OK;
}

__global__ void zero_ints_kernel(int *x, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = 0;
}

int zero_ints(int *x, int n, hipStream_t st) {
    if (n <= 0) return AVA_OK;
    zero_ints_kernel<<<ceil_div(n, 256), 256, 0, st>>>(x, n);
    AVA_LAUNCHED("zero_ints");
    return AVA_OK;
}

}  // namespace ava

extern "C" int ava_mem_chunk(const float *q, const float *k, const float *e, const float *v, const float *la,
                             const float *b, int BH, int T, int hs, int g, float m, float cap, float *F, float *S,
                             float *y, ava_stream stream) {
    AVA_REQUIRE(hs == HS, AVA_ERR_UNSUPPORTED, "mem_chunk: head size %d (this build runs 64)", hs);
    AVA_REQUIRE(BH >= 0 && T >= 0, AVA_ERR_SHAPE, "mem_chunk: BH=%d T=%d", BH, T);
    return ava::mem_chunk_strided(q, k, e, v, la, b, BH, T, 1, HS, g, g, m, cap, F, S, y, HS, (hipStream_t)stream);
}

extern "C" int ava_mem_scan(const float *q, const float *k, const float *e, const float *v, const float *la,
                            const float *b, int BH, int T, int hs, int g, float m, float cap, float *F, float *S,
                            float *y, ava_stream stream) {
    AVA_REQUIRE(hs == HS, AVA_ERR_UNSUPPORTED, "mem_scan: head size %d (this build runs 64)", hs);
    AVA_REQUIRE(BH >= 0 && T >= 0, AVA_ERR_SHAPE, "mem_scan: BH=%d T=%d", BH, T);
    // [BH][T][64]: one head per "batch row", time stride 64; gates [BH][T][g]
    return ava::mem_scan_strided(q, k, e, v, la, b, BH, T, 1, HS, g, g, m, cap, F, S, y, HS, (hipStream_t)stream);
}
