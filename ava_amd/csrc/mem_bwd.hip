// The backward of the fast-weight (delta-rule) memory recurrence for gfx950, one workgroup per head
// (delta_rec's gradient, gpu/arch.rs:1091-1136; the CUDA forms memg_bwd / memg_bwd4,
// gpu/lif.cu:3411-3888).
//
// Forward, per head and step: r = F^T e;  u_ij = b_i k_i v_j - a_i b_i e_i r_j;  S' = M S + u;
// P = a_i F_ij + S'_ij (M = 0: + u_ij);  F' = clamp(P, +-cap);  y = F'^T q.
// Backward, from the last step (dF, dS carried): gP = (dF + q dy^T) where |F'| < cap, else 0;
//   dq_i = sum_j dy_j F'_ij;  dalpha_i += sum_j gP_ij F_ij;  du = gP + dS;  dS <- M du;
//   dv_j = sum_i du_ij b_i k_i;  dr_j = -sum_i du_ij a_i b_i e_i;
//   with sv_i = sum_j du_ij v_j and sr_i = sum_j du_ij r_j:  dk_i = b_i sv_i;
//   db_i = k_i sv_i - a_i e_i sr_i;  dalpha_i -= b_i e_i sr_i;  de_i = -a_i b_i sr_i + sum_j dr_j F_ij;
//   dF <- a_i gP_ij + e_i dr_j;  dla = dalpha a (summed over the head's rows for per-head gates).
//
// Columns of F never mix in the forward, nor in the carried gradients; only the row sums above
// (over all 64 columns) couple them. So wave w owns columns 16w..16w+15 outright, and lane l of it
// a 4 x 4 block: rows 4 (l & 15).., columns 16w + 4 (l >> 4)... A column sum (r, dr, dv) is 4 FMAs
// in the lane and 4 DPP adds over the 16 lanes of a DPP row; a row sum is 4 in the lane and two
// lane swaps over the wave's column groups, then the four waves' partials add up in LDS once per
// CK steps.
//
// States for the backward come from recomputation: pass 1 replays the forward and parks (F, S)
// every CK steps in the caller's workspace; pass 2 walks the checkpoints from the last, replays CK
// steps from each with every state F_t kept in registers (CK + 1 of them, and r_t), and walks those
// steps back. The inputs of CK steps are staged in LDS; the next group's are loaded meanwhile.
// Workspace: BH x ceil(T / CK) x (1 or 2 with momentum) x 16 KB.
#include <stdlib.h>

#include "common.h"

namespace {

constexpr int HS = 64, CK = 4;

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// The sum over the 16 lanes of v's DPP row (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), in every one of them.
__device__ __forceinline__ float sum16(float v) {
    v += dppf<0xB1>(v);
    v += dppf<0x4E>(v);
    v += dppf<0x141>(v);
    return v + dppf<0x140>(v);
}
// v[l] + v[l ^ 16] + v[l ^ 32] + v[l ^ 48] in every lane (the gfx950 lane swaps).
__device__ __forceinline__ float sum_cols(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// v[0..19] summed over the four 16-lane groups of the wave; lane group g gets the sums of
// v[5 g .. 5 g + 4] in w. Each lane swap exchanges a pair of values between groups, so a stage adds
// two values per swap: v_permlane32_swap pairs v[q] with v[q + 10] across the wave's halves, then
// v_permlane16_swap pairs u[q] with u[q + 5] across the 16-lane groups of each half.
__device__ __forceinline__ void rs_rows(const float (&v)[20], float (&w)[5]) {
    float u[10];
#pragma unroll
    for (int q = 0; q < 10; q++) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[q]), __float_as_uint(v[q + 10]), false, false);
        u[q] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
#pragma unroll
    for (int q = 0; q < 5; q++) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(u[q]), __float_as_uint(u[q + 5]), false, false);
        w[q] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
}

struct MemBwdArgs {
    const float *q, *k, *e, *v, *la, *b, *F0, *S0, *dy, *dFT, *dST;
    float *dq, *dk, *de, *dv, *dla, *db, *dF0, *dS0, *ck, *part;
    int T;
    float m, cap;
};

struct Stage {
    float q[CK][HS], k[CK][HS], e[CK][HS], v[CK][HS], a[CK][HS], b[CK][HS], bk[CK][HS], abe[CK][HS], dy[CK][HS];
};

// One forward step on the lane's 4 x CPL block (rows i0.., columns j0..): r (the block's CPL columns of
// e^T F, summed over all rows) is returned for the backward.
template <bool MOM, int CPL>
__device__ __forceinline__ void fwd_step(float (&F)[4 * CPL], float (&S)[4 * CPL], const Stage &sg, int s, int i0,
                                         int j0, float M, float cap, float (&r)[CPL]) {
    const f32x4 e4 = *reinterpret_cast<const f32x4 *>(&sg.e[s][i0]);
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        float x = e4[0] * F[c];
        x = fmaf(e4[1], F[CPL + c], x);
        x = fmaf(e4[2], F[2 * CPL + c], x);
        x = fmaf(e4[3], F[3 * CPL + c], x);
        r[c] = sum16(x);
    }
    float v4[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) v4[c] = sg.v[s][j0 + c];
    const f32x4 a4 = *reinterpret_cast<const f32x4 *>(&sg.a[s][i0]);
    const f32x4 k4 = *reinterpret_cast<const f32x4 *>(&sg.bk[s][i0]);
    const f32x4 x4 = *reinterpret_cast<const f32x4 *>(&sg.abe[s][i0]);
#pragma unroll
    for (int ri = 0; ri < 4; ri++)
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int m = CPL * ri + c;
            const float u = fmaf(-x4[ri], r[c], k4[ri] * v4[c]);
            float f;
            if (MOM) {
                S[m] = fmaf(M, S[m], u);
                f = fmaf(a4[ri], F[m], S[m]);
            } else {
                f = fmaf(a4[ri], F[m], u);
            }
            F[m] = __builtin_amdgcn_fmed3f(f, -cap, cap);
        }
}

// NCG workgroups per head, each owning 64 / NCG of its value columns: NCG = 1, wave w owns columns
// 16w.. and lane group g = lane / 16 four of them (CPL = 4); NCG = 4 (few heads: four times the
// workgroups), workgroup cg owns columns 16cg.., wave w four of them and lane group g one (CPL = 1).
// The rows' sums over the workgroup's columns then go to `part` [BH][NCG][T][5][64] and mem_bwd_rows
// adds the column groups in order.
template <bool G1, bool MOM, int NCG>
__global__ __launch_bounds__(256, 2) void mem_bwd_kernel(MemBwdArgs p) {
    constexpr int CPL = 4 / NCG, NE = 4 * CPL;
    __shared__ __attribute__((aligned(16))) Stage sg;
    __shared__ float red[CK][4][5][HS];  // per step, wave and row: dq, sum gP F, sv, sr, sum dr F

    const int wg = blockIdx.x, bh = wg / NCG, cg = wg - bh * NCG;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i0 = 4 * (lane & 15);
    const int j0 = (NCG == 1 ? 16 * wave : 16 * cg + 4 * wave) + CPL * (lane >> 4);
    const int T = p.T, nck = (T + CK - 1) / CK;
    constexpr int NS = MOM ? 2 : 1;
    const size_t hb = (size_t)bh * T * HS;
    const size_t gb = G1 ? (size_t)bh * T : hb;
    // a workgroup's checkpoints: 256 lanes x NE floats per state
    float *ckh = p.ck + (size_t)wg * nck * NS * (256 * NE) + (size_t)tid * NE;
    const float M = p.m, cap = p.cap;

    float F[NE], S[NE];
    {
        const size_t o0 = (size_t)bh * HS * HS;
#pragma unroll
        for (int m = 0; m < NE; m++) {
            const size_t o = o0 + (size_t)(i0 + m / CPL) * HS + j0 + m % CPL;
            F[m] = p.F0 ? p.F0[o] : 0.0f;
            S[m] = (MOM && p.S0) ? p.S0[o] : 0.0f;
        }
    }

    // staging: thread -> (step st of the group, channel cc); the loads of a group are issued one
    // group ahead
    const int st = tid >> 6, cc = tid & 63;
    float lq = 0, lk = 0, le = 0, lv = 0, ll = 0, lb = 0, ld = 0;
    auto load = [&](int t0, bool bwd) {
        const int t = t0 + st;
        if (t < T && t0 >= 0) {
            const size_t o = hb + (size_t)t * HS + cc;
            lk = p.k[o];
            le = p.e[o];
            lv = p.v[o];
            const size_t og = G1 ? gb + t : o;
            ll = p.la[og];
            lb = p.b[og];
            if (bwd) {
                lq = p.q[o];
                ld = p.dy[o];
            }
        } else {
            lq = lk = le = lv = ll = lb = ld = 0.0f;
        }
    };
    auto stage = [&]() {
        const float a = expf(ll);
        sg.q[st][cc] = lq;
        sg.k[st][cc] = lk;
        sg.e[st][cc] = le;
        sg.v[st][cc] = lv;
        sg.a[st][cc] = a;
        sg.b[st][cc] = lb;
        sg.bk[st][cc] = lb * lk;
        sg.abe[st][cc] = (a * lb) * le;
        sg.dy[st][cc] = ld;
    };
    auto park = [&](int c, const float (&X)[NE], int which) {
        float *dst = ckh + ((size_t)c * NS + which) * (256 * NE);
#pragma unroll
        for (int z = 0; z < NE / 4; z++)
            *reinterpret_cast<f32x4 *>(dst + 4 * z) = f32x4{X[4 * z], X[4 * z + 1], X[4 * z + 2], X[4 * z + 3]};
    };
    auto unpark = [&](int c, float (&X)[NE], int which) {
        const float *src = ckh + ((size_t)c * NS + which) * (256 * NE);
#pragma unroll
        for (int z = 0; z < NE / 4; z++) {
            const f32x4 x = *reinterpret_cast<const f32x4 *>(src + 4 * z);
            X[4 * z] = x[0];
            X[4 * z + 1] = x[1];
            X[4 * z + 2] = x[2];
            X[4 * z + 3] = x[3];
        }
    };

    // 1. the forward, parking the state at the start of every group of CK steps
    load(0, false);
    for (int c = 0; c < nck; c++) {
        __syncthreads();
        stage();
        __syncthreads();
        load((c + 1) * CK, false);
        park(c, F, 0);
        if (MOM) park(c, S, 1);
        const int n = min(CK, T - c * CK);
#pragma unroll
        for (int s = 0; s < CK; s++) {
            if (s < n) {
                float r[CPL];
                fwd_step<MOM, CPL>(F, S, sg, s, i0, j0, M, cap, r);
            }
        }
    }

    // 2. backwards, group by group
    float dF[NE], dS[NE];
    {
        const size_t o0 = (size_t)bh * HS * HS;
#pragma unroll
        for (int m = 0; m < NE; m++) {
            const size_t o = o0 + (size_t)(i0 + m / CPL) * HS + j0 + m % CPL;
            dF[m] = p.dFT ? p.dFT[o] : 0.0f;
            dS[m] = (MOM && p.dST) ? p.dST[o] : 0.0f;
        }
    }
    load((nck - 1) * CK, true);
    for (int c = nck - 1; c >= 0; c--) {
        const int t0 = c * CK, n = min(CK, T - t0);
        __syncthreads();  // the previous group's combine is done with the staging and red
        stage();
        __syncthreads();
        load(t0 - CK, true);  // nothing past the first group (t0 - CK < 0)
        float Ft[CK + 1][NE], rt[CK][CPL];
        unpark(c, Ft[0], 0);
        if (MOM) unpark(c, S, 1);
#pragma unroll
        for (int s = 0; s < CK; s++) {
            if (s < n) {
#pragma unroll
                for (int m = 0; m < NE; m++) Ft[s + 1][m] = Ft[s][m];
                fwd_step<MOM, CPL>(Ft[s + 1], S, sg, s, i0, j0, M, cap, rt[s]);
            }
        }
#pragma unroll
        for (int s = CK - 1; s >= 0; s--) {
            if (s < n) {
                const float(&Fa)[NE] = Ft[s];      // F before the step
                const float(&Fb)[NE] = Ft[s + 1];  // after it
                const f32x4 q4 = *reinterpret_cast<const f32x4 *>(&sg.q[s][i0]);
                const f32x4 e4 = *reinterpret_cast<const f32x4 *>(&sg.e[s][i0]);
                const f32x4 a4 = *reinterpret_cast<const f32x4 *>(&sg.a[s][i0]);
                const f32x4 k4 = *reinterpret_cast<const f32x4 *>(&sg.bk[s][i0]);
                const f32x4 x4 = *reinterpret_cast<const f32x4 *>(&sg.abe[s][i0]);
                float v4[CPL], y4[CPL];
#pragma unroll
                for (int cj = 0; cj < CPL; cj++) {
                    v4[cj] = sg.v[s][j0 + cj];
                    y4[cj] = sg.dy[s][j0 + cj];
                }
                float pdq[4], pal[4], psv[4], psr[4], pde[4], cdr[CPL], cdv[CPL];
#pragma unroll
                for (int z = 0; z < 4; z++) pdq[z] = pal[z] = psv[z] = psr[z] = pde[z] = 0.0f;
#pragma unroll
                for (int z = 0; z < CPL; z++) cdr[z] = cdv[z] = 0.0f;
#pragma unroll
                for (int ri = 0; ri < 4; ri++)
#pragma unroll
                    for (int cj = 0; cj < CPL; cj++) {
                        const int m = CPL * ri + cj;
                        pdq[ri] = fmaf(y4[cj], Fb[m], pdq[ri]);
                        float gP = fmaf(q4[ri], y4[cj], dF[m]);
                        gP = fabsf(Fb[m]) < cap ? gP : 0.0f;
                        pal[ri] = fmaf(gP, Fa[m], pal[ri]);
                        float du = gP;
                        if (MOM) {
                            du = gP + dS[m];
                            dS[m] = M * du;
                        }
                        psv[ri] = fmaf(du, v4[cj], psv[ri]);
                        psr[ri] = fmaf(du, rt[s][cj], psr[ri]);
                        cdr[cj] = fmaf(-du, x4[ri], cdr[cj]);
                        cdv[cj] = fmaf(du, k4[ri], cdv[cj]);
                        dF[m] = a4[ri] * gP;
                    }
#pragma unroll
                for (int cj = 0; cj < CPL; cj++) {
                    cdr[cj] = sum16(cdr[cj]);
                    cdv[cj] = sum16(cdv[cj]);
                }
#pragma unroll
                for (int ri = 0; ri < 4; ri++)
#pragma unroll
                    for (int cj = 0; cj < CPL; cj++) {
                        const int m = CPL * ri + cj;
                        pde[ri] = fmaf(cdr[cj], Fa[m], pde[ri]);
                        dF[m] = fmaf(e4[ri], cdr[cj], dF[m]);
                    }
                {
                    // the 20 row partials (quantity z, row ri: index 4 z + ri) summed over the wave's four
                    // lane groups by a reduce-scatter: lane group g ends with the sums of 5 g .. 5 g + 4
                    float v[20];
#pragma unroll
                    for (int ri = 0; ri < 4; ri++) {
                        v[ri] = pdq[ri];
                        v[4 + ri] = pal[ri];
                        v[8 + ri] = psv[ri];
                        v[12 + ri] = psr[ri];
                        v[16 + ri] = pde[ri];
                    }
                    float w[5];
                    rs_rows(v, w);
                    const int g = lane >> 4;
#pragma unroll
                    for (int z = 0; z < 5; z++) {
                        const int k = 5 * g + z;
                        red[s][wave][k >> 2][i0 + (k & 3)] = w[z];
                    }
                }
                if ((lane & 15) == 0) {
                    float *dvp = p.dv + hb + (size_t)(t0 + s) * HS + j0;
                    if (CPL == 4) *reinterpret_cast<f32x4 *>(dvp) = f32x4{cdv[0], cdv[CPL > 1 ? 1 : 0], cdv[CPL > 2 ? 2 : 0], cdv[CPL > 3 ? 3 : 0]};
                    else dvp[0] = cdv[0];
                }
            }
        }
        __syncthreads();
        // the rows' gradients: thread -> (step st, row cc), the four waves' partials added
        if (st < n) {
            const int t = t0 + st;
            float x[5];
#pragma unroll
            for (int z = 0; z < 5; z++) x[z] = ((red[st][0][z][cc] + red[st][1][z][cc]) + red[st][2][z][cc]) + red[st][3][z][cc];
            if (NCG > 1) {
                // this workgroup's columns only: mem_bwd_rows adds the groups
                float *pp = p.part + (((size_t)bh * NCG + cg) * T + t) * (5 * HS) + cc;
#pragma unroll
                for (int z = 0; z < 5; z++) pp[z * HS] = x[z];
            } else {
                const float a = sg.a[st][cc], b = sg.b[st][cc], k = sg.k[st][cc], e = sg.e[st][cc];
                const size_t o = hb + (size_t)t * HS + cc;
                p.dq[o] = x[0];
                p.dk[o] = b * x[2];
                p.de[o] = fmaf(-(a * b), x[3], x[4]);
                const float dal = fmaf(-(b * e), x[3], x[1]);
                const float dbr = fmaf(-(a * e), x[3], k * x[2]);
                if (G1) {
                    const float sa = ava::wave_sum(dal * a), sb = ava::wave_sum(dbr);
                    if (cc == 0) {
                        p.dla[gb + t] = sa;
                        p.db[gb + t] = sb;
                    }
                } else {
                    p.dla[o] = dal * a;
                    p.db[o] = dbr;
                }
            }
        }
    }
    {
        const size_t o0 = (size_t)bh * HS * HS;
#pragma unroll
        for (int m = 0; m < NE; m++) {
            const size_t o = o0 + (size_t)(i0 + m / CPL) * HS + j0 + m % CPL;
            if (p.dF0) p.dF0[o] = dF[m];
            if (MOM && p.dS0) p.dS0[o] = dS[m];
        }
    }
}

// The rows' gradients from the column groups' partial sums (NCG > 1): thread -> (step, row), the groups
// added in order, then the combine of mem_bwd_kernel.
template <bool G1, int NCG>
__global__ __launch_bounds__(256) void mem_bwd_rows(MemBwdArgs p) {
    const int T = p.T, tid = threadIdx.x, cc = tid & 63;
    const int t = blockIdx.x * 4 + (tid >> 6), bh = blockIdx.y;
    if (t >= T) return;  // whole waves (4 steps per workgroup, one wave each)
    float x[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < NCG; g++) {
        const float *pp = p.part + (((size_t)bh * NCG + g) * T + t) * (5 * HS) + cc;
#pragma unroll
        for (int z = 0; z < 5; z++) x[z] = g ? x[z] + pp[z * HS] : pp[z * HS];
    }
    const size_t hb = (size_t)bh * T * HS, gb = G1 ? (size_t)bh * T : hb;
    const size_t o = hb + (size_t)t * HS + cc, og = G1 ? gb + t : o;
    const float a = expf(p.la[og]), b = p.b[og], k = p.k[o], e = p.e[o];
    p.dq[o] = x[0];
    p.dk[o] = b * x[2];
    p.de[o] = fmaf(-(a * b), x[3], x[4]);
    const float dal = fmaf(-(b * e), x[3], x[1]);
    const float dbr = fmaf(-(a * e), x[3], k * x[2]);
    if (G1) {
        const float sa = ava::wave_sum(dal * a), sb = ava::wave_sum(dbr);
        if (cc == 0) {
            p.dla[gb + t] = sa;
            p.db[gb + t] = sb;
        }
    } else {
        p.dla[o] = dal * a;
        p.db[o] = dbr;
    }
}

// Column groups per head: four when there are too few heads to fill the GPU with one workgroup each
// (AVA_MEM_BWD_GROUPS=1 or 4 chooses).
int mem_bwd_groups(int BH) {
    static const int forced = getenv("AVA_MEM_BWD_GROUPS") ? atoi(getenv("AVA_MEM_BWD_GROUPS")) : 0;
    if (forced == 1 || forced == 4) return forced;
    return BH < 512 ? 4 : 1;
}

}  // namespace

extern "C" size_t ava_mem_scan_bwd_workspace(int BH, int T, int momentum) {
    if (BH <= 0 || T <= 0) return 0;
    const int ncg = mem_bwd_groups(BH);
    const size_t ck = (size_t)BH * ((T + CK - 1) / CK) * (momentum ? 2 : 1) * HS * HS * sizeof(float);
    const size_t part = ncg > 1 ? (size_t)BH * ncg * T * 5 * HS * sizeof(float) : 0;
    return ck + part;
}

// The backward of ava_mem_scan (same layout and gates), from the initial state F0, S0 (nullable:
// zeros) and the gradients dy of y and dF_T, dS_T of the final state (nullable: zeros): dq, dk, de,
// dv [BH][T][hs]; dla, db [BH][T][g]; dF0, dS0 (nullable) the gradients of the initial state.
extern "C" int ava_mem_scan_bwd(const float *q, const float *k, const float *e, const float *v, const float *la,
                                const float *b, int BH, int T, int hs, int g, float m, float cap, const float *F0,
                                const float *S0, const float *dy, const float *dF_T, const float *dS_T, float *dq,
                                float *dk, float *de, float *dv, float *dla, float *db, float *dF0, float *dS0,
                                void *work, size_t work_bytes, ava_stream stream) {
    AVA_REQUIRE(hs == HS, AVA_ERR_UNSUPPORTED, "mem_scan_bwd: head size %d (this build runs 64)", hs);
    AVA_REQUIRE(g == 1 || g == HS, AVA_ERR_SHAPE, "mem_scan_bwd: g=%d (1 or hs)", g);
    AVA_REQUIRE(BH > 0 && T > 0, AVA_ERR_SHAPE, "mem_scan_bwd: BH=%d T=%d", BH, T);
    AVA_REQUIRE(q && k && e && v && la && b && dy && dq && dk && de && dv && dla && db && work, AVA_ERR_ARG,
                "mem_scan_bwd: NULL buffer");
    const bool mom = m != 0.0f;
    const size_t need = ava_mem_scan_bwd_workspace(BH, T, mom);
    AVA_REQUIRE(work_bytes >= need, AVA_ERR_SHAPE, "mem_scan_bwd: workspace %zu < %zu bytes", work_bytes, need);
    const int ncg = mem_bwd_groups(BH);
    float *ck = (float *)work;
    float *part = ncg > 1 ? ck + (size_t)BH * ((T + CK - 1) / CK) * (mom ? 2 : 1) * HS * HS : nullptr;
    MemBwdArgs p{q, k, e, v, la, b, F0, mom ? S0 : nullptr, dy, dF_T, mom ? dS_T : nullptr, dq, dk, de, dv, dla, db,
                 dF0, mom ? dS0 : nullptr, ck, part, T, m, cap};
    const hipStream_t st = (hipStream_t)stream;
#define AVA_MB(G1_, MOM_)                                                                           \
    do {                                                                                             \
        if (ncg > 1) {                                                                               \
            mem_bwd_kernel<G1_, MOM_, 4><<<BH * 4, 256, 0, st>>>(p);                                 \
            mem_bwd_rows<G1_, 4><<<dim3(ava::ceil_div(T, 4), BH), 256, 0, st>>>(p);                       \
        } else {                                                                                     \
            mem_bwd_kernel<G1_, MOM_, 1><<<BH, 256, 0, st>>>(p);                                     \
        }                                                                                            \
    } while (0)
    if (g == 1) {
        if (mom) AVA_MB(true, true);
        else AVA_MB(true, false);
    } else {
        if (mom) AVA_MB(false, true);
        else AVA_MB(false, false);
    }
#undef AVA_MB
    AVA_LAUNCHED("mem_scan_bwd");
    return AVA_OK;
}
