// The gated delta rule in its chunked (WY / UT) form for gfx950: per head, chunks of 64 tokens,
// the state F [64][64] (row = key channel, column = value channel) resident in LDS for the whole
// sequence. The algebra is the reference's delta_rule_from (gpu/model.rs:744-799); inside a chunk,
// with cum = the running sum of log alpha, Gamma_i = exp(cum_i), D_ij = exp(cum_i - cum_j) for
// j <= i (0 above), M = on/below the diagonal:
//   A_ij = beta_i k_i.k_j (j < i);  Tw = (I + A)^-1;  Tu = (I + A o D)^-1 = D o Tw (D's ratios
//   factor through the triangular inverse: (I + A o D) = G (I + A) G^-1 with G = diag(Gamma), formed
//   here pairwise as exp(cum_i - cum_j) so no Gamma alone can underflow)
//   W = Tw diag(beta) K;  U = Tu diag(beta) V;  WF = W F
//   Y = diag(Gamma) (Q F - (QK^T o M) WF) + (QK^T o D o M) U
//   F <- Gamma_c (F - K^T WF) + K^T diag(Gamma_c / Gamma) U
// With gates, and without gates when no workspace is given, one kernel walks a head's chunks with
// every 64 x 64 x 64 product on the fp32 MFMA (v_mfma_f32_32x32x2_f32, one 32 x 32 quadrant per wave,
// operands straight from LDS rows of odd stride, so a column read hits 32 different banks). Without
// gates (alpha = 1, config[2]) the two read-outs merge: Y = Q F + (QK^T o M)(U - W F) and
// F <- F + K^T (U - W F). The unit lower-triangular inverse is a left-looking forward substitution
// spread over the 4 waves (16 columns each, 4 lanes per column); the reference doubles blocks
// (gpu/model.rs:720-742): both are exact inverses, equal up to rounding. The next chunk's q, k, v
// are loaded into registers while the current chunk is computed. Without gates and with a workspace,
// the work splits in two phases (the inverses of all chunks at once, then the walk as six products
// per chunk on the bf16 matrix cores in split terms): see the second half of this file.
#include "common.h"

namespace {

constexpr int C = 64, LD = 65;  // chunk length / head size, LDS row stride (odd: conflict-free columns)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct DeltaArgs {
    const float *q, *k, *v, *la, *beta;  // [BH][T][64], la/beta [BH][T] (la NULL: alpha = 1)
    int T;
    float *F, *y;
};

// acc += A B over one 32 x 32 quadrant: lane l supplies A(l & 31, x + (l >> 5)) and B(x + (l >> 5), l & 31)
// for x = 0, 2, .., 62 (fa, fb take quadrant-relative rows/columns and absolute k).
template <class FA, class FB>
__device__ __forceinline__ void mq(f32x16 &acc, int lane, FA fa, FB fb) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll 8
    for (int x = 0; x < C; x += 2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa(r, x + h), fb(x + h, r), acc, 0, 0, 0);
}
// v[l] + v[l ^ 16] and v[l] + v[l ^ 32] in every lane l, through the VALU lane swaps of gfx950
// (v_permlane16_swap / v_permlane32_swap: the swap leaves v[l] in one result and the partner's in the
// other, and both lanes add the same two values).
__device__ __forceinline__ float xsum16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xsum32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Register i of a quadrant's accumulator: row (i / 4) 8 + (l / 32) 4 + i % 4, column l % 32.
__device__ __forceinline__ int qrow(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

// One chunk without gates (alpha = 1), state F in sF, the chunk's K, Q, V staged:
//   D = (I + A)^-1 diag(beta) (V - K F)   (= U - W F: one triangular solve replaces Tw, W, U and W F)
//   Y = Q F + (QK^T o M) D;  F <- F + K^T D
// Six 64 x 64 x 64 products and one solve with 64 right-hand sides; Q F stays in registers until Y.
// Ends with a barrier (the next chunk may overwrite the staged inputs).
template <class NEXT>
__device__ __forceinline__ void solve_chunk(const float *sK, const float *sQ, const float *sV, float *sA, float *sD,
                                            float *sR, float *sF, float *sX, const float *s_beta, float *yh, int t0,
                                            int lane, int wave, int row0, int col0, int lc, NEXT next) {
    f32x16 qf = {};
    {
        f32x16 aq = {}, ak = {}, kf = {};
        mq(aq, lane, [&](int r, int x) { return sQ[(row0 + r) * LD + x]; },
           [&](int x, int c) { return sK[(col0 + c) * LD + x]; });
        mq(ak, lane, [&](int r, int x) { return sK[(row0 + r) * LD + x]; },
           [&](int x, int c) { return sK[(col0 + c) * LD + x]; });
        mq(kf, lane, [&](int r, int x) { return sK[(row0 + r) * LD + x]; },
           [&](int x, int c) { return sF[x * LD + col0 + c]; });
        mq(qf, lane, [&](int r, int x) { return sQ[(row0 + r) * LD + x]; },
           [&](int x, int c) { return sF[x * LD + col0 + c]; });
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = row0 + qrow(i, lane), c = col0 + lc, o = r * LD + c;
            sX[o] = aq[i];
            sA[o] = c < r ? s_beta[r] * ak[i] : 0.0f;
            sR[o] = s_beta[r] * (sV[o] - kf[i]);
        }
    }
    __syncthreads();
    next();  // Q, V and beta of this chunk are read: the next chunk's may land in their place
    // D = (I + A)^-1 R, column by column, left-looking: d_i = R_i - sum_{j<i} A_ij d_j. Wave w solves
    // columns 16w..16w+15; lane l holds column c = 16w + (l & 15) and rows j = 4m + (l >> 4) of its
    // solution in registers (rows not solved yet hold 0, so their terms vanish without a mask). A row's
    // sum is split over the column's 4 lanes and added with the lane swaps: a step's dependency chain
    // is one fma and two swaps.
    {
        const int c = wave * 16 + (lane & 15), q = lane >> 4;
        float xr[16];
#pragma unroll
        for (int m = 0; m < 16; m++) xr[m] = 0.0f;
        // row i's A values and right-hand side are read one step ahead (cur / nxt), so the LDS
        // latency is not on the step's dependency chain
        float cur[16], nxt[16], rc = sR[c], rn = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; m++) cur[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < C; i++) {
            if (i + 1 < C) {
#pragma unroll
                for (int m = 0; 4 * m < i + 1; m++) nxt[m] = sA[(i + 1) * LD + 4 * m + q];
                rn = sR[(i + 1) * LD + c];
                AVA_ISSUE_FENCE();
            }
            float part = 0.0f;
#pragma unroll
            for (int m = 0; 4 * m < i; m++) part = fmaf(cur[m], xr[m], part);
            const float di = rc - xsum32(xsum16(part));
            if (q == (i & 3)) xr[i >> 2] = di;
#pragma unroll
            for (int m = 0; m < 16; m++) cur[m] = nxt[m];
            rc = rn;
        }
#pragma unroll
        for (int m = 0; m < 16; m++) sD[(4 * m + q) * LD + c] = xr[m];
    }
    __syncthreads();
    // Y = Q F + (QK o M) D;  F <- F + K^T D (Y no longer reads F: the update needs no barrier before it)
    {
        mq(qf, lane, [&](int r, int x) { return x <= row0 + r ? sX[(row0 + r) * LD + x] : 0.0f; },
           [&](int x, int c) { return sD[x * LD + col0 + c]; });
#pragma unroll
        for (int i = 0; i < 16; i++) yh[(size_t)(t0 + row0 + qrow(i, lane)) * C + col0 + lc] = qf[i];
        f32x16 a = {};
        mq(a, lane, [&](int r, int x) { return sK[x * LD + row0 + r]; },
           [&](int x, int c) { return sD[x * LD + col0 + c]; });
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int o = (row0 + qrow(i, lane)) * LD + col0 + lc;
            sF[o] = sF[o] + a[i];
        }
    }
}

// global_load_lds_dword: 4 bytes per lane from g + lane to the LDS row at l (l wave-uniform), so one
// instruction fills a 64-float row of a padded LDS matrix. The address-space cast exists only in the
// device pass.
__device__ __forceinline__ void dma_row(const float *g, float *l) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 4, 0, 0);
#endif
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt((0) | (7 << 4) | (15 << 8)); }

// Without gates: the chunk loop with the next chunk's k, q, v and beta brought straight into LDS
// (dword rows, 4 waves x 48 + 1 loads) while the current chunk's solve runs. K alternates between two
// buffers (the current chunk's K is read until its state update); Q, V and beta are dead after the
// first products and are overwritten in place.
__global__ __launch_bounds__(256) void delta_plain_kernel(DeltaArgs p) {
    extern __shared__ float sm[];
    float *sK = sm, *sQ = sK + C * LD, *sV = sQ + C * LD, *sA = sV + C * LD, *sD = sA + C * LD;
    float *sR = sD + C * LD, *sK2 = sR + C * LD, *sF = sK2 + C * LD, *sX = sF + C * LD;
    float *s_beta = sX + C * LD;

    const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = (wave >> 1) * 32, col0 = (wave & 1) * 32, lc = lane & 31;
    const float *qh = p.q + (size_t)bh * p.T * C, *kh = p.k + (size_t)bh * p.T * C, *vh = p.v + (size_t)bh * p.T * C;
    const float *bth = p.beta + (size_t)bh * p.T;
    float *Fh = p.F + (size_t)bh * C * C, *yh = p.y + (size_t)bh * p.T * C;

    for (int i = tid; i < C * C; i += 256) sF[(i >> 6) * LD + (i & 63)] = Fh[i];
    auto issue = [&](int t0, float *kd) {
        for (int r = wave; r < C; r += 4) {
            const size_t o = (size_t)(t0 + r) * C + lane;
            dma_row(kh + o, kd + r * LD);
            dma_row(qh + o, sQ + r * LD);
            dma_row(vh + o, sV + r * LD);
        }
        if (wave == 0) dma_row(bth + t0 + lane, s_beta);
    };
    float *kc = sK, *kn = sK2;
    issue(0, kc);
    for (int t0 = 0; t0 < p.T; t0 += C) {
        wait_vm0();
        __syncthreads();  // the chunk's rows are in LDS, and the previous chunk's state update is done
        float *knext = kn;
        solve_chunk(kc, sQ, sV, sA, sD, sR, sF, sX, s_beta, yh, t0, lane, wave, row0, col0, lc, [&]() {
            if (t0 + C < p.T) issue(t0 + C, knext);
        });
        kn = kc;
        kc = knext;
    }
    __syncthreads();
    for (int i = tid; i < C * C; i += 256) Fh[i] = sF[(i >> 6) * LD + (i & 63)];
}

// ------------------------------------------------------------------ the plain rule in two phases
//
// The chunk's triangular inverse does not depend on the state, so it leaves the sequential walk:
//   phase 1 (every (head, chunk) at once): T' = (I + A)^-1 diag(beta), A_ij = beta_i k_i.k_j (j < i),
//           written to a workspace [BH][T / 64][64][64];
//   phase 2 (one workgroup per head, chunk after chunk): R = V - K F, D = T' R, Y = Q F + (QK^T o M) D,
//           F <- F + K^T D.
// Phase 2 is six products per chunk and no solve (on the bf16 matrix cores, below).

struct DeltaInvArgs {
    const float *k, *beta;
    int T, nch;
    float *Tp;
};

// (I + A)^-1 in two levels of 32: the diagonal blocks' inverses T11 and T22 by left-looking substitution
// (waves 0-1 and 2-3 at once, 32 steps each), then T21 = -T22 A21 T11 by two 32 x 32 x 32 products.
// Exact inverses both, equal to the 64-step substitution up to rounding.
__global__ __launch_bounds__(256) void delta_inv_kernel(DeltaInvArgs p) {
    __shared__ float sK[C * LD], sA[C * LD], s_beta[C];
    const int bh = blockIdx.x / p.nch, ch = blockIdx.x - bh * p.nch;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = (wave >> 1) * 32, col0 = (wave & 1) * 32, lc = lane & 31;
    const float *kh = p.k + ((size_t)bh * p.T + (size_t)ch * C) * C;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = tid + 256 * j, r = idx >> 4, c = (idx & 15) * 4;
        const f32x4 x = *reinterpret_cast<const f32x4 *>(kh + (size_t)r * C + c);
#pragma unroll
        for (int z = 0; z < 4; z++) sK[r * LD + c + z] = x[z];
    }
    if (wave == 0) s_beta[lane] = p.beta[(size_t)bh * p.T + (size_t)ch * C + lane];
    __syncthreads();
    {
        f32x16 ak = {};
        mq(ak, lane, [&](int r, int x) { return sK[(row0 + r) * LD + x]; },
           [&](int x, int c) { return sK[(col0 + c) * LD + x]; });
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = row0 + qrow(i, lane), c = col0 + lc;
            sA[r * LD + c] = c < r ? s_beta[r] * ak[i] : 0.0f;
        }
    }
    __syncthreads();
    // the diagonal blocks: waves 0-1 the columns 0..31 of T11, waves 2-3 those of T22 (block base o);
    // lane l holds column c = o + 16 (w & 1) + (l & 15) and block rows j = 4m + (l >> 4), m < 8. Row i's
    // A values are read a step ahead, so the LDS latency is not on the substitution's dependency chain.
    float *sT = sK;  // K is read: its LDS holds T
    {
        const int o = (wave >> 1) * 32, c = o + (wave & 1) * 16 + (lane & 15), q = lane >> 4;
        float xr[8], cur[8], nxt[8];
#pragma unroll
        for (int m = 0; m < 8; m++) {
            xr[m] = 0.0f;
            cur[m] = 0.0f;
            nxt[m] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 32; i++) {
            if (i + 1 < 32) {
#pragma unroll
                for (int m = 0; 4 * m < i + 1; m++) nxt[m] = sA[(o + i + 1) * LD + o + 4 * m + q];
                AVA_ISSUE_FENCE();
            }
            float part = 0.0f;
#pragma unroll
            for (int m = 0; 4 * m < i; m++) part = fmaf(cur[m], xr[m], part);
            const float tot = xsum32(xsum16(part));
            const float xi = (o + i == c ? 1.0f : 0.0f) - tot;
            if (q == (i & 3)) xr[i >> 2] = xi;
#pragma unroll
            for (int m = 0; m < 8; m++) cur[m] = nxt[m];
        }
#pragma unroll
        for (int m = 0; m < 8; m++) {
            sT[(o + 4 * m + q) * LD + c] = xr[m];
            sT[(o + 4 * m + q) * LD + (c ^ 32)] = 0.0f;  // T12 = 0 (rows o.., the other block's columns)
        }
    }
    __syncthreads();
    // M = A21 T11 into the unused upper block of sA, then T21 = -T22 M: wave w takes the 16 x 16 tile
    // (w >> 1, w & 1) of each (v_mfma_f32_16x16x4f32: lane l gives row / column l % 16 at k l / 16)
    {
        const int ti = (wave >> 1) * 16, tj = (wave & 1) * 16, r = lane & 15, kq = lane >> 4;
        f32x4 m = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 32; k += 4)
            m = __builtin_amdgcn_mfma_f32_16x16x4f32(sA[(32 + ti + r) * LD + k + kq], sT[(k + kq) * LD + tj + r], m, 0,
                                                      0, 0);
#pragma unroll
        for (int z = 0; z < 4; z++) sA[(ti + 4 * kq + z) * LD + 32 + tj + r] = m[z];
        __syncthreads();
        f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 32; k += 4)
            t = __builtin_amdgcn_mfma_f32_16x16x4f32(sT[(32 + ti + r) * LD + 32 + k + kq],
                                                      sA[(k + kq) * LD + 32 + tj + r], t, 0, 0, 0);
#pragma unroll
        for (int z = 0; z < 4; z++) sT[(32 + ti + 4 * kq + z) * LD + tj + r] = -t[z];
    }
    __syncthreads();
    float *Th = p.Tp + ((size_t)bh * p.nch + ch) * C * C;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = tid + 256 * j, r = idx >> 4, c = (idx & 15) * 4;
        f32x4 x;
#pragma unroll
        for (int z = 0; z < 4; z++) x[z] = sT[r * LD + c + z] * s_beta[c + z];
        *reinterpret_cast<f32x4 *>(Th + (size_t)r * C + c) = x;
    }
}

// ------------------------------------------------------------------ phase 2 on the bf16 matrix cores
//
// The six products of a chunk run as v_mfma_f32_32x32x16_bf16 on operands split into bf16 terms,
// x = t0 + t1 + t2 (each term the rest rounded again to bf16). A product of order P keeps the terms
// a_i b_j with i + j < P, with f32 accumulation: order 3 (six products per k step) leaves about 2^-24
// of |a b|, as an f32 product does; order 2 (three) about 2^-17. All six products are of order 3:
// with order 2 the config[2] walk came 1.1e-5 from the float64 recurrence (order 3: 2.4e-7) and a key
// read right after its write missed the 1e-4 read-back bar (R = V - K F cancels there).
// Every operand lives in LDS as a term buffer: up to three planes of a 64 x 64 matrix, each row (the
// output row of an A operand, the output column of a B operand) holding its 64 k values
// contiguously, 72 apart (a 16-byte load per lane per k step, no bank conflicts across 8 lanes). The
// state F stays f32 in the accumulator registers of each wave's quadrant; its bf16 terms are rewritten
// after each update. Per chunk:
//   P1  KF = K F, QF = Q F (kept), X^T = K Q^T          (A: K rows, Q rows; B: F columns, Q rows)
//   P2  R = V - K F (f32) -> terms; X masked -> terms; D = T' R
//   P3  Y = QF + X D, F += K^T D
// and the next chunk's K, Q, V, T' arrive in registers during the chunk and are split into LDS at its end.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int PST = 72;  // bf16 per row of a term plane
constexpr int PLANE = C * PST;
constexpr int NTMAX = 3;  // term planes per buffer

template <int N>
__device__ __forceinline__ void splitn(float x, __bf16 (&o)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) {
        o[i] = (__bf16)x;
        x = x - (float)o[i];
    }
}

// Products over the wave's quadrant, k = 0..63: A's rows ar0 .. ar0 + 31 and B's columns bc0 .. bc0 + 31
// of term buffers. The leading term's product and the cross terms go to separate accumulators (added
// at the end, small ones first), and products that share an operand run in one k loop, so consecutive
// matrix instructions rarely wait on each other's results.
template <int P>
struct Frag {
    bf16x8 t[P];
};
template <int P>
__device__ __forceinline__ Frag<P> ldf(const __bf16 *B, int row, int k) {
    Frag<P> f;
#pragma unroll
    for (int i = 0; i < P; i++) f.t[i] = *reinterpret_cast<const bf16x8 *>(B + i * PLANE + row * PST + k);
    return f;
}
struct Acc3 {
    f32x16 m, x, y;  // t0 t0; t0 t1 + t1 t0; the terms of order 3
};
template <int P>
__device__ __forceinline__ void mfma_terms(Acc3 &c, const Frag<P> &a, const Frag<P> &b) {
    c.m = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.t[0], b.t[0], c.m, 0, 0, 0);
    c.x = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.t[0], b.t[1], c.x, 0, 0, 0);
    c.x = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.t[1], b.t[0], c.x, 0, 0, 0);
    if constexpr (P > 2) {
        c.y = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.t[0], b.t[2], c.y, 0, 0, 0);
        c.y = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.t[1], b.t[1], c.y, 0, 0, 0);
        c.y = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.t[2], b.t[0], c.y, 0, 0, 0);
    }
}
template <int P>
__device__ __forceinline__ f32x16 total(const Acc3 &c) {
    if constexpr (P > 2) return c.m + (c.x + c.y);
    return c.m + c.x;
}
// acc (+)= A B
template <int P>
__device__ __forceinline__ void mq_bf(f32x16 &acc, const __bf16 *A, int ar0, const __bf16 *B, int bc0, int lane) {
    const int r = lane & 31, k0 = 8 * (lane >> 5);
    Acc3 c{acc, {}, {}};
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
        mfma_terms<P>(c, ldf<P>(A, ar0 + r, k0 + 16 * ks), ldf<P>(B, bc0 + r, k0 + 16 * ks));
    acc = total<P>(c);
}
// acc1 (+)= A1 B and acc2 (+)= A2 B (one B operand)
template <int P>
__device__ __forceinline__ void mq_bf_2a(f32x16 &acc1, const __bf16 *A1, int a1r0, f32x16 &acc2, const __bf16 *A2,
                                         int a2r0, const __bf16 *B, int bc0, int lane) {
    const int r = lane & 31, k0 = 8 * (lane >> 5);
    Acc3 c1{acc1, {}, {}}, c2{acc2, {}, {}};
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const Frag<P> b = ldf<P>(B, bc0 + r, k0 + 16 * ks);
        mfma_terms<P>(c1, ldf<P>(A1, a1r0 + r, k0 + 16 * ks), b);
        mfma_terms<P>(c2, ldf<P>(A2, a2r0 + r, k0 + 16 * ks), b);
    }
    acc1 = total<P>(c1);
    acc2 = total<P>(c2);
}

// An accumulator quadrant (rows row0.., columns col0..) into a term buffer with its columns as the
// buffer's rows ("column" layout, the B operand of a product over the quadrant's rows), P terms: lane
// l's column is col0 + l % 32, and registers 4g .. 4g + 3 are 4 consecutive rows.
template <int P>
__device__ __forceinline__ void put_cols(__bf16 *B, const f32x16 &x, int row0, int col0, int lane) {
    const int c = col0 + (lane & 31);
#pragma unroll
    for (int g = 0; g < 4; g++) {
        bf16x4 t[P];
#pragma unroll
        for (int z = 0; z < 4; z++) {
            __bf16 o[P];
            splitn<P>(x[4 * g + z], o);
#pragma unroll
            for (int i = 0; i < P; i++) t[i][z] = o[i];
        }
        const int r = row0 + g * 8 + (lane >> 5) * 4;
#pragma unroll
        for (int i = 0; i < P; i++) *reinterpret_cast<bf16x4 *>(B + i * PLANE + c * PST + r) = t[i];
    }
}

// 4 consecutive values of a row into a term buffer (row layout) at row r, columns c .. c + 3
template <int P>
__device__ __forceinline__ void put_row4(__bf16 *B, int r, int c, const f32x4 &x) {
    bf16x4 t[P];
#pragma unroll
    for (int z = 0; z < 4; z++) {
        __bf16 o[P];
        splitn<P>(x[z], o);
#pragma unroll
        for (int i = 0; i < P; i++) t[i][z] = o[i];
    }
#pragma unroll
    for (int i = 0; i < P; i++) *reinterpret_cast<bf16x4 *>(B + i * PLANE + r * PST + c) = t[i];
}

constexpr size_t DELTA_BF_LDS = 5 * (size_t)NTMAX * PLANE * sizeof(__bf16) + sizeof(float) * C * LD;

// acc (+)= A B over k = 32 half .. 32 half + 31 only
template <int P>
__device__ __forceinline__ void mq_bf_half(f32x16 &acc, const __bf16 *A, int ar0, const __bf16 *B, int bc0, int half,
                                           int lane) {
    const int r = lane & 31, k0 = 8 * (lane >> 5) + 32 * half;
    Acc3 c{acc, {}, {}};
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
        mfma_terms<P>(c, ldf<P>(A, ar0 + r, k0 + 16 * ks), ldf<P>(B, bc0 + r, k0 + 16 * ks));
    acc = total<P>(c);
}

// Eight waves, two per SIMD: wave w < 4 ("reader" waves) owns quadrant w of Y and computes K F, Q F and
// Y; wave w >= 4 ("state" waves) owns quadrant w - 4 of F (f32 in its registers) and computes X^T and the
// update K^T D; D = T' R splits its k range between the two sets (the state waves' half added through
// the LDS that held V). Each phase thus has two waves per SIMD to overlap.
__global__ __launch_bounds__(512) void delta_seq_bf_kernel(DeltaArgs p, const float *__restrict__ Tp) {
    extern __shared__ __attribute__((aligned(16))) float smb[];
    __bf16 *B1 = reinterpret_cast<__bf16 *>(smb);  // F columns (P1), then R columns (P2)
    __bf16 *B2 = B1 + NTMAX * PLANE;                // Q rows (P1), then X rows (P3)
    __bf16 *B3 = B2 + NTMAX * PLANE;                // T' rows (P2), then D columns (P3)
    __bf16 *B4 = B3 + NTMAX * PLANE;                // K rows
    __bf16 *B5 = B4 + NTMAX * PLANE;                // K columns (K^T rows)
    float *sV = reinterpret_cast<float *>(B5 + NTMAX * PLANE);  // V, f32 [64][LD]; then D's second half

    const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool reader = wave < 4;
    const int qd = wave & 3, row0 = (qd >> 1) * 32, col0 = (qd & 1) * 32, lc = lane & 31;
    const int nch = p.T / C;
    const float *qh = p.q + (size_t)bh * p.T * C, *kh = p.k + (size_t)bh * p.T * C, *vh = p.v + (size_t)bh * p.T * C;
    const float *Th = Tp + (size_t)bh * nch * C * C;
    float *Fh = p.F + (size_t)bh * C * C, *yh = p.y + (size_t)bh * p.T * C;

    f32x16 Fr = {};  // the state waves' quadrant of F
    if (!reader) {
#pragma unroll
        for (int i = 0; i < 16; i++) Fr[i] = Fh[(row0 + qrow(i, lane)) * C + col0 + lc];
        put_cols<3>(B1, Fr, row0, col0, lane);
    }

    // the next chunk's inputs in registers: float4 j of thread t is row (t + 512 j) / 16, columns
    // 4 ((t + 512 j) % 16) .. + 3
    f32x4 pk[2], pq[2], pv[2], pt[2];
    auto fetch = [&](int ch) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int idx = tid + 512 * j;
            const size_t o = (size_t)(ch * C + (idx >> 4)) * C + (idx & 15) * 4;
            pk[j] = *reinterpret_cast<const f32x4 *>(kh + o);
            pq[j] = *reinterpret_cast<const f32x4 *>(qh + o);
            pv[j] = *reinterpret_cast<const f32x4 *>(vh + o);
            pt[j] = *reinterpret_cast<const f32x4 *>(Th + (size_t)ch * C * C + (idx >> 4) * C + (idx & 15) * 4);
        }
    };
    // K rows (B4) and K columns (B5) from one split, Q rows (B2), T' rows (B3); V as f32
    auto stage = [&]() {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int idx = tid + 512 * j, r = idx >> 4, c = (idx & 15) * 4;
            bf16x4 kt[3];
#pragma unroll
            for (int z = 0; z < 4; z++) {
                __bf16 o[3];
                splitn<3>(pk[j][z], o);
#pragma unroll
                for (int i = 0; i < 3; i++) {
                    kt[i][z] = o[i];
                    B5[i * PLANE + (c + z) * PST + r] = o[i];
                }
                sV[r * LD + c + z] = pv[j][z];
            }
#pragma unroll
            for (int i = 0; i < 3; i++) *reinterpret_cast<bf16x4 *>(B4 + i * PLANE + r * PST + c) = kt[i];
            put_row4<3>(B2, r, c, pq[j]);
            put_row4<3>(B3, r, c, pt[j]);
        }
    };
    fetch(0);
    stage();
    f32x16 qf, kf, xt;
    for (int ch = 0; ch < nch; ch++) {
        const int t0 = ch * C;
        __syncthreads();  // the chunk's operands and F's terms are in LDS
        if (ch + 1 < nch) fetch(ch + 1);
        // P1: readers K F, Q F; state waves X^T = K Q^T (rows s, columns t)
        qf = f32x16{};
        kf = f32x16{};
        xt = f32x16{};
        if (reader) mq_bf_2a<3>(kf, B4, row0, qf, B2, row0, B1, col0, lane);
        else mq_bf<3>(xt, B4, row0, B2, col0, lane);
        __syncthreads();  // F's terms and Q's rows are read
        // readers: R = V - K F into B1 (columns); state waves: X (s <= t) into B2 as rows t
        if (reader) {
            f32x16 rr;
#pragma unroll
            for (int i = 0; i < 16; i++) rr[i] = sV[(row0 + qrow(i, lane)) * LD + col0 + lc] - kf[i];
            put_cols<3>(B1, rr, row0, col0, lane);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int s = row0 + qrow(i, lane), t = col0 + lc;
                xt[i] = s <= t ? xt[i] : 0.0f;
            }
            put_cols<3>(B2, xt, row0, col0, lane);  // row t of X = column t of X^T
        }
        __syncthreads();  // R is complete; V is read
        // D = T' R: readers take k 0..31, state waves k 32..63 and leave their half in the V buffer
        f32x16 d = {};
        mq_bf_half<3>(d, B3, row0, B1, col0, reader ? 0 : 1, lane);
        if (!reader) {
#pragma unroll
            for (int i = 0; i < 16; i++) sV[(row0 + qrow(i, lane)) * LD + col0 + lc] = d[i];
        }
        __syncthreads();  // T' is read; D's second half is in LDS
        if (reader) {
#pragma unroll
            for (int i = 0; i < 16; i++) d[i] = d[i] + sV[(row0 + qrow(i, lane)) * LD + col0 + lc];
            put_cols<3>(B3, d, row0, col0, lane);
        }
        __syncthreads();
        // P3: readers Y = Q F + X D; state waves F += K^T D and F's new terms (B1: R was read before
        // the barrier above)
        if (reader) {
            mq_bf<3>(qf, B2, row0, B3, col0, lane);
#pragma unroll
            for (int i = 0; i < 16; i++) yh[(size_t)(t0 + row0 + qrow(i, lane)) * C + col0 + lc] = qf[i];
        } else {
            f32x16 a = {};
            mq_bf<3>(a, B5, row0, B3, col0, lane);
#pragma unroll
            for (int i = 0; i < 16; i++) Fr[i] = Fr[i] + a[i];
            put_cols<3>(B1, Fr, row0, col0, lane);
        }
        __syncthreads();  // every read of this chunk's operands is done
        if (ch + 1 < nch) stage();
    }
    if (!reader) {
#pragma unroll
        for (int i = 0; i < 16; i++) Fh[(row0 + qrow(i, lane)) * C + col0 + lc] = Fr[i];
    }
}

__global__ __launch_bounds__(256) void delta_chunk_kernel(DeltaArgs p) {
    extern __shared__ float sm[];
    float *sK = sm, *sQ = sK + C * LD, *sV = sQ + C * LD, *sA = sV + C * LD, *sT = sA + C * LD;
    float *sW = sT + C * LD, *sU = sW + C * LD, *sF = sU + C * LD, *sX = sF + C * LD;
    float *s_cum = sX + C * LD, *s_beta = s_cum + C;

    const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = (wave >> 1) * 32, col0 = (wave & 1) * 32, lc = lane & 31;
    const float *qh = p.q + (size_t)bh * p.T * C, *kh = p.k + (size_t)bh * p.T * C, *vh = p.v + (size_t)bh * p.T * C;
    float *Fh = p.F + (size_t)bh * C * C, *yh = p.y + (size_t)bh * p.T * C;
    const bool gated = p.la != nullptr;

    for (int i = tid; i < C * C; i += 256) sF[(i >> 6) * LD + (i & 63)] = Fh[i];

    // the next chunk in registers: float4 j of thread t is row (t + 256 j) / 16, columns 4 ((t + 256 j) % 16)
    f32x4 pk[4], pq[4], pv[4];
    float pbeta = 0.0f, pla = 0.0f;
    auto fetch = [&](int t0) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int idx = tid + 256 * j, r = idx >> 4, c = (idx & 15) * 4;
            const size_t o = (size_t)(t0 + r) * C + c;
            pk[j] = *reinterpret_cast<const f32x4 *>(kh + o);
            pq[j] = *reinterpret_cast<const f32x4 *>(qh + o);
            pv[j] = *reinterpret_cast<const f32x4 *>(vh + o);
        }
        if (wave == 0) {
            pbeta = p.beta[(size_t)bh * p.T + t0 + lane];
            pla = gated ? p.la[(size_t)bh * p.T + t0 + lane] : 0.0f;
        }
    };
    auto put = [&](const f32x16 &acc, float *dst) {
#pragma unroll
        for (int i = 0; i < 16; i++) dst[(row0 + qrow(i, lane)) * LD + col0 + lc] = acc[i];
    };
    fetch(0);

    for (int t0 = 0; t0 < p.T; t0 += C) {
        // ---- stage the chunk; start the next one's loads
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int idx = tid + 256 * j, r = idx >> 4, c = (idx & 15) * 4;
#pragma unroll
            for (int z = 0; z < 4; z++) {
                sK[r * LD + c + z] = pk[j][z];
                sQ[r * LD + c + z] = pq[j][z];
                sV[r * LD + c + z] = pv[j][z];
            }
        }
        if (wave == 0) {
            s_beta[lane] = pbeta;
            if (gated) {
                // cum = running sum of log alpha, in token order
                float run = 0.0f;
                for (int i = 0; i < C; i++) {
                    run = run + __shfl(pla, i, 64);
                    if (lane == i) s_cum[i] = run;
                }
            }
        }
        __syncthreads();
        if (t0 + C < p.T) fetch(t0 + C);

        // ---- QK = Q K^T -> sX;  A = strict_lower(beta_i k_i . k_j) -> sA
        {
            f32x16 aq = {}, ak = {};
            mq(aq, lane, [&](int r, int x) { return sQ[(row0 + r) * LD + x]; },
               [&](int x, int c) { return sK[(col0 + c) * LD + x]; });
            mq(ak, lane, [&](int r, int x) { return sK[(row0 + r) * LD + x]; },
               [&](int x, int c) { return sK[(col0 + c) * LD + x]; });
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int r = row0 + qrow(i, lane), c = col0 + lc;
                sX[r * LD + c] = aq[i];
                sA[r * LD + c] = c < r ? s_beta[r] * ak[i] : 0.0f;
            }
        }
        __syncthreads();

        // ---- Tw = (I + A)^-1 -> sT, column by column, left-looking: x_i = [i == c] - sum_{j<i} A_ij x_j.
        //      Wave w solves columns 16w..16w+15; lane l holds column c = 16w + (l & 15) and the rows
        //      j = 4m + (l >> 4) of its solution in registers. A row's sum is split over the column's 4
        //      lanes and added with the lane swaps, so a step's dependency chain is one fma and two swaps
        //      (the other products and the A row's reads do not wait for the previous row).
        {
            const int c = wave * 16 + (lane & 15), q = lane >> 4;
            float xr[16];  // rows not solved yet hold 0, so their terms vanish without a mask
#pragma unroll
            for (int m = 0; m < 16; m++) xr[m] = 0.0f;
#pragma unroll
            for (int i = 0; i < C; i++) {
                float part = 0.0f;
#pragma unroll
                for (int m = 0; 4 * m < i; m++) part = fmaf(sA[i * LD + 4 * m + q], xr[m], part);
                const float tot = xsum32(xsum16(part));
                const float xi = (i == c ? 1.0f : 0.0f) - tot;
                if (q == (i & 3)) xr[i >> 2] = xi;
            }
#pragma unroll
            for (int m = 0; m < 16; m++) sT[(4 * m + q) * LD + c] = xr[m];
        }
        __syncthreads();

        // ---- W = Tw (beta K) -> sW;  U = (D o Tw) (beta V) -> sU
        {
            f32x16 aw = {}, au = {};
            mq(aw, lane, [&](int r, int x) { return sT[(row0 + r) * LD + x]; },
               [&](int x, int c) { return s_beta[x] * sK[x * LD + col0 + c]; });
            mq(au, lane,
               [&](int r, int x) {
                   const int i = row0 + r;
                   return x <= i ? sT[i * LD + x] * expf(s_cum[i] - s_cum[x]) : 0.0f;
               },
               [&](int x, int c) { return s_beta[x] * sV[x * LD + col0 + c]; });
            put(aw, sW);
            put(au, sU);
        }
        __syncthreads();

        // ---- WF = W F -> sA
        {
            f32x16 a = {};
            mq(a, lane, [&](int r, int x) { return sW[(row0 + r) * LD + x]; },
               [&](int x, int c) { return sF[x * LD + col0 + c]; });
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int o = (row0 + qrow(i, lane)) * LD + col0 + lc;
                sA[o] = a[i];
            }
        }
        __syncthreads();

        // ---- Y = diag(Gamma) (Q F - (QK o M) WF) + (QK o D o M) U
        {
            f32x16 a1 = {};
            mq(a1, lane, [&](int r, int x) { return sQ[(row0 + r) * LD + x]; },
               [&](int x, int c) { return sF[x * LD + col0 + c]; });
            {
                f32x16 a2 = {};
                mq(a1, lane, [&](int r, int x) { return x <= row0 + r ? -sX[(row0 + r) * LD + x] : 0.0f; },
                   [&](int x, int c) { return sA[x * LD + col0 + c]; });
                mq(a2, lane,
                   [&](int r, int x) {
                       const int i = row0 + r;
                       return x <= i ? sX[i * LD + x] * expf(s_cum[i] - s_cum[x]) : 0.0f;
                   },
                   [&](int x, int c) { return sU[x * LD + col0 + c]; });
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int r = row0 + qrow(i, lane);
                    yh[(size_t)(t0 + r) * C + col0 + lc] = a1[i] * expf(s_cum[r]) + a2[i];
                }
            }
        }
        __syncthreads();  // every read of F for this chunk is done

        // ---- F <- Gamma_c (F - K^T WF) + K^T diag(Gamma_c / Gamma) U
        {
            f32x16 a = {};
            mq(a, lane, [&](int r, int x) { return sK[x * LD + row0 + r]; },
               [&](int x, int c) { return sA[x * LD + col0 + c]; });
            {
                f32x16 b = {};
                const float cl = s_cum[C - 1], gc = expf(cl);
                mq(b, lane, [&](int r, int x) { return sK[x * LD + row0 + r]; },
                   [&](int x, int c) { return sU[x * LD + col0 + c] * expf(cl - s_cum[x]); });
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int o = (row0 + qrow(i, lane)) * LD + col0 + lc;
                    sF[o] = (sF[o] - a[i]) * gc + b[i];
                }
            }
        }
        __syncthreads();
        }

    for (int i = tid; i < C * C; i += 256) Fh[i] = sF[(i >> 6) * LD + (i & 63)];
}

}  // namespace

extern "C" size_t ava_delta_chunk_workspace(int BH, int T) {
    return BH > 0 && T > 0 ? (size_t)BH * T * C * sizeof(float) : 0;
}

extern "C" int ava_delta_chunk(const float *q, const float *k, const float *v, const float *la, const float *beta,
                               int BH, int T, int hs, float *F, float *y, void *work, size_t work_bytes,
                               ava_stream stream) {
    AVA_REQUIRE(q && k && v && beta && F && y, AVA_ERR_ARG, "delta_chunk: NULL buffer");
    AVA_REQUIRE(hs == C, AVA_ERR_UNSUPPORTED, "delta_chunk: head size %d (this build runs 64)", hs);
    AVA_REQUIRE(BH >= 0 && T >= 0 && T % C == 0, AVA_ERR_SHAPE, "delta_chunk: BH=%d T=%d (T a multiple of 64)", BH, T);
    if (BH == 0 || T == 0) return AVA_OK;
    const hipStream_t st = (hipStream_t)stream;
    const size_t lds = sizeof(float) * (9 * C * LD + 2 * C);
    DeltaArgs a{q, k, v, la, beta, T, F, y};
    if (!la && work) {
        AVA_REQUIRE(work_bytes >= ava_delta_chunk_workspace(BH, T), AVA_ERR_SHAPE,
                    "delta_chunk: the workspace holds %zu bytes, %zu needed", work_bytes,
                    ava_delta_chunk_workspace(BH, T));
        const size_t lds2 = DELTA_BF_LDS;
        if (int r = ava::lds_opt_in((const void *)delta_seq_bf_kernel, lds2)) return r;
        const int nch = T / C;
        DeltaInvArgs ia{k, beta, T, nch, reinterpret_cast<float *>(work)};
        delta_inv_kernel<<<BH * nch, 256, 0, st>>>(ia);
        AVA_LAUNCHED("delta_inv");
        delta_seq_bf_kernel<<<BH, 512, lds2, st>>>(a, reinterpret_cast<const float *>(work));
        AVA_LAUNCHED("delta_seq");
        return AVA_OK;
    }
    if (int r = ava::lds_opt_in((const void *)delta_chunk_kernel, lds)) return r;
    if (int r = ava::lds_opt_in((const void *)delta_plain_kernel, lds)) return r;
    if (la) delta_chunk_kernel<<<BH, 256, lds, st>>>(a);
    else delta_plain_kernel<<<BH, 256, lds, st>>>(a);
    AVA_LAUNCHED("delta_chunk");
    return AVA_OK;
}
