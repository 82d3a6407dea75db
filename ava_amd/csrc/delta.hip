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
// Every 64 x 64 x 64 product runs on the fp32 MFMA (v_mfma_f32_32x32x2_f32, one 32 x 32 quadrant per
// wave, operands straight from LDS rows of odd stride, so a column read hits 32 different banks).
// Without gates (alpha = 1, config[2]) the two read-outs merge: Y = Q F + (QK^T o M)(U - W F) and
// F <- F + K^T (U - W F). The unit lower-triangular inverse is a left-looking forward substitution
// spread over the 4 waves (16 columns each, 4 lanes per column); the reference doubles blocks
// (gpu/model.rs:720-742): both are exact inverses, equal up to rounding. The next chunk's q, k, v
// are loaded into registers while the current chunk is computed.
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

extern "C" int ava_delta_chunk(const float *q, const float *k, const float *v, const float *la, const float *beta,
                               int BH, int T, int hs, float *F, float *y, ava_stream stream) {
    AVA_REQUIRE(q && k && v && beta && F && y, AVA_ERR_ARG, "delta_chunk: NULL buffer");
    AVA_REQUIRE(hs == C, AVA_ERR_UNSUPPORTED, "delta_chunk: head size %d (this build runs 64)", hs);
    AVA_REQUIRE(BH >= 0 && T >= 0 && T % C == 0, AVA_ERR_SHAPE, "delta_chunk: BH=%d T=%d (T a multiple of 64)", BH, T);
    if (BH == 0 || T == 0) return AVA_OK;
    const size_t lds = sizeof(float) * (9 * C * LD + 2 * C);
    if (int r = ava::lds_opt_in((const void *)delta_chunk_kernel, lds)) return r;
    if (int r = ava::lds_opt_in((const void *)delta_plain_kernel, lds)) return r;
    DeltaArgs a{q, k, v, la, beta, T, F, y};
    if (la) delta_chunk_kernel<<<BH, 256, lds, (hipStream_t)stream>>>(a);
    else delta_plain_kernel<<<BH, 256, lds, (hipStream_t)stream>>>(a);
    AVA_LAUNCHED("delta_chunk");
    return AVA_OK;
}
