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
// The unit lower-triangular inverse is a forward substitution, one lane per column of Tw (the
// reference doubles blocks, gpu/model.rs:720-742; both are exact inverses, equal up to rounding).
// Every 64 x 64 x 64 product runs on 256 threads with a 4 x 4 register block each.
#include "common.h"

namespace {

constexpr int C = 64, LD = 68;  // chunk length / head size, padded LDS row (float4-aligned)

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct DeltaArgs {
    const float *q, *k, *v, *la, *beta;  // [BH][T][64], la/beta [BH][T] (la NULL: alpha = 1)
    int T;
    float *F, *y;
};

// acc[a][b] += sum_x A(r0 + a, x) B(x, c0 + b), A and B read through the accessors.
template <class FA, class FB>
__device__ __forceinline__ void mm4(float (&acc)[4][4], FA fa, FB fb) {
#pragma unroll 4
    for (int x = 0; x < C; x++) {
        float av[4], bv[4];
#pragma unroll
        for (int a = 0; a < 4; a++) av[a] = fa(a, x);
        const f32x4 b4 = fb(x);
#pragma unroll
        for (int b = 0; b < 4; b++) bv[b] = b4[b];
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) acc[a][b] = fmaf(av[a], bv[b], acc[a][b]);
    }
}

__global__ __launch_bounds__(256) void delta_chunk_kernel(DeltaArgs p) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float *sK = sm, *sQ = sK + C * LD, *sV = sQ + C * LD, *sA = sV + C * LD, *sT = sA + C * LD;
    float *sW = sT + C * LD, *sU = sW + C * LD, *sF = sU + C * LD, *sX = sF + C * LD;
    float *s_cum = sX + C * LD, *s_beta = s_cum + C;

    const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ty = tid >> 4, tx = tid & 15, r0 = ty * 4, c0 = tx * 4;
    const float *qh = p.q + (size_t)bh * p.T * C, *kh = p.k + (size_t)bh * p.T * C, *vh = p.v + (size_t)bh * p.T * C;
    float *Fh = p.F + (size_t)bh * C * C, *yh = p.y + (size_t)bh * p.T * C;
    const bool gated = p.la != nullptr;

    for (int i = tid; i < C * C / 4; i += 256) {
        const int r = i >> 4, c = (i & 15) * 4;
        *reinterpret_cast<f32x4 *>(sF + r * LD + c) = reinterpret_cast<const f32x4 *>(Fh)[i];
    }

    for (int t0 = 0; t0 < p.T; t0 += C) {
        // ---- load the chunk
        for (int i = tid; i < C * C / 4; i += 256) {
            const int r = i >> 4, c = (i & 15) * 4;
            const size_t o = (size_t)(t0 + r) * C + c;
            *reinterpret_cast<f32x4 *>(sK + r * LD + c) = *reinterpret_cast<const f32x4 *>(kh + o);
            *reinterpret_cast<f32x4 *>(sQ + r * LD + c) = *reinterpret_cast<const f32x4 *>(qh + o);
            *reinterpret_cast<f32x4 *>(sV + r * LD + c) = *reinterpret_cast<const f32x4 *>(vh + o);
        }
        if (wave == 0) {
            s_beta[lane] = p.beta[(size_t)bh * p.T + t0 + lane];
            // cum = running sum of log alpha, in token order (one lane does the serial sum)
            float la = gated ? p.la[(size_t)bh * p.T + t0 + lane] : 0.0f;
            float run = 0.0f;
            for (int i = 0; i < C; i++) {
                const float li = __shfl(la, i, 64);
                run = run + li;
                if (lane == i) s_cum[i] = run;
            }
        }
        __syncthreads();

        // ---- A = strict_lower(beta_i k_i . k_j)
        {
            float acc[4][4] = {};
            mm4(acc, [&](int a, int x) { return sK[(r0 + a) * LD + x]; },
                [&](int x) { return f32x4{sK[(c0 + 0) * LD + x], sK[(c0 + 1) * LD + x], sK[(c0 + 2) * LD + x],
                                          sK[(c0 + 3) * LD + x]}; });
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int i = r0 + a, j = c0 + b;
                    sA[i * LD + j] = j < i ? s_beta[i] * acc[a][b] : 0.0f;
                }
        }
        __syncthreads();

        // ---- Tw = (I + A)^-1: lane = column c, forward substitution over rows (one wave)
        if (wave == 0) {
            const int c = lane;
            float t[C];
#pragma unroll
            for (int i = 0; i < C; i++) {
                float s = i == c ? 1.0f : 0.0f;
#pragma unroll
                for (int j = 0; j < i; j++) s = fmaf(-sA[i * LD + j], t[j], s);
                t[i] = s;
            }
#pragma unroll
            for (int i = 0; i < C; i++) sT[i * LD + c] = t[i];
        }
        __syncthreads();

        // ---- W = Tw (beta K) -> sW;  U = (D o Tw) (beta V) -> sU
        {
            float aw[4][4] = {}, au[4][4] = {};
            mm4(aw, [&](int a, int x) { return sT[(r0 + a) * LD + x]; },
                [&](int x) {
                    const f32x4 kk = *reinterpret_cast<const f32x4 *>(sK + x * LD + c0);
                    return kk * s_beta[x];
                });
            if (gated) {
                mm4(au, [&](int a, int x) {
                        const int i = r0 + a;
                        return x <= i ? sT[i * LD + x] * expf(s_cum[i] - s_cum[x]) : 0.0f;
                    },
                    [&](int x) {
                        const f32x4 vv = *reinterpret_cast<const f32x4 *>(sV + x * LD + c0);
                        return vv * s_beta[x];
                    });
            } else {
                mm4(au, [&](int a, int x) { return sT[(r0 + a) * LD + x]; },
                    [&](int x) {
                        const f32x4 vv = *reinterpret_cast<const f32x4 *>(sV + x * LD + c0);
                        return vv * s_beta[x];
                    });
            }
#pragma unroll
            for (int a = 0; a < 4; a++) {
                *reinterpret_cast<f32x4 *>(sW + (r0 + a) * LD + c0) = f32x4{aw[a][0], aw[a][1], aw[a][2], aw[a][3]};
                *reinterpret_cast<f32x4 *>(sU + (r0 + a) * LD + c0) = f32x4{au[a][0], au[a][1], au[a][2], au[a][3]};
            }
        }
        __syncthreads();

        // ---- WF = W F -> sA;  QK = Q K^T -> sX
        {
            float aw[4][4] = {}, aq[4][4] = {};
            mm4(aw, [&](int a, int x) { return sW[(r0 + a) * LD + x]; },
                [&](int x) { return *reinterpret_cast<const f32x4 *>(sF + x * LD + c0); });
            mm4(aq, [&](int a, int x) { return sQ[(r0 + a) * LD + x]; },
                [&](int x) { return f32x4{sK[(c0 + 0) * LD + x], sK[(c0 + 1) * LD + x], sK[(c0 + 2) * LD + x],
                                          sK[(c0 + 3) * LD + x]}; });
#pragma unroll
            for (int a = 0; a < 4; a++) {
                *reinterpret_cast<f32x4 *>(sA + (r0 + a) * LD + c0) = f32x4{aw[a][0], aw[a][1], aw[a][2], aw[a][3]};
                *reinterpret_cast<f32x4 *>(sX + (r0 + a) * LD + c0) = f32x4{aq[a][0], aq[a][1], aq[a][2], aq[a][3]};
            }
        }
        __syncthreads();

        // ---- Y = diag(Gamma) (Q F - (QK o M) WF) + (QK o D o M) U
        {
            float qf[4][4] = {}, mw[4][4] = {}, du[4][4] = {};
            mm4(qf, [&](int a, int x) { return sQ[(r0 + a) * LD + x]; },
                [&](int x) { return *reinterpret_cast<const f32x4 *>(sF + x * LD + c0); });
            mm4(mw, [&](int a, int x) { return x <= r0 + a ? sX[(r0 + a) * LD + x] : 0.0f; },
                [&](int x) { return *reinterpret_cast<const f32x4 *>(sA + x * LD + c0); });
            if (gated) {
                mm4(du, [&](int a, int x) {
                        const int i = r0 + a;
                        return x <= i ? sX[i * LD + x] * expf(s_cum[i] - s_cum[x]) : 0.0f;
                    },
                    [&](int x) { return *reinterpret_cast<const f32x4 *>(sU + x * LD + c0); });
            } else {
                mm4(du, [&](int a, int x) { return x <= r0 + a ? sX[(r0 + a) * LD + x] : 0.0f; },
                    [&](int x) { return *reinterpret_cast<const f32x4 *>(sU + x * LD + c0); });
            }
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const int i = r0 + a;
                const float g = gated ? expf(s_cum[i]) : 1.0f;
                f32x4 o;
#pragma unroll
                for (int b = 0; b < 4; b++) o[b] = (qf[a][b] - mw[a][b]) * g + du[a][b];
                *reinterpret_cast<f32x4 *>(yh + (size_t)(t0 + i) * C + c0) = o;
            }
        }
        __syncthreads();  // every read of F for this chunk is done

        // ---- F <- Gamma_c (F - K^T WF) + K^T diag(Gamma_c / Gamma) U
        {
            float kw[4][4] = {}, ku[4][4] = {};
            const float cl = s_cum[C - 1];
            mm4(kw, [&](int a, int x) { return sK[x * LD + r0 + a]; },
                [&](int x) { return *reinterpret_cast<const f32x4 *>(sA + x * LD + c0); });
            mm4(ku, [&](int a, int x) { return sK[x * LD + r0 + a]; },
                [&](int x) {
                    const f32x4 uu = *reinterpret_cast<const f32x4 *>(sU + x * LD + c0);
                    return gated ? uu * expf(cl - s_cum[x]) : uu;
                });
            const float gc = gated ? expf(cl) : 1.0f;
#pragma unroll
            for (int a = 0; a < 4; a++) {
                f32x4 f = *reinterpret_cast<const f32x4 *>(sF + (r0 + a) * LD + c0);
#pragma unroll
                for (int b = 0; b < 4; b++) f[b] = (f[b] - kw[a][b]) * gc + ku[a][b];
                *reinterpret_cast<f32x4 *>(sF + (r0 + a) * LD + c0) = f;
            }
        }
        __syncthreads();
    }

    for (int i = tid; i < C * C / 4; i += 256) {
        const int r = i >> 4, c = (i & 15) * 4;
        reinterpret_cast<f32x4 *>(Fh)[i] = *reinterpret_cast<const f32x4 *>(sF + r * LD + c);
    }
}

}  // namespace

extern "C" int ava_delta_chunk(const float *q, const float *k, const float *v, const float *la, const float *beta,
                               int BH, int T, int hs, float *F, float *y, ava_stream stream) {
    AVA_REQUIRE(q && k && v && beta && F && y, AVA_ERR_ARG, "delta_chunk: NULL buffer");
    AVA_REQUIRE(hs == C, AVA_ERR_UNSUPPORTED, "delta_chunk: head size %d (this build runs 64)", hs);
    AVA_REQUIRE(BH >= 0 && T >= 0 && T % C == 0, AVA_ERR_SHAPE, "delta_chunk: BH=%d T=%d (T a multiple of 64)", BH, T);
    if (BH == 0 || T == 0) return AVA_OK;
    const size_t lds = sizeof(float) * (9 * C * LD + 2 * C);
    static bool attr = false;
    if (!attr) {
        AVA_HIP(hipFuncSetAttribute((const void *)delta_chunk_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds));
        attr = true;
    }
    DeltaArgs a{q, k, v, la, beta, T, F, y};
    delta_chunk_kernel<<<BH, 256, lds, (hipStream_t)stream>>>(a);
    AVA_LAUNCHED("delta_chunk");
    return AVA_OK;
}
