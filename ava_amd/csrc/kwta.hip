// k-winners-take-all for gfx950: one wavefront per row, the row held in registers.
//
// The k-th largest value of a row is exact. As soon as some threshold t has exactly k values at or
// above it, the answer is the smallest of those values (one wave min). Such a t is searched in value
// space first: the count of values >= t is monotone in t, so t is interpolated (alternating with
// midpoints) inside a bracket whose counts straddle k; a continuous row needs a handful of counts.
// When ties make the count skip k, an exact bisection over the order-preserving uint32 image of
// the floats (larger float <=> larger key) takes over: the candidate key prefix|bit is kept when at
// least k keys are >= it, which ends at the k-th largest key (duplicates counted). Each count is a
// wave ballot per register and a popcount: no LDS, no atomics, no barriers, so a SIMD interleaves
// several rows' waves while their loads are in flight. HBM traffic is one read of u and one
// write of the output per element.
//
// The mask is then the reference's: keep u_i when u_i - kth >= 0 (ties kept: more than k units
// can win), a = relu(u · mask), squared with relu2 (gpu/model/fstep/arch.rs:976-989,
// gpu/lif.cu:4629-4655). Optionally the kernel emits the split-plane int8 form of a (the input
// of the W2 product) instead of f32.
#include "common.h"

namespace {

__device__ __forceinline__ uint32_t key_of(float f) {
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float float_of_key(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float uni(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }



// Row reductions: over the wave (a wave per row), or over the row's RW waves through LDS (a
// workgroup per row, for few rows), combined pairwise in a fixed order. Results are wave-uniform
// (readfirstlane) either way; the leading barrier keeps a reduction from overwriting slots the
// previous one is still reading.
template <int N, class T, class F>
__device__ __forceinline__ T tree(const T *r, F op) {
    if constexpr (N == 1) return r[0];
    else return op(tree<N / 2>(r, op), tree<N / 2>(r + N / 2, op));
}
template <int RW>
struct RowRed {
    float *fs;
    int *is;
    template <class T, class F>
    __device__ __forceinline__ T across(T v, T *slots, F op) {
        if constexpr (RW > 1) {
            __syncthreads();
            if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
            __syncthreads();
            v = tree<RW>(slots, op);
        }
        return v;
    }
    __device__ __forceinline__ float fsum(float v) {
        return uni(across(ava::wave_sum(v), fs, [](float a, float b) { return a + b; }));
    }
    __device__ __forceinline__ float fmin(float v) {
        return uni(across(ava::wave_min(v), fs, [](float a, float b) { return fminf(a, b); }));
    }
    __device__ __forceinline__ float fmax(float v) {
        return uni(across(ava::wave_max(v), fs, [](float a, float b) { return fmaxf(a, b); }));
    }
    __device__ __forceinline__ int isum(int v) {  // v wave-uniform
        return __builtin_amdgcn_readfirstlane(across(v, is, [](int a, int b) { return a + b; }));
    }
    __device__ __forceinline__ uint32_t umin(uint32_t v) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
        int r = across((int)v, is, [](int a, int b) { return (int)min((uint32_t)a, (uint32_t)b); });
        return (uint32_t)__builtin_amdgcn_readfirstlane(r);
    }
};

// NV float4 chunks per lane. A wave per row (RW = 1): h <= 256 NV, chunk c = 64 i + lane; a
// workgroup of RW waves per row (RW = 4): h <= 256 RW NV, chunk c = 64 RW i + thread (8 and 16 waves
// per row measured slower on the decode rows). OUT: 0 = f32 a, P>0 = P int8 planes + row exponent.
template <int NV, int P, bool FULL, int RW = 1>
__global__ __launch_bounds__(RW > 4 ? 64 * RW : 256) void kwta_kernel(const float *__restrict__ u, int n, int h, int k,
                                                                      int relu2, float *__restrict__ a,
                                                                      float *__restrict__ kth_out,
                                                                      int8_t *__restrict__ xq,
                                                                      int32_t *__restrict__ xexp, int ldq) {
    constexpr bool WG = RW > 1;
    __shared__ float s_f[RW > 4 ? RW : 4];
    __shared__ int s_i[RW > 4 ? RW : 4];
    RowRed<RW> red{s_f, s_i};
    constexpr int LANES = 64 * RW;  // threads of a row
    const int lane = WG ? (int)threadIdx.x : (int)(threadIdx.x & 63);
    const int row = WG ? (int)blockIdx.x : (int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    if (row >= n) return;  // uniform over the row's threads
    const float *ur = u + (size_t)row * h;
    const int nq = h >> 2;  // float4 chunks in the row

    f32x4 x[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * LANES + lane;
        if (FULL || c < nq) x[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(ur) + c);
        else x[i] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // never counted: see below
    }

    float kth = -INFINITY;
    const bool all = k >= h;
    constexpr bool full = FULL;  // h == LANES NV * 4: every chunk real, no padding lanes
    // count of the row's values >= t (padding chunks are -inf and never counted for finite t)
    auto count_ge = [&](float t) {
        int c = 0;
#pragma unroll
        for (int i = 0; i < NV; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) c += __popcll(__ballot(x[i][j] >= t));
        return red.isum(c);
    };
    // the k-th largest once exactly k values are >= t: the smallest of them. A zero result is
    // -0 when a -0 is among them (in the order of the keys, -0 < +0), else +0.
    auto smallest_at_or_above = [&](float t) {
        float mn = INFINITY;
#pragma unroll
        for (int i = 0; i < NV; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) mn = x[i][j] >= t ? fminf(mn, x[i][j]) : mn;
        mn = red.fmin(mn);
        if (mn == 0.0f) {
            bool neg = false;
#pragma unroll
            for (int i = 0; i < NV; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) neg |= x[i][j] >= t && __float_as_uint(x[i][j]) == 0x80000000u;
            mn = red.isum(__ballot(neg) ? 1 : 0) ? -0.0f : 0.0f;
        }
        return mn;
    };
    if (!all) {
        // 1. search in value space: count(>= t) is monotone; interpolate t between a bracket
        //    lo (count > k) and hi (count < k) until exactly k values are >= t, which for
        //    continuous rows takes a handful of counts. Ties can make the count skip k: then
        //    (or on non-finite values) fall through to the exact bisection.
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool real = full || i * LANES + lane < nq;
                if (real) {
                    lo = fminf(lo, x[i][j]);
                    hi = fmaxf(hi, x[i][j]);
                }
            }
        // wave-uniform (readfirstlane), so the search's control flow is scalar
        lo = red.fmin(lo);
        hi = red.fmax(hi);
        bool done = false, found = false;
        float tk = 0.0f;  // a threshold with exactly k values at or above it
        if (isfinite(lo) && isfinite(hi)) {
            int clo = h, chi = count_ge(hi);
            if (chi >= k) {  // the maximum is the k-th largest (ties at the top)
                kth = hi;
                done = true;
            }
            // Two first guesses from the row's mean and deviation as if it were normal: the quantile
            // of the kept fraction, then one Newton step on the count with the normal density. They
            // only place the bracket (any guess gives the same exact answer); on wide-layer rows they
            // land within a few per cent of k, so the interpolation below needs a few counts more.
            if (!done) {
                float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
                for (int i = 0; i < NV; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const bool real = full || i * LANES + lane < nq;
                        s1 += real ? x[i][j] : 0.0f;
                        s2 += real ? x[i][j] * x[i][j] : 0.0f;
                    }
                s1 = red.fsum(s1);
                s2 = red.fsum(s2);
                const float mu = s1 / (float)h, sd = sqrtf(fmaxf(s2 / (float)h - mu * mu, 0.0f));
                const float z = ava::normal_upper_quantile((float)k / (float)h);
                const float dens = (float)h * 0.39894228f * __expf(-0.5f * z * z) / fmaxf(sd, 1e-30f);
                float t = uni(mu + z * sd);
                for (int g = 0; g < 2 && !found; g++) {
                    if (!(t > lo && t < hi)) break;
                    const int c = count_ge(t);
                    if (c == k) {
                        tk = t;
                        found = true;
                    } else if (c > k) {
                        lo = t;
                        clo = c;
                    } else {
                        hi = t;
                        chi = c;
                    }
                    t = uni(t + (float)(c - k) / dens);
                }
            }
            for (int it = 0; it < 24 && !done && !found; it++) {
                // interpolation on even steps, midpoint on odd ones (guards slow one-sided convergence)
                float t = (it & 1) ? lo * 0.5f + hi * 0.5f
                                   : lo + (hi - lo) * ((float)(clo - k) / (float)(clo - chi));
                if (!(t > lo && t < hi)) t = lo * 0.5f + hi * 0.5f;
                if (!(t > lo && t < hi)) break;  // lo, hi adjacent floats: ties
                const int c = count_ge(t);
                if (c == k) {
                    tk = t;
                    found = true;
                } else if (c > k) {
                    lo = t;
                    clo = c;
                } else {
                    hi = t;
                    chi = c;
                }
            }
        }
        if (found) {  // outside the search loop, so the keys are not hoisted into registers of their own
            kth = smallest_at_or_above(tk);
            done = true;
        }
        if (!done) {
            // 2. exact bisection over the order-preserving key image (any input, ties included). The
            //    keys replace the values in place (padding: key 0, below every real key) and the
            //    values come back after, so the row stays in one set of registers.
#pragma unroll
            for (int i = 0; i < NV; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const bool real = full || i * LANES + lane < nq;
                    x[i][j] = __uint_as_float(real ? key_of(x[i][j]) : 0u);
                }
            uint32_t prefix = 0;
            for (int bit = 31; bit >= 0; bit--) {
                const uint32_t cand = prefix | (1u << bit);
                int cnt = 0;
#pragma unroll
                for (int i = 0; i < NV; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) cnt += __popcll(__ballot(__float_as_uint(x[i][j]) >= cand));
                cnt = red.isum(cnt);
                if (cnt >= k) prefix = cand;
                if (cnt == k) {
                    // exactly k keys are >= cand: the k-th largest is the smallest of them
                    uint32_t mn = 0xffffffffu;
#pragma unroll
                    for (int i = 0; i < NV; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const uint32_t kk = __float_as_uint(x[i][j]);
                            mn = kk >= cand ? min(mn, kk) : mn;
                        }
                    prefix = red.umin(mn);
                    break;
                }
            }
            kth = float_of_key(prefix);
#pragma unroll
            for (int i = 0; i < NV; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const bool real = full || i * LANES + lane < nq;
                    x[i][j] = real ? float_of_key(__float_as_uint(x[i][j])) : -INFINITY;
                }
        }
    }
    if (kth_out && lane == 0) kth_out[row] = kth;

    // a = relu(u · mask)^(1 or 2)
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = x[i][j];
            const float keep = all ? 1.0f : ((v - kth >= 0.0f) ? 1.0f : 0.0f);
            float y = v * keep;
            y = y > 0.0f ? y : 0.0f;
            y = relu2 ? y * y : y;
            x[i][j] = y;
            amax = fmaxf(amax, y);
        }

    if constexpr (P == 0) {
        float *ar = a + (size_t)row * h;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int c = i * LANES + lane;
            if (full || c < nq) __builtin_nontemporal_store(x[i], reinterpret_cast<f32x4 *>(ar) + c);
        }
    } else {
        amax = red.fmax(amax);
        const int e = ava::plane_exp(amax);
        if (lane == 0) xexp[row] = e;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int c = i * LANES + lane;
            if (full || c < nq) {
                int q0[P], q1[P], q2[P], q3[P];
                ava::to_planes<P>(x[i][0], e, q0);
                ava::to_planes<P>(x[i][1], e, q1);
                ava::to_planes<P>(x[i][2], e, q2);
                ava::to_planes<P>(x[i][3], e, q3);
#pragma unroll
                for (int p = 0; p < P; p++)
                    __builtin_nontemporal_store(ava::pack4(q0[p], q1[p], q2[p], q3[p]),
                                                reinterpret_cast<uint32_t *>(xq + ((size_t)p * n + row) * ldq) + c);
            }
        }
        // zero the K padding of the planes (ldq > h)
        for (int c = h + lane * 4; c < ldq; c += 4 * LANES)
#pragma unroll
            for (int p = 0; p < P; p++)
                *reinterpret_cast<uint32_t *>(xq + ((size_t)p * n + row) * ldq + c) = 0u;
    }
}

// Rows at most this many take a workgroup each: with few rows a wave per row leaves most of the chip
// idle and each row's search is a chain of counts.
constexpr int WG_ROWS = 2048;

template <int P>
int launch(const float *u, int n, int h, int k, int relu2, float *a, float *kth, int8_t *xq, int32_t *xexp,
           int ldq, hipStream_t st) {
    if (n <= WG_ROWS && h <= 4096) {
        const int nv4 = (h + 1023) / 1024;
#define AVA_KWG(NV_)                                                                                           \
    if (nv4 <= NV_) {                                                                                          \
        if (h == NV_ * 1024)                                                                                   \
            kwta_kernel<NV_, P, true, 4><<<n, 256, 0, st>>>(u, n, h, k, relu2, a, kth, xq, xexp, ldq);          \
        else                                                                                                   \
            kwta_kernel<NV_, P, false, 4><<<n, 256, 0, st>>>(u, n, h, k, relu2, a, kth, xq, xexp, ldq);         \
        AVA_LAUNCHED("kwta");                                                                                  \
        return AVA_OK;                                                                                         \
    }
        AVA_KWG(1) AVA_KWG(2) AVA_KWG(4)
#undef AVA_KWG
    }
    const int nv = (h + 255) / 256;
    dim3 grid(ava::ceil_div(n, 4)), block(256);
#define AVA_KW(NV_)                                                                                      \
    if (nv <= NV_) {                                                                                     \
        if (h == NV_ * 256)                                                                              \
            kwta_kernel<NV_, P, true><<<grid, block, 0, st>>>(u, n, h, k, relu2, a, kth, xq, xexp, ldq);  \
        else                                                                                             \
            kwta_kernel<NV_, P, false><<<grid, block, 0, st>>>(u, n, h, k, relu2, a, kth, xq, xexp, ldq); \
        AVA_LAUNCHED("kwta");                                                                            \
        return AVA_OK;                                                                                   \
    }
    AVA_KW(1) AVA_KW(2) AVA_KW(4) AVA_KW(8) AVA_KW(16) AVA_KW(32)
#undef AVA_KW
    return ava::fail(AVA_ERR_SHAPE, "kwta: row width %d > 8192", h);
}

}  // namespace

namespace ava {

// kWTA with the split-plane int8 output (the W2 input of a block): xq [P][n][ldq], xexp [n].
int kwta_planes(const float *u, int n, int h, int k, int relu2, int planes, int8_t *xq, int32_t *xexp, int ldq,
                float *kth, hipStream_t st) {
    AVA_REQUIRE(h % 4 == 0 && ldq % 4 == 0 && ldq >= h, AVA_ERR_SHAPE, "kwta_planes: h=%d ldq=%d", h, ldq);
    if (planes == 1) return launch<1>(u, n, h, k, relu2, nullptr, kth, xq, xexp, ldq, st);
    if (planes == 2) return launch<2>(u, n, h, k, relu2, nullptr, kth, xq, xexp, ldq, st);
    if (planes == 3) return launch<3>(u, n, h, k, relu2, nullptr, kth, xq, xexp, ldq, st);
    return fail(AVA_ERR_ARG, "kwta_planes: planes %d (1..3)", planes);
}

}  // namespace ava

extern "C" int ava_kwta(const float *u, int n, int h, int k, int relu2, float *a, float *kth_out,
                        ava_stream stream) {
    AVA_REQUIRE(u && a, AVA_ERR_ARG, "kwta: NULL buffer");
    AVA_REQUIRE(n >= 0 && h > 0 && k > 0, AVA_ERR_SHAPE, "kwta: n=%d h=%d k=%d", n, h, k);
    AVA_REQUIRE(h % 4 == 0, AVA_ERR_SHAPE, "kwta: row width %d must be a multiple of 4", h);
    if (n == 0) return AVA_OK;
    return launch<0>(u, n, h, k, relu2, a, kth_out, nullptr, nullptr, 0, (hipStream_t)stream);
}
