// The cerebellum head (CB) and its online table (CB2) for gfx950: the granule code, the read-out with
// the table's share, and the online learning step.
//
// Reference: gpu/v51b.rs:18-32 (the part), :242-265 (wiring), :327-337 (cb_code), :373-389
// (CbOnline::add); gpu/model/fstep/arch_f3.rs:225-299 (the one-row forward); gpu/fast4/cb.rs:25-84
// (the learning step). The wiring is built on the host (model.cpp) from the same seed.
//
// Per row the code is:
//   u = [xf, rmsnorm(E[id], 1)] (2d); h_j = sum over the unit's 4 inputs of u[idx] * sgn, from 0 in order;
//   kth = the k-th largest of h (k = G / 32); a_j = relu(h_j) where h_j - kth >= 0, else 0;
//   c = a / (sqrt(sum a^2) + 1e-6).
// One workgroup per row holds h in registers (G / 256 units per thread). The k-th largest is exact:
// a threshold t is interpolated (alternating with midpoints) inside a bracket whose block-wide counts
// straddle k until exactly k values are >= t, the answer then being the smallest of them; ties that
// make the count skip k fall back to an exact bisection over the order-preserving key image.
#include "common.h"

namespace {

constexpr int NT = 256;
constexpr float NORM_EPS = 1e-5f;  // gpu/model.rs:36

__device__ __forceinline__ uint32_t key_of(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float float_of_key(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Block-wide reductions; every thread gets the result, made wave-uniform
// (readfirstlane) so control flow on it stays scalar. `red` holds 4 slots; the leading barrier
// protects it from the previous reduction's reads.
__device__ __forceinline__ float uni(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Block reductions over NWV waves (4 by default: 256 threads) in a fixed pairwise order (for 4 waves
// (r0 + r1) + (r2 + r3)); red holds NWV slots.
template <int NWV, class T, class F>
__device__ __forceinline__ T tree(const T *red, F op) {
    if constexpr (NWV == 1) return red[0];
    else return op(tree<NWV / 2>(red, op), tree<NWV / 2>(red + NWV / 2, op));
}
template <int NWV = 4>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = ava::wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return uni(tree<NWV>(red, [](float a, float b) { return a + b; }));
}
template <int NWV = 4>
__device__ __forceinline__ float block_max(float v, float *red) {
    v = ava::wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return uni(tree<NWV>(red, [](float a, float b) { return fmaxf(a, b); }));
}
template <int NWV = 4>
__device__ __forceinline__ float block_min(float v, float *red) {
    v = ava::wave_min(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return uni(tree<NWV>(red, [](float a, float b) { return fminf(a, b); }));
}
template <int NWV = 4>
__device__ __forceinline__ int block_isum(int v, int *red) {
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;  // v is wave-uniform (ballot counts)
    __syncthreads();
    return uni(tree<NWV>(red, [](int a, int b) { return a + b; }));
}
template <int NWV = 4>
__device__ __forceinline__ uint32_t block_umin(uint32_t v, uint32_t *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (uint32_t)uni((int)tree<NWV>(red, [](uint32_t a, uint32_t b) { return min(a, b); }));
}

// The granule code of rows n: code [n][g]. With keep != NULL, each stream's last position (row
// b T + T - 1) is also written to keep [b][g] (the code the learning step uses).
// With lcnt != NULL the row's non-zero units are also listed in unit order: lidx/lval [n][lcap] (unit,
// value) and lcnt [n] = their number (beyond lcap only the first lcap are listed; readers then use the
// dense code).
constexpr int APPLY_LCAP = 1024;  // unit lists the read-out takes through LDS

// With AP > 0 (a row per workgroup of NTH >= d threads, the unit lists on) the kernel goes on to the
// read-out and its planes: thread c forms out[row][c] with cb_apply_cols_kernel's sums in its order
// (the list kept in LDS as it is written), then the row's AP planes for the head as
// quant_rows_kernel writes them (xq [AP][n][ldq], xexp [n]): one launch instead of three.
struct ApplyArgs {
    const float *w, *tab;
    const double *scale;
    float *out;
    int8_t *xq;
    int32_t *xexp;
    int ldq;
};
template <int GPT, int NTH, int AP = 0>
__global__ __launch_bounds__(NTH) void cb_code_kernel(const float *__restrict__ xf, const int32_t *__restrict__ ids,
                                                     const float *__restrict__ emb, int d, int vocab,
                                                     const uint32_t *__restrict__ widx,
                                                     const float *__restrict__ wsgn, int g, int k, int T,
                                                     float *__restrict__ code, float *__restrict__ keep,
                                                     int *__restrict__ lcnt, int *__restrict__ lidx,
                                                     float *__restrict__ lval, int lcap, ApplyArgs ap) {
    __shared__ float su[2048];
    __shared__ int s_lu[AP > 0 ? APPLY_LCAP : 1];
    __shared__ float s_lv[AP > 0 ? APPLY_LCAP : 1];
    constexpr int NWV = NTH / 64;
    __shared__ float fred[NWV];
    __shared__ int ired[NWV];
    __shared__ uint32_t ured[NWV];
    __shared__ int s_wc[NWV][GPT];
    const int row = blockIdx.x, tid = threadIdx.x;
    int id = ids[row];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // an id outside [0, vocab) reads the nearest row
    const float *xr = xf + (size_t)row * d, *er = emb + (size_t)id * d;

    // u = [xf, rmsnorm(emb row, 1)]
    float ss = 0.0f;
    for (int c = tid; c < d; c += NTH) {
        su[c] = xr[c];
        const float e = er[c];
        ss += e * e;
    }
    ss = block_sum<NWV>(ss, fred);
    const float inv = 1.0f / sqrtf((ss * (1.0f / (float)d) + 0.0f) * 1.0f + NORM_EPS);
    for (int c = tid; c < d; c += NTH) su[d + c] = (er[c] * inv) * 1.0f;
    __syncthreads();

    // h: unit j = tid + NTH i (padding units are -inf: never counted, never kept)
    float h[GPT];
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        const int j = tid + i * NTH;
        if (j < g) {
            const uint4 ix = reinterpret_cast<const uint4 *>(widx)[j];
            const float4 sv = reinterpret_cast<const float4 *>(wsgn)[j];
            float acc = 0.0f;
            acc += su[ix.x] * sv.x;
            acc += su[ix.y] * sv.y;
            acc += su[ix.z] * sv.z;
            acc += su[ix.w] * sv.w;
            h[i] = acc;
        } else {
            h[i] = -INFINITY;
        }
    }
    auto count_ge = [&](float t) {
        int c = 0;
#pragma unroll
        for (int i = 0; i < GPT; i++) c += __popcll(__ballot(h[i] >= t));
        return block_isum<NWV>(c, ired);
    };

    float kth = -INFINITY;
    if (k < g) {
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int i = 0; i < GPT; i++)
            if (tid + i * NTH < g) {
                lo = fminf(lo, h[i]);
                hi = fmaxf(hi, h[i]);
            }
        lo = block_min<NWV>(lo, fred);
        hi = block_max<NWV>(hi, fred);
        bool done = false, found = false;
        float tk = 0.0f;
        if (isfinite(lo) && isfinite(hi)) {
            int clo = g, chi = count_ge(hi);
            if (chi >= k) {
                kth = hi;
                done = true;
            }
            // two first guesses from the units' mean and deviation as if normal (the quantile of the kept
            // fraction, then a Newton step on the count): they only place the bracket
            if (!done) {
                float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
                for (int i = 0; i < GPT; i++)
                    if (tid + i * NTH < g) {
                        s1 += h[i];
                        s2 += h[i] * h[i];
                    }
                s1 = block_sum<NWV>(s1, fred);
                s2 = block_sum<NWV>(s2, fred);
                const float mu = s1 / (float)g, sd = sqrtf(fmaxf(s2 / (float)g - mu * mu, 0.0f));
                const float z = ava::normal_upper_quantile((float)k / (float)g);
                const float dens = (float)g * 0.39894228f * __expf(-0.5f * z * z) / fmaxf(sd, 1e-30f);
                float t = uni(mu + z * sd);
                for (int gi = 0; gi < 2 && !found; gi++) {
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
            for (int it = 0; it < 40 && !done && !found; it++) {
                float t = (it & 1) ? lo * 0.5f + hi * 0.5f : lo + (hi - lo) * ((float)(clo - k) / (float)(clo - chi));
                if (!(t > lo && t < hi)) t = lo * 0.5f + hi * 0.5f;
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
            }
        }
        if (found) {
            // the smallest value >= tk; a zero is -0 when a -0 is among them (key order -0 < +0)
            float mn = INFINITY;
#pragma unroll
            for (int i = 0; i < GPT; i++) mn = h[i] >= tk ? fminf(mn, h[i]) : mn;
            mn = block_min<NWV>(mn, fred);
            if (mn == 0.0f) {
                int neg = 0;
#pragma unroll
                for (int i = 0; i < GPT; i++)
                    neg += __popcll(__ballot(h[i] >= tk && __float_as_uint(h[i]) == 0x80000000u));
                mn = block_isum<NWV>(neg, ired) ? -0.0f : 0.0f;
            }
            kth = mn;
            done = true;
        }
        if (!done) {
            // exact bisection over the keys (padding: key 0, below every real key)
            uint32_t prefix = 0;
            for (int bit = 31; bit >= 0; bit--) {
                const uint32_t cand = prefix | (1u << bit);
                int c = 0;
#pragma unroll
                for (int i = 0; i < GPT; i++)
                    c += __popcll(__ballot(tid + i * NTH < g && key_of(h[i]) >= cand));
                const int cnt = block_isum<NWV>(c, ired);
                if (cnt >= k) prefix = cand;
                if (cnt == k) {
                    uint32_t mn = 0xffffffffu;
#pragma unroll
                    for (int i = 0; i < GPT; i++) {
                        const uint32_t kk = key_of(h[i]);
                        mn = (tid + i * NTH < g && kk >= cand) ? min(mn, kk) : mn;
                    }
                    prefix = block_umin<NWV>(mn, ured);
                    break;
                }
            }
            kth = float_of_key(prefix);
        }
    }

    // relu on the winners, then unit length
    float s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        const float v = h[i];
        float a = v * ((k >= g || v - kth >= 0.0f) ? 1.0f : 0.0f);
        a = a > 0.0f ? a : 0.0f;
        h[i] = tid + i * NTH < g ? a : 0.0f;
        s2 += h[i] * h[i];
    }
    s2 = block_sum<NWV>(s2, fred);
    const float len = sqrtf(s2) * 1.0f + (float)1e-6;
    float *cr = code + (size_t)row * g;
    float *kr = (keep && row % T == T - 1) ? keep + (size_t)(row / T) * g : nullptr;
#pragma unroll
    for (int i = 0; i < GPT; i++) {
        const int j = tid + i * NTH;
        h[i] = j < g ? h[i] / len : 0.0f;
        if (j < g) {
            cr[j] = h[i];
            if (kr) kr[j] = h[i];
        }
    }
    if (lcnt) {
        // unit j = tid + NTH i: in unit order the i-th group of NTH comes after all earlier groups
        const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
        for (int i = 0; i < GPT; i++) {
            const int c = __popcll(__ballot(h[i] != 0.0f));
            if (lane == 0) s_wc[wave][i] = c;
        }
        __syncthreads();
        int base = 0;
        int *li = lidx + (size_t)row * lcap;
        float *lv = lval + (size_t)row * lcap;
#pragma unroll
        for (int i = 0; i < GPT; i++) {
            const uint64_t bm = __ballot(h[i] != 0.0f);
            int before = 0;
            for (int w = 0; w < wave; w++) before += s_wc[w][i];
            const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0));
            const int pos = base + before + rank;
            if (h[i] != 0.0f && pos < lcap) {
                li[pos] = tid + i * NTH;
                lv[pos] = h[i];
            }
            if constexpr (AP > 0)
                if (h[i] != 0.0f && pos < APPLY_LCAP) {
                    s_lu[pos] = tid + i * NTH;
                    s_lv[pos] = h[i];
                }
#pragma unroll
            for (int w = 0; w < NWV; w++) base += s_wc[w][i];
        }
        if (tid == 0) lcnt[row] = base;
        if constexpr (AP > 0) {
            __syncthreads();  // the LDS list (and this row's code in memory) are complete
            const int cnt = base, c = tid, b = row / T;
            const bool listed = cnt <= lcap && cnt <= APPLY_LCAP;
            float o = 0.0f;
            if (c < d) {
                const double sc = ap.scale ? ap.scale[b] : 1.0;
                const float *tb = ap.tab ? ap.tab + (size_t)b * g * d + c : nullptr;
                float acc = 0.0f, acc2 = 0.0f;
                if (listed) {
                    constexpr int QB = 16;
                    if (ap.w) {
                        for (int q0 = 0; q0 < cnt; q0 += QB) {
                            float v[QB];
#pragma unroll
                            for (int z = 0; z < QB; z++) v[z] = ap.w[(size_t)s_lu[min(q0 + z, cnt - 1)] * d + c];
                            AVA_ISSUE_FENCE();
#pragma unroll
                            for (int z = 0; z < QB; z++)
                                if (q0 + z < cnt) acc += v[z] * s_lv[q0 + z];
                        }
                    }
                    if (tb) {
                        for (int q0 = 0; q0 < cnt; q0 += QB) {
                            float v[QB];
#pragma unroll
                            for (int z = 0; z < QB; z++)  // non-temporal: rows of a 12.9 GB table, read once
                                v[z] = __builtin_nontemporal_load(tb + (size_t)s_lu[min(q0 + z, cnt - 1)] * d);
                            AVA_ISSUE_FENCE();
#pragma unroll
                            for (int z = 0; z < QB; z++)
                                if (q0 + z < cnt) {
                                    const float x = sc == 1.0 ? s_lv[q0 + z] : (float)((double)s_lv[q0 + z] * sc);
                                    acc2 += x * v[z];
                                }
                        }
                    }
                } else {
                    for (int j = 0; j < g; j++) {
                        const float cj = cr[j];
                        if (cj == 0.0f) continue;
                        if (ap.w) acc += ap.w[(size_t)j * d + c] * cj;
                        if (tb) acc2 += (sc == 1.0 ? cj : (float)((double)cj * sc)) * tb[(size_t)j * d];
                    }
                }
                o = xr[c] + acc;
                if (tb) o = o + acc2;
                ap.out[(size_t)row * d + c] = o;
            }
            const int e = ava::plane_exp(block_max<NWV>(c < d ? fabsf(o) : 0.0f, fred));
            if (tid == 0) ap.xexp[row] = e;
            for (int cc = tid; cc < ap.ldq; cc += NTH) {
                int qv[AP];
                ava::to_planes<AP>(cc < d ? o : 0.0f, e, qv);
#pragma unroll
                for (int p = 0; p < AP; p++) ap.xq[((size_t)p * gridDim.x + row) * ap.ldq + cc] = (int8_t)qv[p];
            }
        }
    }
}

// out [n][d] = xf + sum over the non-zero units j in order of W[j] c_j (W NULL: nothing), then + the
// table's share sum x_j tab[b][j] with x_j = c_j or (float)((double)c_j * scale[b]), from the row's
// unit list (cb_code's lidx/lval) or, when the list overflowed, the dense code. Block (row, 256
// columns), one column per thread: the table rows are read 1 KB per wave, coalesced.
__global__ __launch_bounds__(NT) void cb_apply_cols_kernel(const float *__restrict__ xf, const float *__restrict__ code,
                                                           int g, int d, const float *__restrict__ w,
                                                           const float *__restrict__ tab,
                                                           const double *__restrict__ scale, int T,
                                                           const int *__restrict__ lcnt, const int *__restrict__ lidx,
                                                           const float *__restrict__ lval, int lcap,
                                                           float *__restrict__ out) {
    __shared__ int s_j[APPLY_LCAP];
    __shared__ float s_c[APPLY_LCAP];
    const int row = blockIdx.x, tid = threadIdx.x, c = blockIdx.y * NT + tid;
    const int cnt = lcnt[row];
    const bool listed = cnt <= lcap && cnt <= APPLY_LCAP;
    if (listed)
        for (int q = tid; q < cnt; q += NT) {
            s_j[q] = lidx[(size_t)row * lcap + q];
            s_c[q] = lval[(size_t)row * lcap + q];
        }
    __syncthreads();
    if (c >= d) return;
    const int b = row / T;
    const double sc = scale ? scale[b] : 1.0;
    const float *tb = tab ? tab + (size_t)b * g * d + c : nullptr;
    const float *cr = code + (size_t)row * g;
    float acc = 0.0f, acc2 = 0.0f;
    if (listed) {
        // rows in batches of 16 whose loads are all issued before the adds (in unit order) use them
        constexpr int QB = 16;
        if (w) {
            for (int q0 = 0; q0 < cnt; q0 += QB) {
                float v[QB];
#pragma unroll
                for (int z = 0; z < QB; z++) v[z] = w[(size_t)s_j[min(q0 + z, cnt - 1)] * d + c];
                AVA_ISSUE_FENCE();
#pragma unroll
                for (int z = 0; z < QB; z++)
                    if (q0 + z < cnt) acc += v[z] * s_c[q0 + z];
            }
        }
        if (tb) {
            for (int q0 = 0; q0 < cnt; q0 += QB) {
                float v[QB];
#pragma unroll
                for (int z = 0; z < QB; z++) v[z] = tb[(size_t)s_j[min(q0 + z, cnt - 1)] * d];
                AVA_ISSUE_FENCE();
#pragma unroll
                for (int z = 0; z < QB; z++)
                    if (q0 + z < cnt) {
                        const float x = sc == 1.0 ? s_c[q0 + z] : (float)((double)s_c[q0 + z] * sc);
                        acc2 += x * v[z];
                    }
            }
        }
    } else {
        for (int j = 0; j < g; j++) {
            const float cj = cr[j];
            if (cj == 0.0f) continue;
            if (w) acc += w[(size_t)j * d + c] * cj;
            if (tb) acc2 += (sc == 1.0 ? cj : (float)((double)cj * sc)) * tb[(size_t)j * d];
        }
    }
    float o = xf[(size_t)row * d + c] + acc;
    if (tb) o = o + acc2;
    out[(size_t)row * d + c] = o;
}

// ------------------------------------------------------------------ the learning step

// err [B][V] = softmax(logits row) - onehot(next) (max, exp(z - max), the sum, p / sum); nats [B]
// (nullable) = -ln max(p_next, 1e-30). Rows whose next is outside [0, V) are skipped (err zeroed,
// nats NaN): the reference's IGNORE.
// err[b] = softmax(logits[b]) - onehot(next[b]) and nats[b] = -ln p(next), one workgroup per row;
// rows with next outside [0, V) get err = 0 and nats = NaN. KV > 0: the row (V <= KV NT) is read once
// into registers, all loads in flight together; KV = 0: any V, three passes over the row. Both add
// the same terms in the same order. Thread 0 also steps the row's table scale: rows with a valid next
// fade by `fade` (2^(-1/half), host-computed; 1 = no fading); below 1e-18 the row is marked for
// folding (fold[b] = the old scale) and its scale returns to 1.
template <int KV>
__global__ __launch_bounds__(NT) void cb_err_kernel(const float *__restrict__ logits, int ldl, int V,
                                                    const int32_t *__restrict__ next, float *__restrict__ err,
                                                    double *__restrict__ nats, double fade, double *__restrict__ scale,
                                                    double *__restrict__ fold) {
    __shared__ float fred[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float *z = logits + (size_t)b * ldl;
    float *er = err + (size_t)b * V;
    const int y = next[b];
    const bool live = y >= 0 && y < V;
    if (tid == 0) {
        double f = 0.0;
        if (live && fade != 1.0) {
            double sc = scale[b] * fade;
            if (sc < 1e-18) {
                f = sc;
                sc = 1.0;
            }
            scale[b] = sc;
        }
        fold[b] = f;
    }
    if (!live) {
        for (int j = tid; j < V; j += NT) er[j] = 0.0f;
        if (nats && tid == 0) nats[b] = __longlong_as_double(0x7ff8000000000000ll);
        return;
    }
    if constexpr (KV > 0) {
        float zv[KV];
#pragma unroll
        for (int i = 0; i < KV; i++) {
            const int j = tid + i * NT;
            zv[i] = j < V ? z[j] : 0.0f;
        }
        AVA_ISSUE_FENCE();
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < KV; i++)
            if (tid + i * NT < V) mx = fmaxf(mx, zv[i]);
        mx = block_max(mx, fred);
        float den = 0.0f;
#pragma unroll
        for (int i = 0; i < KV; i++)
            if (tid + i * NT < V) den += expf(zv[i] - mx);
        den = block_sum(den, fred);
#pragma unroll
        for (int i = 0; i < KV; i++) {
            const int j = tid + i * NT;
            if (j >= V) continue;
            const float p = expf(zv[i] - mx) / den;
            er[j] = p - (j == y ? 1.0f : 0.0f);
            if (nats && j == y) nats[b] = -log((double)(p > 1e-30f ? p : 1e-30f));
        }
    } else {
        float mx = -INFINITY;
        for (int j = tid; j < V; j += NT) mx = fmaxf(mx, z[j]);
        mx = block_max(mx, fred);
        float den = 0.0f;
        for (int j = tid; j < V; j += NT) den += expf(z[j] - mx);
        den = block_sum(den, fred);
        for (int j = tid; j < V; j += NT) {
            const float p = expf(z[j] - mx) / den;
            er[j] = p - (j == y ? 1.0f : 0.0f);
            if (nats && j == y) nats[b] = -log((double)(p > 1e-30f ? p : 1e-30f));
        }
    }
}

// part [ks][B][d] = err [B][V] slice ks . E [V][d] slice ks, fp32 MFMA (v_mfma_f32_32x32x2_f32): block
// = 64 rows x 64 columns, 4 waves of 32 x 32, K in steps of 32 through LDS.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__global__ __launch_bounds__(NT) void cb_delta_kernel(const float *__restrict__ err, int B, int V,
                                                      const float *__restrict__ E, int d, int kslice,
                                                      float *__restrict__ part) {
    __shared__ float sa[64][33];
    __shared__ float sb[32][64 + 4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * 64, c0 = blockIdx.y * 64, ks = blockIdx.z;
    const int kb = ks * kslice, ke = min(V, kb + kslice);
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    f32x16 acc = {};
    // the next K tile is loaded into registers while the current one is multiplied
    float ra[8], rb[8];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int z = 0; z < 8; z++) {
            const int i = tid + z * NT;
            const int r = i >> 5, kk = i & 31;
            ra[z] = (r0 + r < B && k0 + kk < ke) ? err[(size_t)(r0 + r) * V + k0 + kk] : 0.0f;
            const int kb2 = i >> 6, c = i & 63;
            rb[z] = (k0 + kb2 < ke && c0 + c < d) ? E[(size_t)(k0 + kb2) * d + c0 + c] : 0.0f;
        }
    };
    if (kb < ke) fetch(kb);
    for (int k0 = kb; k0 < ke; k0 += 32) {
        __syncthreads();
#pragma unroll
        for (int z = 0; z < 8; z++) {
            const int i = tid + z * NT;
            sa[i >> 5][i & 31] = ra[z];
            sb[i >> 6][i & 63] = rb[z];
        }
        __syncthreads();
        if (k0 + 32 < ke) fetch(k0 + 32);
#pragma unroll
        for (int s = 0; s < 32; s += 2) {
            const float a = sa[wr + (lane & 31)][s + (lane >> 5)];
            const float bb = sb[s + (lane >> 5)][wc + (lane & 31)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bb, acc, 0, 0, 0);
        }
    }
    // accumulator layout: register r -> row (r / 4) * 8 + (lane / 32) * 4 + r % 4, column lane % 32
    float *pr = part + (size_t)ks * B * d;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int row = r0 + wr + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), col = c0 + wc + (lane & 31);
        if (row < B && col < d) pr[(size_t)row * d + col] = acc[r];
    }
}

// delta [B][d] = sum over ks in order of part [ks]
__global__ void cb_delta_sum_kernel(const float *__restrict__ part, int nks, int total, float *__restrict__ delta) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    float s = part[i];
    for (int k = 1; k < nks; k++) s += part[(size_t)k * total + i];
    delta[i] = s;
}

// tab[b][u] -= s_u delta[b] for the non-zero units u of the kept code, s_u = lr * c_u (divided by
// the scale in double when it is not 1). Block (b, slice of g / TSPLIT units): the slice's code is read
// 256 units at a time and its non-zero units gathered in LDS (wave ballots), then every thread updates
// 4 columns of each gathered unit's row (float4; d a multiple of 4, d <= 1024). A row marked for
// folding (fold[b] != 0, a rare event) first has every unit of the slice scaled,
// tab = (float)((double)tab * fold[b]), by the same threads and columns that then update it.
constexpr int TSPLIT = 4;
__global__ __launch_bounds__(NT) void cb_table_kernel(const float *__restrict__ keep, int g, int d,
                                                      const float *__restrict__ delta, const int32_t *__restrict__ next,
                                                      int V, float lr, const double *__restrict__ scale,
                                                      const double *__restrict__ fold, float *__restrict__ tab) {
    __shared__ int s_u[NT];
    __shared__ float s_s[NT];
    __shared__ int s_wc[4];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int y = next[b];
    if (y < 0 || y >= V) return;
    const double sc = scale[b];
    const float *kc = keep + (size_t)b * g;
    float *tb = tab + (size_t)b * g * d;
    const int per = (g + TSPLIT - 1) / TSPLIT, ub = blockIdx.y * per, ue = min(g, ub + per);
    const int c4 = tid * 4;
    typedef float f4 __attribute__((ext_vector_type(4)));
    const double fo = fold[b];
    if (fo != 0.0 && c4 < d)
        for (int u = ub; u < ue; u++) {
            f4 *tr = reinterpret_cast<f4 *>(tb + (size_t)u * d + c4);
            f4 t = *tr;
#pragma unroll
            for (int z = 0; z < 4; z++) t[z] = (float)((double)t[z] * fo);
            *tr = t;
        }
    f4 dv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (c4 < d) dv = *reinterpret_cast<const f4 *>(delta + (size_t)b * d + c4);
    for (int u0 = ub; u0 < ue; u0 += NT) {
        const int u = u0 + tid;
        const float c = u < ue ? kc[u] : 0.0f;
        const uint64_t bm = __ballot(c != 0.0f);
        __syncthreads();  // the previous chunk's list is consumed
        if (lane == 0) s_wc[wave] = __popcll(bm);
        __syncthreads();
        int before = 0;
        for (int w = 0; w < wave; w++) before += s_wc[w];
        const int total = (s_wc[0] + s_wc[1]) + (s_wc[2] + s_wc[3]);
        if (c != 0.0f) {
            const int pos = before + __builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0));
            float s = lr * c;
            if (sc != 1.0) s = (float)((double)s / sc);
            s_u[pos] = u;
            s_s[pos] = s;
        }
        __syncthreads();
        if (c4 < d) {
#pragma unroll 4
            for (int q = 0; q < total; q++) {
                f4 *tr = reinterpret_cast<f4 *>(tb + (size_t)s_u[q] * d + c4);
                const float s = s_s[q];
                f4 t = __builtin_nontemporal_load(tr);  // a kept unit's row, read and written once
#pragma unroll
                for (int z = 0; z < 4; z++) t[z] -= s * dv[z];
                __builtin_nontemporal_store(t, tr);
            }
        }
    }
}

}  // namespace

namespace ava {

int cb_code(const float *xf, const int32_t *ids, const float *emb, int n, int d, int vocab, const uint32_t *widx,
            const float *wsgn, int g, int k, int T, float *code, float *keep, int *lcnt, int *lidx, float *lval,
            int lcap, hipStream_t st) {
    AVA_REQUIRE(d <= 1024 && d % 4 == 0 && g > 0 && g <= 16384 && T > 0, AVA_ERR_SHAPE, "cb_code: d=%d g=%d", d, g);
    AVA_REQUIRE(!lcnt || (lidx && lval && lcap > 0), AVA_ERR_ARG, "cb_code: unit list without storage");
    // few rows (a decode step): 1024 threads per row, so each wave's share of the search is short;
    // many rows: 256
#define AVA_CBC(G_, N_)                                                                                        \
    cb_code_kernel<G_, N_><<<n, N_, 0, st>>>(xf, ids, emb, d, vocab, widx, wsgn, g, k, T, code, keep, lcnt, lidx, \
                                             lval, lcap, ApplyArgs{})
    if (n <= 1024) {
        const int gpt = (g + 1023) / 1024;
        if (gpt <= 2) AVA_CBC(2, 1024);
        else if (gpt <= 4) AVA_CBC(4, 1024);
        else if (gpt <= 8) AVA_CBC(8, 1024);
        else if (gpt <= 12) AVA_CBC(12, 1024);
        else AVA_CBC(16, 1024);
    } else {
        const int gpt = (g + NT - 1) / NT;
        if (gpt <= 2) AVA_CBC(2, NT);
        else if (gpt <= 8) AVA_CBC(8, NT);
        else if (gpt <= 16) AVA_CBC(16, NT);
        else if (gpt <= 32) AVA_CBC(32, NT);
        else if (gpt <= 48) AVA_CBC(48, NT);
        else AVA_CBC(64, NT);
    }
#undef AVA_CBC
    AVA_LAUNCHED("cb_code");
    return AVA_OK;
}

bool cb_head_fits(int n, int d, int g, int planes) { return n <= 1024 && d <= 1024 && g <= 16384 && planes == 3; }

int cb_head(const float *xf, const int32_t *ids, const float *emb, int n, int d, int vocab, const uint32_t *widx,
            const float *wsgn, int g, int k, int T, float *code, float *keep, int *lcnt, int *lidx, float *lval,
            int lcap, const float *w, const float *tab, const double *scale, float *out, int planes, int8_t *xq,
            int32_t *xexp, hipStream_t st) {
    AVA_REQUIRE(cb_head_fits(n, d, g, planes) && d % 4 == 0 && lcnt && lidx && lval && lcap > 0 && T > 0,
                AVA_ERR_SHAPE, "cb_head: n=%d d=%d g=%d planes=%d", n, d, g, planes);
    const ApplyArgs ap{w, tab, scale, out, xq, xexp, q8_ldk(d)};
    const int gpt = (g + 1023) / 1024;
#define AVA_CBH(G_)                                                                                            \
    cb_code_kernel<G_, 1024, 3><<<n, 1024, 0, st>>>(xf, ids, emb, d, vocab, widx, wsgn, g, k, T, code, keep, lcnt, \
                                                    lidx, lval, lcap, ap)
    if (gpt <= 2) AVA_CBH(2);
    else if (gpt <= 4) AVA_CBH(4);
    else if (gpt <= 8) AVA_CBH(8);
    else if (gpt <= 12) AVA_CBH(12);
    else AVA_CBH(16);
#undef AVA_CBH
    AVA_LAUNCHED("cb_code");
    return AVA_OK;
}

int cb_apply_list(const float *xf, const float *code, int n, int g, int d, const float *w, const float *tab,
                  const double *scale, int T, const int *lcnt, const int *lidx, const float *lval, int lcap, float *out,
                  hipStream_t st) {
    AVA_REQUIRE(d > 0 && g > 0 && lcnt && lidx && lval && lcap > 0, AVA_ERR_ARG, "cb_apply: d=%d g=%d", d, g);
    cb_apply_cols_kernel<<<dim3(n, ceil_div(d, NT)), NT, 0, st>>>(xf, code, g, d, w, tab, scale, T, lcnt, lidx, lval,
                                                                  lcap, out);
    AVA_LAUNCHED("cb_apply");
    return AVA_OK;
}

int cb_learn(const float *logits, int ldl, int V, const int32_t *next, int B, const float *emb, int d,
             const float *keep, int g, float lr, double fade, double *scale, float *tab, float *err, float *part,
             int nks, float *delta, double *fold, double *nats, hipStream_t st) {
    AVA_REQUIRE(B > 0 && V > 0 && d > 0 && nks > 0, AVA_ERR_SHAPE, "cb_learn: B=%d V=%d d=%d", B, V, d);
    if (V <= 32 * NT) cb_err_kernel<32><<<B, NT, 0, st>>>(logits, ldl, V, next, err, nats, fade, scale, fold);
    else cb_err_kernel<0><<<B, NT, 0, st>>>(logits, ldl, V, next, err, nats, fade, scale, fold);
    AVA_LAUNCHED("cb_err");
    const int kslice = ((V + nks - 1) / nks + 31) / 32 * 32;
    cb_delta_kernel<<<dim3(ceil_div(B, 64), ceil_div(d, 64), nks), NT, 0, st>>>(err, B, V, emb, d, kslice, part);
    AVA_LAUNCHED("cb_delta");
    cb_delta_sum_kernel<<<ceil_div(B * d, 256), 256, 0, st>>>(part, nks, B * d, delta);
    AVA_LAUNCHED("cb_delta_sum");
    AVA_REQUIRE(d % 4 == 0 && d <= 4 * NT, AVA_ERR_SHAPE, "cb_learn: d=%d (a multiple of 4, <= 1024)", d);
    cb_table_kernel<<<dim3(B, TSPLIT), NT, 0, st>>>(keep, g, d, delta, next, V, lr, scale, fold, tab);
    AVA_LAUNCHED("cb_table");
    return AVA_OK;
}

}  // namespace ava
