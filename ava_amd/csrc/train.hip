// The kernels of the float32 training step (train.cpp composes them with the scans' backward kernels
// and the library GEMMs): RMSNorm, the memory's input preparation and read-out, causal attention's
// backward, the cross-entropy head, the embedding's scatter and the reductions that turn per-row
// terms into parameter gradients. Every kernel is a stream over [rows][channels] f32 in HBM; rows
// are tokens (b-major), a wave owns a row (or a row's head of 64 channels) so per-row sums are wave
// reductions, and every parameter gradient is reduced in a fixed order (no float atomics) except the
// embedding's scatter, whose rows repeat with the token ids.
#include "common.h"
#include "train.h"

namespace {

constexpr int WG = 256;
constexpr float RMS_EPS = 1e-5f;  // gpu/model.rs:458-462
constexpr float UNIT_EPS = 1e-6f; // gpu/model.rs:589-592

__device__ __forceinline__ float sigm(float z) { return 1.0f / (1.0f + expf(-z)); }
// log sigmoid(z) = -(relu(-z) + ln(1 + exp(-|z|))) (gpu/model.rs:618-622)
__device__ __forceinline__ float logsigm(float z) { return -(fmaxf(-z, 0.0f) + log1pf(expf(-fabsf(z)))); }

// ---------------------------------------------------------------- RMSNorm: y = x r g, r = (mean x^2 + eps)^-1/2

// one wave per row; d a multiple of 64 and <= 1024 (each lane holds d / 64 channels: c = lane + 64 j)
__global__ __launch_bounds__(WG) void rms_fwd_kernel(const float *__restrict__ x, int n, int d,
                                                     const float *__restrict__ g, float *__restrict__ y,
                                                     float *__restrict__ inv) {
    const int row = blockIdx.x * (WG / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= n) return;
    const float *xr = x + (size_t)row * d;
    float ss = 0.0f;
    for (int c = lane; c < d; c += 64) ss = fmaf(xr[c], xr[c], ss);
    ss = ava::wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)d + RMS_EPS);
    float *yr = y + (size_t)row * d;
    for (int c = lane; c < d; c += 64) yr[c] = xr[c] * r * g[c];
    if (lane == 0) inv[row] = r;
}

// dx += r g dy - x r^3 / d sum_c(g dy x); part[wg][d] = this workgroup's share of dg_c = sum_n dy x r.
// Rows go to workgroups in contiguous runs, each run's rows one per wave in turn.
__global__ __launch_bounds__(WG) void rms_bwd_kernel(const float *__restrict__ x, const float *__restrict__ inv,
                                                     const float *__restrict__ g, const float *__restrict__ dy,
                                                     int n, int d, int rows_per_wg, float *__restrict__ dx,
                                                     float *__restrict__ part) {
    __shared__ float red[WG / 64][1024];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nj = d >> 6;
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;
    const int r0 = blockIdx.x * rows_per_wg, r1 = min(n, r0 + rows_per_wg);
    for (int row = r0 + wv; row < r1; row += WG / 64) {
        const float *xr = x + (size_t)row * d, *dr = dy + (size_t)row * d;
        const float r = inv[row];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (j < nj) {
                const int c = lane + 64 * j;
                s = fmaf(g[c] * dr[c], xr[c], s);
                acc[j] = fmaf(dr[c] * xr[c], r, acc[j]);
            }
        s = ava::wave_sum(s);
        const float k = r * r * r * s / (float)d;
        float *o = dx + (size_t)row * d;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (j < nj) {
                const int c = lane + 64 * j;
                o[c] += r * g[c] * dr[c] - xr[c] * k;
            }
    }
#pragma unroll
    for (int j = 0; j < 16; j++)
        if (j < nj) red[wv][lane + 64 * j] = acc[j];
    __syncthreads();
    for (int c = threadIdx.x; c < d; c += WG) {
        float s = red[0][c];
#pragma unroll
        for (int w = 1; w < WG / 64; w++) s += red[w][c];
        part[(size_t)blockIdx.x * d + c] = s;
    }
}

// ---------------------------------------------------------------- column sums in a fixed order

// part[chunk][c] = sum over the chunk's rows of x[r][c] (rows of ld floats); lane = column
__global__ __launch_bounds__(WG) void colsum_part_kernel(const float *__restrict__ x, int rows, int cols, int ld,
                                                         int rows_per_chunk, float *__restrict__ part) {
    const int c = blockIdx.x * WG + threadIdx.x;
    if (c >= cols) return;
    const int r0 = blockIdx.y * rows_per_chunk, r1 = min(rows, r0 + rows_per_chunk);
    float s = 0.0f;
    for (int r = r0; r < r1; r++) s += x[(size_t)r * ld + c];
    part[(size_t)blockIdx.y * cols + c] = s;
}

// out[c] (+)= sum_k part[k][c] (+ sign extra[c] when extra): a workgroup per 64 columns, wave w adding
// parts w, w + 4, ... (four running sums each, so several loads are in flight), then the waves' sums in
// wave order: a fixed order for any launch.
__global__ __launch_bounds__(WG) void colsum_final_kernel(const float *__restrict__ part, int nparts, int cols,
                                                          float *__restrict__ out, int accumulate,
                                                          const float *__restrict__ extra, float sign) {
    __shared__ float red[WG / 64][64];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, c = blockIdx.x * 64 + lane;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    if (c < cols) {
        int k = wv;
        for (; k + 12 < nparts; k += 16) {
            s0 += part[(size_t)k * cols + c];
            s1 += part[(size_t)(k + 4) * cols + c];
            s2 += part[(size_t)(k + 8) * cols + c];
            s3 += part[(size_t)(k + 12) * cols + c];
        }
        for (; k < nparts; k += 4) s0 += part[(size_t)k * cols + c];
    }
    red[wv][lane] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (wv == 0 && c < cols) {
        float s = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
        if (extra) s += sign * extra[c];
        out[c] = accumulate ? out[c] + s : s;
    }
}

// out[0] = sum_i a_i b_i over n, via per-workgroup partials then one ordered wave sum
__global__ __launch_bounds__(WG) void dot_part_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                                      size_t n, float *__restrict__ part) {
    __shared__ float red[WG / 64];
    float s = 0.0f;
    for (size_t i = (size_t)blockIdx.x * WG + threadIdx.x; i < n; i += (size_t)gridDim.x * WG) s = fmaf(a[i], b[i], s);
    s = ava::wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

__global__ __launch_bounds__(64) void sum_final_kernel(const float *__restrict__ part, int nparts,
                                                       float *__restrict__ out, int accumulate) {
    float s = 0.0f;
    for (int k = threadIdx.x; k < nparts; k += 64) s += part[k];
    s = ava::wave_sum(s);
    if (threadIdx.x == 0) out[0] = accumulate ? out[0] + s : s;
}

// ---------------------------------------------------------------- small elementwise pieces

// ps [4][d] = sigmoid(beta_p) | theta | sigmoid(arho) | again (rho, gain 0 without ALIF); omb = 1 - beta
__global__ void lif_params_kernel(const float *beta_p, const float *theta, const float *arho, const float *again,
                                  int d, int alif, float *ps, float *omb) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= d) return;
    const float b = sigm(beta_p[c]);
    ps[c] = b;
    ps[d + c] = theta[c];
    ps[2 * d + c] = alif ? sigm(arho[c]) : 0.0f;
    ps[3 * d + c] = alif ? again[c] : 0.0f;
    omb[c] = 1.0f - b;
}

// y[r][c] = x[r][c] * s[c]
__global__ void scale_cols_kernel(const float *__restrict__ x, const float *__restrict__ s, size_t n, int d,
                                  float *__restrict__ y) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = x[i] * s[i % d];
}

__global__ void i8_to_f32_kernel(const int8_t *__restrict__ s, size_t n, float *__restrict__ y) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (float)s[i];
}

__global__ void axpy_kernel(float *__restrict__ y, const float *__restrict__ x, float a, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = y[i] + a * x[i];
}

// the chain rule through a sigmoid-squashed parameter: dp[c] = dq[c] q (1 - q), q = sigmoid(p[c])
__global__ void sigmoid_chain_kernel(const float *__restrict__ p, const float *__restrict__ dq, int n,
                                     float *__restrict__ dp) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    const float q = sigm(p[c]);
    dp[c] = dq[c] * q * (1.0f - q);
}

// an id outside [0, V) reads a zero row (and passes no gradient)
__global__ void embed_kernel(const int32_t *__restrict__ ids, const float *__restrict__ emb, int n, int d, int V,
                             float *__restrict__ x) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * d) return;
    const size_t r = i / d, c = i - r * d;
    const int id = ids[r];
    x[i] = (id >= 0 && id < V) ? emb[(size_t)id * d + c] : 0.0f;
}

// dE[ids[r]] += dx[r] (rows repeat with the token ids: float atomics, so the order of the adds into
// one row is not fixed)
__global__ void embed_bwd_kernel(const int32_t *__restrict__ ids, const float *__restrict__ dx, int n, int d, int V,
                                 float *__restrict__ dE) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * d) return;
    const size_t r = i / d, c = i - r * d;
    const int id = ids[r];
    if (id >= 0 && id < V) atomicAdd(dE + (size_t)id * d + c, dx[i]);
}

// ---------------------------------------------------------------- the memory's inputs (mem_arch, gpu/arch.rs:1873-1941)

// One wave per (row, head), lane = channel. Raw projections q, k, v, we [N][d] (rows of d), the head gate
// inputs zab [N][2 nh] (h Wa | h Wb), the rank-r read-outs lra, lrb [N][d] ((h Wa1) Wa2, (h Wb1) Wb2);
// out: unit q, unit k, e = unit(k + we), the residual value, log alpha and b, head-major [B nh][T][64].
__global__ __launch_bounds__(WG) void prep_fwd_kernel(TrainPrep p) {
    const int item = blockIdx.x * (WG / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int N = p.B * p.T;
    if (item >= N * p.nh) return;
    const int row = item / p.nh, h = item - row * p.nh;
    const int bi = row / p.T, t = row - bi * p.T;
    const int d = p.nh * 64, c = h * 64 + lane;
    const size_t rc = (size_t)row * d + c;
    const float q = p.q[rc], k = p.k[rc], ek = k + p.we[rc];
    const float rq = 1.0f / sqrtf(ava::wave_sum(q * q) + UNIT_EPS);
    const float rk = 1.0f / sqrtf(ava::wave_sum(k * k) + UNIT_EPS);
    const float re = 1.0f / sqrtf(ava::wave_sum(ek * ek) + UNIT_EPS);
    float v = p.v[rc];
    if (p.vfirst) v = v * (1.0f + p.vres[0]) + p.vfirst[rc] * p.vres[1];
    const float za = ((p.zab[(size_t)row * 2 * p.nh + h] + p.ba[h]) + p.off[c]) + p.lra[rc];
    const float zb = (p.zab[(size_t)row * 2 * p.nh + p.nh + h] + p.bb[h]) + p.lrb[rc];
    const size_t o = (((size_t)bi * p.nh + h) * p.T + t) * 64 + lane;
    p.hq[o] = q * rq;
    p.hk[o] = k * rk;
    p.he[o] = ek * re;
    p.hv[o] = v;
    p.hla[o] = logsigm(za);
    p.hb[o] = 2.0f * sigm(zb);
}

// The backward of prep_fwd_kernel, from the memory scan's gradients (head-major dq, dk, de, dv, dla, db)
// to row-major gradients of the raw projections (dq, dk, dv, dwe), of the gate pre-activations per channel
// (dza, dzb [N][d], which are also the read-outs' gradients) and per head (dzab [N][2 nh]); dvfirst +=
// dv p1 and the value residual's two parameters' per-(row, head) shares vres_part [N nh][2].
__global__ __launch_bounds__(WG) void prep_bwd_kernel(TrainPrep p, TrainPrepGrad g) {
    const int item = blockIdx.x * (WG / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int N = p.B * p.T;
    if (item >= N * p.nh) return;
    const int row = item / p.nh, h = item - row * p.nh;
    const int bi = row / p.T, t = row - bi * p.T;
    const int d = p.nh * 64, c = h * 64 + lane;
    const size_t rc = (size_t)row * d + c;
    const size_t o = (((size_t)bi * p.nh + h) * p.T + t) * 64 + lane;
    const float q = p.q[rc], k = p.k[rc], ek = k + p.we[rc];
    const float rq = 1.0f / sqrtf(ava::wave_sum(q * q) + UNIT_EPS);
    const float rk = 1.0f / sqrtf(ava::wave_sum(k * k) + UNIT_EPS);
    const float re = 1.0f / sqrtf(ava::wave_sum(ek * ek) + UNIT_EPS);
    // unit(x) = x r: dx = r du - x r^3 <x, du>
    const float gq = g.dq[o], gk = g.dk[o], ge = g.de[o];
    const float sq = ava::wave_sum(q * gq), sk = ava::wave_sum(k * gk), se = ava::wave_sum(ek * ge);
    const float dq = rq * gq - q * (rq * rq * rq) * sq;
    const float dk_unit = rk * gk - k * (rk * rk * rk) * sk;
    const float dek = re * ge - ek * (re * re * re) * se;
    g.dq_raw[rc] = dq;
    g.dk_raw[rc] = dk_unit + dek;
    g.dwe[rc] = dek;
    const float dvp = g.dv[o];
    float vres0 = 0.0f, vres1 = 0.0f;
    if (p.vfirst) {
        g.dv_raw[rc] = dvp * (1.0f + p.vres[0]);
        g.dvfirst[rc] += dvp * p.vres[1];
        vres0 = ava::wave_sum(dvp * p.v[rc]);
        vres1 = ava::wave_sum(dvp * p.vfirst[rc]);
    } else {
        g.dv_raw[rc] = dvp;
    }
    const float za = ((p.zab[(size_t)row * 2 * p.nh + h] + p.ba[h]) + p.off[c]) + p.lra[rc];
    const float zb = (p.zab[(size_t)row * 2 * p.nh + p.nh + h] + p.bb[h]) + p.lrb[rc];
    // d logsigmoid(z) / dz = sigmoid(-z); d 2 sigmoid(z) / dz = 2 s (1 - s)
    const float dza = g.dla[o] * sigm(-za);
    const float sb = sigm(zb);
    const float dzb = g.db[o] * 2.0f * sb * (1.0f - sb);
    g.dza[rc] = dza;
    g.dzb[rc] = dzb;
    const float ha = ava::wave_sum(dza), hb = ava::wave_sum(dzb);
    if (lane == 0) {
        g.dzab[(size_t)row * 2 * p.nh + h] = ha;
        g.dzab[(size_t)row * 2 * p.nh + p.nh + h] = hb;
        if (g.vres_part) {
            g.vres_part[(size_t)item * 2] = vres0;
            g.vres_part[(size_t)item * 2 + 1] = vres1;
        }
    }
}

// ---------------------------------------------------------------- the memory's read-out (gpu/model.rs:583-604)

// o = head_norm(y) silu(g): y head-major [B nh][T][64], g and o row-major [N][d]; one wave per (row, head)
__global__ __launch_bounds__(WG) void readout_fwd_kernel(const float *__restrict__ y, const float *__restrict__ g,
                                                         int B, int T, int nh, float *__restrict__ o) {
    const int item = blockIdx.x * (WG / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (item >= B * T * nh) return;
    const int row = item / nh, h = item - row * nh, bi = row / T, t = row - bi * T;
    const size_t rc = (size_t)row * nh * 64 + h * 64 + lane;
    const float yv = y[(((size_t)bi * nh + h) * T + t) * 64 + lane];
    const float r = 1.0f / sqrtf(ava::wave_sum(yv * yv) / 64.0f + RMS_EPS);
    const float gv = g[rc];
    o[rc] = (yv * r) * (gv * sigm(gv));
}

// dy (head-major) and dg (row-major) from do (row-major)
__global__ __launch_bounds__(WG) void readout_bwd_kernel(const float *__restrict__ y, const float *__restrict__ g,
                                                         const float *__restrict__ dout, int B, int T, int nh,
                                                         float *__restrict__ dy, float *__restrict__ dg) {
    const int item = blockIdx.x * (WG / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (item >= B * T * nh) return;
    const int row = item / nh, h = item - row * nh, bi = row / T, t = row - bi * T;
    const size_t rc = (size_t)row * nh * 64 + h * 64 + lane;
    const size_t hm = (((size_t)bi * nh + h) * T + t) * 64 + lane;
    const float yv = y[hm];
    const float r = 1.0f / sqrtf(ava::wave_sum(yv * yv) / 64.0f + RMS_EPS);
    const float gv = g[rc], sg = sigm(gv), silu = gv * sg, dov = dout[rc];
    const float dhn = dov * silu;
    const float s = ava::wave_sum(yv * dhn);
    dy[hm] = r * dhn - yv * (r * r * r) * s / 64.0f;
    dg[rc] = dov * (yv * r) * (sg * (1.0f + gv * (1.0f - sg)));
}

// ---------------------------------------------------------------- causal attention's backward

// Rows of q, k, v, o, do: [B*T][de], head hh at dims hh*hd .. (hd = 32 or 64). Both kernels run the
// forward read's register layout (the engram read's attend_fa_kernel): v_mfma_f32_32x32x2f32 products
// whose k-step s takes dims s and HD/2 + s in the two lane halves (so a lane's row operand is HD/2
// contiguous dims), and an accumulator that leaves lane l column l % 32 and rows
// kappa(r, l / 32) = 8 (r / 4) + 4 (l / 32) + r % 4, r = 0..15; products over those rows take them in
// the order kappa(t, 0), kappa(t, 1) at k-step t, so the lane's own register t is the B operand and A is
// read in place (lanes 0..31 one row, 32..63 another). Scores are kept in base-2 units (s log2 e).
typedef float f32x16t __attribute__((ext_vector_type(16)));
typedef float f32x4t __attribute__((ext_vector_type(4)));
constexpr float LOG2E = 1.44269504088896341f;

template <int N>
__device__ __forceinline__ void row_load(const float *p, float (&x)[N]) {
#pragma unroll
    for (int c = 0; c < N / 4; c++) {
        const f32x4t v = reinterpret_cast<const f32x4t *>(p)[c];
#pragma unroll
        for (int z = 0; z < 4; z++) x[4 * c + z] = v[z];
    }
}
__device__ __forceinline__ float swap_max(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float swap_sum(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ int kap(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// One wave per (32 queries, stream, head): first the rows' log-sum-exp over keys 0..t (base 2) and
// D = <do, o>, then per key tile S^T = K Q^T, P = 2^(S - lse), dP^T = V dO^T, dS = P (dP - D) and
// dQ^T += K^T dS^T; dq = scale dQ. lse and D are kept for the second kernel.
template <int HD>
__global__ __launch_bounds__(64) void attn_bwd_dq_kernel(TrainAttn a) {
    constexpr int HH = HD / 2, NO = HD / 32;
    const int T = a.T, de = a.de, nh = a.nh, nqb = (T + 31) >> 5;
    const int L = (int)blockIdx.x, sh = L / nqb, qb = (nqb - 1 - (L - sh * nqb)) * 32;
    const int bi = sh / nh, hh = sh - bi * nh;
    const int lane = threadIdx.x, lq = lane & 31, h = lane >> 5;
    const int qrow = qb + lq, qc = min(qrow, T - 1);
    const float sc2 = a.scale * LOG2E;
    const size_t rb = (size_t)bi * T;  // the stream's first row
    const float *kb = a.k + rb * de + hh * HD, *vb = a.v + rb * de + hh * HD;
    float qf[HH], df[HH];
    row_load<HH>(a.q + (rb + qc) * de + hh * HD + HH * h, qf);
    row_load<HH>(a.dout + (rb + qc) * de + hh * HD + HH * h, df);
    float D;
    {
        float of[HH];
        row_load<HH>(a.o + (rb + qc) * de + hh * HD + HH * h, of);
        float x = 0.0f;
#pragma unroll
        for (int c = 0; c < HH; c++) x = fmaf(df[c], of[c], x);
        D = swap_sum(x);
    }
    const int kend = min(qb + 32, T), nt = (kend + 31) >> 5;
    auto scores = [&](int k0) {
        float kx[HH];
        row_load<HH>(kb + (size_t)min(k0 + lq, T - 1) * de + HH * h, kx);
        f32x16t s = {};
#pragma unroll
        for (int c = 0; c < HH; c++) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kx[c], qf[c], s, 0, 0, 0);
        const bool edge = k0 + 31 > qb;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float x = s[r] * sc2;
            if (edge && k0 + kap(r, h) > qrow) x = -INFINITY;
            s[r] = x;
        }
        return s;
    };
    // the log-sum-exp (base 2)
    float m = -INFINITY, den = 0.0f;
    for (int j = 0; j < nt; j++) {
        const f32x16t s = scores(32 * j);
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) tmax = fmaxf(tmax, s[r]);
        const float nm = fmaxf(m, swap_max(tmax));
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) ps += s[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[r] - nm);
        den = (m == -INFINITY ? 0.0f : den * __builtin_amdgcn_exp2f(m - nm)) + swap_sum(ps);
        m = nm;
    }
    const float lse = m + __log2f(den);
    f32x16t dq[NO];
#pragma unroll
    for (int u = 0; u < NO; u++) dq[u] = f32x16t{};
    for (int j = 0; j < nt; j++) {
        const int k0 = 32 * j;
        f32x16t s = scores(k0);
        float vx[HH];
        row_load<HH>(vb + (size_t)min(k0 + lq, T - 1) * de + HH * h, vx);
        f32x16t dp = {};
#pragma unroll
        for (int c = 0; c < HH; c++) dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vx[c], df[c], dp, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p = s[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[r] - lse);
            s[r] = p * (dp[r] - D);  // dS
        }
#pragma unroll
        for (int u = 0; u < NO; u++)
#pragma unroll
            for (int t = 0; t < 16; t++) {
                const float kt = kb[(size_t)min(k0 + kap(t, h), T - 1) * de + 32 * u + lq];
                dq[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(kt, s[t], dq[u], 0, 0, 0);
            }
    }
    if (qrow < T) {
        float *op = a.dq + (rb + qrow) * de + hh * HD + 4 * h;
#pragma unroll
        for (int u = 0; u < NO; u++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                f32x4t w;
#pragma unroll
                for (int z = 0; z < 4; z++) w[z] = dq[u][4 * g + z] * a.scale;
                *reinterpret_cast<f32x4t *>(op + 32 * u + 8 * g) = w;
            }
        if (h == 0) {
            a.lse[(rb + qrow) * nh + hh] = lse;
            a.dsum[(rb + qrow) * nh + hh] = D;
        }
    }
}

// One wave per (32 keys, stream, head), over the query tiles at and after the keys: S = Q K^T (lane:
// key, registers: queries), P = 2^(S - lse), dP = dO V^T, dS = P (dP - D); dV^T += dO^T P and
// dK^T += Q^T dS; dk = scale dK.
template <int HD>
__global__ __launch_bounds__(64) void attn_bwd_dkv_kernel(TrainAttn a) {
    constexpr int HH = HD / 2, NO = HD / 32;
    const int T = a.T, de = a.de, nh = a.nh, nkb = (T + 31) >> 5;
    const int L = (int)blockIdx.x, sh = L / nkb, kb0 = (L - sh * nkb) * 32;  // the earliest keys (most queries) first
    const int bi = sh / nh, hh = sh - bi * nh;
    const int lane = threadIdx.x, lq = lane & 31, h = lane >> 5;
    const int key = kb0 + lq, kc = min(key, T - 1);
    const float sc2 = a.scale * LOG2E;
    const size_t rb = (size_t)bi * T;
    const float *qb = a.q + rb * de + hh * HD, *ob = a.dout + rb * de + hh * HD;
    float kf[HH], vf[HH];
    row_load<HH>(a.k + (rb + kc) * de + hh * HD + HH * h, kf);
    row_load<HH>(a.v + (rb + kc) * de + hh * HD + HH * h, vf);
    f32x16t dk[NO], dv[NO];
#pragma unroll
    for (int u = 0; u < NO; u++) dk[u] = dv[u] = f32x16t{};
    for (int q0 = kb0; q0 < T; q0 += 32) {
        float qx[HH], ox[HH];
        const int qr = min(q0 + lq, T - 1);
        row_load<HH>(qb + (size_t)qr * de + HH * h, qx);
        row_load<HH>(ob + (size_t)qr * de + HH * h, ox);
        f32x16t s = {}, dp = {};
#pragma unroll
        for (int c = 0; c < HH; c++) {
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(qx[c], kf[c], s, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ox[c], vf[c], dp, 0, 0, 0);
        }
        const bool edge = q0 < kb0 + 31;  // a query of the tile lies before the block's last key
        float pr[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int qi = q0 + kap(r, h);
            const bool ok = qi < T && (!edge || qi >= key);
            const size_t ri = (rb + min(qi, T - 1)) * nh + hh;
            const float p = ok ? __builtin_amdgcn_exp2f(s[r] * sc2 - a.lse[ri]) : 0.0f;
            pr[r] = p;
            s[r] = p * (dp[r] - a.dsum[ri]);  // dS
        }
#pragma unroll
        for (int u = 0; u < NO; u++)
#pragma unroll
            for (int t = 0; t < 16; t++) {
                const size_t rr = (size_t)min(q0 + kap(t, h), T - 1) * de + 32 * u + lq;
                dv[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(ob[rr], pr[t], dv[u], 0, 0, 0);
                dk[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(qb[rr], s[t], dk[u], 0, 0, 0);
            }
    }
    if (key < T) {
        float *kp = a.dk + (rb + key) * de + hh * HD + 4 * h, *vp = a.dv + (rb + key) * de + hh * HD + 4 * h;
#pragma unroll
        for (int u = 0; u < NO; u++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                f32x4t wk, wv;
#pragma unroll
                for (int z = 0; z < 4; z++) {
                    wk[z] = dk[u][4 * g + z] * a.scale;
                    wv[z] = dv[u][4 * g + z];
                }
                *reinterpret_cast<f32x4t *>(kp + 32 * u + 8 * g) = wk;
                *reinterpret_cast<f32x4t *>(vp + 32 * u + 8 * g) = wv;
            }
    }
}

// ---------------------------------------------------------------- the head's cross-entropy

// per row: lse of the logits, the row's loss lse - logit[target] (0 for a target outside [0, V)) and
// whether it counts; one workgroup per row
__global__ __launch_bounds__(WG) void ce_row_kernel(const float *__restrict__ logits, const int32_t *__restrict__ tgt,
                                                   int V, float *__restrict__ lse, float *__restrict__ loss_row,
                                                   float *__restrict__ valid) {
    __shared__ float red[WG / 64];
    const int row = blockIdx.x;
    const float *lr = logits + (size_t)row * V;
    float m = -INFINITY;
    for (int c = threadIdx.x; c < V; c += WG) m = fmaxf(m, lr[c]);
    m = ava::wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
    for (int c = threadIdx.x; c < V; c += WG) s += expf(lr[c] - m);
    s = ava::wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float l = m + logf(((red[0] + red[1]) + red[2]) + red[3]);
        const int t = tgt[row];
        const bool ok = t >= 0 && t < V;
        lse[row] = l;
        loss_row[row] = ok ? l - lr[t] : 0.0f;
        valid[row] = ok ? 1.0f : 0.0f;
    }
}

// loss = sum(loss_row) / max(1, sum(valid)); scal[0] = 1 / max(1, count) for the gradient
__global__ __launch_bounds__(64) void ce_total_kernel(const float *__restrict__ loss_row, const float *__restrict__ valid,
                                                      int n, float *__restrict__ loss, float *__restrict__ scal) {
    float s = 0.0f, c = 0.0f;
    for (int r = threadIdx.x; r < n; r += 64) {
        s += loss_row[r];
        c += valid[r];
    }
    s = ava::wave_sum(s);
    c = ava::wave_sum(c);
    if (threadIdx.x == 0) {
        const float inv = 1.0f / fmaxf(c, 1.0f);
        loss[0] = s * inv;
        scal[0] = inv;
    }
}

// dlogits = (softmax - onehot(target)) / count, in place over the logits
__global__ __launch_bounds__(WG) void ce_grad_kernel(float *__restrict__ logits, const int32_t *__restrict__ tgt,
                                                     const float *__restrict__ lse, const float *__restrict__ scal,
                                                     int V) {
    const int row = blockIdx.x;
    float *lr = logits + (size_t)row * V;
    const int t = tgt[row];
    const bool ok = t >= 0 && t < V;
    const float l = lse[row], inv = scal[0];
    for (int c = threadIdx.x; c < V; c += WG) {
        const float p = ok ? expf(lr[c] - l) : 0.0f;
        lr[c] = (p - (c == t ? 1.0f : 0.0f)) * inv;
    }
}

unsigned grid1(size_t n, int block = WG) { return (unsigned)((n + block - 1) / block); }

}  // namespace

namespace ava {
namespace train {

int rms_fwd(const float *x, int n, int d, const float *g, float *y, float *inv, hipStream_t st) {
    AVA_REQUIRE(d % 64 == 0 && d <= 1024, AVA_ERR_SHAPE, "train rms: d=%d (a multiple of 64, <= 1024)", d);
    if (n == 0) return AVA_OK;
    rms_fwd_kernel<<<grid1(n, WG / 64), WG, 0, st>>>(x, n, d, g, y, inv);
    AVA_LAUNCHED("train rms_fwd");
    return AVA_OK;
}

size_t rms_bwd_part_floats(int n, int d) { return (size_t)std::max(1, std::min(n, 1024)) * d; }

int rms_bwd(const float *x, const float *inv, const float *g, const float *dy, int n, int d, float *dx, float *dg,
            float *part, hipStream_t st) {
    AVA_REQUIRE(d % 64 == 0 && d <= 1024, AVA_ERR_SHAPE, "train rms_bwd: d=%d", d);
    const int nwg = std::max(1, std::min(n, 1024));
    const int per = (n + nwg - 1) / std::max(nwg, 1);
    rms_bwd_kernel<<<nwg, WG, 0, st>>>(x, inv, g, dy, n, d, std::max(per, 1), dx, part);
    AVA_LAUNCHED("train rms_bwd");
    colsum_final_kernel<<<grid1(d, 64), WG, 0, st>>>(part, nwg, d, dg, 0, nullptr, 0.0f);
    AVA_LAUNCHED("train rms_bwd colsum");
    return AVA_OK;
}

size_t colsum_part_floats(int rows, int cols) { return (size_t)std::max(1, std::min(rows, 256)) * cols; }

int colsum(const float *x, int rows, int cols, int ld, float *out, int accumulate, float *part, hipStream_t st,
           const float *extra, float sign) {
    const int nch = std::max(1, std::min(rows, 256));
    const int per = std::max(1, (rows + nch - 1) / nch);
    colsum_part_kernel<<<dim3(grid1(cols), nch), WG, 0, st>>>(x, rows, cols, ld, per, part);
    AVA_LAUNCHED("train colsum");
    colsum_final_kernel<<<grid1(cols, 64), WG, 0, st>>>(part, nch, cols, out, accumulate, extra, sign);
    AVA_LAUNCHED("train colsum final");
    return AVA_OK;
}

size_t dot_part_floats() { return 1024; }

int dot(const float *a, const float *b, size_t n, float *out, int accumulate, float *part, hipStream_t st) {
    const int nwg = (int)std::max<size_t>(1, std::min<size_t>(1024, (n + WG - 1) / WG));
    dot_part_kernel<<<nwg, WG, 0, st>>>(a, b, n, part);
    AVA_LAUNCHED("train dot");
    sum_final_kernel<<<1, 64, 0, st>>>(part, nwg, out, accumulate);
    AVA_LAUNCHED("train dot final");
    return AVA_OK;
}

int lif_params(const float *beta_p, const float *theta, const float *arho, const float *again, int d, int alif,
               float *ps, float *omb, hipStream_t st) {
    lif_params_kernel<<<grid1(d), WG, 0, st>>>(beta_p, theta, arho, again, d, alif, ps, omb);
    AVA_LAUNCHED("train lif_params");
    return AVA_OK;
}

int scale_cols(const float *x, const float *s, size_t rows, int d, float *y, hipStream_t st) {
    const size_t n = rows * d;
    if (n == 0) return AVA_OK;
    scale_cols_kernel<<<grid1(n), WG, 0, st>>>(x, s, n, d, y);
    AVA_LAUNCHED("train scale_cols");
    return AVA_OK;
}

int i8_to_f32(const int8_t *s, size_t n, float *y, hipStream_t st) {
    if (n == 0) return AVA_OK;
    i8_to_f32_kernel<<<grid1(n), WG, 0, st>>>(s, n, y);
    AVA_LAUNCHED("train i8_to_f32");
    return AVA_OK;
}

int axpy(float *y, const float *x, float a, size_t n, hipStream_t st) {
    if (n == 0) return AVA_OK;
    axpy_kernel<<<grid1(n), WG, 0, st>>>(y, x, a, n);
    AVA_LAUNCHED("train axpy");
    return AVA_OK;
}

int sigmoid_chain(const float *p, const float *dq, int n, float *dp, hipStream_t st) {
    sigmoid_chain_kernel<<<grid1(n), WG, 0, st>>>(p, dq, n, dp);
    AVA_LAUNCHED("train sigmoid_chain");
    return AVA_OK;
}

int embed(const int32_t *ids, const float *emb, int n, int d, int V, float *x, hipStream_t st) {
    embed_kernel<<<grid1((size_t)n * d), WG, 0, st>>>(ids, emb, n, d, V, x);
    AVA_LAUNCHED("train embed");
    return AVA_OK;
}

int embed_bwd(const int32_t *ids, const float *dx, int n, int d, int V, float *dE, hipStream_t st) {
    embed_bwd_kernel<<<grid1((size_t)n * d), WG, 0, st>>>(ids, dx, n, d, V, dE);
    AVA_LAUNCHED("train embed_bwd");
    return AVA_OK;
}

int prep_fwd(const TrainPrep &p, hipStream_t st) {
    const size_t items = (size_t)p.B * p.T * p.nh;
    prep_fwd_kernel<<<grid1(items, WG / 64), WG, 0, st>>>(p);
    AVA_LAUNCHED("train prep_fwd");
    return AVA_OK;
}

int prep_bwd(const TrainPrep &p, const TrainPrepGrad &g, hipStream_t st) {
    const size_t items = (size_t)p.B * p.T * p.nh;
    prep_bwd_kernel<<<grid1(items, WG / 64), WG, 0, st>>>(p, g);
    AVA_LAUNCHED("train prep_bwd");
    return AVA_OK;
}

int readout_fwd(const float *y, const float *g, int B, int T, int nh, float *o, hipStream_t st) {
    readout_fwd_kernel<<<grid1((size_t)B * T * nh, WG / 64), WG, 0, st>>>(y, g, B, T, nh, o);
    AVA_LAUNCHED("train readout_fwd");
    return AVA_OK;
}

int readout_bwd(const float *y, const float *g, const float *dout, int B, int T, int nh, float *dy, float *dg,
                hipStream_t st) {
    readout_bwd_kernel<<<grid1((size_t)B * T * nh, WG / 64), WG, 0, st>>>(y, g, dout, B, T, nh, dy, dg);
    AVA_LAUNCHED("train readout_bwd");
    return AVA_OK;
}

int attn_bwd(const TrainAttn &a, hipStream_t st) {
    AVA_REQUIRE(a.hd == 32 || a.hd == 64, AVA_ERR_SHAPE, "train attn_bwd: head size %d (32 or 64)", a.hd);
    AVA_REQUIRE(a.de % 4 == 0 && a.de == a.nh * a.hd && a.T > 0 && a.B > 0, AVA_ERR_SHAPE,
                "train attn_bwd: B=%d T=%d de=%d nh=%d hd=%d", a.B, a.T, a.de, a.nh, a.hd);
    const int blocks = ceil_div(a.T, 32) * a.B * a.nh;
    if (a.hd == 32) attn_bwd_dq_kernel<32><<<blocks, 64, 0, st>>>(a);
    else attn_bwd_dq_kernel<64><<<blocks, 64, 0, st>>>(a);
    AVA_LAUNCHED("train attn_bwd_dq");
    if (a.hd == 32) attn_bwd_dkv_kernel<32><<<blocks, 64, 0, st>>>(a);
    else attn_bwd_dkv_kernel<64><<<blocks, 64, 0, st>>>(a);
    AVA_LAUNCHED("train attn_bwd_dkv");
    return AVA_OK;
}

int cross_entropy(float *logits, const int32_t *tgt, int n, int V, float *lse, float *loss_row, float *valid,
                  float *loss, float *scal, hipStream_t st) {
    ce_row_kernel<<<n, WG, 0, st>>>(logits, tgt, V, lse, loss_row, valid);
    AVA_LAUNCHED("train ce_row");
    ce_total_kernel<<<1, 64, 0, st>>>(loss_row, valid, n, loss, scal);
    AVA_LAUNCHED("train ce_total");
    ce_grad_kernel<<<n, WG, 0, st>>>(logits, tgt, lse, scal, V);
    AVA_LAUNCHED("train ce_grad");
    return AVA_OK;
}

}  // namespace train
}  // namespace ava

// ---------------------------------------------------------------- the dense mix and small products

namespace {

// out = raw + sum_j w[j] S_j in j order (raw = S_{ns-1}, the block's output; w on the device)
struct TrainMix {
    const float *s[17];
    const float *w;
    float *out;
    int ns;
    size_t n;
};

__global__ __launch_bounds__(WG) void mix_kernel(TrainMix a) {
    const size_t i = (size_t)blockIdx.x * WG + threadIdx.x;
    if (i >= a.n) return;
    float x = a.s[a.ns - 1][i];
    for (int j = 0; j < a.ns; j++) x = x + a.s[j][i] * a.w[j];
    a.out[i] = x;
}

__global__ void mul_kernel(const float *__restrict__ a, const float *__restrict__ b, size_t n, float *__restrict__ y) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] * b[i];
}

}  // namespace

namespace ava {
namespace train {

int mix(float *out, const float *const *streams, int ns, const float *w, size_t n, hipStream_t st) {
    AVA_REQUIRE(ns >= 2 && ns <= 17, AVA_ERR_SHAPE, "train mix: %d streams", ns);
    TrainMix a;
    for (int j = 0; j < ns; j++) a.s[j] = streams[j];
    a.w = w;
    a.out = out;
    a.ns = ns;
    a.n = n;
    mix_kernel<<<grid1(n), WG, 0, st>>>(a);
    AVA_LAUNCHED("train mix");
    return AVA_OK;
}

int mul(const float *a, const float *b, size_t n, float *y, hipStream_t st) {
    if (n == 0) return AVA_OK;
    mul_kernel<<<grid1(n), WG, 0, st>>>(a, b, n, y);
    AVA_LAUNCHED("train mul");
    return AVA_OK;
}

}  // namespace train
}  // namespace ava
