// The per-row kernels between the products of one Ava-0.4 block (gfx950): the token embedding,
// RMSNorm fused with the split-plane int8 quantizer, the memory's key/value/gate preparation and its
// read-out (head norm times silu(g)), the f32 gate projections, the engram's causal read, and the
// dense (DenseFormer) mix.
//
// Row kernels run one wavefront per row with the row in registers (d <= 2048: NV float4 per lane),
// so a row is read once from HBM and every reduction is a wave reduction (no LDS, no barrier).
// Element-wise arithmetic follows the reference's operation order (gpu/model.rs:458-622,
// gpu/arch.rs:1873-2020, gpu/model/fstep.rs:207-292); the reductions sum in a tree, not in the
// reference's sequential order, which moves results by float rounding only.
#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float NORM_EPS = 1e-5f;  // gpu/model.rs:36

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (expf(-x) * 1.0f + 1.0f); }
__device__ __forceinline__ float log_sigmoid_ref(float x) {
    const float soft = logf(expf(-fabsf(x)) * 1.0f + 1.0f);
    const float r = -x > 0.0f ? -x : 0.0f;
    return -(r + soft);
}

// Write one row's P planes (the row's values in registers, NV float4 chunks per lane at columns
// 4 (i*64 + lane)), its exponent, and zero the K padding [k, ldq).
template <int P, int NV>
__device__ __forceinline__ void put_planes(const f32x4 (&x)[NV], int lane, int k, int ldq, size_t m, size_t row,
                                           int8_t *__restrict__ xq, int32_t *__restrict__ xexp) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) amax = fmaxf(amax, fabsf(x[i][c]));
    amax = ava::wave_max(amax);
    const int e = ava::plane_exp(amax);
    if (lane == 0) xexp[row] = e;
    const int nq = k >> 2;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        if (c < nq) {
            int q0[P], q1[P], q2[P], q3[P];
            ava::to_planes<P>(x[i][0], e, q0);
            ava::to_planes<P>(x[i][1], e, q1);
            ava::to_planes<P>(x[i][2], e, q2);
            ava::to_planes<P>(x[i][3], e, q3);
#pragma unroll
            for (int p = 0; p < P; p++)
                reinterpret_cast<uint32_t *>(xq + ((size_t)p * m + row) * ldq)[c] = ava::pack4(q0[p], q1[p], q2[p], q3[p]);
        }
    }
    for (int c = k + lane * 4; c < ldq; c += 256)
#pragma unroll
        for (int p = 0; p < P; p++) *reinterpret_cast<uint32_t *>(xq + ((size_t)p * m + row) * ldq + c) = 0u;
}

// ------------------------------------------------------------------ embedding

// x[n] = tok_emb[ids[n]] (and a copy into the dense mix's stream 0). One wave per row.
template <int NV>
__global__ __launch_bounds__(256) void embed_kernel(const int32_t *__restrict__ ids, const float *__restrict__ emb,
                                                    int n, int d, int vocab, float *__restrict__ x,
                                                    float *__restrict__ x0) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    int id = ids[row];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // an id outside [0, vocab) reads the nearest row, never out of bounds
    const f32x4 *src = reinterpret_cast<const f32x4 *>(emb + (size_t)id * d);
    f32x4 *dst = reinterpret_cast<f32x4 *>(x + (size_t)row * d);
    f32x4 *dst0 = x0 ? reinterpret_cast<f32x4 *>(x0 + (size_t)row * d) : nullptr;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        if (c < (d >> 2)) {
            const f32x4 v = src[c];
            dst[c] = v;
            if (dst0) dst0[c] = v;
        }
    }
}

// ------------------------------------------------------------------ RMSNorm -> planes

// h = x (mean(x^2) + eps)^-1/2 * gain (gpu/model.rs:458-462); its planes, and h itself when hout.
template <int P, int NV>
__global__ __launch_bounds__(256) void rms_planes_kernel(const float *__restrict__ x, int n, int d,
                                                         const float *__restrict__ gain, int8_t *__restrict__ xq,
                                                         int32_t *__restrict__ xexp, int ldq, float *__restrict__ hout) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const int nq = d >> 2;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + (size_t)row * d);
    f32x4 v[NV];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        v[i] = c < nq ? xr[c] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int z = 0; z < 4; z++) ss += v[i][z] * v[i][z];
    }
    ss = ava::wave_sum(ss);
    const float ms = ss * (1.0f / (float)d) + 0.0f;
    const float inv = 1.0f / sqrtf(ms * 1.0f + NORM_EPS);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        if (c < nq) {
            const f32x4 g = reinterpret_cast<const f32x4 *>(gain)[c];
#pragma unroll
            for (int z = 0; z < 4; z++) v[i][z] = (v[i][z] * inv) * g[z];
            if (hout) reinterpret_cast<f32x4 *>(hout + (size_t)row * d)[c] = v[i];
        }
    }
    put_planes<P, NV>(v, lane, d, ldq, (size_t)n, (size_t)row, xq, xexp);
}

// ------------------------------------------------------------------ f32 gate projections

// G [n][nc] = h [n][d] . W [d][nc] in f32 (the reference keeps the gate projections f32:
// gpu/arch.rs:1914-1936). 64 rows x nc (<= 128) columns per block; K in steps of 32 through LDS.
constexpr int GR = 64, GK = 32;
__global__ __launch_bounds__(256) void gate_gemm_kernel(const float *__restrict__ h, int n, int d,
                                                        const float *__restrict__ w, int nc, float *__restrict__ g) {
    __shared__ float sh[GR][GK + 1];
    __shared__ float sw[GK][128];
    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * GR;
    // thread -> rows (tid / 16) * 4 .. +3, columns (tid % 16) + 16 c, c < nc/16
    const int tr = (tid >> 4) * 4, tc = tid & 15;
    float acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 8; b++) acc[a][b] = 0.0f;
    for (int k0 = 0; k0 < d; k0 += GK) {
        for (int i = tid; i < GR * GK; i += 256) {
            const int rr = i / GK, kk = i % GK;
            const int row = r0 + rr;
            sh[rr][kk] = (row < n && k0 + kk < d) ? h[(size_t)row * d + k0 + kk] : 0.0f;
        }
        for (int i = tid; i < GK * 128; i += 256) {
            const int kk = i / 128, cc = i % 128;
            sw[kk][cc] = (cc < nc && k0 + kk < d) ? w[(size_t)(k0 + kk) * nc + cc] : 0.0f;
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < GK; kk++) {
            float hv[4], wv[8];
#pragma unroll
            for (int a = 0; a < 4; a++) hv[a] = sh[tr + a][kk];
#pragma unroll
            for (int b = 0; b < 8; b++) wv[b] = sw[kk][tc + 16 * b];
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 8; b++) acc[a][b] = fmaf(hv[a], wv[b], acc[a][b]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int row = r0 + tr + a;
        if (row >= n) continue;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int c = tc + 16 * b;
            if (c < nc) g[(size_t)row * nc + c] = acc[a][b];
        }
    }
}

// ------------------------------------------------------------------ memory preparation

// Per (row, head), one wave, lane = channel c of the head (gpu/arch.rs:1873-1941, gpu/lif.cu's
// wprepc semantics): from P = [q | k | v | we | g] (raw projections, [n][5d]) and G = [za | zb |
// z1a | z1b] ([n][2 nh + 2 r]):
//   q <- q / |q|, k <- k / |k|, e = (k_raw + we) / |k_raw + we|   (|x| = (sum x^2 + 1e-6)^1/2)
//   v <- v (1 + p0) + v0 p1 (value residual, blocks after the first; v0 = the first block's v)
//   la_c = logsig(((za_h + ba_h) + off_c) + (z1a . Wa2)_c),  b_c = 2 sigmoid((zb_h + bb_h) + (z1b . Wb2)_c)
// written in place (q, k, v; e over the we columns) and into la, b [n][d]. With vfirst_out the raw
// v is saved for later blocks.
struct PrepArgs {
    float *P;  // [n][5d]
    const float *G;
    int n, d, nh, r;
    const float *ba, *bb, *off, *wa2, *wb2;  // [nh], [nh], [d], [r][d], [r][d]
    const float *vres;                        // [2] or NULL
    const float *v0;                          // [n][d] or NULL
    float *v0_out;                            // [n][d] or NULL
    float *la, *b;                            // [n][d]
};

__global__ __launch_bounds__(256) void mem_prep_kernel(PrepArgs p) {
    extern __shared__ float smem[];  // wa2, wb2 slices of this head: [2][r][64]
    const int hh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *swa = smem, *swb = smem + p.r * 64;
    for (int i = tid; i < p.r * 64; i += 256) {
        const int rr = i >> 6, c = i & 63;
        swa[i] = p.wa2[(size_t)rr * p.d + hh * 64 + c];
        swb[i] = p.wb2[(size_t)rr * p.d + hh * 64 + c];
    }
    __syncthreads();
    const int d = p.d, ldp = 5 * d, ldg = 2 * p.nh + 2 * p.r;
    const int c = hh * 64 + lane;
    const float offc = p.off[c], bah = p.ba[hh], bbh = p.bb[hh];
    float p0 = 0.0f, p1 = 0.0f;
    if (p.vres) {
        p0 = p.vres[0] * 1.0f + 1.0f;
        p1 = p.vres[1];
    }
    // 16 rows per block: 4 waves x 4 rows
    for (int rr = 0; rr < 4; rr++) {
        const int row = blockIdx.x * 16 + wave * 4 + rr;
        if (row >= p.n) break;
        float *Pr = p.P + (size_t)row * ldp;
        const float *Gr = p.G + (size_t)row * ldg;
        const float q = Pr[c], kr = Pr[d + c], v = Pr[2 * d + c], we = Pr[3 * d + c];
        const float ek = kr + we;
        const float sq = ava::wave_sum(q * q), sk = ava::wave_sum(kr * kr), se = ava::wave_sum(ek * ek);
        Pr[c] = q * (1.0f / sqrtf(sq * 1.0f + 1e-6f));
        Pr[d + c] = kr * (1.0f / sqrtf(sk * 1.0f + 1e-6f));
        Pr[3 * d + c] = ek * (1.0f / sqrtf(se * 1.0f + 1e-6f));
        if (p.v0_out) p.v0_out[(size_t)row * d + c] = v;
        if (p.v0) Pr[2 * d + c] = v * p0 + p.v0[(size_t)row * d + c] * p1;
        const float za = Gr[hh] + bah, zb = Gr[p.nh + hh] + bbh;
        // lanes 0..r-1 hold z1a, lanes 32..32+r-1 hold z1b; each is broadcast with readlane
        const int zl_i = lane < 32 ? lane : lane - 32 + p.r;
        const float zl = (lane & 31) < p.r ? Gr[2 * p.nh + zl_i] : 0.0f;
        const int zbits = __float_as_int(zl);
        float lra = 0.0f, lrb = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            if (j < p.r) {
                const float za_j = __int_as_float(__builtin_amdgcn_readlane(zbits, j));
                const float zb_j = __int_as_float(__builtin_amdgcn_readlane(zbits, 32 + j));
                lra = fmaf(za_j, swa[j * 64 + lane], lra);
                lrb = fmaf(zb_j, swb[j * 64 + lane], lrb);
            }
        }
        p.la[(size_t)row * d + c] = log_sigmoid_ref((za + offc) + lra);
        p.b[(size_t)row * d + c] = sigmoid_ref(zb + lrb) * 2.0f + 0.0f;
    }
}

// ------------------------------------------------------------------ memory read-out

// o = head_norm(y) * silu(g) (gpu/model.rs:583-604), then its planes (the Wo input). One wave per
// row; lane l holds channels 16l..16l+15, so a head (64 channels) is 4 consecutive lanes.
template <int P>
__global__ __launch_bounds__(256) void mem_post_kernel(const float *__restrict__ y, int n, int d,
                                                       const float *__restrict__ g, int ldg, int8_t *__restrict__ xq,
                                                       int32_t *__restrict__ xexp, int ldq) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    constexpr int NV = 4;  // d = 1024: 16 channels per lane (d < 1024 leaves lanes idle)
    const int c0 = lane * 16;
    const bool on = c0 < d;
    f32x4 v[NV];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        v[i] = on ? reinterpret_cast<const f32x4 *>(y + (size_t)row * d + c0)[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int z = 0; z < 4; z++) ss += v[i][z] * v[i][z];
    }
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    const float inv = 1.0f / sqrtf(ss * (1.0f / 64.0f) + 0.0f + NORM_EPS);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const f32x4 gv = on ? reinterpret_cast<const f32x4 *>(g + (size_t)row * ldg + c0)[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int z = 0; z < 4; z++) {
            const float gz = gv[z];
            const float s = gz / (1.0f + expf(-gz));
            v[i][z] = (v[i][z] * inv) * s;
            amax = fmaxf(amax, fabsf(v[i][z]));
        }
    }
    amax = ava::wave_max(amax);
    const int e = ava::plane_exp(amax);
    if (lane == 0) xexp[row] = e;
    if (on) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            int q0[P], q1[P], q2[P], q3[P];
            ava::to_planes<P>(v[i][0], e, q0);
            ava::to_planes<P>(v[i][1], e, q1);
            ava::to_planes<P>(v[i][2], e, q2);
            ava::to_planes<P>(v[i][3], e, q3);
#pragma unroll
            for (int p = 0; p < P; p++)
                *reinterpret_cast<uint32_t *>(xq + ((size_t)p * n + row) * ldq + c0 + 4 * i) =
                    ava::pack4(q0[p], q1[p], q2[p], q3[p]);
        }
    }
}

// ------------------------------------------------------------------ engram read

// Causal single-head attention of one stream's T queries against its store: query t (store
// position n0 + t) reads entries 0..n0 + t with softmax(q.k / sqrt(de)) (gpu/model.rs:543-562,
// gpu/model/fstep.rs:303-329). de == 64. Block = 64 queries x 256 threads; keys and values in
// tiles of 64 through LDS; the softmax is the online (running max) form, equal to the reference's
// two-pass form up to rounding. out [B*T][64].
__global__ __launch_bounds__(256) void attend_kernel(const float *__restrict__ q, int ldq, const float *__restrict__ ks,
                                                     const float *__restrict__ vs, int cap, int n0, int T, float scale,
                                                     float *__restrict__ out) {
    __shared__ float sk[64][65];
    __shared__ float sv[64][64];
    __shared__ float sp[64][65];
    const int bi = blockIdx.y, qb = blockIdx.x * 64;
    const int tid = threadIdx.x;
    const int r = tid >> 2, sub = tid & 3;  // query row, quarter (16 keys / 16 output dims)
    const float *kb = ks + (size_t)bi * cap * 64, *vb = vs + (size_t)bi * cap * 64;
    float qr[64];
    {
        const bool ok = qb + r < T;
        const f32x4 *src = reinterpret_cast<const f32x4 *>(q + ((size_t)bi * T + qb + r) * ldq);
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const f32x4 v = ok ? src[c] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int z = 0; z < 4; z++) qr[4 * c + z] = v[z];
        }
    }
    float mx = -INFINITY, den = 0.0f, o[16];
#pragma unroll
    for (int z = 0; z < 16; z++) o[z] = 0.0f;
    const int qpos = n0 + qb + r;                  // this row's store position
    const int kend = min(n0 + qb + 64, n0 + T);    // keys the block's last row reads
    for (int k0 = 0; k0 < kend; k0 += 64) {
        __syncthreads();
        for (int i = tid; i < 64 * 64; i += 256) {
            const int rr = i >> 6, cc = i & 63;
            const bool ok = k0 + rr < kend;
            sk[rr][cc] = ok ? kb[(size_t)(k0 + rr) * 64 + cc] : 0.0f;
            sv[rr][cc] = ok ? vb[(size_t)(k0 + rr) * 64 + cc] : 0.0f;
        }
        __syncthreads();
        float s[16], tmax = -INFINITY;
#pragma unroll
        for (int z = 0; z < 16; z++) {
            const int kk = sub * 16 + z;
            float a = 0.0f;
#pragma unroll
            for (int c = 0; c < 64; c++) a = fmaf(sk[kk][c], qr[c], a);
            a = a * scale + 0.0f;
            s[z] = (k0 + kk <= qpos) ? a : -INFINITY;
            tmax = fmaxf(tmax, s[z]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 1, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 2, 64));
        const float nmx = fmaxf(mx, tmax);
        const float corr = (mx == -INFINITY) ? 0.0f : expf(mx - nmx);
        float psum = 0.0f;
#pragma unroll
        for (int z = 0; z < 16; z++) {
            const float e = (s[z] == -INFINITY) ? 0.0f : expf(s[z] - nmx);
            sp[r][sub * 16 + z] = e;
            psum += e;
        }
        psum += __shfl_xor(psum, 1, 64);
        psum += __shfl_xor(psum, 2, 64);
        den = den * corr + psum;
        mx = nmx;
        __syncthreads();
#pragma unroll
        for (int z = 0; z < 16; z++) o[z] *= corr;
        for (int kk = 0; kk < 64; kk++) {
            const float pk = sp[r][kk];
#pragma unroll
            for (int z = 0; z < 16; z++) o[z] = fmaf(pk, sv[kk][sub * 16 + z], o[z]);
        }
    }
    if (qb + r < T) {
        float *orow = out + ((size_t)bi * T + qb + r) * 64 + sub * 16;
#pragma unroll
        for (int z = 0; z < 16; z++) orow[z] = o[z] / den;
    }
}

// Append this forward's keys and values to the store: store[b][n0 + t] = kv[b T + t].
__global__ void store_append_kernel(const float *__restrict__ kv, int ldkv, int T, int B, int cap, int n0,
                                    float *__restrict__ ks, float *__restrict__ vs) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // over B*T*64
    if (i >= B * T * 64) return;
    const int c = i & 63, row = i >> 6, bi = row / T, t = row - bi * T;
    const size_t dst = ((size_t)bi * cap + n0 + t) * 64 + c;
    ks[dst] = kv[(size_t)row * ldkv + c];
    vs[dst] = kv[(size_t)row * ldkv + 64 + c];
}

// ------------------------------------------------------------------ dense mix

// DenseFormer (gpu/arch.rs:1492-1500): stream[i+1] = x; x <- x + sum_{j <= i+1} w_j stream_j, the
// terms added one at a time in j order.
struct DenseArgs {
    float *x;
    float *streams[17];
    float w[17];
    int ns;  // i + 2 terms (the last is the stream being written)
    size_t n4;
};

__global__ __launch_bounds__(256) void dense_mix_kernel(DenseArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n4) return;
    const f32x4 x = reinterpret_cast<const f32x4 *>(a.x)[i];
    reinterpret_cast<f32x4 *>(a.streams[a.ns - 1])[i] = x;
    f32x4 mix = x;
    for (int j = 0; j < a.ns; j++) {
        const f32x4 s = j == a.ns - 1 ? x : reinterpret_cast<const f32x4 *>(a.streams[j])[i];
        const float w = a.w[j];
#pragma unroll
        for (int z = 0; z < 4; z++) mix[z] = mix[z] + s[z] * w;
    }
    reinterpret_cast<f32x4 *>(a.x)[i] = mix;
}

}  // namespace

namespace ava {

int embed(const int32_t *ids, const float *emb, int n, int d, int vocab, float *x, float *x0, hipStream_t st) {
    AVA_REQUIRE(d % 4 == 0 && d <= 2048, AVA_ERR_SHAPE, "embed: d=%d", d);
    dim3 grid(ceil_div(n, 4)), block(256);
    if (d <= 1024) embed_kernel<4><<<grid, block, 0, st>>>(ids, emb, n, d, vocab, x, x0);
    else embed_kernel<8><<<grid, block, 0, st>>>(ids, emb, n, d, vocab, x, x0);
    AVA_LAUNCHED("embed");
    return AVA_OK;
}

int rms_planes(const float *x, int n, int d, const float *gain, int planes, int8_t *xq, int32_t *xexp, int ldq,
               float *hout, hipStream_t st) {
    AVA_REQUIRE(d % 4 == 0 && d <= 2048 && ldq >= d && ldq % 4 == 0, AVA_ERR_SHAPE, "rms_planes: d=%d ldq=%d", d, ldq);
    dim3 grid(ceil_div(n, 4)), block(256);
#define AVA_RP(P_, NV_) rms_planes_kernel<P_, NV_><<<grid, block, 0, st>>>(x, n, d, gain, xq, xexp, ldq, hout)
    if (d <= 1024) {
        if (planes == 1) AVA_RP(1, 4);
        else if (planes == 2) AVA_RP(2, 4);
        else AVA_RP(3, 4);
    } else {
        if (planes == 1) AVA_RP(1, 8);
        else if (planes == 2) AVA_RP(2, 8);
        else AVA_RP(3, 8);
    }
#undef AVA_RP
    AVA_LAUNCHED("rms_planes");
    return AVA_OK;
}

int gate_gemm(const float *h, int n, int d, const float *w, int nc, float *g, hipStream_t st) {
    AVA_REQUIRE(nc <= 128, AVA_ERR_SHAPE, "gate_gemm: %d columns (<= 128)", nc);
    gate_gemm_kernel<<<ceil_div(n, GR), 256, 0, st>>>(h, n, d, w, nc, g);
    AVA_LAUNCHED("gate_gemm");
    return AVA_OK;
}

int mem_prep(float *P, const float *G, int n, int d, int nh, int r, const float *ba, const float *bb, const float *off,
             const float *wa2, const float *wb2, const float *vres, const float *v0, float *v0_out, float *la, float *b,
             hipStream_t st) {
    AVA_REQUIRE(d == nh * 64 && r > 0 && r <= 32, AVA_ERR_SHAPE, "mem_prep: d=%d nh=%d r=%d", d, nh, r);
    PrepArgs a{P, G, n, d, nh, r, ba, bb, off, wa2, wb2, vres, v0, v0_out, la, b};
    dim3 grid(ceil_div(n, 16), nh), block(256);
    mem_prep_kernel<<<grid, block, sizeof(float) * 2 * r * 64, st>>>(a);
    AVA_LAUNCHED("mem_prep");
    return AVA_OK;
}

int mem_post(const float *y, int n, int d, const float *g, int ldg, int planes, int8_t *xq, int32_t *xexp, int ldq,
             hipStream_t st) {
    AVA_REQUIRE(d % 64 == 0 && d <= 1024, AVA_ERR_SHAPE, "mem_post: d=%d (<= 1024)", d);
    dim3 grid(ceil_div(n, 4)), block(256);
    if (planes == 1) mem_post_kernel<1><<<grid, block, 0, st>>>(y, n, d, g, ldg, xq, xexp, ldq);
    else if (planes == 2) mem_post_kernel<2><<<grid, block, 0, st>>>(y, n, d, g, ldg, xq, xexp, ldq);
    else mem_post_kernel<3><<<grid, block, 0, st>>>(y, n, d, g, ldg, xq, xexp, ldq);
    AVA_LAUNCHED("mem_post");
    return AVA_OK;
}

int engram_read(const float *qkv, int ldqkv, int B, int T, float *ks, float *vs, int cap, int n0, float *out,
                hipStream_t st) {
    AVA_REQUIRE(n0 + T <= cap, AVA_ERR_SHAPE, "engram: store of %d entries holds %d + %d", cap, n0, T);
    const int total = B * T * 64;
    store_append_kernel<<<ceil_div(total, 256), 256, 0, st>>>(qkv + 64, ldqkv, T, B, cap, n0, ks, vs);
    AVA_LAUNCHED("store_append");
    dim3 grid(ceil_div(T, 64), B);
    attend_kernel<<<grid, 256, 0, st>>>(qkv, ldqkv, ks, vs, cap, n0, T, (float)(1.0 / sqrt(64.0)), out);
    AVA_LAUNCHED("attend");
    return AVA_OK;
}

int dense_mix(float *x, float *const *streams, const float *w, int ns, size_t n, hipStream_t st) {
    AVA_REQUIRE(ns >= 2 && ns <= 17 && n % 4 == 0, AVA_ERR_SHAPE, "dense_mix: %d streams", ns);
    DenseArgs a;
    a.x = x;
    for (int j = 0; j < ns; j++) {
        a.streams[j] = streams[j];
        a.w[j] = w[j];
    }
    a.ns = ns;
    a.n4 = n / 4;
    dense_mix_kernel<<<(unsigned)((a.n4 + 255) / 256), 256, 0, st>>>(a);
    AVA_LAUNCHED("dense_mix");
    return AVA_OK;
}

}  // namespace ava
