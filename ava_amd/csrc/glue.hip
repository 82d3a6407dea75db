// The per-row kernels between the products of one Ava-0.4 block (gfx950): the token embedding,
// RMSNorm fused with the split-plane int8 quantizer, the memory's read-out (head norm times silu(g)),
// the f32 gate projections, the engram's causal read, and the dense (DenseFormer) mix. (The memory's
// key/value/gate preparation is fused into its scan, mem.hip.)
//
// Row kernels run one wavefront per row with the row in registers (d <= 2048: NV float4 per lane),
// so a row is read once from HBM and every reduction is a wave reduction (no LDS, no barrier).
// Element-wise arithmetic follows the reference's operation order (gpu/model.rs:458-622,
// gpu/arch.rs:1873-2020, gpu/model/fstep.rs:207-292); the reductions sum in a tree, not in the
// reference's sequential order, which moves results by float rounding only.
#include <hip/hip_fp16.h>

#include <algorithm>

#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float NORM_EPS = 1e-5f;  // gpu/model.rs:36


// Write one row's P planes (the row's values in registers, NV float4 chunks per lane at columns
// 4 (i*64 + lane)), its exponent, and zero the K padding [k, ldq).
template <int P, int NV>
__device__ __forceinline__ void put_planes(const f32x4 (&x)[NV], int lane, int k, int ldq, size_t m, size_t row,
                                           int8_t *__restrict__ xq, int32_t *__restrict__ xexp) {
    if (!xq) return;  // the row's planes are written elsewhere
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

// h = x (mean(x^2) + eps)^-1/2 * gain (gpu/model.rs:458-462) of one row held in a wave's registers
// (NV float4 chunks per lane, zero past d); its planes, and h itself when hout.
template <int P, int NV>
__device__ __forceinline__ float row_rms_planes(f32x4 (&v)[NV], int lane, int d, const float *__restrict__ gain,
                                                size_t n, size_t row, int8_t *__restrict__ xq,
                                                int32_t *__restrict__ xexp, int ldq, float *__restrict__ hout) {
    const int nq = d >> 2;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
#pragma unroll
        for (int z = 0; z < 4; z++) ss += v[i][z] * v[i][z];
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
            if (hout) reinterpret_cast<f32x4 *>(hout + row * d)[c] = v[i];
        }
    }
    put_planes<P, NV>(v, lane, d, ldq, n, row, xq, xexp);
    return inv;  // the row's 1 / rms, the same value for every lane
}

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
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        v[i] = c < nq ? xr[c] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    row_rms_planes<P, NV>(v, lane, d, gain, (size_t)n, (size_t)row, xq, xexp, ldq, hout);
}

// ------------------------------------------------------------------ f32 gate projections

// G [n][nc] = h [n][d] . W [d][nc] at f32 accuracy (the reference keeps the gate projections f32:
// gpu/arch.rs:1914-1936) on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16): every operand value is
// split into three bf16 terms, x = t0 + t1 + t2 (each term the rest rounded again), and the products
// a_i b_j with i + j < 3 are kept, which leaves about 2^-24 of |a b| per product as an f32 product
// does; the leading product t0 t0 and the five cross products accumulate apart (f32) and are added at
// the end. Six bf16 products per 16 k cost a third of the eight f32 ones (v_mfma_f32_32x32x2_f32) they
// replace. Block = 128 rows x NC columns (NC = nc rounded up to 32, <= 128); wave w owns rows
// 32w..32w+31; K in steps of 32 through LDS, where each operand is held as its three term planes with
// k contiguous (a 16-byte fragment read per lane and term); the next step's tiles are in flight meanwhile.
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int GR = 128, GK = 32, GKP = GK + 8;  // GKP: bf16 per LDS row (80 bytes: conflict-free fragments)
__device__ __forceinline__ void split3(const float (&x)[8], bf16x8 (&t)[3]) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float r = x[e];
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const __bf16 o = (__bf16)r;
            t[i][e] = o;
            r = r - (float)o;
        }
    }
}
// The K loop and stores of gate_mfma_kernel for the 128-row block at r0. The block's rows come from
// h, or, with NORM, from x normed as they are staged: h = (x * s_inv[row]) * gain[k], the two
// roundings of row_rms_planes, so G gets the same bits either way.
template <int NCB, bool NORM>
__device__ __forceinline__ void gate_block(const float *__restrict__ h, int n, int d, const float *__restrict__ w,
                                           int nc, float *__restrict__ g, int r0, const float *s_inv,
                                           const float *__restrict__ gain) {
    __shared__ __attribute__((aligned(16))) __bf16 sh[3][GR][GKP];        // h rows: k contiguous
    __shared__ __attribute__((aligned(16))) __bf16 sw[3][NCB * 32][GKP];  // W columns: k contiguous
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int last = min(GR, n - r0) - 1;  // the block's last row (rows past n repeat it, unstored)
    f32x16 acc[NCB], crs[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        acc[cb] = f32x16{};
        crs[cb] = f32x16{};
    }
    // staging items of 8 consecutive k: h (row, k group) 128 x 4, W (column, k group) NCB 32 x 4
    constexpr int HI = GR * (GK / 8) / 256, WI = (NCB * 32 * (GK / 8) + 255) / 256;
    float hv[HI][8], wv[WI][8];
    f32x4 gr[HI][2];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int j = 0; j < HI; j++) {
            const int it = tid + j * 256, rr = min(it >> 2, last), kk = k0 + (it & 3) * 8;
            const f32x4 *src = reinterpret_cast<const f32x4 *>(h + (size_t)(r0 + rr) * d + kk);
            const f32x4 u0 = src[0], u1 = src[1];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                hv[j][e] = u0[e];
                hv[j][4 + e] = u1[e];
            }
            if (NORM) {
                gr[j][0] = reinterpret_cast<const f32x4 *>(gain + kk)[0];
                gr[j][1] = reinterpret_cast<const f32x4 *>(gain + kk)[1];
            }
        }
#pragma unroll
        for (int j = 0; j < WI; j++) {
            const int it = tid + j * 256, cc = it % (NCB * 32), kk = k0 + (it / (NCB * 32)) * 8;
            const bool on = it < NCB * 32 * (GK / 8) && cc < nc;
#pragma unroll
            for (int e = 0; e < 8; e++) wv[j][e] = on ? w[(size_t)(kk + e) * nc + cc] : 0.0f;
        }
    };
    fetch(0);
    for (int k0 = 0; k0 < d; k0 += GK) {
        __syncthreads();  // the previous step's tiles are read
#pragma unroll
        for (int j = 0; j < HI; j++) {
            const int it = tid + j * 256, rr = it >> 2, kg = (it & 3) * 8;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                x[e] = hv[j][e];
                if (NORM) x[e] = (x[e] * s_inv[min(rr, last)]) * gr[j][e >> 2][e & 3];
            }
            bf16x8 t[3];
            split3(x, t);
#pragma unroll
            for (int i = 0; i < 3; i++) *reinterpret_cast<bf16x8 *>(&sh[i][rr][kg]) = t[i];
        }
#pragma unroll
        for (int j = 0; j < WI; j++) {
            const int it = tid + j * 256;
            if (it < NCB * 32 * (GK / 8)) {
                const int cc = it % (NCB * 32), kg = (it / (NCB * 32)) * 8;
                bf16x8 t[3];
                split3(wv[j], t);
#pragma unroll
                for (int i = 0; i < 3; i++) *reinterpret_cast<bf16x8 *>(&sw[i][cc][kg]) = t[i];
            }
        }
        if (k0 + GK < d) fetch(k0 + GK);
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < GK; ks += 16) {
            const int kf = ks + 8 * (lane >> 5);
            bf16x8 a[3];
#pragma unroll
            for (int i = 0; i < 3; i++) a[i] = *reinterpret_cast<const bf16x8 *>(&sh[i][wave * 32 + (lane & 31)][kf]);
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                bf16x8 b[3];
#pragma unroll
                for (int i = 0; i < 3; i++) b[i] = *reinterpret_cast<const bf16x8 *>(&sw[i][cb * 32 + (lane & 31)][kf]);
                acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc[cb], 0, 0, 0);
                crs[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], crs[cb], 0, 0, 0);
                crs[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], crs[cb], 0, 0, 0);
                crs[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], crs[cb], 0, 0, 0);
                crs[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], crs[cb], 0, 0, 0);
                crs[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], crs[cb], 0, 0, 0);
            }
        }
    }
    // lane holds rows (r/4)*8 + (lane/32)*4 + r%4 of column lane%32 of each 32 x 32 block
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        const int col = cb * 32 + (lane & 31);
        if (col >= nc) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = r0 + wave * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (row < n) g[(size_t)row * nc + col] = acc[cb][r] + crs[cb][r];
        }
    }
}

template <int NCB>  // column blocks of 32
__global__ __launch_bounds__(256) void gate_mfma_kernel(const float *__restrict__ h, int n, int d,
                                                        const float *__restrict__ w, int nc, float *__restrict__ g) {
    gate_block<NCB, false>(h, n, d, w, nc, g, blockIdx.x * GR, nullptr, nullptr);
}

// RMSNorm, planes and gate projections of many rows in one launch (the prefill form of
// rms_gate_kernel), d = 1024, a 128-row block per workgroup: wave w norms the block's rows
// 32w..32w+31 one at a time as rms_planes_kernel does (planes to xq; each row's loads issued before
// the previous row's norm), keeping the rows' 1 / rms in LDS; the block then runs gate_mfma_kernel's
// K loop on the rows normed again as they are staged. G and the planes get the bits of
// rms_planes_kernel + gate_mfma_kernel, and h makes no round trip through HBM (x is read a second
// time, partly from the cache hierarchy).
template <int P, int NCB>
__global__ __launch_bounds__(256, 2) void rms_gate_mfma_kernel(const float *__restrict__ x, int n,
                                                               const float *__restrict__ gain, int8_t *__restrict__ xq,
                                                               int32_t *__restrict__ xexp, int ldq,
                                                               const float *__restrict__ w, int nc,
                                                               float *__restrict__ g) {
    constexpr int d = 1024, NV = 4;
    __shared__ float s_inv[GR];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * GR, w0 = r0 + wave * 32;
    // the next two rows' loads in flight while a row is normed
    f32x4 cur[NV], nx1[NV], nx2[NV];
    auto load_row = [&](int row, f32x4 (&v)[NV]) {
        const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + (size_t)min(row, n - 1) * d);
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = xr[i * 64 + lane];
    };
    load_row(w0, cur);
    load_row(w0 + 1, nx1);
    for (int j = 0; j < 32; j++) {
        if (j + 2 < 32) load_row(w0 + j + 2, nx2);
        if (w0 + j < n) {  // wave-uniform
            const float inv =
                row_rms_planes<P, NV>(cur, lane, d, gain, (size_t)n, (size_t)(w0 + j), xq, xexp, ldq, nullptr);
            if (lane == 0) s_inv[wave * 32 + j] = inv;
        }
#pragma unroll
        for (int i = 0; i < NV; i++) {
            cur[i] = nx1[i];
            nx1[i] = nx2[i];
        }
    }
    __syncthreads();  // every row's 1 / rms is in s_inv (gate_block's first barrier follows too)
    gate_block<NCB, true>(x, n, d, w, nc, g, r0, s_inv, gain);
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
    f32x4 v[NV], gvs[NV];
    // the row's y and g loads all in flight before the first use
#pragma unroll
    for (int i = 0; i < NV; i++) {
        v[i] = on ? reinterpret_cast<const f32x4 *>(y + (size_t)row * d + c0)[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        gvs[i] = on ? reinterpret_cast<const f32x4 *>(g + (size_t)row * ldg + c0)[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    AVA_ISSUE_FENCE();
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
#pragma unroll
        for (int z = 0; z < 4; z++) ss += v[i][z] * v[i][z];
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    const float inv = 1.0f / sqrtf(ss * (1.0f / 64.0f) + 0.0f + NORM_EPS);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const f32x4 gv = gvs[i];
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

// The engram store's element: f32 (the reference's store) or fp16 (a KV cache at half the bytes).
__device__ __forceinline__ float kv_get(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float kv_get(const __half *p, size_t i) { return __half2float(p[i]); }
__device__ __forceinline__ void kv_put(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void kv_put(__half *p, size_t i, float v) { p[i] = __float2half_rn(v); }

// 16-byte loads of the store: DPL elements per lane (4 f32 or 8 fp16), widened to f32; load16: 16
// consecutive elements. `load` (the decode read, which streams each entry once) is non-temporal:
// 386 -> 370 us for 256 streams x 32,768 fp16 entries of 64 dims (5.55 -> 5.81 TB/s, the same bits).
template <typename KV>
struct KvLane;
template <>
struct KvLane<float> {
    static constexpr int DPL = 4;
    static __device__ __forceinline__ void load(const float *p, float (&x)[4]) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
#pragma unroll
        for (int z = 0; z < 4; z++) x[z] = v[z];
    }
    static __device__ __forceinline__ void load16(const float *p, float (&x)[16]) {
        f32x4 v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = reinterpret_cast<const f32x4 *>(p)[c];
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int z = 0; z < 4; z++) x[4 * c + z] = v[c][z];
    }
};
template <>
struct KvLane<__half> {
    static constexpr int DPL = 8;
    static __device__ __forceinline__ void load(const __half *p, float (&x)[8]) {
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
        const uint32_t w[4] = {u[0], u[1], u[2], u[3]};
#pragma unroll
        for (int z = 0; z < 4; z++) {
            const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&w[z]));
            x[2 * z] = f.x;
            x[2 * z + 1] = f.y;
        }
    }
    static __device__ __forceinline__ void load16(const __half *p, float (&x)[16]) {
        const uint4 u0 = reinterpret_cast<const uint4 *>(p)[0], u1 = reinterpret_cast<const uint4 *>(p)[1];
        const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int z = 0; z < 8; z++) {
            const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&w[z]));
            x[2 * z] = f.x;
            x[2 * z + 1] = f.y;
        }
    }
};

// Causal attention of one stream's T queries against its store (gpu/model.rs:543-562,
// gpu/model/fstep.rs:303-329): query t (store position n0 + t) reads entries 0..n0 + t with
// softmax(q.k / sqrt(head size)). On the fp32 MFMA (v_mfma_f32_32x32x2_f32), for query blocks of 64:
// per 64-key tile, S = Q K^T (wave w: a 32 x 32 quadrant), scaled and masked into LDS; the online
// (running max) softmax by row, 4 threads per row with 16 scores each (the running max, the rescale
// factor of the previous tiles, exp); then O = O corr + P V (wave w: its quadrant of the 64 x 64
// output, kept in the MFMA accumulator across tiles); O / den at the end. Equal to the reference's
// two-pass softmax up to rounding.
// Heads: the store's rows hold nh heads of HD dims (de = nh HD, the reference's heads of 32,
// gpu/memory.rs:610-700); workgroup (query block, b nh + h) reads head h: its query, key and value
// dims h HD .. h HD + HD - 1. The Q, K and V tiles are HD wide; for HD = 32, P V has one 32-column
// output: the two waves of a row half each take half of the tile's keys.
template <typename KV, int HD>
__global__ __launch_bounds__(256) void attend_mfma_kernel(const float *__restrict__ q, int ldq,
                                                          const KV *__restrict__ ks, const KV *__restrict__ vs,
                                                          int cap, int n0, const int *n0p, int T, float scale,
                                                          int de, int nh, float *__restrict__ out) {
    static_assert(HD == 32 || HD == 64, "head size 32 or 64");
    if (n0p) n0 = min(*n0p, cap - T);  // the store length on the device (a replayed graph)
    constexpr int L = 65;               // LDS row stride (odd: a column read hits 32 banks)
    constexpr int LK = HD + 1;          // the same for the head's Q, K and V tiles (HD 32: 3 workgroups per CU)
    // scores in base-2 units (s log2 e), so the softmax's exponentials are the hardware 2^x
    // (v_exp_f32): with m the running max in those units, 2^(s log2 e - m) = e^(s - m ln 2), and
    // the normalized weights are the softmax's up to rounding
    const float scale2 = scale * 1.44269504088896341f;
    // Q lives in registers (each wave's MFMA operand column of its 32 query rows); sK stages it first
    __shared__ float sK[64 * LK], sV[64 * LK], sP[64 * L];
    __shared__ float s_corr[64], s_den[64];
    const int bi = blockIdx.y / nh, hh = blockIdx.y - bi * nh, qb = blockIdx.x * 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lc = lane & 31;
    const int row0 = (wave >> 1) * 32, col0 = (wave & 1) * 32;
    const int r = tid >> 2, sub = tid & 3;  // the softmax's row and quarter
    const KV *kb = ks + (size_t)bi * cap * de + hh * HD, *vb = vs + (size_t)bi * cap * de + hh * HD;
    for (int i = tid; i < 64 * HD; i += 256) {
        const int rr = i / HD, cc = i % HD;
        sK[rr * LK + cc] = qb + rr < T ? q[((size_t)bi * T + qb + rr) * ldq + hh * HD + cc] : 0.0f;
    }
    __syncthreads();
    float qf[HD / 2];  // lane (fr, h): Q[row0 + fr][x + h] for x = 0, 2, ..
#pragma unroll
    for (int x = 0; x < HD; x += 2) qf[x >> 1] = sK[(row0 + (lane & 31)) * LK + x + (lane >> 5)];
    auto qrow = [&](int i) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); };
    float mx = -INFINITY, den = 0.0f;
    f32x16 o = {};
    const int qpos = n0 + qb + r;                // the softmax row's store position
    const int kend = min(n0 + qb + 64, n0 + T);  // keys the block's last row reads
    // thread (r, sub) stages key/value row r, dims 16 sub .. 16 sub + 15; the next tile's are loaded
    // into registers while this tile is computed
    float kr[16] = {}, vr[16] = {};
    auto fetch = [&](int k0) {
        if (sub * 16 >= HD) return;  // HD = 32: the threads of dims 32..63 stage nothing
        const bool ok = k0 + r < kend;
        const size_t o16 = (size_t)(k0 + (ok ? r : 0)) * de + (ok ? sub * 16 : 0);
        KvLane<KV>::load16(kb + o16, kr);
        KvLane<KV>::load16(vb + o16, vr);
        if (!ok)
#pragma unroll
            for (int z = 0; z < 16; z++) kr[z] = vr[z] = 0.0f;
    };
    fetch(0);
    for (int k0 = 0; k0 < kend; k0 += 64) {
        __syncthreads();  // the previous tile's K, V and P (the first time: Q) are read
#pragma unroll
        for (int z = 0; z < 16; z++) {
            if (sub * 16 < HD) {
                sK[r * LK + sub * 16 + z] = kr[z];
                sV[r * LK + sub * 16 + z] = vr[z];
            }
        }
        if (k0 + 64 < kend) fetch(k0 + 64);
        __syncthreads();
        {
            f32x16 sa = {};
            const int fr = lane & 31, h = lane >> 5;
#pragma unroll
            for (int x = 0; x < HD; x += 2)
                sa = __builtin_amdgcn_mfma_f32_32x32x2f32(qf[x >> 1], sK[(col0 + fr) * LK + x + h], sa, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int rr = row0 + qrow(i), cc = col0 + lc;
                const float a = sa[i] * scale2;
                sP[rr * L + cc] = (k0 + cc <= n0 + qb + rr) ? a : -INFINITY;
            }
        }
        __syncthreads();
        {
            float sc[16], tmax = -INFINITY;
#pragma unroll
            for (int z = 0; z < 16; z++) {
                sc[z] = sP[r * L + sub * 16 + z];
                tmax = fmaxf(tmax, sc[z]);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 1, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 2, 64));
            const float nmx = fmaxf(mx, tmax);
            const float corr = (mx == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mx - nmx);
            float psum = 0.0f;
#pragma unroll
            for (int z = 0; z < 16; z++) {
                const float e = (sc[z] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc[z] - nmx);
                sP[r * L + sub * 16 + z] = e;
                psum += e;
            }
            psum += __shfl_xor(psum, 1, 64);
            psum += __shfl_xor(psum, 2, 64);
            den = den * corr + psum;
            mx = nmx;
            if (sub == 0) s_corr[r] = corr;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 16; i++) o[i] *= s_corr[row0 + qrow(i)];
        {
            const int fr = lane & 31, h = lane >> 5;
            if constexpr (HD == 64) {
#pragma unroll 8
                for (int x = 0; x < 64; x += 2)
                    o = __builtin_amdgcn_mfma_f32_32x32x2f32(sP[(row0 + fr) * L + x + h], sV[(x + h) * LK + col0 + fr],
                                                             o, 0, 0, 0);
            } else {
                // one 32-column output: the wave pair of a row half splits the tile's keys, each
                // keeping its partial sum (both scale by the same corrections); added at the end
                const int kh = col0;
#pragma unroll 8
                for (int x = 0; x < 32; x += 2)
                    o = __builtin_amdgcn_mfma_f32_32x32x2f32(sP[(row0 + fr) * L + kh + x + h],
                                                             sV[(kh + x + h) * LK + fr], o, 0, 0, 0);
            }
        }
    }
    if constexpr (HD == 32) {
        // the second key half's partials through sK (no wave reads sK after its last S product,
        // which every wave passed before the last tile's softmax barrier)
        if (col0)
#pragma unroll
            for (int i = 0; i < 16; i++) sK[(row0 + qrow(i)) * LK + lc] = o[i];
    }
    if (sub == 0) s_den[r] = den;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int rr = row0 + qrow(i);
        if constexpr (HD == 64) {
            if (qb + rr < T) out[((size_t)bi * T + qb + rr) * de + hh * HD + col0 + lc] = o[i] / s_den[rr];
        } else {
            if (qb + rr < T && col0 == 0)
                out[((size_t)bi * T + qb + rr) * de + hh * HD + lc] = (o[i] + sK[rr * LK + lc]) / s_den[rr];
        }
    }
}

// The same read with S, P and O in registers (flash-attention form), one wave per (32 queries, stream,
// head); the tiled read of both head sizes. S^T = K Q^T on v_mfma_f32_32x32x2f32: A is 32 key rows x 2 dims (lane l:
// key l % 32, dim slot l / 32), B the wave's Q^T, loaded once; k-step s takes dims s (lanes 0..31) and
// HD/2 + s (lanes 32..63), so a lane's key and query operands are HD/2 contiguous dims of one row. The
// accumulator gives lane l query l % 32 and keys kappa(r, l / 32) = 8 (r / 4) + 4 (l / 32) + r % 4,
// r = 0..15: a query's 32 scores are two lanes' 16, and the online softmax's max and sum take one lane
// swap each. O^T += V^T P^T with the keys taken in the order kappa(t, 0), kappa(t, 1) at k-step t, so B
// is the lane's own P[t] and A is value dims read in place (lanes 0..31 one key row, 32..63 another:
// 128-byte rows). No LDS and no barrier; the next key tile's loads are in flight during each tile. The
// query blocks go heaviest (latest) first. Equal to the reference's two-pass softmax up to rounding.
template <typename KV, int N>
__device__ __forceinline__ void load_row(const KV *p, float (&x)[N]) {
    if constexpr (sizeof(KV) == 4) {
#pragma unroll
        for (int c = 0; c < N / 4; c++) {
            const f32x4 v = reinterpret_cast<const f32x4 *>(p)[c];
#pragma unroll
            for (int z = 0; z < 4; z++) x[4 * c + z] = v[z];
        }
    } else {
#pragma unroll
        for (int c = 0; c < N / 8; c++) {
            const uint4 u = reinterpret_cast<const uint4 *>(p)[c];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int z = 0; z < 4; z++) {
                const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&w[z]));
                x[8 * c + 2 * z] = f.x;
                x[8 * c + 2 * z + 1] = f.y;
            }
        }
    }
}
__device__ __forceinline__ float swap32max(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float swap32sum(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Buffer loads of the store (rows past the resource's range read 0).
template <typename KV>
__device__ __forceinline__ float kv_load(BufRes r, unsigned voff, unsigned soff) {
    if constexpr (sizeof(KV) == 4) {
        return load_f32(r, voff, soff);
    } else {
#if defined(__HIP_DEVICE_COMPILE__)
        const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
        return __half2float(__ushort_as_half(u));
#else
        return 0.0f;
#endif
    }
}
template <typename KV, int N>
__device__ __forceinline__ void kv_load_row(BufRes r, unsigned voff, float (&x)[N]) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef int i32x4_ __attribute__((ext_vector_type(4)));
    if constexpr (sizeof(KV) == 4) {
#pragma unroll
        for (int c = 0; c < N / 4; c++) {
            const i32x4_ v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(voff + 16 * c), 0, 0);
#pragma unroll
            for (int z = 0; z < 4; z++) x[4 * c + z] = __int_as_float(v[z]);
        }
    } else {
#pragma unroll
        for (int c = 0; c < N / 8; c++) {
            const i32x4_ v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(voff + 16 * c), 0, 0);
#pragma unroll
            for (int z = 0; z < 4; z++) {
                const unsigned w = (unsigned)v[z];
                const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&w));
                x[8 * c + 2 * z] = f.x;
                x[8 * c + 2 * z + 1] = f.y;
            }
        }
    }
#endif
}

template <typename KV, int HD>
__global__ __launch_bounds__(64, HD == 32 ? 4 : 2) void attend_fa_kernel(const float *__restrict__ q, int ldq,
                                                      const KV *__restrict__ ks, const KV *__restrict__ vs, int cap,
                                                      int n0, const int *n0p, int T, float scale, int de, int nh,
                                                      float *__restrict__ out) {
    static_assert(HD == 32 || HD == 64, "head size 32 or 64");
    constexpr int HH = HD / 2;   // dims per lane half in S^T's k-steps
    constexpr int NO = HD / 32;  // 32-dim tiles of O^T
    constexpr unsigned SZ = sizeof(KV);
    if (n0p) n0 = min(*n0p, cap - T);
    const int nqb = (T + 31) >> 5, nsh = (int)gridDim.x / nqb;
    // workgroups are dealt to the 8 XCDs round-robin: with (stream, head) pairs a multiple of 8, every
    // query block of a pair gets the same id mod 8, so one XCD's L2 holds the pair's keys and values
    const int L = (int)blockIdx.x;
    int sh, qi;
    if (nsh % 8 == 0) {
        sh = (L & 7) + 8 * ((L >> 3) / nqb);
        qi = (L >> 3) % nqb;
    } else {
        sh = L / nqb;
        qi = L % nqb;
    }
    const int qb = (nqb - 1 - qi) * 32;  // the latest (heaviest) query blocks first
    const int bi = sh / nh, hh = sh - bi * nh;
    const int lane = threadIdx.x, lq = lane & 31, h = lane >> 5;
    const float scale2 = scale * 1.44269504088896341f;  // scores in base-2 units (as attend_mfma_kernel)
    const int qrow = qb + lq;
    float qf[HH];
    load_row<float, HH>(q + ((size_t)bi * T + min(qrow, T - 1)) * ldq + hh * HD + HH * h, qf);
    const int qpos = n0 + qrow;                // this lane's store position
    const int kend = n0 + min(qb + 32, T);     // keys the block reads: 0 .. kend - 1
    const int kmax = n0 + T - 1;               // the store's last key
    const int nt = (kend + 31) >> 5;           // key tiles
    // the stream's rows 0 .. kmax of the store; lane offsets carry the head's dims
    const unsigned rowb = (unsigned)de * SZ, range = (unsigned)(kmax + 1) * rowb;
    const BufRes kr = buf_res((float *)(ks + (size_t)bi * cap * de), range);
    const BufRes vr = buf_res((float *)(vs + (size_t)bi * cap * de), range);
    const unsigned kcol = (unsigned)(hh * HD + HH * h) * SZ, vcol = (unsigned)(hh * HD + lq) * SZ;
    // K rows of tile k0: lane row k0 + lq (past kmax: zeros)
    auto fetchK = [&](int k0, float (&kx)[HH]) { kv_load_row<KV, HH>(kr, (unsigned)(k0 + lq) * rowb + kcol, kx); };
    // V of tile k0 in the order of the P V k-steps: t -> key k0 + 8 (t / 4) + 4 h + t % 4
    auto fetchV = [&](int k0, float (&vx)[NO][16]) {
        if (k0 + 31 <= kmax) {
            const unsigned vo = (unsigned)(k0 + 4 * h) * rowb + vcol;
#pragma unroll
            for (int t = 0; t < 16; t++)
#pragma unroll
                for (int u = 0; u < NO; u++)
                    vx[u][t] = kv_load<KV>(vr, vo + 32u * u * SZ, (unsigned)(8 * (t >> 2) + (t & 3)) * rowb);
        } else {  // the store's last tile: rows past kmax fall outside the resource and read 0
#pragma unroll
            for (int t = 0; t < 16; t++)
#pragma unroll
                for (int u = 0; u < NO; u++)
                    vx[u][t] = kv_load<KV>(vr, (unsigned)(k0 + 8 * (t >> 2) + 4 * h + (t & 3)) * rowb + vcol + 32u * u * SZ, 0u);
        }
    };
    auto scores = [&](const float (&kx)[HH]) {
        f32x16 sa = {};
#pragma unroll
        for (int s = 0; s < HH; s++) sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kx[s], qf[s], sa, 0, 0, 0);
        return sa;
    };
    float m = -INFINITY, den = 0.0f;
    f32x16 o[NO];
#pragma unroll
    for (int u = 0; u < NO; u++) o[u] = f32x16{};
    float kx[HH], vx[NO][16];
    // tile j's scores are formed during tile j - 1 (its softmax does not wait on them): the loop enters
    // each tile with its scores sc and the next tile's keys in kx
    fetchK(0, kx);
    fetchV(0, vx);
    f32x16 sc = scores(kx);
    if (nt > 1) fetchK(32, kx);
    for (int j = 0; j < nt; j++) {
        const int k0 = 32 * j;
        const bool more = j + 1 < nt;
        f32x16 sn = {};
        if (more) sn = scores(kx);
        if (j + 2 < nt) fetchK(k0 + 64, kx);
        const bool edge = k0 + 31 > n0 + qb;  // a key of the tile lies past the block's first query
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float x = sc[r] * scale2;
            if (edge && k0 + 8 * (r >> 2) + 4 * h + (r & 3) > qpos) x = -INFINITY;
            sc[r] = x;
            tmax = fmaxf(tmax, x);
        }
        tmax = swap32max(tmax);
        const float nm = fmaxf(m, tmax);
        const float corr = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - nm);
        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float e = (sc[r] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc[r] - nm);
            sc[r] = e;
            psum += e;
        }
        psum = swap32sum(psum);
        den = den * corr + psum;
        m = nm;
#pragma unroll
        for (int u = 0; u < NO; u++) {
#pragma unroll
            for (int r = 0; r < 16; r++) o[u][r] *= corr;
#pragma unroll
            for (int t = 0; t < 16; t++) o[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(vx[u][t], sc[t], o[u], 0, 0, 0);
        }
        if (more) fetchV(k0 + 32, vx);
        sc = sn;
    }
    if (qrow < T) {
        float *op = out + ((size_t)bi * T + qrow) * de + hh * HD + 4 * h;
#pragma unroll
        for (int u = 0; u < NO; u++)
#pragma unroll
            for (int a = 0; a < 4; a++) {
                f32x4 w;
#pragma unroll
                for (int z = 0; z < 4; z++) w[z] = o[u][4 * a + z] / den;
                *reinterpret_cast<f32x4 *>(op + 32 * u + 8 * a) = w;
            }
    }
}

// The decode form of the same read (flash-decoding), for a few queries per stream: query row
// (b, t) at store position n0 + t reads keys 0..n0 + t. Its keys are cut into chunks of ACH; workgroup
// (s, row) reads chunk s, each wave a quarter of it, 32 keys per iteration, 16 bytes per lane per
// load (attend_split_kernel's lane layout); the lanes of a key add their partial dot products by DPP,
// each lane group keeps its own running max, sum and output dims, and a workgroup's groups merge in
// LDS into one partial (max, sum, o[64]) per (row, chunk): part [row][nsplit][66]; attend_combine
// merges the chunks.
constexpr int ACH = 1024;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// The sum over the 16 lanes of each DPP row, in every lane (quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror).
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

// The sum over each group of 8 lanes (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror), in every lane.
__device__ __forceinline__ float row_sum8(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0x141>(v);
}

// The sum over each group of 4 lanes (quad_perm [1,0,3,2], [2,3,0,1]), in every lane.
__device__ __forceinline__ float row_sum4(float v) {
    v += dpp_f<0xB1>(v);
    return v + dpp_f<0x4E>(v);
}

// Lane layout: a key's HD dims are read by LPK = HD / DPL lanes (HD 64: 16 for f32, 8 for fp16; HD 32:
// 8 and 4), so a wave holds G = 64 / LPK key groups and reads G whole keys per 16-byte load
// instruction; each group takes U = 32 / G keys of a 32-key iteration (keys G j + group). Heads: the
// store's rows hold nh heads of HD dims; workgroup (s, row nh + h) reads head h of the row's query.
// part [row nh + h][nsplit][HD + 2].
template <typename KV, int HD>
__global__ __launch_bounds__(256) void attend_split_kernel(const float *__restrict__ q, int ldq,
                                                           const KV *__restrict__ ks, const KV *__restrict__ vs,
                                                           int cap, int n0, const int *n0p, int T, float scale,
                                                           int de, int nh, int nsplit, float *__restrict__ part) {
    if (n0p) n0 = min(*n0p, cap - T);  // the store length on the device: chunks past it are empty
    constexpr int DPL = KvLane<KV>::DPL, LPK = HD / DPL, G = 64 / LPK, U = 32 / G, NG = 4 * G;
    static_assert(LPK == 4 || LPK == 8 || LPK == 16, "lanes per key");
    __shared__ float sm[NG], sl[NG];
    __shared__ float so[NG][HD];
    const int s = blockIdx.x, rh = blockIdx.y, row = rh / nh, hh = rh - row * nh;
    const int b = row / T, t = row - b * T;
    const int klen = n0 + t + 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = lane / LPK, cl = (lane % LPK) * DPL;
    float qv[DPL];
#pragma unroll
    for (int z = 0; z < DPL; z++) qv[z] = q[(size_t)row * ldq + hh * HD + cl + z];
    const int kb = s * ACH + wave * (ACH / 4), ke = min(kb + ACH / 4, klen);
    const KV *kbase = ks + (size_t)b * cap * de + hh * HD + cl, *vbase = vs + (size_t)b * cap * de + hh * HD + cl;
    float m = -INFINITY, l = 0.0f, o[DPL];
#pragma unroll
    for (int z = 0; z < DPL; z++) o[z] = 0.0f;
    for (int k0 = kb; k0 < ke; k0 += 32) {
        float kv[U][DPL], vv[U][DPL];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const int kk = k0 + G * j + grp;
            if (kk < ke) {
                KvLane<KV>::load(kbase + (size_t)kk * de, kv[j]);
                KvLane<KV>::load(vbase + (size_t)kk * de, vv[j]);
            } else {
#pragma unroll
                for (int z = 0; z < DPL; z++) kv[j][z] = vv[j][z] = 0.0f;
            }
        }
        float sc[U], bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < U; j++) {
            float a = kv[j][0] * qv[0];
#pragma unroll
            for (int z = 1; z < DPL; z++) a = fmaf(kv[j][z], qv[z], a);
            a = (LPK == 16 ? row_sum16(a) : LPK == 8 ? row_sum8(a) : row_sum4(a)) * scale;
            sc[j] = (k0 + G * j + grp < ke) ? a : -INFINITY;
            bm = fmaxf(bm, sc[j]);
        }
        const float nm = fmaxf(m, bm);
        if (nm == -INFINITY) continue;  // no key of this group yet
        const float corr = expf(m - nm);  // m = -inf: 0
        l *= corr;
#pragma unroll
        for (int z = 0; z < DPL; z++) o[z] *= corr;
#pragma unroll
        for (int j = 0; j < U; j++) {
            const float p = expf(sc[j] - nm);  // -inf: 0
            l += p;
#pragma unroll
            for (int z = 0; z < DPL; z++) o[z] = fmaf(p, vv[j][z], o[z]);
        }
        m = nm;
    }
    const int gi = wave * G + grp;
    if (lane % LPK == 0) {
        sm[gi] = m;
        sl[gi] = l;
    }
#pragma unroll
    for (int z = 0; z < DPL; z++) so[gi][cl + z] = o[z];
    __syncthreads();
    if (threadIdx.x < HD) {
        const int c = threadIdx.x;
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < NG; i++) M = fmaxf(M, sm[i]);
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int i = 0; i < NG; i++) {
                const float w = sm[i] == -INFINITY ? 0.0f : expf(sm[i] - M);
                L = fmaf(sl[i], w, L);
                O = fmaf(so[i][c], w, O);
            }
        }
        float *pr = part + ((size_t)rh * nsplit + s) * (HD + 2);
        if (c == 0) {
            pr[0] = M;
            pr[1] = L;
        }
        pr[2 + c] = O;
    }
}

// out [row][h HD + c] = the merge of head h's chunk partials: M = max m_s, L = sum l_s e^(m_s - M),
// o = sum o_s e^(m_s - M) / L, the terms added in chunk order. Lane s takes chunk s's (m, l) and
// weight; every lane's o_s loads for 16 chunks are in flight together. Workgroup row nh + h.
// With P > 0 (one head of 64) the row's planes (quant_rows_kernel's, the next product's input) are
// written too, and with adv the store length on the device advances by T (store_advance_kernel's
// step: every reader of it in this forward, the store append and the chunk reads, ran before this
// kernel).
template <int P, int HD>
__global__ __launch_bounds__(64) void attend_combine_kernel(const float *__restrict__ part, int nsplit,
                                                            float *__restrict__ out, int8_t *__restrict__ xq,
                                                            int32_t *__restrict__ xexp, int ldq, int *adv, int T,
                                                            int cap, int de, int nh) {
    static_assert(P == 0 || HD == 64, "planes need one head of 64");
    constexpr int PS = HD + 2;
    const int rh = blockIdx.x, row = rh / nh, hh = rh - row * nh, c = threadIdx.x;
    const float *pr = part + (size_t)rh * nsplit * PS;
    float M = -INFINITY;
    for (int s0 = 0; s0 < nsplit; s0 += 64)
        if (s0 + c < nsplit) M = fmaxf(M, pr[(size_t)(s0 + c) * PS]);
    M = ava::wave_max(M);
    float L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += 64) {
        const int cnt = min(64, nsplit - s0);
        float ms = -INFINITY, ls = 0.0f;
        if (c < cnt) {
            ms = pr[(size_t)(s0 + c) * PS];
            ls = pr[(size_t)(s0 + c) * PS + 1];
        }
        const float w = ms == -INFINITY ? 0.0f : expf(ms - M);
        for (int j0 = 0; j0 < cnt; j0 += 16) {
            float ov[16];
#pragma unroll
            for (int j = 0; j < 16; j++)
                ov[j] = j0 + j < cnt && c < HD ? pr[(size_t)(s0 + j0 + j) * PS + 2 + c] : 0.0f;
            AVA_ISSUE_FENCE();
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int sj = j0 + j;
                if (sj >= cnt) break;
                if (__shfl(ms, sj) == -INFINITY) continue;
                const float wj = __shfl(w, sj);
                L = fmaf(__shfl(ls, sj), wj, L);
                O = fmaf(ov[j], wj, O);
            }
        }
    }
    const float o = O / L;
    if (c < HD) out[(size_t)row * de + hh * HD + c] = o;
    if constexpr (P > 0) {
        const int e = ava::plane_exp(ava::wave_max(fabsf(o)));
        if (c == 0) xexp[row] = e;
        int qv[P];
        ava::to_planes<P>(o, e, qv);
        const int nrows = gridDim.x;
#pragma unroll
        for (int p = 0; p < P; p++) {
            int8_t *qr = xq + ((size_t)p * nrows + row) * ldq;
            qr[c] = (int8_t)qv[p];
            for (int z = 64 + c; z < ldq; z += 64) qr[z] = 0;
        }
    }
    if (adv && rh == 0 && c == 0) *adv = min(*adv + T, cap);
}

// The device store length advances by T after a forward, saturating at the store's capacity (the
// host refuses forwards that would not fit; a replayed graph cannot ask, so this keeps it in bounds).
__global__ void store_advance_kernel(int *n0p, int T, int cap) {
    if (threadIdx.x == 0) *n0p = min(*n0p + T, cap);
}

// Append this forward's keys and values to the store: store[b][n0 + t] = kv[b T + t], de values each
// (keys at kv's columns 0..de-1, values at de..2de-1; n0 from the device when n0p).
template <typename KV>
__global__ void store_append_kernel(const float *__restrict__ kv, int ldkv, int T, int B, int cap, int n0,
                                    const int *n0p, int de, KV *__restrict__ ks, KV *__restrict__ vs) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // over B*T*de
    if (i >= B * T * de) return;
    if (n0p) n0 = min(*n0p, cap - T);
    const int row = i / de, c = i - row * de, bi = row / T, t = row - bi * T;
    const size_t dst = ((size_t)bi * cap + n0 + t) * de + c;
    kv_put(ks, dst, kv[(size_t)row * ldkv + c]);
    kv_put(vs, dst, kv[(size_t)row * ldkv + de + c]);
}

// ------------------------------------------------------------------ dense mix

// DenseFormer (gpu/arch.rs:1492-1500): stream[i+1] = x; x <- x + sum_{j <= i+1} w_j stream_j, the
// terms added one at a time in j order. The caller hands the block's output over as stream[i+1]
// itself (a buffer exchange on the host, not a copy), and the mixed rows go to a separate `x`.
struct DenseArgs {
    float *x;                    // out: the mixed rows
    const float *streams[17];    // streams[ns - 1]: the block's output (x before the mix)
    float w[17];
    int ns;  // i + 2 terms (the last is the block's output)
    size_t n4;
};

__global__ __launch_bounds__(256) void dense_mix_kernel(DenseArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n4) return;
    const f32x4 x = reinterpret_cast<const f32x4 *>(a.streams[a.ns - 1])[i];
    f32x4 mix = x;
    for (int j = 0; j < a.ns; j++) {
        const f32x4 s = j == a.ns - 1 ? x : reinterpret_cast<const f32x4 *>(a.streams[j])[i];
        const float w = a.w[j];
#pragma unroll
        for (int z = 0; z < 4; z++) mix[z] = mix[z] + s[z] * w;
    }
    reinterpret_cast<f32x4 *>(a.x)[i] = mix;
}

// The dense mix of whole rows (the same terms in the same order as dense_mix_kernel) followed by the
// next norm's planes of the mixed row (row_rms_planes): one wave per row, so the row is read once.
// The earlier streams go in batches of 4 with the loads of all the lane's chunks in flight together
// (a batch is one memory round trip, not one per chunk), non-temporal (each stream row is read once
// here and not again before the next block's mix: 5.67 -> 5.41 ms per config[3] forward; the same
// hint on the read-out's y and g loads, which the producers wrote just before, doubled its time).
template <int P, int NV>
__global__ __launch_bounds__(256) void dense_rms_kernel(DenseArgs a, int n, int d, const float *__restrict__ gain,
                                                        int8_t *__restrict__ xq, int32_t *__restrict__ xexp, int ldq,
                                                        float *__restrict__ hout) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= n) return;
    const int nq = d >> 2;
    const size_t base = (size_t)row * nq;
    f32x4 x[NV], v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = min(i * 64 + lane, nq - 1);
        x[i] = reinterpret_cast<const f32x4 *>(a.streams[a.ns - 1])[base + c];
        v[i] = x[i];
    }
    for (int j0 = 0; j0 < a.ns - 1; j0 += 4) {
        f32x4 sv[4][NV];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const f32x4 *sp = reinterpret_cast<const f32x4 *>(a.streams[min(j0 + q, a.ns - 2)]) + base;
#pragma unroll
            for (int i = 0; i < NV; i++) sv[q][i] = __builtin_nontemporal_load(sp + min(i * 64 + lane, nq - 1));
        }
        AVA_ISSUE_FENCE();
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (j0 + q < a.ns - 1) {
                const float w = a.w[j0 + q];
#pragma unroll
                for (int i = 0; i < NV; i++)
#pragma unroll
                    for (int z = 0; z < 4; z++) v[i][z] = v[i][z] + sv[q][i][z] * w;
            }
    }
    const float wl = a.w[a.ns - 1];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        if (c < nq) {
#pragma unroll
            for (int z = 0; z < 4; z++) v[i][z] = v[i][z] + x[i][z] * wl;
            __builtin_nontemporal_store(v[i], reinterpret_cast<f32x4 *>(a.x) + base + c);
        } else {
            v[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    row_rms_planes<P, NV>(v, lane, d, gain, (size_t)n, (size_t)row, xq, xexp, ldq, hout);
}

// The embedding rows (as embed_kernel) followed by the first block's norm planes.
template <int P, int NV>
__global__ __launch_bounds__(256) void embed_rms_kernel(const int32_t *__restrict__ ids, const float *__restrict__ emb,
                                                        int n, int d, int vocab, float *__restrict__ x,
                                                        float *__restrict__ x0, const float *__restrict__ gain,
                                                        int8_t *__restrict__ xq, int32_t *__restrict__ xexp, int ldq) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    int id = ids[row];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(emb + (size_t)id * d);
    f32x4 *dst = reinterpret_cast<f32x4 *>(x + (size_t)row * d);
    f32x4 *dst0 = x0 ? reinterpret_cast<f32x4 *>(x0 + (size_t)row * d) : nullptr;
    f32x4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = i * 64 + lane;
        if (c < (d >> 2)) {
            v[i] = src[c];
            dst[c] = v[i];
            if (dst0) dst0[c] = v[i];
        } else {
            v[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    row_rms_planes<P, NV>(v, lane, d, gain, (size_t)n, (size_t)row, xq, xexp, ldq, nullptr);
}

// ------------------------------------------------------------------ the least-read rule's counts
//
// gpu/memory.rs:700-738 (StoreUse::count_reads): after a read of T queries per stream, slot j of the
// store gets the attention mass of every query that sees it before its own key (the old slots j < n0,
// and new slot n0 + i for the queries after i), averaged over the heads, and its age (the number of
// later queries that could see it) advances: old slots by T, new slot n0 + i to T - 1 - i. The read
// kernels keep their softmax online and never form a probability, so the counts take two passes of
// their own: the max and the sum of each (query, head)'s scores, then each slot's mass. Scores are the
// oracle's: s = (q . k) with the dot product as one fma chain in dim order, times 1 / sqrt(hd).

template <class KV>
__device__ __forceinline__ float kv_at(const KV *p) {
    if constexpr (sizeof(KV) == 2) return __half2float(*reinterpret_cast<const __half *>(p));
    else return *reinterpret_cast<const float *>(p);
}

template <class KV>
__device__ __forceinline__ float eng_score(const float *qr, const KV *kr, int hd) {
    float s = kv_at(kr) * qr[0];
    for (int a = 1; a < hd; a++) s = fmaf(kv_at(kr + a), qr[a], s);
    return s;
}

// One wave per (query row b T + t, head h): ml[2 w] = max_j s_j, ml[2 w + 1] = sum_j exp(s_j - max) over
// the slots 0..n0 + t.
template <class KV>
__global__ __launch_bounds__(256) void engram_ml_kernel(const float *__restrict__ q, int ldq, const KV *__restrict__ ks,
                                                        int cap, int de, int hd, int nh, int B, int T, int n0,
                                                        float scale, float *__restrict__ ml) {
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (w >= B * T * nh) return;
    const int row = w / nh, h = w - row * nh, b = row / T, t = row - b * T, n = n0 + t + 1;
    const float *qr = q + (size_t)row * ldq + h * hd;
    const KV *kb = ks + (size_t)b * cap * de + h * hd;
    float mx = -INFINITY;
    for (int j = lane; j < n; j += 64) mx = fmaxf(mx, eng_score(qr, kb + (size_t)j * de, hd) * scale + 0.0f);
    mx = ava::wave_max(mx);
    float l = 0.0f;
    for (int j = lane; j < n; j += 64) l += expf((eng_score(qr, kb + (size_t)j * de, hd) * scale + 0.0f) - mx);
    l = ava::wave_sum(l);
    if (lane == 0) {
        ml[2 * w] = mx;
        ml[2 * w + 1] = l;
    }
}

// One thread per (stream b, slot j < n0 + T): the mass from the queries that see j before their own
// key, summed over queries within each head and then over heads, times 1 / nh; then the counts.
template <class KV>
__global__ __launch_bounds__(256) void engram_got_kernel(const float *__restrict__ q, int ldq, const KV *__restrict__ ks,
                                                         int cap, int de, int hd, int nh, int T, int n0, float scale,
                                                         const float *__restrict__ ml, float *__restrict__ reads,
                                                         float *__restrict__ age) {
    const int b = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n0 + T) return;
    const KV *kr = ks + ((size_t)b * cap + j) * de;
    const int t0 = j < n0 ? 0 : j - n0 + 1;  // the first query that sees j before its own key
    float got = 0.0f;
    for (int h = 0; h < nh; h++) {
        float acc = 0.0f;
        for (int t = t0; t < T; t++) {
            const size_t row = (size_t)b * T + t, w = row * nh + h;
            const float s = eng_score(q + row * ldq + h * hd, kr + h * hd, hd) * scale + 0.0f;
            acc += expf(s - ml[2 * w]) / ml[2 * w + 1];
        }
        got += acc;
    }
    got = got * (1.0f / (float)nh);
    float *rd = reads + (size_t)b * cap, *ag = age + (size_t)b * cap;
    if (j < n0) {
        rd[j] = rd[j] + got;
        ag[j] = ag[j] + (float)T;
    } else {
        rd[j] = 0.0f + got;
        ag[j] = (float)(T - 1 - (j - n0));
    }
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

// Few rows (decode): 4 rows per workgroup on the VALU, 1024 threads. Thread t takes column t % 128
// over the K eighth t / 128, with the rows' inputs staged in LDS and 32 weight loads in flight (an L2
// round trip is ~0.5 us, so the loop is load-latency bound); the eighths add in order at the end.
constexpr int GRR = 4, GKS = 8;
__global__ __launch_bounds__(1024) void gate_rows_kernel(const float *__restrict__ h, int n, int d,
                                                         const float *__restrict__ w, int nc, float *__restrict__ g) {
    __shared__ float sh[GRR][1024];
    __shared__ float sacc[GKS][GRR][128];
    const int tid = threadIdx.x, c = tid & 127, ks = tid >> 7, r0 = blockIdx.x * GRR;
    for (int i = tid; i < GRR * d; i += 1024) {
        const int r = i / d, k = i - r * d;
        sh[r][k] = r0 + r < n ? h[(size_t)(r0 + r) * d + k] : 0.0f;
    }
    __syncthreads();
    float acc[GRR] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (c < nc) {
        const int kb = ks * (d / GKS), ke = kb + d / GKS;  // (ke - kb) % 32 == 0 (launcher)
        for (int k0 = kb; k0 < ke; k0 += 32) {
            float wv[32];  // the 32 loads are issued before any is used
#pragma unroll
            for (int j = 0; j < 32; j++) wv[j] = w[(size_t)(k0 + j) * nc + c];
            AVA_ISSUE_FENCE();
#pragma unroll
            for (int j = 0; j < 32; j++)
#pragma unroll
                for (int r = 0; r < GRR; r++) acc[r] = fmaf(sh[r][k0 + j], wv[j], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < GRR; r++) sacc[ks][r][c] = acc[r];
    __syncthreads();
    if (tid < GRR * 128) {
        const int r = tid >> 7;
        if (c < nc && r0 + r < n) {
            float v = sacc[0][r][c];
#pragma unroll
            for (int q = 1; q < GKS; q++) v += sacc[q][r][c];
            g[(size_t)(r0 + r) * nc + c] = v;
        }
    }
}

// The norm of 4 rows (waves 0..3, one row each, as rms_planes_kernel: planes to xq) and then, from
// the normed rows kept in LDS, their gate projections (all 16 waves, as gate_rows_kernel): for few
// rows, one launch instead of two and no round trip of h.
template <int P, int RR>  // RR rows per workgroup (1: the most workgroups, for the fewest rows)
__global__ __launch_bounds__(1024) void rms_gate_kernel(const float *__restrict__ x, int n, int d,
                                                        const float *__restrict__ gain, int8_t *__restrict__ xq,
                                                        int32_t *__restrict__ xexp, int ldq,
                                                        const float *__restrict__ w, int nc, float *__restrict__ g) {
    __shared__ __attribute__((aligned(16))) float sh[RR][1024];
    __shared__ float sacc[GKS][RR][128];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r0 = blockIdx.x * RR;
    if (wave < RR) {
        const int row = r0 + wave, nq = d >> 2;
        f32x4 v[4];
        if (row < n) {
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + (size_t)row * d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = i * 64 + lane;
                v[i] = c < nq ? xr[c] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            row_rms_planes<P, 4>(v, lane, d, gain, (size_t)n, (size_t)row, xq, xexp, ldq, nullptr);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = i * 64 + lane;
            if (c < nq) *reinterpret_cast<f32x4 *>(&sh[wave][4 * c]) = v[i];
        }
    }
    __syncthreads();
    const int c = tid & 127, ks = tid >> 7;
    float acc[RR];
#pragma unroll
    for (int r = 0; r < RR; r++) acc[r] = 0.0f;
    if (c < nc) {
        const int kb = ks * (d / GKS), ke = kb + d / GKS;
        for (int k0 = kb; k0 < ke; k0 += 32) {
            float wv[32];
#pragma unroll
            for (int j = 0; j < 32; j++) wv[j] = w[(size_t)(k0 + j) * nc + c];
            AVA_ISSUE_FENCE();
#pragma unroll
            for (int j = 0; j < 32; j++)
#pragma unroll
                for (int r = 0; r < RR; r++) acc[r] = fmaf(sh[r][k0 + j], wv[j], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RR; r++) sacc[ks][r][c] = acc[r];
    __syncthreads();
    if (tid < RR * 128) {
        const int r = tid >> 7;
        if (c < nc && r0 + r < n) {
            float v = sacc[0][r][c];
#pragma unroll
            for (int q = 1; q < GKS; q++) v += sacc[q][r][c];
            g[(size_t)(r0 + r) * nc + c] = v;
        }
    }
}

// Few rows: workgroup (8 rows, 16 gate columns), so a workgroup reads 64 KB of W instead of all of it.
// Every workgroup norms its 8 rows (two per wave, as rms_planes_kernel) into LDS; those of column group
// 0 also write the planes. Thread (row half, K eighth, column) then forms 4 rows' partial sums over its
// eighth with all its weight loads in flight, and the eighths add in order: the same operations in the
// same order as rms_gate_kernel, so the same bits.
constexpr int GCR = 8, GCC = 16;
template <int P>
__global__ __launch_bounds__(256) void rms_gate_cols_kernel(const float *__restrict__ x, int n, int d,
                                                            const float *__restrict__ gain, int8_t *__restrict__ xq,
                                                            int32_t *__restrict__ xexp, int ldq,
                                                            const float *__restrict__ w, int nc, float *__restrict__ g) {
    // the K eighths of a row sit 4 floats apart in banks, so a wave's four eighths read without conflict
    __shared__ __attribute__((aligned(16))) float sh[GCR][1024 + 4 * GKS];
    auto at = [](int k) { return k + (k >> 7) * 4; };
    __shared__ float sacc[GKS][GCR][GCC];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * GCR, c0 = blockIdx.y * GCC, nq = d >> 2;
    {
        f32x4 v[2][4];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = r0 + 2 * wave + h;
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + (size_t)min(row, n - 1) * d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = i * 64 + lane;
                v[h][i] = c < nq && row < n ? xr[c] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        AVA_ISSUE_FENCE();
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int rl = 2 * wave + h, row = r0 + rl;
            if (row < n)
                row_rms_planes<P, 4>(v[h], lane, d, gain, (size_t)n, (size_t)row, blockIdx.y == 0 ? xq : nullptr,
                                     xexp, ldq, nullptr);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = i * 64 + lane;
                if (c < nq) *reinterpret_cast<f32x4 *>(&sh[rl][at(4 * c)]) = v[h][i];
            }
        }
    }
    __syncthreads();
    const int cl = tid & (GCC - 1), ks = (tid >> 4) & (GKS - 1), rh = tid >> 7, c = c0 + cl;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (c < nc) {
        const int kb = ks * (d / GKS), ke = kb + d / GKS;  // (ke - kb) % 32 == 0 (rms_gate_fits)
        // 32 weights per step; the next step's 32 are in flight while this step's are used
        float wv[32], wn[32];
#pragma unroll
        for (int j = 0; j < 32; j++) wv[j] = w[(size_t)(kb + j) * nc + c];
        for (int k0 = kb; k0 < ke; k0 += 32) {
            if (k0 + 32 < ke) {
#pragma unroll
                for (int j = 0; j < 32; j++) wn[j] = w[(size_t)(k0 + 32 + j) * nc + c];
            }
            AVA_ISSUE_FENCE();
#pragma unroll
            for (int h = 0; h < 2; h++) {
                // the 4 rows' 16 inputs as float4 LDS reads, all issued before the first fma
                f32x4 hv[4][4];
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        hv[r][q] = *reinterpret_cast<const f32x4 *>(&sh[rh * 4 + r][at(k0 + 16 * h + 4 * q)]);
#pragma unroll
                for (int j = 0; j < 16; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[r] = fmaf(hv[r][j >> 2][j & 3], wv[16 * h + j], acc[r]);
            }
#pragma unroll
            for (int j = 0; j < 32; j++) wv[j] = wn[j];
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) sacc[ks][rh * 4 + r][cl] = acc[r];
    __syncthreads();
    if (tid < GCR * GCC) {
        const int r = tid / GCC, cc = tid % GCC, row = r0 + r;
        if (c0 + cc < nc && row < n) {
            float v = sacc[0][r][cc];
#pragma unroll
            for (int q = 1; q < GKS; q++) v += sacc[q][r][cc];
            g[(size_t)row * nc + c0 + cc] = v;
        }
    }
}

bool rms_gate_fits(int n, int d, int nc) {
    return ceil_div(n, GR) < 64 && d <= 1024 && d % (GKS * 32) == 0 && nc <= 128;
}

int rms_gate(const float *x, int n, int d, const float *gain, int planes, int8_t *xq, int32_t *xexp, int ldq,
             const float *w, int nc, float *g, hipStream_t st) {
    AVA_REQUIRE(rms_gate_fits(n, d, nc) && ldq >= d && ldq % 4 == 0, AVA_ERR_SHAPE, "rms_gate: n=%d d=%d nc=%d", n,
                d, nc);
    // (8 rows, 16 columns) per workgroup while that still fills the chip with a few rounds, else four
    // rows and all columns
    const bool cols = n <= 1024;
    const dim3 grid(ceil_div(n, GRR)), block(1024), cgrid(ceil_div(n, GCR), ceil_div(nc, GCC));
#define AVA_RG(P_)                                                                                            \
    if (cols) rms_gate_cols_kernel<P_><<<cgrid, 256, 0, st>>>(x, n, d, gain, xq, xexp, ldq, w, nc, g);        \
    else rms_gate_kernel<P_, GRR><<<grid, block, 0, st>>>(x, n, d, gain, xq, xexp, ldq, w, nc, g)
    if (planes == 1) AVA_RG(1);
    else if (planes == 2) AVA_RG(2);
    else AVA_RG(3);
#undef AVA_RG
    AVA_LAUNCHED("rms_gate");
    return AVA_OK;
}

// From 512 blocks of rows (two per CU) the one launch beats the two (131,072 rows: 430 against 520 us);
// with fewer, its norms run on too few workgroups.
bool rms_gate_many_fits(int n, int d, int nc) { return n >= 512 * GR && d == 1024 && nc > 0 && nc <= 96; }

int rms_gate_many(const float *x, int n, int d, const float *gain, int planes, int8_t *xq, int32_t *xexp, int ldq,
                  const float *w, int nc, float *g, hipStream_t st) {
    AVA_REQUIRE(rms_gate_many_fits(n, d, nc) && ldq >= d && ldq % 4 == 0, AVA_ERR_SHAPE,
                "rms_gate_many: n=%d d=%d nc=%d", n, d, nc);
    const int blocks = ceil_div(n, GR);
#define AVA_RGM(P_, C_) rms_gate_mfma_kernel<P_, C_><<<blocks, 256, 0, st>>>(x, n, gain, xq, xexp, ldq, w, nc, g)
#define AVA_RGMP(P_)                                  \
    switch ((nc + 31) / 32) {                         \
    case 1: AVA_RGM(P_, 1); break;                    \
    case 2: AVA_RGM(P_, 2); break;                    \
    default: AVA_RGM(P_, 3); break;                   \
    }
    if (planes == 1) AVA_RGMP(1)
    else if (planes == 2) AVA_RGMP(2)
    else AVA_RGMP(3)
#undef AVA_RGMP
#undef AVA_RGM
    AVA_LAUNCHED("rms_gate_many");
    return AVA_OK;
}

int gate_gemm(const float *h, int n, int d, const float *w, int nc, float *g, hipStream_t st) {
    AVA_REQUIRE(nc > 0 && nc <= 128 && d % GK == 0, AVA_ERR_SHAPE, "gate_gemm: %d columns (<= 128), d=%d", nc, d);
    const int blocks = ceil_div(n, GR);
    if (blocks < 64 && d <= 1024 && d % (GKS * 32) == 0) {
        gate_rows_kernel<<<ceil_div(n, GRR), 1024, 0, st>>>(h, n, d, w, nc, g);
        AVA_LAUNCHED("gate_gemm");
        return AVA_OK;
    }
    switch ((nc + 31) / 32) {
    case 1: gate_mfma_kernel<1><<<blocks, 256, 0, st>>>(h, n, d, w, nc, g); break;
    case 2: gate_mfma_kernel<2><<<blocks, 256, 0, st>>>(h, n, d, w, nc, g); break;
    case 3: gate_mfma_kernel<3><<<blocks, 256, 0, st>>>(h, n, d, w, nc, g); break;
    default: gate_mfma_kernel<4><<<blocks, 256, 0, st>>>(h, n, d, w, nc, g); break;
    }
    AVA_LAUNCHED("gate_gemm");
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

size_t engram_split_floats(int B, int T, int n0, int de, int nh) {
    const int hd = de / (nh > 0 ? nh : 1);
    return T <= ENGRAM_SPLIT_T ? (size_t)B * T * nh * ceil_div(n0 + T, ACH) * (hd + 2) : 0;
}

// With n0p (the store length on the device) the chunk grid covers the whole store, so a captured
// launch serves every length; chunks past the length are empty and merge as nothing.
template <typename KV, int HD>
int attend_t(const float *q, int ldq, const KV *ks, const KV *vs, int cap, int n0, const int *n0p, int B, int T,
             int de, int nh, float *out, float *part, size_t part_floats, const PostRead &post, hipStream_t st) {
    const float scale = (float)(1.0 / sqrt((double)HD));
    if (T <= ENGRAM_SPLIT_T) {
        const int span = n0p ? cap - T : n0;
        const int nsplit = ceil_div(span + T, ACH);
        const size_t need = engram_split_floats(B, T, span, de, nh);
        AVA_REQUIRE(part && part_floats >= need, AVA_ERR_ARG, "attend: the decode read needs %zu floats of partials",
                    need);
        attend_split_kernel<KV, HD><<<dim3(nsplit, B * T * nh), 256, 0, st>>>(q, ldq, ks, vs, cap, n0, n0p, T, scale,
                                                                              de, nh, nsplit, part);
        AVA_LAUNCHED("attend_split");
        if constexpr (HD == 64) {
#define AVA_AC(P_)                                                                                                 \
    attend_combine_kernel<P_, 64><<<B * T * nh, 64, 0, st>>>(part, nsplit, out, post.xq, post.xexp, post.ldq, post.adv, \
                                                             T, cap, de, nh)
            if (!post.xq) AVA_AC(0);
            else if (post.planes == 1) AVA_AC(1);
            else if (post.planes == 2) AVA_AC(2);
            else AVA_AC(3);
#undef AVA_AC
        } else {
            attend_combine_kernel<0, HD><<<B * T * nh, 64, 0, st>>>(part, nsplit, out, nullptr, nullptr, 0, post.adv, T,
                                                                     cap, de, nh);
        }
        AVA_LAUNCHED("attend_combine");
        return AVA_OK;
    }
    // the register-resident form (AVA_ATTEND_FA=0: the LDS-tiled one)
    static const bool fa = !(getenv("AVA_ATTEND_FA") && atoi(getenv("AVA_ATTEND_FA")) == 0);
    bool done = false;
    {
        // the buffer resources' byte offsets are 32-bit
        if (fa && (size_t)cap * de * sizeof(KV) < (1ull << 31)) {
            attend_fa_kernel<KV, HD><<<ceil_div(T, 32) * B * nh, 64, 0, st>>>(q, ldq, ks, vs, cap, n0, n0p, T, scale,
                                                                               de, nh, out);
            done = true;
        }
    }
    if (!done) {
        dim3 grid(ceil_div(T, 64), B * nh);
        attend_mfma_kernel<KV, HD><<<grid, 256, 0, st>>>(q, ldq, ks, vs, cap, n0, n0p, T, scale, de, nh, out);
    }
    AVA_LAUNCHED("attend");
    return AVA_OK;
}

int attend(const float *q, int ldq, const void *ks, const void *vs, int kv_half, int cap, int n0, const int *n0p,
           int B, int T, int de, int nh, float *out, float *part, size_t part_floats, hipStream_t st,
           const PostRead &post) {
    AVA_REQUIRE(B > 0 && T > 0 && n0 >= 0 && n0 + T <= cap, AVA_ERR_SHAPE,
                "attend: B=%d T=%d, a store of %d entries holds %d + %d", B, T, cap, n0, T);
    AVA_REQUIRE(nh >= 1 && de % nh == 0 && (de / nh == 32 || de / nh == 64) && de % 64 == 0 && de <= 4096,
                AVA_ERR_SHAPE, "attend: %d dims in %d heads (heads of 32 or 64, a multiple of 64 dims)", de, nh);
    AVA_REQUIRE(ldq >= de && ldq % 4 == 0, AVA_ERR_SHAPE, "attend: ldq %d for %d dims", ldq, de);
    AVA_REQUIRE(!post.xq || (nh == 1 && de == 64 && post.planes >= 1 && post.planes <= 3 && post.ldq >= 64 &&
                             post.ldq % 64 == 0),
                AVA_ERR_ARG, "attend: planes %d, ldq %d (planes: one head of 64)", post.planes, post.ldq);
    const bool h32 = de / nh == 32;
    if (kv_half) {
        const __half *k = (const __half *)ks, *v = (const __half *)vs;
        return h32 ? attend_t<__half, 32>(q, ldq, k, v, cap, n0, n0p, B, T, de, nh, out, part, part_floats, post, st)
                   : attend_t<__half, 64>(q, ldq, k, v, cap, n0, n0p, B, T, de, nh, out, part, part_floats, post, st);
    }
    const float *k = (const float *)ks, *v = (const float *)vs;
    return h32 ? attend_t<float, 32>(q, ldq, k, v, cap, n0, n0p, B, T, de, nh, out, part, part_floats, post, st)
               : attend_t<float, 64>(q, ldq, k, v, cap, n0, n0p, B, T, de, nh, out, part, part_floats, post, st);
}

int engram_read(const float *qkv, int ldqkv, int B, int T, int de, int nh, void *ks, void *vs, int kv_half, int cap,
                int n0, int *n0p, float *out, float *part, size_t part_floats, hipStream_t st, const PostRead &post) {
    AVA_REQUIRE(n0 + T <= cap, AVA_ERR_SHAPE, "engram: store of %d entries holds %d + %d", cap, n0, T);
    AVA_REQUIRE(ldqkv >= 3 * de, AVA_ERR_SHAPE, "engram: ldqkv %d for %d dims", ldqkv, de);
    const int total = B * T * de;
    if (kv_half)
        store_append_kernel<__half><<<ceil_div(total, 256), 256, 0, st>>>(qkv + de, ldqkv, T, B, cap, n0, n0p, de,
                                                                           (__half *)ks, (__half *)vs);
    else
        store_append_kernel<float><<<ceil_div(total, 256), 256, 0, st>>>(qkv + de, ldqkv, T, B, cap, n0, n0p, de,
                                                                          (float *)ks, (float *)vs);
    AVA_LAUNCHED("store_append");
    return attend(qkv, ldqkv, ks, vs, kv_half, cap, n0, n0p, B, T, de, nh, out, part, part_floats, st, post);
}

int engram_advance(int *n0p, int T, int cap, hipStream_t st) {
    store_advance_kernel<<<1, 64, 0, st>>>(n0p, T, cap);
    AVA_LAUNCHED("store_advance");
    return AVA_OK;
}

int engram_count(const float *q, int ldq, const void *ks, int kv_half, int cap, int n0, int B, int T, int de, int nh,
                 float *ml, float *reads, float *age, hipStream_t st) {
    AVA_REQUIRE(q && ks && ml && reads && age, AVA_ERR_ARG, "engram_count: NULL buffer");
    AVA_REQUIRE(B > 0 && T > 0 && nh > 0 && de % nh == 0 && n0 >= 0 && n0 + T <= cap, AVA_ERR_SHAPE,
                "engram_count: B=%d T=%d n0=%d cap=%d de=%d heads=%d", B, T, n0, cap, de, nh);
    const int hd = de / nh;
    const float scale = (float)(1.0 / sqrt((double)hd));
    const int waves = B * T * nh;
    if (kv_half) {
        engram_ml_kernel<__half><<<ceil_div(waves, 4), 256, 0, st>>>(q, ldq, (const __half *)ks, cap, de, hd, nh, B, T,
                                                                    n0, scale, ml);
        engram_got_kernel<__half><<<dim3(ceil_div(n0 + T, 256), B), 256, 0, st>>>(
            q, ldq, (const __half *)ks, cap, de, hd, nh, T, n0, scale, ml, reads, age);
    } else {
        engram_ml_kernel<float><<<ceil_div(waves, 4), 256, 0, st>>>(q, ldq, (const float *)ks, cap, de, hd, nh, B, T, n0,
                                                                   scale, ml);
        engram_got_kernel<float><<<dim3(ceil_div(n0 + T, 256), B), 256, 0, st>>>(
            q, ldq, (const float *)ks, cap, de, hd, nh, T, n0, scale, ml, reads, age);
    }
    AVA_LAUNCHED("engram_count");
    return AVA_OK;
}

int dense_rms(float *x, float *const *streams, const float *w, int ns, int n, int d, const float *gain, int planes,
              int8_t *xq, int32_t *xexp, int ldq, float *hout, hipStream_t st) {
    AVA_REQUIRE(ns >= 2 && ns <= 17 && d % 4 == 0 && d <= 1024 && ldq >= d && ldq % 4 == 0, AVA_ERR_SHAPE,
                "dense_rms: %d streams, d=%d", ns, d);
    for (int j = 0; j < ns; j++) AVA_REQUIRE(streams[j] != x, AVA_ERR_ARG, "dense_rms: x is stream %d", j);
    DenseArgs a;
    a.x = x;
    for (int j = 0; j < ns; j++) {
        a.streams[j] = streams[j];
        a.w[j] = w[j];
    }
    a.ns = ns;
    a.n4 = (size_t)n * d / 4;
    // few rows: one wave per workgroup, so the rows spread over more CUs
    const int rpb = n <= 1024 ? 1 : 4;
    const dim3 grid(ceil_div(n, rpb)), block(64 * rpb);
    if (planes == 1) dense_rms_kernel<1, 4><<<grid, block, 0, st>>>(a, n, d, gain, xq, xexp, ldq, hout);
    else if (planes == 2) dense_rms_kernel<2, 4><<<grid, block, 0, st>>>(a, n, d, gain, xq, xexp, ldq, hout);
    else dense_rms_kernel<3, 4><<<grid, block, 0, st>>>(a, n, d, gain, xq, xexp, ldq, hout);
    AVA_LAUNCHED("dense_rms");
    return AVA_OK;
}

int embed_rms(const int32_t *ids, const float *emb, int n, int d, int vocab, float *x, float *x0, const float *gain,
              int planes, int8_t *xq, int32_t *xexp, int ldq, hipStream_t st) {
    AVA_REQUIRE(d % 4 == 0 && d <= 1024 && ldq >= d && ldq % 4 == 0, AVA_ERR_SHAPE, "embed_rms: d=%d", d);
    const dim3 grid(ceil_div(n, 4)), block(256);
    if (planes == 1) embed_rms_kernel<1, 4><<<grid, block, 0, st>>>(ids, emb, n, d, vocab, x, x0, gain, xq, xexp, ldq);
    else if (planes == 2) embed_rms_kernel<2, 4><<<grid, block, 0, st>>>(ids, emb, n, d, vocab, x, x0, gain, xq, xexp, ldq);
    else embed_rms_kernel<3, 4><<<grid, block, 0, st>>>(ids, emb, n, d, vocab, x, x0, gain, xq, xexp, ldq);
    AVA_LAUNCHED("embed_rms");
    return AVA_OK;
}

int dense_mix(float *x, float *const *streams, const float *w, int ns, size_t n, hipStream_t st) {
    AVA_REQUIRE(ns >= 2 && ns <= 17 && n % 4 == 0, AVA_ERR_SHAPE, "dense_mix: %d streams", ns);
    for (int j = 0; j < ns; j++) AVA_REQUIRE(streams[j] != x, AVA_ERR_ARG, "dense_mix: x is stream %d", j);
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

extern "C" size_t ava_attend_part_floats(int B, int T, int n0) { return ava::engram_split_floats(B, T, n0); }

extern "C" int ava_attend(const float *q, int ldq, const void *ks, const void *vs, int kv_half, int cap, int n0, int B,
                          int T, float *out, float *part, size_t part_floats, ava_stream stream) {
    AVA_REQUIRE(q && ks && vs && out, AVA_ERR_ARG, "attend: NULL argument");
    return ava::attend(q, ldq, ks, vs, kv_half, cap, n0, nullptr, B, T, 64, 1, out, part, part_floats,
                       (hipStream_t)stream);
}

extern "C" size_t ava_attend_heads_part_floats(int B, int T, int n0, int de, int heads) {
    return heads >= 1 ? ava::engram_split_floats(B, T, n0, de, heads) : 0;
}

extern "C" int ava_attend_heads(const float *q, int ldq, const void *ks, const void *vs, int kv_half, int cap, int n0,
                                int B, int T, int de, int heads, float *out, float *part, size_t part_floats,
                                ava_stream stream) {
    AVA_REQUIRE(q && ks && vs && out, AVA_ERR_ARG, "attend_heads: NULL argument");
    return ava::attend(q, ldq, ks, vs, kv_half, cap, n0, nullptr, B, T, de, heads, out, part, part_floats,
                       (hipStream_t)stream);
}
