// The gradients around the scans for gfx950: the kWTA-relu² backward and the dense (DenseFormer)
// mix backward. Both are streams over HBM; every lane moves 16-byte vectors.
#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// kWTA then relu²: a = relu(u) where u - kth >= 0 (ties kept), out = a². Its backward (candle's sqr
// backward through the mask, gpu/lif.cu:4666-4679): gu = (a ga) 2 where a > 0, else 0, with a = u on
// the kept units. The mask is re-formed from u and the row's kth (the forward's own compare), so
// the forward keeps no copy of a.
__global__ __launch_bounds__(256) void relu2_bwd_kernel(const float *__restrict__ u, const float *__restrict__ kth,
                                                        const float *__restrict__ ga, float *__restrict__ gu, int h4,
                                                        size_t n4) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float th = kth[i / h4];
    const f32x4 x = reinterpret_cast<const f32x4 *>(u)[i];
    const f32x4 g = reinterpret_cast<const f32x4 *>(ga)[i];
    f32x4 o;
#pragma unroll
    for (int z = 0; z < 4; z++) o[z] = (x[z] - th >= 0.0f && x[z] > 0.0f) ? (x[z] * g[z]) * 2.0f : 0.0f;
    reinterpret_cast<f32x4 *>(gu)[i] = o;
}

// The dense mix of block i, mix_i = raw_i + sum_{j <= i + 1} w_ij S_j, has the backward
//   dL/dS_c  = base + sum_{k = i0 .. L-1} w_k[c] G_k   (G_k = dL/d(the mix after block k), base = the
//              gradient that reaches S_c directly),
//   dL/dw_ij = <G_i, S_j>  (a dot product over all rows and channels).
// wf holds block k's k + 2 weights from offset k (k + 3) / 2.
//
// One workgroup owns a chunk of DB_CHUNK consecutive floats. It loads its chunk of `base` into
// registers once and uses it twice: as the start of the gradient sum (the G_k streamed through, each
// term rounded in block order, so the sum has the oracle's bits), and as the left operand of the nd
// dot products, each of which streams one S_j chunk through and leaves one partial per (j, chunk).
// The partials are stored j-major (part[j][chunk]) and reduced by one wave per j in a fixed order,
// so dw does not depend on scheduling.
constexpr int DB_THREADS = 256, DB_PER_THREAD = 4;  // f32x4 vectors per thread
constexpr int DB_CHUNK4 = DB_THREADS * DB_PER_THREAD;  // f32x4 vectors per workgroup
constexpr int DB_MAXD = 32;

struct DenseBackArgs {
    const float *S, *G, *wf, *base;
    float *out, *part;
    int col, i0, L, nd, nchunk;
    size_t M4;
};

__global__ __launch_bounds__(DB_THREADS) void dense_grad_kernel(DenseBackArgs a) {
    __shared__ float wsum[DB_MAXD][DB_THREADS / 64];
    const size_t M = a.M4 * 4;
    const size_t c0 = (size_t)blockIdx.x * DB_CHUNK4;
    f32x4 bs[DB_PER_THREAD];
    bool in[DB_PER_THREAD];
#pragma unroll
    for (int r = 0; r < DB_PER_THREAD; r++) {
        const size_t i = c0 + r * DB_THREADS + threadIdx.x;
        in[r] = i < a.M4;
        bs[r] = in[r] ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.base) + i) : f32x4{0, 0, 0, 0};
    }
    // the gradient into stream `col`, block terms in order
    f32x4 acc[DB_PER_THREAD];
#pragma unroll
    for (int r = 0; r < DB_PER_THREAD; r++) acc[r] = bs[r];
    for (int k = a.i0; k < a.L; k++) {
        const float w = a.wf[k * (k + 3) / 2 + a.col];
        const f32x4 *gk = reinterpret_cast<const f32x4 *>(a.G + (size_t)k * M);
        f32x4 g[DB_PER_THREAD];
#pragma unroll
        for (int r = 0; r < DB_PER_THREAD; r++)
            g[r] = in[r] ? __builtin_nontemporal_load(gk + c0 + r * DB_THREADS + threadIdx.x) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < DB_PER_THREAD; r++)
#pragma unroll
            for (int z = 0; z < 4; z++) acc[r][z] = acc[r][z] + w * g[r][z];
    }
#pragma unroll
    for (int r = 0; r < DB_PER_THREAD; r++)
        if (in[r]) __builtin_nontemporal_store(acc[r], reinterpret_cast<f32x4 *>(a.out) + c0 + r * DB_THREADS + threadIdx.x);
    if (a.nd == 0) return;
    // the weight gradients: <base, S_j> over this chunk, one j at a time
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int j = 0; j < a.nd; j++) {
        const f32x4 *sj = reinterpret_cast<const f32x4 *>(a.S + (size_t)j * M);
        float d = 0.0f;
#pragma unroll
        for (int r = 0; r < DB_PER_THREAD; r++) {
            const f32x4 s = in[r] ? __builtin_nontemporal_load(sj + c0 + r * DB_THREADS + threadIdx.x) : f32x4{0, 0, 0, 0};
#pragma unroll
            for (int z = 0; z < 4; z++) d = fmaf(bs[r][z], s[z], d);
        }
        d = ava::wave_sum(d);
        if (lane == 0) wsum[j][wv] = d;
    }
    __syncthreads();
    if ((int)threadIdx.x < a.nd) {
        const int j = threadIdx.x;
        float s = wsum[j][0];
#pragma unroll
        for (int w = 1; w < DB_THREADS / 64; w++) s += wsum[j][w];
        a.part[(size_t)j * a.nchunk + blockIdx.x] = s;
    }
}

// dw[j] = the sum of row j of part [nd][nchunk]: one wave per j, lane l adding chunks l, l + 64, ...
// in order, then the wave's butterfly.
__global__ __launch_bounds__(64) void dense_grad_sum_kernel(const float *__restrict__ part, int nchunk,
                                                            float *__restrict__ dw) {
    const float *row = part + (size_t)blockIdx.x * nchunk;
    float s = 0.0f;
    for (int c = threadIdx.x; c < nchunk; c += 64) s += row[c];
    s = ava::wave_sum(s);
    if (threadIdx.x == 0) dw[blockIdx.x] = s;
}

int dense_back_chunks(size_t M4) { return (int)std::max<size_t>(1, (M4 + DB_CHUNK4 - 1) / DB_CHUNK4); }

}  // namespace

extern "C" int ava_kwta_relu2_bwd(const float *u, const float *kth, int n, int h, const float *ga, float *gu,
                                  ava_stream stream) {
    AVA_REQUIRE(u && kth && ga && gu, AVA_ERR_ARG, "kwta_relu2_bwd: NULL buffer");
    AVA_REQUIRE(n >= 0 && h > 0 && h % 4 == 0, AVA_ERR_SHAPE, "kwta_relu2_bwd: n=%d h=%d (h a multiple of 4)", n, h);
    const size_t n4 = (size_t)n * h / 4;
    if (n4 == 0) return AVA_OK;
    relu2_bwd_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, (hipStream_t)stream>>>(u, kth, ga, gu, h / 4, n4);
    AVA_LAUNCHED("kwta_relu2_bwd");
    return AVA_OK;
}

extern "C" size_t ava_dense_back_part_floats(long long M, int nd) {
    return M > 0 && nd > 0 ? (size_t)dense_back_chunks((size_t)M / 4) * nd : 0;
}

extern "C" int ava_dense_back(const float *S, const float *G, const float *wf, const float *base, float *out, float *dw,
                              int col, int i0, int L, int nd, long long M, float *part, size_t part_floats,
                              ava_stream stream) {
    AVA_REQUIRE(G && wf && base && out, AVA_ERR_ARG, "dense_back: NULL buffer");
    AVA_REQUIRE(M > 0 && M % 4 == 0, AVA_ERR_SHAPE, "dense_back: M=%lld (a multiple of 4)", M);
    AVA_REQUIRE(nd >= 0 && nd <= DB_MAXD && i0 >= 0 && i0 <= L && col >= 0 && col <= L + 1, AVA_ERR_SHAPE,
                "dense_back: col=%d i0=%d L=%d nd=%d (nd <= %d)", col, i0, L, nd, DB_MAXD);
    for (int k = i0; k < L; k++)
        AVA_REQUIRE(col <= k + 1, AVA_ERR_SHAPE, "dense_back: block %d has no weight %d", k, col);
    AVA_REQUIRE(nd == 0 || (S && dw && part), AVA_ERR_ARG, "dense_back: nd=%d needs S, dw and part", nd);
    const size_t M4 = (size_t)M / 4;
    const int nchunk = dense_back_chunks(M4);
    AVA_REQUIRE(nd == 0 || part_floats >= (size_t)nchunk * nd, AVA_ERR_SHAPE,
                "dense_back: part holds %zu < %zu floats", part_floats, (size_t)nchunk * nd);
    const hipStream_t st = (hipStream_t)stream;
    DenseBackArgs a{S, G, wf, base, out, part, col, i0, L, nd, nchunk, M4};
    dense_grad_kernel<<<nchunk, DB_THREADS, 0, st>>>(a);
    AVA_LAUNCHED("dense_back");
    if (nd > 0) {
        dense_grad_sum_kernel<<<nd, 64, 0, st>>>(part, nchunk, dw);
        AVA_LAUNCHED("dense_back_sum");
    }
    return AVA_OK;
}
