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

// The dense mix of block i, out = raw + sum_{j <= i + 1} w_ij S_j (S_{i+1} = raw), has the backward
//   dL/dS_c = base + sum_{k = i0 .. L-1} w_k[c] G_k    (G_k = dL/d(the mix after block k)),
//   dL/dw_ij = sum_e G_i,e S_j,e.
// Here: out = base + sum_k w_k[col] G_k over e, and part[wg][j] = this workgroup's share of
// sum_e base_e S_j,e for j < nd (the products, as gpu/lif.cu:4922-4971's dense_back). wf holds block
// k's k + 2 weights from k (k + 3) / 2.
constexpr int DENSE_MAXD = 32, DENSE_WG = 1024;

struct DenseBackArgs {
    const float *S, *G, *wf, *base;
    float *out, *part;
    int col, i0, L, nd;
    size_t M4;
};

__global__ __launch_bounds__(256) void dense_back_kernel(DenseBackArgs a) {
    __shared__ float red[4][DENSE_MAXD];
    float acc[DENSE_MAXD];
#pragma unroll
    for (int j = 0; j < DENSE_MAXD; j++) acc[j] = 0.0f;
    const size_t M = a.M4 * 4;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < a.M4; i += (size_t)gridDim.x * 256) {
        const f32x4 g = reinterpret_cast<const f32x4 *>(a.base)[i];
        f32x4 x = g;
        for (int k = a.i0; k < a.L; k++) {
            const float w = a.wf[k * (k + 3) / 2 + a.col];
            const f32x4 gk = reinterpret_cast<const f32x4 *>(a.G + (size_t)k * M)[i];
#pragma unroll
            for (int z = 0; z < 4; z++) x[z] = x[z] + w * gk[z];
        }
        reinterpret_cast<f32x4 *>(a.out)[i] = x;
#pragma unroll
        for (int j = 0; j < DENSE_MAXD; j++)
            if (j < a.nd) {
                const f32x4 s = reinterpret_cast<const f32x4 *>(a.S + (size_t)j * M)[i];
                acc[j] = fmaf(g[0], s[0], acc[j]);
                acc[j] = fmaf(g[1], s[1], acc[j]);
                acc[j] = fmaf(g[2], s[2], acc[j]);
                acc[j] = fmaf(g[3], s[3], acc[j]);
            }
    }
    if (a.nd == 0) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < DENSE_MAXD; j++)
        if (j < a.nd) {
            const float s = ava::wave_sum(acc[j]);
            if (lane == 0) red[w][j] = s;
        }
    __syncthreads();
    if ((int)threadIdx.x < a.nd) {
        const int j = threadIdx.x;
        a.part[(size_t)blockIdx.x * a.nd + j] = ((red[0][j] + red[1][j]) + red[2][j]) + red[3][j];
    }
}

// dw[j] = the workgroups' shares added in workgroup order (one thread per j).
__global__ void dense_back_sum_kernel(const float *__restrict__ part, int nwg, int nd, float *__restrict__ dw) {
    const int j = threadIdx.x;
    if (j >= nd) return;
    float s = 0.0f;
    for (int g = 0; g < nwg; g++) s += part[(size_t)g * nd + j];
    dw[j] = s;
}

int dense_back_grid(size_t M4) { return (int)std::min<size_t>(DENSE_WG, std::max<size_t>(1, (M4 + 255) / 256)); }

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
    return M > 0 && nd > 0 ? (size_t)dense_back_grid((size_t)M / 4) * nd : 0;
}

extern "C" int ava_dense_back(const float *S, const float *G, const float *wf, const float *base, float *out, float *dw,
                              int col, int i0, int L, int nd, long long M, float *part, size_t part_floats,
                              ava_stream stream) {
    AVA_REQUIRE(G && wf && base && out, AVA_ERR_ARG, "dense_back: NULL buffer");
    AVA_REQUIRE(M > 0 && M % 4 == 0, AVA_ERR_SHAPE, "dense_back: M=%lld (a multiple of 4)", M);
    AVA_REQUIRE(nd >= 0 && nd <= DENSE_MAXD && i0 >= 0 && i0 <= L && col >= 0 && col <= L + 1, AVA_ERR_SHAPE,
                "dense_back: col=%d i0=%d L=%d nd=%d (nd <= %d)", col, i0, L, nd, DENSE_MAXD);
    for (int k = i0; k < L; k++)
        AVA_REQUIRE(col <= k + 1, AVA_ERR_SHAPE, "dense_back: block %d has no weight %d", k, col);
    AVA_REQUIRE(nd == 0 || (S && dw && part), AVA_ERR_ARG, "dense_back: nd=%d needs S, dw and part", nd);
    const size_t M4 = (size_t)M / 4;
    const int grid = dense_back_grid(M4);
    AVA_REQUIRE(nd == 0 || part_floats >= (size_t)grid * nd, AVA_ERR_SHAPE, "dense_back: part holds %zu < %zu floats",
                part_floats, (size_t)grid * nd);
    const hipStream_t st = (hipStream_t)stream;
    DenseBackArgs a{S, G, wf, base, out, part, col, i0, L, nd, M4};
    dense_back_kernel<<<grid, 256, 0, st>>>(a);
    AVA_LAUNCHED("dense_back");
    if (nd > 0) {
        dense_back_sum_kernel<<<1, 64, 0, st>>>(part, grid, nd, dw);
        AVA_LAUNCHED("dense_back_sum");
    }
    return AVA_OK;
}
