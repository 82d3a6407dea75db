// int8 weights, split-plane activations and the i8 MFMA product for gfx950.
//
// Weights: W [din][dout] f32 -> qt [dout][ldk] int8 (each output column's weights contiguous in K,
// the B operand of v_mfma_i32_32x32x32_i8) and one f32 scale per output column, the reference's
// quantizer (parts/src/quant.rs:18-31).
//
// Activations: P planes of int8 under a power-of-two row scale (common.h: plane_exp / to_planes),
// [P][m][ldk]. Every plane's products are exact int32 sums; the epilogue combines them with one
// rounding, so a P = 3 product differs from the reference's f32 fma chain only by its 2^-22
// relative activation error, and integer inputs (spikes) give the reference's bits exactly.
//
// Product kernels: for many rows, a persistent grid of 8-wave workgroups over 128 x 256 output
// tiles with the operands brought into LDS by direct-to-LDS buffer loads (two stages; the next
// tile's first K step loads during the current tile's epilogue); for few rows (decode), 32-row
// blocks whose K steps are spread over the waves. Both order the tiles so that the workgroups of one
// XCD share its L2 for the rows and weight columns they read.
#include <stdlib.h>

#include <type_traits>

#include <algorithm>
#include <mutex>
#include <set>
#include <utility>

#include "common.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ weights

// One thread per output column: the column's absmax over din, then scale = amax/127 (1 if zero).
__global__ void q8_scale_kernel(const float *__restrict__ w, int din, int dout, float *__restrict__ scale) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= dout) return;
    float m = 0.0f;
    for (int j = 0; j < din; j++) m = fmaxf(m, fabsf(w[(size_t)j * dout + c]));
    scale[c] = m > 0.0f ? m / 127.0f : 1.0f;
}

// qt[c][j] = clamp(round(w[j][c] / scale[c]), +-127); 0 in the padding j >= din. A 64 x 64 tile
// transposed through LDS so both the reads and the writes are row-contiguous.
__global__ void q8_pack_kernel(const float *__restrict__ w, int din, int dout, int ldk,
                               const float *__restrict__ scale, int8_t *__restrict__ qt) {
    __shared__ int8_t tile[64][68];
    const int j0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 256 threads: 4 rows per pass
    for (int r = ty; r < 64; r += 4) {
        const int j = j0 + r, c = c0 + tx;
        int8_t q = 0;
        if (j < din && c < dout) {
            float t = roundf(w[(size_t)j * dout + c] / scale[c]);
            t = fminf(fmaxf(t, -127.0f), 127.0f);
            q = (int8_t)t;
        }
        tile[r][tx] = q;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int c = c0 + r, j = j0 + tx;
        if (c < dout && j < ldk) qt[(size_t)c * ldk + j] = tile[tx][r];
    }
}

// ------------------------------------------------------------------ activations

// One wave per row: the row's absmax, its exponent, then its planes (padding zeroed).
template <int P>
__global__ __launch_bounds__(256) void quant_rows_kernel(const float *__restrict__ x, int m, int k, int ldx,
                                                         int8_t *__restrict__ xq, int32_t *__restrict__ xexp,
                                                         int ldq) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float *xr = x + (size_t)row * ldx;
    float amax = 0.0f;
    for (int j = lane; j < k; j += 64) amax = fmaxf(amax, fabsf(xr[j]));
    amax = ava::wave_max(amax);
    const int e = ava::plane_exp(amax);
    if (lane == 0) xexp[row] = e;
    for (int j = lane * 4; j < ldq; j += 256) {
        int q[4][P];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v = (j + i < k) ? xr[j + i] : 0.0f;
            ava::to_planes<P>(v, e, q[i]);
        }
#pragma unroll
        for (int p = 0; p < P; p++)
            *reinterpret_cast<uint32_t *>(xq + ((size_t)p * m + row) * ldq + j) =
                ava::pack4(q[0][p], q[1][p], q[2][p], q[3][p]);
    }
}

// ------------------------------------------------------------------ the product

enum Epi { EPI_ACC = 0, EPI_STORE = ava::Q8_STORE, EPI_MUL = ava::Q8_MUL, EPI_ADD = ava::Q8_ADD, EPI_LIF = 4 };



// Epilogue parameters: y [m][ldy] (f32 or, for EPI_ACC, int32 [P][m][n]); colv [n] (EPI_MUL).
struct EpiArgs {
    void *y;
    int ldy;
    const float *colv;
    int group;  // row blocks per tile group (tile_origin)
    ava::LifEpi lif;  // EPI_LIF (few-rows kernel only): the LIF step on the product
};

// The output tile of tile index idx in a grid of `grid` workgroups (a workgroup takes indices
// blockIdx.x, blockIdx.x + grid, ...). Workgroups are dealt round-robin to the 8 XCDs, each with its
// own L2, so when both counts are multiples of 8 the indices of XCD x (idx mod 8 = x) are mapped to
// the x-th contiguous eighth of the tiles. The tiles go in groups of
// `group` row blocks, rows fastest: a weight column tile is then fetched from beyond L2 once per
// group, not once per row block, while the group's activation rows stay in L2 as the group sweeps
// the columns. group <= 1 is plain row-major order.
__device__ __forceinline__ void tile_origin(int idx, int grid, int tiles_m, int tiles_n, int group, int &mt, int &nt) {
    const int total = tiles_m * tiles_n;
    int t = idx;
    if (total % 8 == 0 && grid % 8 == 0) t = (idx & 7) * (total >> 3) + (idx >> 3);
    if (group <= 1) {
        mt = t / tiles_n;
        nt = t - mt * tiles_n;
        return;
    }
    const int span = group * tiles_n, g = t / span, r = t - g * span;
    const int rows = min(group, tiles_m - g * group);  // the last group may be short
    mt = g * group + r % rows;
    nt = r / rows;
}

// LDS position of 16-byte chunk c of tile row r: the chunk index XOR a function of the row, so that
// the fragment reads (32 consecutive rows, one chunk) and the staging writes (whole rows) do not
// collide in banks. For 64-byte rows, c ^ ((r >> 2) & 3) measured conflict-free on gfx950 (207 of
// about 210 B/clk/CU for ds_read_b128, against 61 unswizzled and 117 for c ^ (((r>>1)^(r>>3)) & 3)).
// CPR = chunks per row (4 or 8).
template <int CPR>
__device__ __forceinline__ int swz(int r, int c) {
    if (CPR == 4) return c ^ ((r >> 2) & 3);
    return c ^ ((r >> 1) & 7);
}

// The product's epilogue for one wave's FM x FN blocks of 32 x 32 outputs at tile rows rw0..,
// columns cw0..: in block (i, j) the lane holds, in register r, plane p's int32 sum for tile row
// rw0 + 32 i + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3) and column cw0 + 32 j + (lane & 31).
// exw is, in lane l, the exponent of wave row rw0 + l less 7 (P - 1); a register's row takes it with
// ds_bpermute. The planes combine exactly (sum_p acc_p 2^(7(P-1-p)), an integer below 2^53) and round
// once to f32: in double (CMB_F64), or for K <= 1024 (CMB_I32) the top two planes first in int32
// (|acc_p| <= 128 x 127 x 1024, so |acc_0 2^7 + acc_1| < 2^31), which leaves P = 2 one int32 -> f32
// conversion (correctly rounded, as the rounding of the double) and P = 3 one fma in double. Spike
// products (one plane, no row exponents: every exponent 0) skip the exponent (CMB_NOEXP).
// sc[j] and cv[j] are column (n0 + cw0 + 32 j + (lane & 31), clamped to n - 1)'s scale and colv
// (EPI_MUL), loaded by the caller.
// An interior tile stores (and, for EPI_ADD, loads) through a buffer resource based at its first
// row: the lane's offset is one VGPR and each register's row offset a wave-uniform SGPR, so no
// element forms a 64-bit address or tests a bound. Edge tiles and the int32 planes take the
// checked path.
enum { CMB_F64 = 0, CMB_I32 = 1, CMB_NOEXP = 2 };
template <int P, int EPI, int BM, int BN, int FM, int FN, int CMB>
__device__ __forceinline__ void epilogue(const i32x16 (&acc)[P][FM][FN], int exw, int m, int n, int m0, int n0,
                                         int rw0, int cw0, const float (&sc)[FN], const float (&cv)[FN],
                                         const EpiArgs &ep, int lane) {
    const int ccol = lane & 31, rsub = (lane >> 5) * 4;
    auto row_exp = [&](int wr) { return __builtin_amdgcn_ds_bpermute(wr << 2, exw); };  // wave row wr's
    // Block row i's exponents in one register: lane 16 q + z holds that of wave row 32 i + 8 (z >> 2) +
    // (z & 3) + 4 (q >> 1), and register r of a block reads it from lane z = r of its DPP row by
    // row_newbcast (every lane of a 16-lane row takes the row's lane r).
    auto exp_row = [&](int i) {
        const int z = lane & 15, q = lane >> 4;
        return row_exp(32 * i + 8 * (z >> 2) + (z & 3) + 4 * (q >> 1));
    };
    auto bcast = [&](int e, int r) {
        switch (r) {  // a constant in the unrolled loops (the DPP control must be one)
#define AVA_BC(R) \
    case R: return __builtin_amdgcn_mov_dpp(e, 0x150 + R, 0xf, 0xf, true);
            AVA_BC(0) AVA_BC(1) AVA_BC(2) AVA_BC(3) AVA_BC(4) AVA_BC(5) AVA_BC(6) AVA_BC(7)
            AVA_BC(8) AVA_BC(9) AVA_BC(10) AVA_BC(11) AVA_BC(12) AVA_BC(13) AVA_BC(14)
#undef AVA_BC
            default: return __builtin_amdgcn_mov_dpp(e, 0x150 + 15, 0xf, 0xf, true);
        }
    };
    auto value = [&](int i, int j, int r) {
        if (P == 1) return (float)acc[0][i][j][r];
        if (CMB == CMB_I32) {
            const int t = (int)((unsigned)acc[0][i][j][r] * 128u + (unsigned)acc[1][i][j][r]);
            if (P == 2) return (float)t;
            return (float)fma((double)t, 128.0, (double)acc[2][i][j][r]);
        }
        double A = (double)acc[0][i][j][r];
#pragma unroll
        for (int p = 1; p < P; p++) A = fma(A, 128.0, (double)acc[p][i][j][r]);
        return (float)A;
    };
    // the value under its row's exponent e (ldexp is exact; CMB_NOEXP: every e is 0)
    auto scaled = [&](int i, int j, int r, int e) {
        const float x = value(i, j, r);
        return CMB == CMB_NOEXP ? x : ldexpf(x, e);
    };
    if (EPI == EPI_ACC) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = n0 + cw0 + j * 32 + ccol;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + rw0 + i * 32 + rsub + (r >> 2) * 8 + (r & 3);
                    if (row < m && col < n)
#pragma unroll
                        for (int p = 0; p < P; p++)
                            reinterpret_cast<int32_t *>(ep.y)[((size_t)p * m + row) * n + col] = acc[p][i][j][r];
                }
        }
        return;
    }
    float *ybase = reinterpret_cast<float *>(ep.y);
    if (m0 + BM <= m && n0 + BN <= n) {
        const BufRes yr = buf_res(ybase + (size_t)m0 * ep.ldy, (unsigned)(BM * ep.ldy) * 4u);
        const unsigned ld4 = (unsigned)ep.ldy * 4u;
        const unsigned voff = ((unsigned)(rw0 + rsub) * (unsigned)ep.ldy + (unsigned)(n0 + cw0 + ccol)) * 4u;
        // block b = (i, j) = (b / FN, b % FN) at a time. EPI_ADD: block b + 1's 16 prior values are
        // loaded after block b's values are formed (in the registers its accumulators held) and before
        // block b's stores: vmcnt counts loads and stores in issue order, so a load issued behind a
        // block's stores is not seen done before those stores are
        constexpr int NB = FM * FN;
        auto row_off = [&](int i, int r) { return (unsigned)(i * 32 + (r >> 2) * 8 + (r & 3)) * ld4; };
        float prev[2][16];
        auto load_prev = [&](int blk, float (&pv)[16]) {
            const int i = blk / FN, j = blk % FN;
#pragma unroll
            for (int r = 0; r < 16; r++) pv[r] = load_f32_nt(yr, voff + j * 128u, row_off(i, r));
        };
        if (EPI != EPI_ADD) {
            // a block row's FN blocks together: each broadcast exponent serves FN outputs
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int er = exp_row(i);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    int eg = er;  // a fresh copy per group of 4 rows (see below)
#if defined(__HIP_DEVICE_COMPILE__)
                    asm volatile("" : "+v"(eg));
#endif
#pragma unroll
                    for (int z = 0; z < 4; z++) {
                        const int r = g * 4 + z, e = CMB == CMB_NOEXP ? 0 : bcast(eg, r);
#pragma unroll
                        for (int j = 0; j < FN; j++) {
                            float v = scaled(i, j, r, e) * sc[j];
                            if (EPI == EPI_MUL) v = v * cv[j];
                            store_f32_nt(yr, voff + j * 128u, row_off(i, r), v);
                        }
                    }
                }
            }
            return;
        }
        load_prev(0, prev[0]);
        AVA_ISSUE_FENCE();
        int er = 0;
#pragma unroll
        for (int blk = 0; blk < NB; blk++) {
            const int i = blk / FN, j = blk % FN;
            if (j == 0) er = exp_row(i);
            float v[16];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                // a fresh copy per group of 4 rows: the broadcasts are not shared between blocks and
                // formed when needed (16 held exponents cost registers the accumulators need)
                int eg = er;
#if defined(__HIP_DEVICE_COMPILE__)
                asm volatile("" : "+v"(eg));
#endif
#pragma unroll
                for (int z = 0; z < 4; z++) {
                    const int r = g * 4 + z;
                    v[r] = scaled(i, j, r, CMB == CMB_NOEXP ? 0 : bcast(eg, r)) * sc[j];
                    if (EPI == EPI_MUL) v[r] = v[r] * cv[j];
                    if (EPI == EPI_ADD) v[r] = prev[blk & 1][r] + v[r];
                }
            }
            if (EPI == EPI_ADD && blk + 1 < NB) {
                AVA_ISSUE_FENCE();
                load_prev(blk + 1, prev[(blk + 1) & 1]);
                AVA_ISSUE_FENCE();
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                if (EPI == EPI_ADD) store_f32(yr, voff + j * 128u, row_off(i, r), v[r]);
                else store_f32_nt(yr, voff + j * 128u, row_off(i, r), v[r]);
            }
        }
        return;
    }
    // an edge tile: every access goes through a resource over the tile's existing rows with the whole
    // offset in the lane operand, so the range check drops rows past m (loads read 0); columns past n
    // are masked per lane
    // (the lane index passes through an empty asm: in a persistent caller, the lane offsets of this
    // rare path are then formed here, per tile, instead of before the tile loop and kept in registers)
    int el = lane;
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(el));
#endif
    const int eccol = el & 31, ersub = (el >> 5) * 4;
    const unsigned rows_ok = (unsigned)min(BM, m - m0);
    const BufRes yr = buf_res(ybase + (size_t)m0 * ep.ldy, rows_ok * (unsigned)ep.ldy * 4u);
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int col = n0 + cw0 + j * 32 + eccol;
        const bool col_ok = col < n;
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int rbase = rw0 + i * 32 + ersub;  // tile row of r = 0
            auto off = [&](int r) {
                return ((unsigned)(rbase + (r >> 2) * 8 + (r & 3)) * (unsigned)ep.ldy + (unsigned)col) * 4u;
            };
            float prev[16];
            if (EPI == EPI_ADD) {
#pragma unroll
                for (int r = 0; r < 16; r++) prev[r] = col_ok ? load_f32(yr, off(r), 0u) : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int tr = rbase + (r >> 2) * 8 + (r & 3);
                float v = scaled(i, j, r, CMB == CMB_NOEXP ? 0 : row_exp(tr - rw0)) * sc[j];
                if (EPI == EPI_MUL) v = v * cv[j];
                if (EPI == EPI_ADD) v = prev[r] + v;
                if (col_ok) store_f32(yr, off(r), 0u, v);
            }
        }
    }
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] in [15:14]
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// global_load_lds_dwordx4: 16 bytes per lane from `g` to LDS at `l` + 16 x lane (l wave-uniform). The
// address-space cast exists only in the device pass (the host pass never sees the body).
__device__ __forceinline__ void dma16(const void *g, void *l) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 16, 0, 0);
#endif
}

// A raw buffer resource over [base, base + bytes) of int8 data (the int8 twin of common.h's buf_res).
#if defined(__HIP_DEVICE_COMPILE__)
typedef __amdgpu_buffer_rsrc_t BufRes8;
__device__ __forceinline__ BufRes8 buf_res8(const int8_t *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, (int)bytes, 0x00020000);
}
#else
typedef const int8_t *BufRes8;
__device__ inline BufRes8 buf_res8(const int8_t *base, unsigned) { return base; }
#endif

// ------------------------------------------------------------------ the product for many rows
//
// A persistent grid (at most one 8-wave workgroup per CU) walks the 128 x 256 output tiles:
// workgroup b takes tile indices b, b + G, b + 2G, ... (G = the grid), placed by tile_origin.
// Operands reach LDS through buffer_load_dwordx4 ... lds: one load instruction writes 64 lanes x 16
// bytes = 1 KB of stage rows contiguously (lane l takes row r0 + l / CPR and the 16-byte chunk that
// lands in slot l % CPR under the row's swizzle). Each operand (a plane of the tile's rows, or the
// tile's weight columns) is read through a buffer resource based at the tile's first row: a lane
// keeps one 32-bit offset per load instruction, the K step is the instruction's uniform offset, and
// rows past the operand's end read as zeros (the resource's range check), so edge tiles need no
// clamping. Load instruction i of wave w covers stage rows (8 i + w) RPI .. + RPI - 1, so instruction
// i reads the same operand in every wave and its resource is fixed at compile time.
//
// Two LDS stages of BK-byte K steps: at step kt a wave waits for its own loads, one barrier makes
// every wave's loads visible and frees the other stage, and step kt is multiplied while the loads of
// step kt + 1 go into the other stage, two after each group of MFMAs (after a tile's last step they
// fetch the next tile's first step, whose latency then hides behind this tile's epilogue; after the
// grid's last tile, this tile's first step again, unused). Each wave owns 64 x 64 outputs per plane,
// 2 x 2 blocks of v_mfma_i32_32x32x32_i8; the fragment reads of the next (K sub-step, plane) group are
// issued before the MFMAs of the current group, so four MFMAs cover their LDS latency (the order is
// fixed with sched_group_barrier). A tile's first step multiplies into zero accumulators (no
// register clearing).
constexpr int GEMM_BM = 128, GEMM_BN = 256, GEMM_WM = 2, GEMM_WN = 4, GEMM_ILV = 2;

__device__ __forceinline__ void dma16_buf(BufRes8 r, unsigned voff, unsigned soff, void *l) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)l, 16, (int)voff,
                                             (int)soff, 0, 0);
#endif
}

// The instruction order of one K step: the first group's fragment reads, then per group g the reads
// of group g + 1 (if any) followed by the FM x FN MFMAs of group g (mask 0x100: LDS reads, 0x008: MFMA).
// After the MFMAs of group g come the next step's global loads ILV g .. ILV g + ILV - 1 (mask 0x020),
// so that they leave between the MFMAs instead of all at once after the barrier.
template <int G, int KS, int P, int FM, int FN, int LPW, int ILV>
__device__ __forceinline__ void frag_schedule() {
    if constexpr (G < KS * P) {
        constexpr int p = G % P, ks = G / P;
        constexpr int reads = (p + 1 < P) ? FM : (ks + 1 < KS ? FN + FM : 0);
        if constexpr (reads > 0) __builtin_amdgcn_sched_group_barrier(0x100, reads, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);
        constexpr int left = LPW - G * ILV;
        if constexpr (left > 0) __builtin_amdgcn_sched_group_barrier(0x020, left < ILV ? left : ILV, 0);
        frag_schedule<G + 1, KS, P, FM, FN, LPW, ILV>();
    }
}

template <int P, int EPI, int BK, int CMB>
__global__ __launch_bounds__(64 * GEMM_WM * GEMM_WN, 1) void q8_gemm_kernel(const int8_t *__restrict__ xq,
                                                                        const int32_t *__restrict__ xexp, int m,
                                                                        int n, int ldk, const int8_t *__restrict__ qt,
                                                                        const float *__restrict__ scale, EpiArgs ep) {
    constexpr int BM = GEMM_BM, BN = GEMM_BN, WM = GEMM_WM, WN = GEMM_WN, NWAVE = WM * WN, NT = 64 * NWAVE;
    constexpr int CPR = BK / 16, RPI = 1024 / BK, KS = BK / 32;
    static_assert(BK == 64 || BK == 128, "K step");
    constexpr int MW = BM / WM, NW = BN / WN, FM = MW / 32, FN = NW / 32;
    constexpr int A_ROWS = P * BM, STAGE = (A_ROWS + BN) * BK;
    constexpr int ROUND = NWAVE * RPI;  // stage rows per load instruction index
    static_assert(BM % ROUND == 0 && BN % ROUND == 0, "an instruction index reads one operand");
    constexpr int LPW = (A_ROWS + BN) / ROUND;  // load instructions per wave per step
    static_assert(BM <= NT, "one row exponent per thread");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];

    const int tiles_n = (n + BN - 1) / BN, tiles_m = (m + BM - 1) / BM, total = tiles_m * tiles_n;
    const int grid = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // per lane, the offset of each load instruction's 16 bytes within its operand (any tile)
    unsigned voff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int srow0 = (i * NWAVE + wave) * RPI, srow = srow0 + lane / CPR;
        const int rr = i * ROUND < A_ROWS ? srow - (i * ROUND / BM) * BM : srow - A_ROWS;
        voff[i] = (unsigned)rr * (unsigned)ldk + swz<CPR>(rr, lane % CPR) * 16;
    }
    BufRes8 rs[P + 1];  // the current tile's planes, then its weight columns
    auto set_rs = [&](int m0, int n0) {
        const unsigned arows = (unsigned)min(BM, m - m0), brows = (unsigned)min(BN, n - n0);
#pragma unroll
        for (int p = 0; p < P; p++) rs[p] = buf_res8(xq + ((size_t)p * m + m0) * ldk, arows * (unsigned)ldk);
        rs[P] = buf_res8(qt + (size_t)n0 * ldk, brows * (unsigned)ldk);
    };
    // load instruction i of step kt of the tile of rs, into `stage`
    auto issue_one = [&](int i, int kt, int stage) {
        const int op = i * ROUND < A_ROWS ? i * ROUND / BM : P;
        dma16_buf(rs[op], voff[i], (unsigned)(kt * BK), smem + stage * STAGE + (i * NWAVE + wave) * 1024);
    };

    const int KT = ldk / BK;
    const int frow = lane & 31, fc = lane >> 5;
    int idx = blockIdx.x, mt, nt;
    tile_origin(idx, grid, tiles_m, tiles_n, ep.group, mt, nt);
    int m0 = mt * BM, n0 = nt * BN;
    set_rs(m0, n0);
#pragma unroll
    for (int i = 0; i < LPW; i++) issue_one(i, 0, 0);
    int sbase = 0;  // the stage holding the tile's first step
    // Whether the previous tile's epilogue issued at least 63 vector memory instructions after this
    // tile's first-step loads. On gfx9 vmcnt counts loads and stores together, decrements in issue
    // order and holds at most 63, so an instruction issued with 63 older ones outstanding waits for
    // the oldest: the first-step loads had then landed before the last of those was issued, and the
    // first step needs no wait (which would also wait for the epilogue's stores to reach L2).
    static_assert(FM * FN * 16 >= 63, "an interior epilogue issues at least 63 stores per wave");
    bool loaded = false;
    // the row exponents through a resource of 0 bytes when there are none: its loads read 0, so the
    // load needs no branch (a branch would make the compiler wait for the value at its join)
    const BufRes xer = buf_res(const_cast<float *>(reinterpret_cast<const float *>(xexp)),
                               EPI != EPI_ACC && xexp ? (unsigned)m * 4u : 0u);
    for (; idx < total; idx += grid) {
        // the exponent of this wave's row wm MW + lane of the tile and each lane's column scales, used
        // by the epilogue: issued before the K loop, so the epilogue does not wait for the next tile's
        // first-step loads issued in the last step. EPI_ADD waits for those anyway (its prior values
        // are loaded after them) and loads its scales after the K loop, which keeps two registers free
        // during it.
        const int ex = __float_as_int(load_f32(xer, (unsigned)min(m0 + wm * MW + lane, m - 1) * 4u, 0u));
        float sc[FN], cv[FN];
        auto load_cols = [&]() {
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = min(n0 + wn * NW + j * 32 + (lane & 31), n - 1);
                sc[j] = EPI != EPI_ACC ? scale[col] : 0.0f;
                cv[j] = EPI == EPI_MUL ? ep.colv[col] : 0.0f;
            }
        };
        if (EPI != EPI_ADD) load_cols();
        i32x16 acc[P][FM][FN];
        int st = sbase;
        auto step = [&](auto first, int kt) {
            constexpr bool FIRST = decltype(first)::value;
            st = (sbase + kt) & 1;
            if (FIRST && loaded) wait_vm<63>();  // holds by itself: see `loaded`
            else wait_vm<0>();  // this wave's loads of step kt (and the previous tile's stores) are done
            __builtin_amdgcn_s_barrier();  // every wave's are; every wave is done with the other stage
            int knext = kt + 1;
            if (kt + 1 == KT) {
                knext = 0;
                if (idx + grid < total) {
                    tile_origin(idx + grid, grid, tiles_m, tiles_n, ep.group, mt, nt);
                    set_rs(mt * BM, nt * BN);
                }
            }
            const int8_t *la = smem + st * STAGE, *lb = la + A_ROWS * BK;
            auto afr = [&](int ks, int p, int i) {
                const int r = wm * MW + i * 32 + frow;
                return *reinterpret_cast<const i32x4 *>(la + (p * BM + r) * BK + swz<CPR>(r, ks * 2 + fc) * 16);
            };
            auto bfr = [&](int ks, int j) {
                const int r = wn * NW + j * 32 + frow;
                return *reinterpret_cast<const i32x4 *>(lb + r * BK + swz<CPR>(r, ks * 2 + fc) * 16);
            };
            // group g = (ks, p): fragments double-buffered across groups
            i32x4 bb[2][FN], aa[2][FM];
#pragma unroll
            for (int j = 0; j < FN; j++) bb[0][j] = bfr(0, j);
#pragma unroll
            for (int i = 0; i < FM; i++) aa[0][i] = afr(0, 0, i);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
#pragma unroll
                for (int p = 0; p < P; p++) {
                    const int g = ks * P + p, cur = g & 1;
                    if (p + 1 < P) {
#pragma unroll
                        for (int i = 0; i < FM; i++) aa[cur ^ 1][i] = afr(ks, p + 1, i);
                    } else if (ks + 1 < KS) {
#pragma unroll
                        for (int j = 0; j < FN; j++) bb[(ks + 1) & 1][j] = bfr(ks + 1, j);
#pragma unroll
                        for (int i = 0; i < FM; i++) aa[cur ^ 1][i] = afr(ks + 1, 0, i);
                    }
#pragma unroll
                    for (int i = 0; i < FM; i++)
#pragma unroll
                        for (int j = 0; j < FN; j++) {
                            const i32x16 c = (FIRST && ks == 0) ? i32x16{} : acc[p][i][j];
                            acc[p][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aa[cur][i], bb[ks & 1][j], c, 0, 0, 0);
                        }
#pragma unroll
                    for (int q = 0; q < GEMM_ILV; q++) {
                        const int li = g * GEMM_ILV + q;
                        if (li < LPW) issue_one(li, knext, st ^ 1);
                    }
                }
            }
            __builtin_amdgcn_sched_group_barrier(0x100, FN + FM, 0);
            frag_schedule<0, KS, P, FM, FN, LPW, GEMM_ILV>();
        };
        step(std::integral_constant<bool, true>{}, 0);
#pragma nounroll
        for (int kt = 1; kt < KT; kt++) step(std::integral_constant<bool, false>{}, kt);
        if (EPI == EPI_ADD) load_cols();
        epilogue<P, EPI, BM, BN, FM, FN, CMB>(acc, ex - 7 * (P - 1), m, n, m0, n0, wm * MW, wn * NW, sc, cv, ep,
                                              lane);
        loaded = EPI != EPI_ACC && m0 + BM <= m && n0 + BN <= n;  // the interior path ran
        m0 = mt * BM;  // the next tile (tile_origin ran at the last step)
        n0 = nt * BN;
        sbase = st ^ 1;
    }
    wait_vm<0>();  // no load into LDS outlives the workgroup
}

// Products of at most this many rows take the few-rows kernel.
constexpr int SMALL_ROWS = 512;
// Few-rows products of at least this many columns take 64-column blocks.
constexpr int SMALL_WIDE_COLS = 4096;

// ------------------------------------------------------------------ the product for few rows
//
// Decode shapes (m <= 512 rows) leave the tiled kernels with a few dozen workgroups. Here a workgroup
// owns a 32 x BN output block (BN = 32 FN) and all of K; its NW waves take the 64-byte K steps
// kt = w, w + NW, ... each on its own: a wave stages its steps (P planes x 32 rows and BN weight
// columns, 64 bytes each) in its own ring of D LDS buffers with direct-to-LDS loads, D - 1 steps ahead
// of the one it multiplies, and waits for its own loads only, so the K loop has no barrier. At the end
// wave w forms its exact plane combination A_w = sum_p acc_p 2^(7(P-1-p)) in double (an integer below
// 2^47); the NW partials are added in LDS (still exact, so in any order) and rounded once as the tiled
// kernels' epilogue does: the same bits as they give, for any m. The staging rate per CU bounds the
// time, so a CU wants 8 waves loading: two 4-wave workgroups when the grid has enough blocks, else
// one of 8 waves (5-7% faster than 4 there).
template <int P, int FN, int D = 2, int NW = 4>
struct SmallCfg {
    static constexpr int BM = 32, BN = 32 * FN, BK = 64, CPR = 4, RPI = 16;  // a 1 KB load = 16 rows
    static constexpr int ROWS = P * BM + BN, LPS = ROWS / RPI, BUF = ROWS * BK;
    static_assert(D >= 2 && (D - 1) * LPS < 64, "ring depth: the loads in flight must fit vmcnt");
    static_assert(NW == 4 || NW == 8, "waves per workgroup");
    static constexpr size_t OPS = (size_t)NW * D * BUF;                       // NW waves x D buffers
    static constexpr size_t ACC = (size_t)NW * P * FN * 16 * 64 * 4;         // int32 planes, EPI_ACC
    static constexpr size_t DBL = (size_t)NW * FN * 16 * 64 * 8;             // doubles, other epilogues
};

// The values the few-rows epilogue reads from memory besides the accumulators: each column's scale (and
// colv, and for EPI_LIF the channel's four parameters), each finished row's exponent and, for EPI_ADD,
// the prior y, for EPI_LIF the membrane state. They are loaded at the start of the kernel, so their
// latency passes during the K loop instead of after it. Wave w finishes rows r = w + NW q of the block
// (q < 16 / NW) in columns n0 + 32 j + (lane & 31); rows past m and columns past n load the last ones
// (in bounds, unused).
template <int EPI, int FN, int NW>
struct SmallPre {
    static constexpr int Q = 16 / NW;
    float sc[FN], cv[FN];
    int ex[Q];
    float y[FN][Q];                            // EPI_ADD: y; EPI_LIF: the membrane v
    float ls[EPI == EPI_LIF ? FN : 1][Q];      // EPI_LIF: the last spike
    float la[EPI == EPI_LIF ? FN : 1][Q];      // EPI_LIF: the trace
    float lp[EPI == EPI_LIF ? FN : 1][4];      // EPI_LIF: beta, theta0, rho, gain
};
template <int P, int EPI, int FN, int NW>
__device__ __forceinline__ void small_prefetch(SmallPre<EPI, FN, NW> &pre, int m, int n, int m0, int n0,
                                               const int32_t *__restrict__ xexp, const float *__restrict__ scale,
                                               const EpiArgs &ep, int lane, int wave) {
    constexpr int Q = 16 / NW;
    if constexpr (EPI == EPI_ACC) return;
    const int rsub = (lane >> 5) * 4;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int r = wave + NW * q, row = min(m0 + (r >> 2) * 8 + rsub + (r & 3), m - 1);
        pre.ex[q] = (xexp ? xexp[row] : 0) - 7 * (P - 1);
    }
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int col = min(n0 + j * 32 + (lane & 31), n - 1);
        pre.sc[j] = scale[col];
        pre.cv[j] = (EPI == EPI_MUL || (EPI == EPI_LIF && ep.colv)) ? ep.colv[col] : 1.0f;
        if constexpr (EPI == EPI_LIF) {
            const ava::LifEpi &L = ep.lif;
#pragma unroll
            for (int z = 0; z < 4; z++) pre.lp[j][z] = L.ps[z * n + col];
        }
#pragma unroll
        for (int q = 0; q < Q; q++) {
            const int r = wave + NW * q, row = min(m0 + (r >> 2) * 8 + rsub + (r & 3), m - 1);
            if constexpr (EPI == EPI_ADD) pre.y[j][q] = reinterpret_cast<const float *>(ep.y)[(size_t)row * ep.ldy + col];
            if constexpr (EPI == EPI_LIF) {
                const size_t o = (size_t)row * n + col;
                pre.y[j][q] = ep.lif.v[o];
                pre.ls[j][q] = ep.lif.s[o];
                pre.la[j][q] = ep.lif.a[o];
            }
        }
    }
}

// The few-rows products' epilogue: wave w's P-plane accumulators of the 32 x 32 FN block combine
// exactly in double; the NW waves' partials add in LDS (smem, 8 NW FN KB; int32 planes for EPI_ACC);
// then one rounding and the epilogue kind, as the tiled kernels' epilogue. Wave w finishes the
// accumulator rows r = w + NW q.
template <int P, int EPI, int FN, int NW>
__device__ __forceinline__ void small_epilogue(const i32x16 (&acc)[P][FN], int8_t *smem, int m, int n, int m0, int n0,
                                               const SmallPre<EPI, FN, NW> &pre, const EpiArgs &ep, int lane,
                                               int wave) {
    const int rsub = (lane >> 5) * 4;
    if (EPI == EPI_ACC) {
        int *si = reinterpret_cast<int *>(smem);  // [wave][p][j][16][64]
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) si[(((wave * P + p) * FN + j) * 16 + r) * 64 + lane] = acc[p][j][r];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = n0 + j * 32 + (lane & 31);
#pragma unroll
            for (int q = 0; q < 16 / NW; q++) {
                const int r = wave + NW * q, row = m0 + (r >> 2) * 8 + rsub + (r & 3);
                if (row < m && col < n)
#pragma unroll
                    for (int p = 0; p < P; p++) {
                        int v = 0;
#pragma unroll
                        for (int w = 0; w < NW; w++) v += si[(((w * P + p) * FN + j) * 16 + r) * 64 + lane];
                        reinterpret_cast<int32_t *>(ep.y)[((size_t)p * m + row) * n + col] = v;
                    }
            }
        }
        return;
    }
    double *sd = reinterpret_cast<double *>(smem);  // [wave][j][16][64]
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            double A = (double)acc[0][j][r];
#pragma unroll
            for (int p = 1; p < P; p++) A = fma(A, 128.0, (double)acc[p][j][r]);
            sd[((wave * FN + j) * 16 + r) * 64 + lane] = A;
        }
    __syncthreads();
    float *ybase = reinterpret_cast<float *>(ep.y);
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int col = n0 + j * 32 + (lane & 31);
        if (col >= n) continue;
        const float sc = pre.sc[j];
        if constexpr (EPI == EPI_LIF) {
            // cur (times colv: the lif-scale factor) into one step of the channel's scan, as
            // lif_scan_kernel's loop body
            const ava::LifEpi &L = ep.lif;
            const float bt = pre.lp[j][0], th0 = pre.lp[j][1], rho = pre.lp[j][2], gain = pre.lp[j][3];
#pragma unroll
            for (int q = 0; q < 16 / NW; q++) {
                const int r = wave + NW * q, row = m0 + (r >> 2) * 8 + rsub + (r & 3);
                if (row >= m) continue;
                const int e = (j * 16 + r) * 64 + lane, ws = FN * 16 * 64;
                double A = sd[e];
#pragma unroll
                for (int w = 1; w < NW; w++) A += sd[w * ws + e];
                float v = ldexpf((float)A, pre.ex[q]) * sc;
                if (ep.colv) v = v * pre.cv[j];
                float vv = pre.y[j][q], sp = pre.ls[j][q], aa = pre.la[j][q];
                const float thp = L.alif ? th0 + aa * gain : th0;
                float tht = th0;
                if (L.alif) {
                    aa = aa * rho + fabsf(sp) * (1.0f - rho);
                    tht = th0 + aa * gain;
                }
                vv = (vv * bt + v) - sp * thp;
                sp = ava::lif_spike(vv, tht, L.levels, L.is_signed);
                const size_t o = (size_t)row * n + col;
                L.v[o] = vv;
                L.s[o] = sp;
                L.a[o] = aa;
                L.spikes[(size_t)row * L.ldspk + col] = (int8_t)sp;
            }
            continue;
        }
#pragma unroll
        for (int q = 0; q < 16 / NW; q++) {
            const int r = wave + NW * q, row = m0 + (r >> 2) * 8 + rsub + (r & 3);
            if (row >= m) continue;
            const int e = (j * 16 + r) * 64 + lane, ws = FN * 16 * 64;
            double A = sd[e];
#pragma unroll
            for (int w = 1; w < NW; w++) A += sd[w * ws + e];
            float v = ldexpf((float)A, pre.ex[q]) * sc;
            if (EPI == EPI_MUL) v = v * pre.cv[j];
            if (EPI == EPI_ADD) v = pre.y[j][q] + v;
            ybase[(size_t)row * ep.ldy + col] = v;
        }
    }
}

// Waits until at most `ahead` steps of LPS loads each are still in flight (ahead < D, wave-uniform).
template <int LPS, int D>
__device__ __forceinline__ void wait_steps(int ahead) {
    if constexpr (D > 1) {
        if (ahead >= D - 1) {
            wait_vm<(D - 1) * LPS>();
            return;
        }
        wait_steps<LPS, D - 1>(ahead);
    } else {
        wait_vm<0>();
    }
}

template <int P, int EPI, int FN, int D, int NW>
__global__ __launch_bounds__(64 * NW) void q8_small_kernel(const int8_t *__restrict__ xq, const int32_t *__restrict__ xexp,
                                                       int m, int n, int ldk, const int8_t *__restrict__ qt,
                                                       const float *__restrict__ scale, EpiArgs ep) {
    using C = SmallCfg<P, FN, D, NW>;
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, CPR = C::CPR, RPI = C::RPI, LPS = C::LPS, BUF = C::BUF;
    static_assert(C::ROWS % RPI == 0, "rows per load");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int mt, nt;
    tile_origin(blockIdx.x, gridDim.x, tiles_m, tiles_n, tiles_m, mt, nt);  // a weight block's row blocks on one XCD
    const int m0 = mt * BM, n0 = nt * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int8_t *wbuf = smem + wave * D * BUF;

    const int8_t *src[LPS];
#pragma unroll
    for (int i = 0; i < LPS; i++) {
        const int srow = i * RPI + lane / CPR;
        if (srow < P * BM) {
            const int p = srow / BM, rr = srow % BM;
            const int row = min(m0 + rr, m - 1);
            src[i] = xq + ((size_t)p * m + row) * ldk + swz<CPR>(rr, lane % CPR) * 16;
        } else {
            const int rr = srow - P * BM;
            const int col = min(n0 + rr, n - 1);
            src[i] = qt + (size_t)col * ldk + swz<CPR>(rr, lane % CPR) * 16;
        }
    }
    // step s of this wave is K step kt = wave + NW s, staged in buffer s % D
    auto issue = [&](int s) {
        int8_t *dst = wbuf + (s % D) * BUF;
        const int off = (wave + NW * s) * BK;
#pragma unroll
        for (int i = 0; i < LPS; i++) dma16(src[i] + off, dst + i * 1024);
    };

    SmallPre<EPI, FN, NW> pre;
    small_prefetch<P, EPI, FN, NW>(pre, m, n, m0, n0, xexp, scale, ep, lane, wave);
    i32x16 acc[P][FN];
#pragma unroll
    for (int p = 0; p < P; p++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[p][j] = i32x16{};
    const int KT = ldk / BK, frow = lane & 31, fc = lane >> 5;
    const int ns = wave < KT ? (KT - wave + NW - 1) / NW : 0;  // this wave's steps
#pragma unroll
    for (int s = 0; s < D - 1; s++)
        if (s < ns) issue(s);
    for (int s = 0; s < ns; s++) {
        // the buffer of step s + D - 1 held step s - 1, whose fragment reads completed last iteration
        if (s + D - 1 < ns) issue(s + D - 1);
        wait_steps<LPS, D>(min(D - 1, ns - 1 - s));  // step s is in LDS; the later ones may be in flight
        const int8_t *la = wbuf + (s % D) * BUF, *lb = la + P * BM * BK;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            i32x4 bf[FN];
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int r = j * 32 + frow;
                bf[j] = *reinterpret_cast<const i32x4 *>(lb + r * BK + swz<CPR>(r, ks * 2 + fc) * 16);
            }
#pragma unroll
            for (int p = 0; p < P; p++) {
                const i32x4 af =
                    *reinterpret_cast<const i32x4 *>(la + (p * BM + frow) * BK + swz<CPR>(frow, ks * 2 + fc) * 16);
#pragma unroll
                for (int j = 0; j < FN; j++) acc[p][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[j], acc[p][j], 0, 0, 0);
            }
        }
        // the buffer is refilled D - 1 steps on: its fragment reads must have completed
#if defined(__HIP_DEVICE_COMPILE__)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
    }
    __syncthreads();  // every wave is done with its buffers
    small_epilogue<P, EPI, FN, NW>(acc, smem, m, n, m0, n0, pre, ep, lane, wave);
}

template <int P, int EPI, int FN, int D, int NW>
int launch_small_fn(const int8_t *xq, const int32_t *xexp, int m, int n, int ldk, const int8_t *qt,
                    const float *scale, EpiArgs ep, hipStream_t st) {
    using C = SmallCfg<P, FN, D, NW>;
    const int total = ((m + C::BM - 1) / C::BM) * ((n + C::BN - 1) / C::BN);
    const size_t lds = std::max(C::OPS, EPI == EPI_ACC ? C::ACC : C::DBL);
    if (int r = ava::lds_opt_in((const void *)q8_small_kernel<P, EPI, FN, D, NW>, lds)) return r;
    q8_small_kernel<P, EPI, FN, D, NW><<<dim3(total), dim3(64 * NW), lds, st>>>(xq, xexp, m, n, ldk, qt, scale, ep);
    AVA_LAUNCHED("q8_gemm");
    return AVA_OK;
}

// 8 waves per workgroup when the grid gives a CU one workgroup or fewer, else 4 (two per CU); single
// planes (spikes) stage so little per step that 4 waves do better.
template <int P, int EPI, int FN>
int launch_small_w(const int8_t *xq, const int32_t *xexp, int m, int n, int ldk, const int8_t *qt, const float *scale,
                   EpiArgs ep, hipStream_t st) {
    using C8 = SmallCfg<P, FN, 2, 8>;
    constexpr bool fits8 = P > 1 && std::max(C8::OPS, EPI == EPI_ACC ? C8::ACC : C8::DBL) <= 163840;  // LDS per CU
    const int nw = ((m + 31) / 32) * ((n + 32 * FN - 1) / (32 * FN)) <= 256 ? 8 : 4;
    if constexpr (fits8)
        if (nw == 8) return launch_small_fn<P, EPI, FN, 2, 8>(xq, xexp, m, n, ldk, qt, scale, ep, st);
    return launch_small_fn<P, EPI, FN, 2, 4>(xq, xexp, m, n, ldk, qt, scale, ep, st);
}

// 64-column blocks for wide products (half the activation re-reads), 32 otherwise (enough blocks).
// Wider blocks (128, 160 columns: one workgroup per CU) and deeper rings measured no faster.
template <int P, int EPI>
int launch_small(const int8_t *xq, const int32_t *xexp, int m, int n, int ldk, const int8_t *qt, const float *scale,
                 EpiArgs ep, hipStream_t st) {
    if (n >= SMALL_WIDE_COLS) return launch_small_w<P, EPI, 2>(xq, xexp, m, n, ldk, qt, scale, ep, st);
    return launch_small_w<P, EPI, 1>(xq, xexp, m, n, ldk, qt, scale, ep, st);
}

// Row blocks per tile group (tile_origin): a weight column tile is fetched past L2 once per 8 row blocks.
constexpr int TILE_GROUP = 8;

// Workgroups for the persistent product: one per CU of the current device.
int gemm_grid(int tiles, int *grid) {
    int c = 0;
    if (int r = ava::device_cus(&c)) return r;
    *grid = std::max(1, std::min(tiles, c));
    return AVA_OK;
}

template <int P, int EPI, int BK>
int launch_tiled(const int8_t *xq, const int32_t *xexp, int m, int n, int ldk, const int8_t *qt, const float *scale,
                 EpiArgs ep, hipStream_t st) {
    const int tiles = ((m + GEMM_BM - 1) / GEMM_BM) * ((n + GEMM_BN - 1) / GEMM_BN);
    int grid = 0;
    if (int r = gemm_grid(tiles, &grid)) return r;
    const size_t lds = (size_t)2 * (P * GEMM_BM + GEMM_BN) * BK;
    auto go = [&](auto kern) -> int {
        if (int r = ava::lds_opt_in((const void *)kern, lds)) return r;
        kern<<<dim3(grid), dim3(64 * GEMM_WM * GEMM_WN), lds, st>>>(xq, xexp, m, n, ldk, qt, scale, ep);
        AVA_LAUNCHED("q8_gemm");
        return AVA_OK;
    };
    // the int32 plane combine holds for K <= 1024; spike products have no row exponents (see epilogue)
    if constexpr (P == 1) {
        if (EPI != EPI_ACC && !xexp) return go(q8_gemm_kernel<P, EPI, BK, CMB_NOEXP>);
    } else {
        if (EPI != EPI_ACC && ldk <= 1024) return go(q8_gemm_kernel<P, EPI, BK, CMB_I32>);
    }
    return go(q8_gemm_kernel<P, EPI, BK, CMB_F64>);
}

template <int P, int EPI>
int launch_gemm(const int8_t *xq, const int32_t *xexp, int m, int n, int ldk, const int8_t *qt, const float *scale,
                EpiArgs ep, hipStream_t st) {
    // few rows (decode): 32-row blocks with the K steps spread over the waves
    if (m <= SMALL_ROWS) return launch_small<P, EPI>(xq, xexp, m, n, ldk, qt, scale, ep, st);
    // 128-byte K steps (whole cache lines per load request) for every plane count: for the single
    // spike plane at 131,072 x 1024 x 1024 they measured 279 us against 340 us for 64-byte steps
    return launch_tiled<P, EPI, 128>(xq, xexp, m, n, ldk, qt, scale, ep, st);
}

template <int EPI>
int gemm_planes(int planes, const int8_t *xq, const int32_t *xexp, int m, int n, int ldk, const int8_t *qt,
                const float *scale, EpiArgs ep, hipStream_t st) {
    if (planes == 1) return launch_gemm<1, EPI>(xq, xexp, m, n, ldk, qt, scale, ep, st);
    if (planes == 2) return launch_gemm<2, EPI>(xq, xexp, m, n, ldk, qt, scale, ep, st);
    if (planes == 3) return launch_gemm<3, EPI>(xq, xexp, m, n, ldk, qt, scale, ep, st);
    return ava::fail(AVA_ERR_ARG, "q8 product: planes %d (1..3)", planes);
}

int check_qw(const ava_qw *w) {
    AVA_REQUIRE(w && w->qt && w->scale, AVA_ERR_ARG, "q8: NULL weights");
    AVA_REQUIRE(w->din > 0 && w->dout > 0 && w->ldk == ava::q8_ldk(w->din), AVA_ERR_SHAPE,
                "q8: weights din=%d dout=%d ldk=%d", w->din, w->dout, w->ldk);
    return AVA_OK;
}

}  // namespace

namespace ava {

int launch_quant_rows(const float *x, int m, int k, int ldx, int planes, int8_t *xq, int32_t *xexp,
                      hipStream_t st) {
    const int ldq = q8_ldk(k);
    dim3 grid(ceil_div(m, 4)), block(256);
    if (planes == 1) quant_rows_kernel<1><<<grid, block, 0, st>>>(x, m, k, ldx, xq, xexp, ldq);
    else if (planes == 2) quant_rows_kernel<2><<<grid, block, 0, st>>>(x, m, k, ldx, xq, xexp, ldq);
    else if (planes == 3) quant_rows_kernel<3><<<grid, block, 0, st>>>(x, m, k, ldx, xq, xexp, ldq);
    else return fail(AVA_ERR_ARG, "quant_rows: planes %d (1..3)", planes);
    AVA_LAUNCHED("quant_rows");
    return AVA_OK;
}

// The product with an epilogue: kind 1 store y, 2 y = v * colv[col], 3 y += v. y [m][ldy].
int q8_gemm(const int8_t *xq, const int32_t *xexp, int planes, int m, const ava_qw *w, int kind, float *y, int ldy,
            const float *colv, hipStream_t st) {
    if (int r = check_qw(w)) return r;
    AVA_REQUIRE(xq && y, AVA_ERR_ARG, "q8 product: NULL buffer");
    if (m == 0) return AVA_OK;
    EpiArgs ep{y, ldy, colv, TILE_GROUP};
    if (kind == EPI_STORE) return gemm_planes<EPI_STORE>(planes, xq, xexp, m, w->dout, w->ldk, w->qt, w->scale, ep, st);
    if (kind == EPI_MUL) return gemm_planes<EPI_MUL>(planes, xq, xexp, m, w->dout, w->ldk, w->qt, w->scale, ep, st);
    if (kind == EPI_ADD) return gemm_planes<EPI_ADD>(planes, xq, xexp, m, w->dout, w->ldk, w->qt, w->scale, ep, st);
    return fail(AVA_ERR_ARG, "q8 product: epilogue %d", kind);
}

int q8_small_rows() { return SMALL_ROWS; }

int q8_gemm_lif(const int8_t *xq, const int32_t *xexp, int planes, int m, const ava_qw *w, const float *colv,
                const LifEpi &lif, hipStream_t st) {
    if (int r = check_qw(w)) return r;
    AVA_REQUIRE(xq && lif.ps && lif.v && lif.s && lif.a && lif.spikes, AVA_ERR_ARG, "q8 lif product: NULL buffer");
    AVA_REQUIRE(m > 0 && m <= SMALL_ROWS, AVA_ERR_SHAPE, "q8 lif product: %d rows (the few-rows form only)", m);
    AVA_REQUIRE(lif.levels == 1 || lif.levels == 2, AVA_ERR_ARG, "q8 lif product: levels %d", lif.levels);
    EpiArgs ep{nullptr, 0, colv, 1, lif};
    if (planes == 1) return launch_small<1, EPI_LIF>(xq, xexp, m, w->dout, w->ldk, w->qt, w->scale, ep, st);
    if (planes == 2) return launch_small<2, EPI_LIF>(xq, xexp, m, w->dout, w->ldk, w->qt, w->scale, ep, st);
    if (planes == 3) return launch_small<3, EPI_LIF>(xq, xexp, m, w->dout, w->ldk, w->qt, w->scale, ep, st);
    return fail(AVA_ERR_ARG, "q8 lif product: planes %d", planes);
}

}  // namespace ava

extern "C" int ava_q8_ldk(int k) { return ava::q8_ldk(k); }

extern "C" int ava_q8_pack(const float *w, int din, int dout, int8_t *qt, float *scale, ava_stream stream) {
    AVA_REQUIRE(w && qt && scale, AVA_ERR_ARG, "q8_pack: NULL buffer");
    AVA_REQUIRE(din > 0 && dout > 0, AVA_ERR_SHAPE, "q8_pack: din=%d dout=%d", din, dout);
    hipStream_t st = (hipStream_t)stream;
    const int ldk = ava::q8_ldk(din);
    q8_scale_kernel<<<ava::ceil_div(dout, 256), 256, 0, st>>>(w, din, dout, scale);
    AVA_LAUNCHED("q8_scale");
    q8_pack_kernel<<<dim3(ava::ceil_div(dout, 64), ava::ceil_div(ldk, 64)), 256, 0, st>>>(w, din, dout, ldk, scale, qt);
    AVA_LAUNCHED("q8_pack");
    return AVA_OK;
}

extern "C" int ava_q8_quant_rows(const float *x, int m, int k, int planes, int8_t *xq, int32_t *xexp,
                                 ava_stream stream) {
    AVA_REQUIRE(x && xq && xexp, AVA_ERR_ARG, "quant_rows: NULL buffer");
    AVA_REQUIRE(m >= 0 && k > 0, AVA_ERR_SHAPE, "quant_rows: m=%d k=%d", m, k);
    if (m == 0) return AVA_OK;
    return ava::launch_quant_rows(x, m, k, k, planes, xq, xexp, (hipStream_t)stream);
}

extern "C" int ava_q8_gemm_acc(const int8_t *xq, int planes, int m, const ava_qw *w, int32_t *acc,
                               ava_stream stream) {
    if (int r = check_qw(w)) return r;
    AVA_REQUIRE(xq && acc, AVA_ERR_ARG, "q8_gemm_acc: NULL buffer");
    if (m == 0) return AVA_OK;
    EpiArgs ep{acc, w->dout, nullptr, TILE_GROUP};
    return gemm_planes<EPI_ACC>(planes, xq, nullptr, m, w->dout, w->ldk, w->qt, w->scale, ep, (hipStream_t)stream);
}

extern "C" size_t ava_q8_workspace(int m, int k, int planes) {
    return (size_t)planes * m * ava::q8_ldk(k) + sizeof(int32_t) * (size_t)m + 256;
}

extern "C" int ava_q8_matmul(const float *x, int m, const ava_qw *w, int planes, float *y, void *ws,
                             size_t ws_bytes, ava_stream stream) {
    if (int r = check_qw(w)) return r;
    AVA_REQUIRE(x && y && ws, AVA_ERR_ARG, "q8_matmul: NULL buffer");
    AVA_REQUIRE(planes >= 1 && planes <= 3, AVA_ERR_ARG, "q8_matmul: planes %d (1..3)", planes);
    AVA_REQUIRE(m >= 0, AVA_ERR_SHAPE, "q8_matmul: m=%d", m);
    AVA_REQUIRE(ws_bytes >= ava_q8_workspace(m, w->din, planes), AVA_ERR_SHAPE,
                "q8_matmul: workspace %zu < %zu bytes", ws_bytes, ava_q8_workspace(m, w->din, planes));
    if (m == 0) return AVA_OK;
    hipStream_t st = (hipStream_t)stream;
    int8_t *xq = (int8_t *)ws;
    int32_t *xe = (int32_t *)(((uintptr_t)(xq + (size_t)planes * m * w->ldk) + 255) & ~(uintptr_t)255);
    if (int r = ava::launch_quant_rows(x, m, w->din, w->din, planes, xq, xe, st)) return r;
    return ava::q8_gemm(xq, xe, planes, m, w, EPI_STORE, y, w->dout, nullptr, st);
}

extern "C" int ava_q8_matmul_i8(const int8_t *s, int m, const ava_qw *w, float *y, ava_stream stream) {
    return ava::q8_gemm(s, nullptr, 1, m, w, EPI_STORE, y, w ? w->dout : 0, nullptr, (hipStream_t)stream);
}

extern "C" int ava_q8_matmul_planes(const int8_t *xq, const int32_t *xexp, int planes, int m, const ava_qw *w,
                                    float *y, ava_stream stream) {
    AVA_REQUIRE(xexp, AVA_ERR_ARG, "q8_matmul_planes: NULL row exponents");
    AVA_REQUIRE(m >= 0, AVA_ERR_SHAPE, "q8_matmul_planes: m=%d", m);
    return ava::q8_gemm(xq, xexp, planes, m, w, EPI_STORE, y, w ? w->dout : 0, nullptr, (hipStream_t)stream);
}

// ------------------------------------------------------------------ the product without allocation

namespace {

// The split planes and row exponents of ava_q8_matmul_noalloc: a file-scope device array, one copy
// per GPU the library runs on, held until the process ends. In host code `scratch` names a host-side
// stand-in, not device memory: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is passed to kernels.
constexpr size_t Q8_SCRATCH_BYTES = (size_t)32 << 20;
__device__ __align__(256) unsigned char scratch[Q8_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch[MAX_DEVICES] = {};

// The device address of `scratch` on the current device (looked up on the first call there).
int scratch_ptr(void **out) {
    int dev = 0;
    AVA_HIP(hipGetDevice(&dev));
    AVA_REQUIRE(dev >= 0 && dev < MAX_DEVICES, AVA_ERR_UNSUPPORTED, "q8_matmul_noalloc: device %d (0..%d)", dev,
                MAX_DEVICES - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        AVA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        AVA_REQUIRE(p, AVA_ERR_HIP, "q8_matmul_noalloc: no device address for the scratch array");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return AVA_OK;
}

}  // namespace

extern "C" int ava_q8_matmul_noalloc(const float *x, int m, const ava_qw *w, int planes, float *y,
                                     ava_stream stream) {
    if (int r = check_qw(w)) return r;
    AVA_REQUIRE(x && y, AVA_ERR_ARG, "q8_matmul_noalloc: NULL buffer");
    AVA_REQUIRE(planes >= 1 && planes <= 3, AVA_ERR_ARG, "q8_matmul_noalloc: planes %d (1..3)", planes);
    AVA_REQUIRE(m >= 0, AVA_ERR_SHAPE, "q8_matmul_noalloc: m=%d", m);
    const size_t need = ava_q8_workspace(m, w->din, planes);
    AVA_REQUIRE(need <= Q8_SCRATCH_BYTES, AVA_ERR_SHAPE,
                "q8_matmul_noalloc: %d rows of %d inputs in %d planes need %zu bytes of scratch; the library's "
                "scratch holds %zu (use ava_q8_matmul with a workspace)", m, w->din, planes, need, Q8_SCRATCH_BYTES);
    if (m == 0) return AVA_OK;
    void *ws = nullptr;
    if (int r = scratch_ptr(&ws)) return r;
    hipStream_t st = (hipStream_t)stream;
    int8_t *xq = (int8_t *)ws;
    int32_t *xe = (int32_t *)(((uintptr_t)(xq + (size_t)planes * m * w->ldk) + 255) & ~(uintptr_t)255);
    if (int r = ava::launch_quant_rows(x, m, w->din, w->din, planes, xq, xe, st)) return r;
    return ava::q8_gemm(xq, xe, planes, m, w, EPI_STORE, y, w->dout, nullptr, st);
}
