// Shared host/device helpers of libava_amd (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ava.h"

// A raw buffer resource over [base, base + bytes): a load or store through it takes a 32-bit lane
// offset and a wave-uniform offset, so no 64-bit address is held per lane (dword 3 = 0x00020000:
// the gfx9-family raw 32-bit format). Accesses past `bytes` in the lane offset are dropped (loads
// return 0) by the hardware range check; the uniform offset is not range checked.
#if defined(__HIP_DEVICE_COMPILE__)
typedef __amdgpu_buffer_rsrc_t BufRes;
__device__ __forceinline__ BufRes buf_res(float *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void store_f32(BufRes r, unsigned voff, unsigned soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ float load_f32(BufRes r, unsigned voff, unsigned soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ float load_f32_nt(BufRes r, unsigned voff, unsigned soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 2));
}
// the same store, non-temporal (cache policy bit 1: `nt`)
__device__ __forceinline__ void store_f32_nt(BufRes r, unsigned voff, unsigned soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)voff, (int)soff, 2);
}
#else
typedef float *BufRes;  // the host pass compiles no kernel bodies
__device__ inline BufRes buf_res(float *base, unsigned) { return base; }
__device__ inline void store_f32(BufRes, unsigned, unsigned, float) {}
__device__ inline float load_f32(BufRes, unsigned, unsigned) { return 0.0f; }
__device__ inline void store_f32_nt(BufRes, unsigned, unsigned, float) {}
__device__ inline float load_f32_nt(BufRes, unsigned, unsigned) { return 0.0f; }
#endif

// A compiler-only barrier: memory operations are not moved across it. Placed after a batch of
// independent loads it keeps the scheduler from spreading them between their uses, so the whole
// batch is in flight at once (each use still waits only for its own load).
#define AVA_ISSUE_FENCE() asm volatile("" ::: "memory")

namespace ava {

// Per-thread last error (ava_last_error).
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);

// Kernels above 64 KiB of dynamic LDS opt in with a function attribute: set once per (device, kernel),
// under a lock (launches may come from several host threads).
int lds_opt_in(const void *fn, size_t bytes);

// The current device's compute units (looked up once per device).
int device_cus(int *cus);

}  // namespace ava

#define AVA_REQUIRE(cond, code, ...)                     \
    do {                                                 \
        if (!(cond)) return ::ava::fail(code, __VA_ARGS__); \
    } while (0)

#define AVA_HIP(call)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess)                                                             \
            return ::ava::fail(AVA_ERR_HIP, "%s: %s (%s:%d)", #call, hipGetErrorString(e_), \
                               __FILE__, __LINE__);                                      \
    } while (0)

// After a kernel launch: report a launch error as AVA_ERR_HIP.
#define AVA_LAUNCHED(name)                                                                   \
    do {                                                                                     \
        hipError_t e_ = hipGetLastError();                                                   \
        if (e_ != hipSuccess)                                                                \
            return ::ava::fail(AVA_ERR_HIP, "%s launch: %s", name, hipGetErrorString(e_));   \
    } while (0)

namespace ava {

static inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// Leading dimension of int8 operands of the i8 MFMA products: K padded to 128 with zeros (an even
// number of 64-byte K steps).
static inline int q8_ldk(int k) { return (k + 127) / 128 * 128; }

// ---- the split-plane activation format (shared by every producer of a dense int8 product input)
// Row exponent: the smallest e with amax * 2^-e < 127.5, so plane 0 = rint(x 2^-e) fits +-127.
__device__ __forceinline__ int plane_exp(float amax) {
    if (!(amax > 0.0f)) return 0;
    int ex;
    frexpf(amax, &ex);
    int e = ex - 7;
    if (ldexpf(amax, -e) >= 127.5f) e += 1;
    return e;
}

// The planes of one value: t0 = x 2^-e, q0 = rint(t0), t1 = (t0 - q0) 128, q1 = rint(t1), ...
// Every step is exact, so x = 2^e (q0 + q1/128 + q2/16384 + r) with |r| <= 2^-15.
template <int P>
__device__ __forceinline__ void to_planes(float x, int e, int (&q)[P]) {
    float t = ldexpf(x, -e);
#pragma unroll
    for (int p = 0; p < P; p++) {
        float qv = rintf(t);
        q[p] = (int)qv;
        t = (t - qv) * 128.0f;
    }
}

static inline __device__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(uint8_t)(int8_t)a | ((uint32_t)(uint8_t)(int8_t)b << 8) |
           ((uint32_t)(uint8_t)(int8_t)c << 16) | ((uint32_t)(uint8_t)(int8_t)d << 24);
}

// z with P(N(0,1) >= z) = p, 0 < p < 1, to about 1e-3 (a search guess only): the rational
// approximation of Abramowitz and Stegun 26.2.23 on the smaller tail.
__device__ __forceinline__ float normal_upper_quantile(float p) {
    const float q = p < 0.5f ? p : 1.0f - p;
    const float w = sqrtf(-2.0f * __logf(fmaxf(q, 1e-30f)));
    const float z = w - (2.515517f + w * (0.802853f + w * 0.010328f)) /
                            (1.0f + w * (1.432788f + w * (0.189269f + w * 0.001308f)));
    return p < 0.5f ? z : -z;
}

// Wave64 reductions.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Kernels launched by other translation units of the library (host launchers).
int launch_quant_rows(const float *x, int m, int k, int ldx, int planes, int8_t *xq, int32_t *xexp,
                      hipStream_t st);

// q8.hip: the i8 MFMA product with an epilogue (kind 1 store, 2 times colv[col], 3 accumulate into y).
enum { Q8_STORE = 1, Q8_MUL = 2, Q8_ADD = 3 };
int q8_gemm(const int8_t *xq, const int32_t *xexp, int planes, int m, const ava_qw *w, int kind, float *y, int ldy,
            const float *colv, hipStream_t st);

// One LIF step (T = 1) fused into a few-rows product's epilogue: row b = stream b, column c = channel c.
struct LifEpi {
    const float *ps;       // [4][n]: beta | theta | rho | gain
    float *v, *s, *a;      // [m][n] state, updated in place
    int8_t *spikes;        // [m][ldspk] out
    int ldspk, levels, is_signed, alif;
};
// y-less product: cur = planes . W (times colv when colv), then the step; m <= the few-rows limit.
int q8_gemm_lif(const int8_t *xq, const int32_t *xexp, int planes, int m, const ava_qw *w, const float *colv,
                const LifEpi &lif, hipStream_t st);
int q8_small_rows();

// The reference's LIF step (gpu/lif_gen.rs:171-180), every operation rounded on its own (the library
// is compiled with -ffp-contract=off): the spike of membrane v at threshold th, levels each side.
__device__ __forceinline__ float lif_spike(float v, float th, int levels, int is_signed) {
    if (!is_signed) return (v - th >= 0.0f) ? 1.0f : 0.0f;
    float h = 0.0f;
    for (int k = 1; k <= levels; k++) {
        const float kth = th * (float)k;
        h += ((v - kth >= 0.0f) ? 1.0f : 0.0f) - ((-v - kth >= 0.0f) ? 1.0f : 0.0f);
    }
    return h;
}

// lif.hip / kwta.hip / mem.hip
// park (nullable): the state (v, s, a) at the start of every LIF_SEG_STEPS-step segment, as
// park [segment][3][B D] (lif_park_floats), for lif_scan_bwd_seg.
int lif_scan(const float *cur, int B, int T, int D, const float *ps, float *v, float *s, float *a, int levels,
             int is_signed, int alif, int8_t *spikes, float *th_out, hipStream_t st, float *park = nullptr);
// The LIF backward in parallel segments of LIF_SEG_STEPS steps (lif_bwd.hip), for few (stream, channel)
// chains; ws holds lif_bwd_seg_floats(B, T, D) floats; park (nullable) the forward's parked states.
constexpr int LIF_SEG_STEPS = 32;
inline size_t lif_park_floats(int B, int T, int D) {
    return (size_t)((T + LIF_SEG_STEPS - 1) / LIF_SEG_STEPS) * 3 * (size_t)B * D;
}
size_t lif_bwd_seg_floats(int B, int T, int D);
int lif_scan_bwd_seg(const float *cur, int B, int T, int D, const float *ps, const float *v0, const float *s0,
                     const float *a0, int levels, int is_signed, int alif, float slope, int reset_grad,
                     const float *g_spk, const float *g_vT, const float *g_aT, float *dI, float *dv0, float *da0,
                     float *dbeta, float *drho, float *dgain, float *ws, size_t ws_floats, const float *park,
                     hipStream_t st);
int kwta_planes(const float *u, int n, int h, int k, int relu2, int planes, int8_t *xq, int32_t *xexp, int ldq,
                float *kth, hipStream_t st);
int mem_scan_strided(const float *q, const float *k, const float *e, const float *v, const float *la, const float *b,
                     int B, int T, int nh, int ld, int g, int ldg, float m, float cap, float *F, float *S, float *y,
                     int ldy, hipStream_t st);

// bad (nullable) [B]: set to 1 for a stream whose memory inputs held a non-finite value in some head;
// that head's F and S are then left as they were.
int mem_block(const float *P, const float *G, int B, int T, int nh, int r, const float *ba, const float *bb,
              const float *off, const float *wa2, const float *wb2, const float *vres, const float *v0, float *v0_out,
              float m, float cap, float *F, float *S, float *y, int *bad, hipStream_t st);
// x[0..n) = 0 with a kernel (a graph may hold it: no memset node).
int zero_ints(int *x, int n, hipStream_t st);

// glue.hip
int embed(const int32_t *ids, const float *emb, int n, int d, int vocab, float *x, float *x0, hipStream_t st);
int rms_planes(const float *x, int n, int d, const float *gain, int planes, int8_t *xq, int32_t *xexp, int ldq,
               float *hout, hipStream_t st);
// G = h . W in f32 (fp32 MFMA tiles; few rows: a VALU kernel over 4 rows per workgroup).
// rms_planes (no h) and gate_gemm of the normed rows in one launch, the same bits as the two; many
// rows (rms_gate_many_fits: at least 65,536, d = 1024, nc <= 96).
bool rms_gate_many_fits(int n, int d, int nc);
int rms_gate_many(const float *x, int n, int d, const float *gain, int planes, int8_t *xq, int32_t *xexp, int ldq,
                  const float *w, int nc, float *g, hipStream_t st);
int gate_gemm(const float *h, int n, int d, const float *w, int nc, float *g, hipStream_t st);
// For few rows: the norm's planes and the gate projections of the normed rows in one launch.
bool rms_gate_fits(int n, int d, int nc);
int rms_gate(const float *x, int n, int d, const float *gain, int planes, int8_t *xq, int32_t *xexp, int ldq,
             const float *w, int nc, float *g, hipStream_t st);
int mem_post(const float *y, int n, int d, const float *g, int ldg, int planes, int8_t *xq, int32_t *xexp, int ldq,
             hipStream_t st);
// The engram read: the tiled causal form for T > ENGRAM_SPLIT_T, the chunk-split decode form (with
// part, engram_split_floats of scratch) for T <= ENGRAM_SPLIT_T. A store row holds de dims in nh heads
// of 32 or 64 (one head of 64: the single-head read; de / 32 heads: the reference's).
constexpr int ENGRAM_SPLIT_T = 4;
size_t engram_split_floats(int B, int T, int n0, int de = 64, int nh = 1);
// Optional work after the decode form's merge: the read's planes for the next product (xq [planes][rows]
// [ldq], xexp [rows]; xq NULL: none), and the device store length advanced by T (adv NULL: none).
struct PostRead {
    int8_t *xq = nullptr;
    int32_t *xexp = nullptr;
    int ldq = 0, planes = 0;
    int *adv = nullptr;
};
int attend(const float *q, int ldq, const void *ks, const void *vs, int kv_half, int cap, int n0, const int *n0p,
           int B, int T, int de, int nh, float *out, float *part, size_t part_floats, hipStream_t st,
           const PostRead &post = {});
int engram_read(const float *qkv, int ldqkv, int B, int T, int de, int nh, void *ks, void *vs, int kv_half, int cap,
                int n0, int *n0p, float *out, float *part, size_t part_floats, hipStream_t st,
                const PostRead &post = {});
int engram_advance(int *n0p, int T, int cap, hipStream_t st);
// The least-read rule's counts after a read of T queries per stream (q rows ldq floats apart, the store
// already holding the T new keys after its n0 old ones): reads and age [B][cap] advance as
// gpu/memory.rs:700-738 keeps them. ml: 2 B T nh floats of scratch.
int engram_count(const float *q, int ldq, const void *ks, int kv_half, int cap, int n0, int B, int T, int de, int nh,
                 float *ml, float *reads, float *age, hipStream_t st);
// cb.hip: the cerebellum head (code with its unit lists, read-out with the online table, learning)
int cb_code(const float *xf, const int32_t *ids, const float *emb, int n, int d, int vocab, const uint32_t *widx,
            const float *wsgn, int g, int k, int T, float *code, float *keep, int *lcnt, int *lidx, float *lval,
            int lcap, hipStream_t st);
// cb_code, cb_apply_list and the planes of its output in one launch, for few rows (cb_head_fits)
bool cb_head_fits(int n, int d, int g, int planes);
int cb_head(const float *xf, const int32_t *ids, const float *emb, int n, int d, int vocab, const uint32_t *widx,
            const float *wsgn, int g, int k, int T, float *code, float *keep, int *lcnt, int *lidx, float *lval,
            int lcap, const float *w, const float *tab, const double *scale, float *out, int planes, int8_t *xq,
            int32_t *xexp, hipStream_t st);
int cb_apply_list(const float *xf, const float *code, int n, int g, int d, const float *w, const float *tab,
                  const double *scale, int T, const int *lcnt, const int *lidx, const float *lval, int lcap, float *out,
                  hipStream_t st);
int cb_learn(const float *logits, int ldl, int V, const int32_t *next, int B, const float *emb, int d,
             const float *keep, int g, float lr, double fade, double *scale, float *tab, float *err, float *part,
             int nks, float *delta, double *fold, double *nats, hipStream_t st);
// The dense mix into x of the ns streams, the last of which is the block's output (x before the mix:
// the caller exchanges the two buffers instead of copying); x must not be any of the streams.
int dense_mix(float *x, float *const *streams, const float *w, int ns, size_t n, hipStream_t st);
// The same dense mix of [n][d] rows, then the planes of rmsnorm(row) * gain (and the normed row when
// hout); the embedding rows, then the first norm's planes. d <= 1024.
int dense_rms(float *x, float *const *streams, const float *w, int ns, int n, int d, const float *gain, int planes,
              int8_t *xq, int32_t *xexp, int ldq, float *hout, hipStream_t st);
int embed_rms(const int32_t *ids, const float *emb, int n, int d, int vocab, float *x, float *x0, const float *gain,
              int planes, int8_t *xq, int32_t *xexp, int ldq, hipStream_t st);

}  // namespace ava
