// The general LIF scan (int2 / ternary / binary spikes, ALIF trace, per-neuron threshold, carried
// state) for gfx950.
//
// Layout: cur [B][T][D] f32, channel-contiguous, so the lanes of a wavefront that own consecutive
// channels of one stream read one contiguous span per time step (64 lanes x VEC x 4 bytes) and
// write their int8 spikes as one contiguous span. Each lane walks T for its VEC channels with the
// membrane, last spike, trace and reset threshold in registers (no global round trip of the
// state); the next PF time steps are loaded while the current PF are processed, so each wave keeps
// PF x 64 x VEC x 4 bytes of reads in flight, which is what hides HBM latency at one or two waves
// per SIMD.
//
// Arithmetic: the reference's step (gpu/lif_gen.rs:171-180) with every operation rounded on its
// own (this file is compiled with -ffp-contract=off), so spikes and final state are bit-identical
// to the CPU loop.
#include "common.h"

namespace {

template <int LEVELS, bool SIGNED>
__device__ __forceinline__ float spike_of(float v, float th) {
    if (!SIGNED) return (v - th >= 0.0f) ? 1.0f : 0.0f;
    float h = 0.0f;
#pragma unroll
    for (int k = 1; k <= LEVELS; k++) {
        float kth = th * (float)k;
        h += ((v - kth >= 0.0f) ? 1.0f : 0.0f) - ((-v - kth >= 0.0f) ? 1.0f : 0.0f);
    }
    return h;
}

template <int VEC>
struct Vec;
template <>
struct Vec<1> {
    typedef float T;
    static __device__ __forceinline__ float get(const T &x, int) { return x; }
};
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <>
struct Vec<2> {
    typedef f32x2 T;
    static __device__ __forceinline__ float get(const T &x, int i) { return x[i]; }
};
template <>
struct Vec<4> {
    typedef f32x4 T;
    static __device__ __forceinline__ float get(const T &x, int i) { return x[i]; }
};

template <int VEC>
__device__ __forceinline__ void store_spikes(int8_t *dst, const float (&s)[VEC]) {
    if constexpr (VEC == 1) {
        *dst = (int8_t)s[0];
    } else if constexpr (VEC == 2) {
        uint16_t w = (uint16_t)(uint8_t)(int8_t)s[0] | ((uint16_t)(uint8_t)(int8_t)s[1] << 8);
        *(uint16_t *)dst = w;
    } else {
        uint32_t w = (uint32_t)(uint8_t)(int8_t)s[0] | ((uint32_t)(uint8_t)(int8_t)s[1] << 8) |
                     ((uint32_t)(uint8_t)(int8_t)s[2] << 16) | ((uint32_t)(uint8_t)(int8_t)s[3] << 24);
        *(uint32_t *)dst = w;
    }
}

// park (VEC = 1 only; nullable): the state (v, s, a) at the start of every ava::LIF_SEG_STEPS-step
// segment, park [segment][3][B D], for the backward in parallel segments.
template <int VEC, int PF, int LEVELS, bool SIGNED, bool ALIF>
__global__ __launch_bounds__(256) void lif_scan_kernel(const float *__restrict__ cur, int B, int T, int D,
                                                       const float *__restrict__ ps, float *__restrict__ v,
                                                       float *__restrict__ s, float *__restrict__ a,
                                                       int8_t *__restrict__ spikes, float *__restrict__ th_out,
                                                       float *__restrict__ park) {
    typedef typename Vec<VEC>::T V;
    const int nv = D / VEC;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= B * nv) return;
    const int b = gid / nv, c0 = (gid - b * nv) * VEC;

    float bt[VEC], th0[VEC], rho[VEC], omr[VEC], gain[VEC], vv[VEC], sp[VEC], aa[VEC], thp[VEC];
#pragma unroll
    for (int i = 0; i < VEC; i++) {
        const int c = c0 + i, st = b * D + c;
        bt[i] = ps[c];
        th0[i] = ps[D + c];
        rho[i] = ps[2 * D + c];
        gain[i] = ps[3 * D + c];
        omr[i] = 1.0f - rho[i];
        vv[i] = v[st];
        sp[i] = s[st];
        aa[i] = a[st];
        thp[i] = ALIF ? th0[i] + aa[i] * gain[i] : th0[i];
    }

    const size_t chains = (size_t)B * D;
    auto put_park = [&](int sg) {
        if constexpr (VEC == 1) {
            float *pk = park + (size_t)sg * 3 * chains + (size_t)b * D + c0;
            pk[0] = vv[0];
            pk[chains] = sp[0];
            pk[2 * chains] = aa[0];
        }
    };
    if (park) put_park(0);

    const V *src = reinterpret_cast<const V *>(cur + (size_t)b * T * D + c0);
    int8_t *dst = spikes + (size_t)b * T * D + c0;
    const size_t stride = (size_t)nv;  // one time step, in V units

    V buf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++)
        if (i < T) buf[i] = __builtin_nontemporal_load(src + (size_t)i * stride);

    for (int t0 = 0; t0 < T; t0 += PF) {
        V nxt[PF];
#pragma unroll
        for (int i = 0; i < PF; i++) {
            const int t = t0 + PF + i;
            if (t < T) nxt[i] = __builtin_nontemporal_load(src + (size_t)t * stride);
        }
#pragma unroll
        for (int i = 0; i < PF; i++) {
            const int t = t0 + i;
            if (t < T) {
                float out[VEC];
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const float x = Vec<VEC>::get(buf[i], j);
                    float tht = th0[j];
                    if (ALIF) {
                        aa[j] = aa[j] * rho[j] + fabsf(sp[j]) * omr[j];
                        tht = th0[j] + aa[j] * gain[j];
                    }
                    vv[j] = (vv[j] * bt[j] + x) - sp[j] * thp[j];
                    sp[j] = spike_of<LEVELS, SIGNED>(vv[j], tht);
                    thp[j] = tht;
                    out[j] = sp[j];
                }
                store_spikes<VEC>(dst + (size_t)t * D, out);
                if (park && (t + 1) % ava::LIF_SEG_STEPS == 0 && t + 1 < T) put_park((t + 1) / ava::LIF_SEG_STEPS);
            }
        }
#pragma unroll
        for (int i = 0; i < PF; i++) buf[i] = nxt[i];
    }

#pragma unroll
    for (int i = 0; i < VEC; i++) {
        const int st = b * D + c0 + i;
        v[st] = vv[i];
        s[st] = sp[i];
        a[st] = aa[i];
        if (th_out) th_out[st] = thp[i];
    }
}

// The same scan for one channel per lane when D is a multiple of 64 (a wave's lanes are 64
// consecutive channels of one stream): the currents are read and the spikes written through buffer
// resources based at the wave's first channel, with the lane's channel as the 32-bit lane offset and
// the time step t D as the wave-uniform offset, so a step costs no 64-bit address arithmetic; whole
// blocks of PF steps run without per-step bound checks, and a segment's parked state is written at the
// end of its block (PF = LIF_SEG_STEPS). The same arithmetic as lif_scan_kernel, so the same bits.
template <int PF, int LEVELS, bool SIGNED, bool ALIF>
__global__ __launch_bounds__(256) void lif_scan_buf_kernel(const float *__restrict__ cur, int B, int T, int D,
                                                           const float *__restrict__ ps, float *__restrict__ v,
                                                           float *__restrict__ s, float *__restrict__ a,
                                                           int8_t *__restrict__ spikes, float *__restrict__ th_out,
                                                           float *__restrict__ park) {
    static_assert(PF == ava::LIF_SEG_STEPS, "a parked segment is one block");
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= B * D) return;  // whole waves (B D is a multiple of 64)
    const int lane = threadIdx.x & 63;
    const int gw = __builtin_amdgcn_readfirstlane(gid - lane);  // the wave's first chain
    const int bw = gw / D, cw = gw - bw * D, c = cw + lane, st = gw + lane;

    const float bt = ps[c], th0 = ps[D + c], rho = ps[2 * D + c], gain = ps[3 * D + c];
    const float omr = 1.0f - rho;
    float vv = v[st], sp = s[st], aa = a[st];
    float thp = ALIF ? th0 + aa * gain : th0;

    const size_t chains = (size_t)B * D;
    auto put_park = [&](int sg) {
        float *pk = park + (size_t)sg * 3 * chains + st;
        pk[0] = vv;
        pk[chains] = sp;
        pk[2 * chains] = aa;
    };
    if (park) put_park(0);

    const size_t slab = (size_t)bw * T * D + cw;  // the wave's first channel at t = 0
    const unsigned span = (unsigned)(T * D - cw);  // elements from there to the slab's end
    const BufRes cr = buf_res(const_cast<float *>(cur) + slab, span * 4u);
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(spikes + slab, 0, (int)span, 0x00020000);
#endif
    const unsigned lv = (unsigned)lane * 4u, row4 = (unsigned)D * 4u;
    auto step = [&](float x, unsigned t) {
        float tht = th0;
        if (ALIF) {
            aa = aa * rho + fabsf(sp) * omr;
            tht = th0 + aa * gain;
        }
        vv = (vv * bt + x) - sp * thp;
        sp = spike_of<LEVELS, SIGNED>(vv, tht);
        thp = tht;
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(int8_t)sp, sr, lane, (int)(t * (unsigned)D), 0);
#endif
    };

    float buf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) buf[i] = load_f32_nt(cr, lv, (unsigned)min(i, T - 1) * row4);
    const int full = T / PF;
    for (int blk = 0; blk < full; blk++) {
        const unsigned t0 = (unsigned)blk * PF;
        float nxt[PF];
        // the next block's currents (past T: the last step again, unused)
#pragma unroll
        for (int i = 0; i < PF; i++) nxt[i] = load_f32_nt(cr, lv, (unsigned)min((int)t0 + PF + i, T - 1) * row4);
#pragma unroll
        for (int i = 0; i < PF; i++) step(buf[i], t0 + i);
        if (park && (int)t0 + PF < T) put_park(blk + 1);
#pragma unroll
        for (int i = 0; i < PF; i++) buf[i] = nxt[i];
    }
    for (int t = full * PF; t < T; t++) step(buf[t - full * PF], (unsigned)t);

    v[st] = vv;
    s[st] = sp;
    a[st] = aa;
    if (th_out) th_out[st] = thp;
}

template <int VEC, int PF>
int launch_vp(const float *cur, int B, int T, int D, const float *ps, float *v, float *s, float *a,
              int levels, int is_signed, int alif, int8_t *spikes, float *th_out, hipStream_t st,
              float *park = nullptr) {
    AVA_REQUIRE(!park || VEC == 1, AVA_ERR_ARG, "lif_scan: parked states need one channel per lane");
    const long threads = (long)B * (D / VEC);
    dim3 grid(ava::ceil_div(threads, 256)), block(256);
    // the buffer form: whole waves per stream, and every offset of a stream's slab in 32 bits
    const bool bufd = VEC == 1 && PF == ava::LIF_SEG_STEPS && D % 64 == 0 && (long)T * D * 4 < (1L << 31);
#define AVA_LIF_GO(L, S, A)                                                                                         \
    do {                                                                                                            \
        if (bufd)                                                                                                   \
            lif_scan_buf_kernel<PF, L, S, A><<<grid, block, 0, st>>>(cur, B, T, D, ps, v, s, a, spikes, th_out,    \
                                                                     park);                                         \
        else                                                                                                        \
            lif_scan_kernel<VEC, PF, L, S, A><<<grid, block, 0, st>>>(cur, B, T, D, ps, v, s, a, spikes, th_out,   \
                                                                      park);                                        \
    } while (0)
    if (!is_signed) {
        if (alif) AVA_LIF_GO(1, false, true);
        else AVA_LIF_GO(1, false, false);
    } else if (levels == 1) {
        if (alif) AVA_LIF_GO(1, true, true);
        else AVA_LIF_GO(1, true, false);
    } else {
        if (alif) AVA_LIF_GO(2, true, true);
        else AVA_LIF_GO(2, true, false);
    }
#undef AVA_LIF_GO
    AVA_LAUNCHED("lif_scan");
    return AVA_OK;
}

}  // namespace

namespace ava {

// One channel per lane, 32 steps in flight: the fastest of 16, 32, 48 and 64 steps and of 1, 2 or 4
// channels per lane at config[1]'s 131,072 lanes and at the block stack's 65,536.
constexpr int LIF_VEC = 1, LIF_PF = 32;

int lif_scan(const float *cur, int B, int T, int D, const float *ps, float *v, float *s, float *a, int levels,
             int is_signed, int alif, int8_t *spikes, float *th_out, hipStream_t st, float *park) {
    AVA_REQUIRE(cur && ps && v && s && a && spikes, AVA_ERR_ARG, "lif_scan: NULL buffer");
    AVA_REQUIRE(B > 0 && T > 0 && D > 0, AVA_ERR_SHAPE, "lif_scan: B=%d T=%d D=%d", B, T, D);
    AVA_REQUIRE(levels == 1 || levels == 2, AVA_ERR_ARG, "lif_scan: levels %d (1 or 2)", levels);
    return launch_vp<LIF_VEC, LIF_PF>(cur, B, T, D, ps, v, s, a, levels, is_signed, alif, spikes, th_out, st, park);
}

}  // namespace ava

extern "C" int ava_lif_scan(const float *cur, int B, int T, int D, const float *ps, float *v, float *s,
                            float *a, int levels, int is_signed, int alif, int8_t *spikes, float *th_out,
                            ava_stream stream) {
    return ava::lif_scan(cur, B, T, D, ps, v, s, a, levels, is_signed, alif, spikes, th_out, (hipStream_t)stream);
}
