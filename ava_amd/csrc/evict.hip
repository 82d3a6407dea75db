// The engram store's cap on the device (EngramCap / evict, gpu/state.rs:37-69, 518-590): after a forward,
// a store that holds more than m entries keeps m of them, in store order.
//   oldest      the last m;
//   least-read  per stream, every slot ranks by (class, value, index): class 1 for a slot some later
//               query could see (age >= 1; value = reads / age, its mean attention mass per later
//               query), class 2 for the slots no later query has seen yet; the last m of the ranking
//               stay (gpu/state.rs:540-590 sorts the same tuples).
// One workgroup per stream. The ranking is a selection, not a sort: every slot's tuple maps to one
// 64-bit key that orders as the tuple does (class in the top bit, the non-negative f32 value's bits,
// then the index), so keys are distinct and the kept slots are exactly those whose key is at least the
// m-th largest, found by a bitwise bisection over the key (64 counting passes). The kept slots then
// move to the front in store order, in rounds of 256: a round reads its rows before any of it writes,
// and a kept slot's index is never below its new position, so no later round's source is overwritten.
// The device length, when kept, becomes m in a second launch.
#include "common.h"

#include <hip/hip_fp16.h>

namespace {

constexpr int EV_THREADS = 256;

struct EvictArgs {
    void *k, *v;            // [B][cap][de] (f32, or fp16 with half)
    float *reads, *age;     // [B][cap] (least-read; also moved with the kept slots when present)
    const int32_t *len_dev; // nullable: the length on the device (read instead of n)
    int cap, n, de, half, m, rule;
};

__device__ __forceinline__ uint64_t slot_key(const float *reads, const float *age, int j) {
    const float a = age[j];
    if (a >= 1.0f) {
        const float value = reads[j] / a;  // >= 0: its bits order as the value
        return ((uint64_t)__float_as_uint(value) << 31) | (uint64_t)j;
    }
    return (1ull << 63) | (uint64_t)j;
}

template <typename E>
__global__ __launch_bounds__(EV_THREADS) void evict_kernel(EvictArgs a) {
    __shared__ int s_cnt[EV_THREADS / 64];
    __shared__ int s_src[EV_THREADS];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = min(a.len_dev ? *a.len_dev : a.n, a.cap);
    const int m = a.m;
    if (n <= m) return;
    const float *reads = a.reads ? a.reads + (size_t)b * a.cap : nullptr;
    const float *age = a.age ? a.age + (size_t)b * a.cap : nullptr;
    const bool ranked = a.rule == 1 && reads && age;

    auto block_count = [&](auto pred) {
        int c = 0;
        for (int j = tid; j < n; j += EV_THREADS) c += pred(j) ? 1 : 0;
        c = (int)ava::wave_sum((float)c);  // at most a few tens of thousands: exact in f32
        __syncthreads();
        if (lane == 0) s_cnt[wv] = c;
        __syncthreads();
        return s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
    };
    // the m-th largest key: bit by bit from the top, keep a bit set while at least m keys are >= it
    uint64_t thr = 0;
    if (ranked) {
        for (int bit = 63; bit >= 0; bit--) {
            const uint64_t cand = thr | (1ull << bit);
            if (block_count([&](int j) { return slot_key(reads, age, j) >= cand; }) >= m) thr = cand;
        }
    }
    auto kept = [&](int j) { return ranked ? slot_key(reads, age, j) >= thr : j >= n - m; };

    E *kb = reinterpret_cast<E *>(a.k) + (size_t)b * a.cap * a.de;
    E *vb = reinterpret_cast<E *>(a.v) + (size_t)b * a.cap * a.de;
    float *rw = a.reads ? a.reads + (size_t)b * a.cap : nullptr;
    float *ag = a.age ? a.age + (size_t)b * a.cap : nullptr;
    int done = 0;  // kept slots placed so far
    for (int j0 = 0; j0 < n; j0 += EV_THREADS) {
        // this round's kept slots in order: a block prefix count over j0 .. j0 + 255
        const int j = j0 + tid;
        const bool kp = j < n && kept(j);
        const unsigned long long bal = __ballot(kp);
        const int before = __popcll(bal & ((1ull << lane) - 1ull));
        __syncthreads();
        if (lane == 0) s_cnt[wv] = __popcll(bal);
        __syncthreads();
        int off = 0;
        for (int w = 0; w < wv; w++) off += s_cnt[w];
        const int cnt = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
        if (kp) s_src[off + before] = j;
        __syncthreads();
        if (cnt > 0) {
            // read every moved row of the round, then write (a destination below done + cnt is never a
            // later round's source)
            const int t = tid;
            float r0 = 0.0f, a0 = 0.0f;
            const int sj = t < cnt ? s_src[t] : 0;
            if (t < cnt && rw) {
                r0 = rw[sj];
                a0 = ag[sj];
            }
            // rows move element by element, the round's threads striding over the rows' de values
            const int total = cnt * a.de;
            constexpr int PER = 16;
            E buf[PER];
            for (int base = 0; base < total; base += EV_THREADS * PER) {
#pragma unroll
                for (int u = 0; u < PER; u++) {
                    const int e = base + u * EV_THREADS + tid;
                    if (e < total) {
                        const int r = e / a.de, c = e - r * a.de;
                        buf[u] = kb[(size_t)s_src[r] * a.de + c];
                    }
                }
                __syncthreads();
#pragma unroll
                for (int u = 0; u < PER; u++) {
                    const int e = base + u * EV_THREADS + tid;
                    if (e < total) {
                        const int r = e / a.de, c = e - r * a.de;
                        kb[(size_t)(done + r) * a.de + c] = buf[u];
                    }
                }
                __syncthreads();
#pragma unroll
                for (int u = 0; u < PER; u++) {
                    const int e = base + u * EV_THREADS + tid;
                    if (e < total) {
                        const int r = e / a.de, c = e - r * a.de;
                        buf[u] = vb[(size_t)s_src[r] * a.de + c];
                    }
                }
                __syncthreads();
#pragma unroll
                for (int u = 0; u < PER; u++) {
                    const int e = base + u * EV_THREADS + tid;
                    if (e < total) {
                        const int r = e / a.de, c = e - r * a.de;
                        vb[(size_t)(done + r) * a.de + c] = buf[u];
                    }
                }
                __syncthreads();
            }
            if (t < cnt && rw) {
                rw[done + t] = r0;
                ag[done + t] = a0;
            }
        }
        done += cnt;
        __syncthreads();
    }
}

// the device length after the eviction (a separate launch: every workgroup of the eviction reads it first)
__global__ void clamp_len_kernel(int32_t *len, int m) {
    if (*len > m) *len = m;
}

}  // namespace

extern "C" int ava_engram_evict(void *k, void *v, float *reads, float *age, int B, int cap, int n, int32_t *len_dev,
                                int de, int kv_half, int eng_max, int rule, ava_stream stream) {
    AVA_REQUIRE(k && v, AVA_ERR_ARG, "engram_evict: NULL store");
    AVA_REQUIRE(rule == 0 || rule == 1, AVA_ERR_ARG, "engram_evict: rule %d (0 oldest, 1 least-read)", rule);
    AVA_REQUIRE(rule == 0 || (reads && age), AVA_ERR_ARG, "engram_evict: the least-read rule needs reads and age");
    AVA_REQUIRE(!reads == !age, AVA_ERR_ARG, "engram_evict: reads and age come together");
    AVA_REQUIRE(B >= 0 && cap > 0 && de > 0 && eng_max > 0 && eng_max < cap && n >= 0 && n <= cap, AVA_ERR_SHAPE,
                "engram_evict: B=%d cap=%d n=%d de=%d eng_max=%d", B, cap, n, de, eng_max);
    if (B == 0 || (!len_dev && n <= eng_max)) return AVA_OK;
    EvictArgs a{k, v, reads, age, len_dev, cap, n, de, kv_half, eng_max, rule};
    const hipStream_t st = (hipStream_t)stream;
    if (kv_half) evict_kernel<__half><<<B, EV_THREADS, 0, st>>>(a);
    else evict_kernel<float><<<B, EV_THREADS, 0, st>>>(a);
    AVA_LAUNCHED("engram_evict");
    if (len_dev) {
        clamp_len_kernel<<<1, 1, 0, st>>>(len_dev, eng_max);
        AVA_LAUNCHED("engram_evict length");
    }
    return AVA_OK;
}
