// The Ava-0.4-shaped int8 block stack on one GPU: weights, scratch and the per-block launch
// sequence (include/ava.h: ava_model_*).
//
// Order of operations per block, as gpu/arch.rs:1592-1867 (block_arch) with carried state as
// gpu/state.rs:870-1071 (block_state):
//   spiking layer   h = rms(x) -> planes -> cur = (h.Win) (1 - beta) -> LIF scan -> x += s.Wout
//   memory          h = rms(x) -> P = h.[Wq|Wk|Wv|We|Wg] (one product), G = h.[Wa|Wb|Wa1|Wb1] (f32)
//                   -> one kernel: prep (unit q, k, e; value residual; log alpha, b) + scan
//                   -> head norm * silu(g) -> x += o.Wo
//   engram (one block)  h = rms(x) -> [q|k|v] -> append k, v to the store -> causal read -> x += o.Wo
//   sparse MLP      h = rms(x) -> u = h.W1 -> kWTA, relu^2 -> planes -> x += a.W2
//   dense mix       stream_{i+1} = x; x += sum_j w_j stream_j
// then the final norm and the head (E^T in int8). Every product input is produced directly in
// split-plane form by the kernel before it (RMSNorm, the read-out, kWTA), so no f32 activation is
// written only to be re-read by a quantizer.
#include <math.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

#include "common.h"

namespace {

// The engram's heads: eng_heads <= 1 is one head of eng_dim.
int eng_nh(const ava_config &c) { return c.eng_heads > 1 ? c.eng_heads : 1; }

struct DevQW {
    ava_qw w{};
};

struct Block {
    float *lif_norm = nullptr, *ps = nullptr, *omb = nullptr;
    DevQW win, wout;
    float *mem_norm = nullptr;
    DevQW wproj;  // [Wq | Wk | Wv | We | Wg], d x 5d
    float *wgate = nullptr;  // [Wa | Wb | Wa1 | Wb1], d x (2 nh + 2 r), f32
    float *ba = nullptr, *bb = nullptr, *off = nullptr, *wa2 = nullptr, *wb2 = nullptr, *vres = nullptr;
    DevQW wo;
    bool eng = false;
    float *eng_norm = nullptr;
    DevQW eqkv, ewo;  // [Wq | Wk | Wv] d x 3de, Wo de x d
    float *mlp_norm = nullptr;
    DevQW w1, w2;
    std::vector<float> dense;  // i + 2 mixing weights (host)
};

struct Timer {
    std::vector<std::pair<const char *, std::pair<hipEvent_t, hipEvent_t>>> pending;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    struct Sum {
        const char *name;  // the launch site's string literal
        int calls;
        double ms;
    };
    std::map<std::string, Sum> sums;
};

}  // namespace

struct ava_model {
    ava_config cfg{};
    int device = 0;
    float *tok_emb = nullptr, *final_norm = nullptr;
    DevQW head;
    std::vector<Block> blocks;
    std::vector<void *> allocs;  // everything the model owns

    // scratch for up to `rows` rows
    size_t rows = 0, scratch_bytes = 0;
    std::vector<void *> scratch;
    float *x = nullptr, *h = nullptr, *cur = nullptr, *P = nullptr, *G = nullptr;
    float *y = nullptr, *v0 = nullptr, *u = nullptr, *qkv = nullptr, *eo = nullptr;
    int8_t *xq = nullptr, *spk = nullptr;
    int32_t *xexp = nullptr;
    std::vector<float *> streams;
    // [rows]: the last forward's streams that met a non-finite memory input (ava_model_nonfinite)
    int *bad = nullptr;
    int bad_n = 0;

    // the cerebellum head (cfg.cb_units > 0): the fixed wiring, the read-out (NULL: zero), the fade
    uint32_t *cb_idx = nullptr;
    float *cb_sgn = nullptr, *cb_w = nullptr;
    int cb_k = 0;
    double cb_fade = 1.0;
    float *cb_codes = nullptr;  // scratch [rows][cb_units]
    int *cb_lcnt = nullptr, *cb_lidx = nullptr;  // the codes' unit lists: [rows], [rows][cb_lcap]
    float *cb_lval = nullptr;
    int cb_lcap = 0;
    // the learning step's scratch for up to cb_rows streams
    int cb_rows = 0;
    float *cb_err = nullptr, *cb_part = nullptr, *cb_delta = nullptr;
    double *cb_fold = nullptr;
    // the decode engram read's chunk partials (grow-only)
    float *att_part = nullptr;
    size_t att_part_floats = 0;
    float *eml = nullptr;  // the least-read counts' per-(query, head) max and sum
    size_t eml_floats = 0;
    // set while captured graphs hold the scratch's addresses: nothing is freed or reallocated
    bool frozen = false;

    // the decision trace (ava_model_set_trace): [layers][tr_rows][...] buffers, the next row tr_pos
    int8_t *tr_spk = nullptr;
    float *tr_u = nullptr, *tr_kth = nullptr;
    size_t tr_rows = 0, tr_pos = 0;

    bool timing = false;
    Timer timer;
    hipStream_t last_stream = nullptr;
    // ava_model_decode_step: the stream the previous token's table step runs on, and the events that
    // fork it from and join it back to the caller's stream (made at build when the model has a table)
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

namespace {

float sigmoid_host(float x) { return 1.0f / (expf(-x) * 1.0f + 1.0f); }  // gpu/model.rs:465-467

int dev_alloc(ava_model *m, void **p, size_t bytes, bool scratch = false) {
    AVA_HIP(hipMalloc(p, bytes < 256 ? 256 : bytes));
    (scratch ? m->scratch : m->allocs).push_back(*p);
    if (scratch) m->scratch_bytes += bytes;
    return AVA_OK;
}

int upload(ava_model *m, float **dst, const float *src, size_t n) {
    AVA_REQUIRE(src, AVA_ERR_ARG, "model: a required parameter is NULL");
    if (int r = dev_alloc(m, (void **)dst, n * sizeof(float))) return r;
    AVA_HIP(hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice));
    return AVA_OK;
}

// Quantize host W [din][dout] (several matrices side by side: parts[i] is [din][cols[i]]) into one
// int8 matrix; per-column scales make the merged product column-for-column the separate ones
// (gpu/int8.rs:89-102, Q8Set::merged).
int quantize(ava_model *m, DevQW *q, int din, const std::vector<std::pair<const float *, int>> &parts) {
    int dout = 0;
    for (auto &p : parts) {
        AVA_REQUIRE(p.first, AVA_ERR_ARG, "model: a required weight matrix is NULL");
        dout += p.second;
    }
    std::vector<float> w((size_t)din * dout);
    int c0 = 0;
    for (auto &p : parts) {
        for (int j = 0; j < din; j++) memcpy(&w[(size_t)j * dout + c0], p.first + (size_t)j * p.second, sizeof(float) * p.second);
        c0 += p.second;
    }
    float *wd = nullptr;
    AVA_HIP(hipMalloc(&wd, w.size() * sizeof(float)));
    AVA_HIP(hipMemcpy(wd, w.data(), w.size() * sizeof(float), hipMemcpyHostToDevice));
    q->w.din = din;
    q->w.dout = dout;
    q->w.ldk = ava::q8_ldk(din);
    int r = dev_alloc(m, (void **)&q->w.qt, (size_t)dout * q->w.ldk);
    if (!r) r = dev_alloc(m, (void **)&q->w.scale, sizeof(float) * dout);
    if (!r) r = ava_q8_pack(wd, din, dout, q->w.qt, q->w.scale, nullptr);
    hipError_t e1 = hipDeviceSynchronize();
    hipError_t e2 = hipFree(wd);
    if (r) return r;
    AVA_REQUIRE(e1 == hipSuccess && e2 == hipSuccess, AVA_ERR_HIP, "model: weight quantization failed: %s",
                hipGetErrorString(e1 != hipSuccess ? e1 : e2));
    return AVA_OK;
}

// The cerebellum's fixed granule wiring (gpu/v51b.rs:242-265): xorshift64 from seed | 1; per unit,
// `fan` distinct inputs of `inputs` drawn as next() % inputs, then one sign per input from next() & 1,
// amplitude 1/sqrt(fan). The seed is the reference's CB_SEED (gpu/v51b.rs:49).
void cb_wiring(int inputs, int g, int fan, std::vector<uint32_t> &idx, std::vector<float> &sgn) {
    uint64_t s = 0x51B0CE7EULL | 1ULL;
    auto next = [&]() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    };
    const float amp = 1.0f / sqrtf((float)fan);
    idx.assign((size_t)g * fan, 0);
    sgn.assign((size_t)g * fan, 0.0f);
    for (int j = 0; j < g; j++) {
        uint32_t picked[8];
        int np = 0;
        while (np < std::min(fan, inputs)) {
            const uint32_t r = (uint32_t)(next() % (uint64_t)inputs);
            bool seen = false;
            for (int a = 0; a < np; a++) seen = seen || picked[a] == r;
            if (!seen) picked[np++] = r;
        }
        for (int a = 0; a < np; a++) {
            idx[(size_t)j * fan + a] = picked[a];
            sgn[(size_t)j * fan + a] = (next() & 1) == 0 ? amp : -amp;
        }
    }
}

int build(ava_model *m, const ava_params *prm) {
    const ava_config &c = m->cfg;
    const int d = c.d, nh = d / c.head_size, r = c.gate_rank, de = c.eng_dim, H = c.hidden;
    AVA_REQUIRE(prm && prm->blocks && prm->tok_emb && prm->final_norm, AVA_ERR_ARG, "model: NULL parameters");
    if (int e = upload(m, &m->tok_emb, prm->tok_emb, (size_t)c.vocab * d)) return e;
    if (int e = upload(m, &m->final_norm, prm->final_norm, d)) return e;
    {
        std::vector<float> et((size_t)d * c.vocab);  // E^T: one scale per vocab row (int8.rs:81-84)
        for (int v = 0; v < c.vocab; v++)
            for (int j = 0; j < d; j++) et[(size_t)j * c.vocab + v] = prm->tok_emb[(size_t)v * d + j];
        if (int e = quantize(m, &m->head, d, {{et.data(), c.vocab}})) return e;
    }
    if (c.cb_units > 0) {
        std::vector<uint32_t> idx;
        std::vector<float> sgn;
        cb_wiring(2 * d, c.cb_units, 4, idx, sgn);
        if (int e = dev_alloc(m, (void **)&m->cb_idx, idx.size() * sizeof(uint32_t))) return e;
        AVA_HIP(hipMemcpy(m->cb_idx, idx.data(), idx.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
        if (int e = upload(m, &m->cb_sgn, sgn.data(), sgn.size())) return e;
        if (prm->cb_w)
            if (int e = upload(m, &m->cb_w, prm->cb_w, (size_t)c.cb_units * d)) return e;
        m->cb_k = c.cb_units / 32;  // gpu/v51b.rs:47 (CB_SPARSITY)
        m->cb_fade = c.cb_half > 0.0f ? exp2(-1.0 / (double)c.cb_half) : 1.0;
        AVA_HIP(hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking));  // default priority
        AVA_HIP(hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming));
        AVA_HIP(hipEventCreateWithFlags(&m->ev_join, hipEventDisableTiming));
    }
    m->blocks.resize(c.layers);
    for (int i = 0; i < c.layers; i++) {
        const ava_block_params &p = prm->blocks[i];
        Block &b = m->blocks[i];
        int e = 0;
        if ((e = upload(m, &b.lif_norm, p.lif_norm, d))) return e;
        AVA_REQUIRE(p.beta_p && p.theta, AVA_ERR_ARG, "model: block %d has no LIF leak/threshold", i);
        AVA_REQUIRE(!c.alif || (p.arho && p.again), AVA_ERR_ARG, "model: block %d: alif needs arho and again", i);
        std::vector<float> ps(4 * (size_t)d), omb(d);
        for (int k = 0; k < d; k++) {
            const float beta = sigmoid_host(p.beta_p[k]);
            ps[k] = beta;
            ps[d + k] = p.theta[k];
            ps[2 * d + k] = c.alif ? sigmoid_host(p.arho[k]) : 0.0f;
            ps[3 * d + k] = c.alif ? p.again[k] : 0.0f;
            omb[k] = beta * -1.0f + 1.0f;  // beta.affine(-1, 1) (arch.rs:1636-1638)
        }
        if ((e = upload(m, &b.ps, ps.data(), ps.size()))) return e;
        if ((e = upload(m, &b.omb, omb.data(), omb.size()))) return e;
        if ((e = quantize(m, &b.win, d, {{p.win, d}}))) return e;
        if ((e = quantize(m, &b.wout, d, {{p.wout, d}}))) return e;
        if ((e = upload(m, &b.mem_norm, p.mem_norm, d))) return e;
        if ((e = quantize(m, &b.wproj, d, {{p.wq, d}, {p.wk, d}, {p.wv, d}, {p.we, d}, {p.wg, d}}))) return e;
        {
            const int nc = 2 * nh + 2 * r;
            AVA_REQUIRE(p.wa && p.wb && p.wa1 && p.wb1, AVA_ERR_ARG, "model: block %d has no gate projections", i);
            std::vector<float> wg((size_t)d * nc);
            for (int j = 0; j < d; j++) {
                float *row = &wg[(size_t)j * nc];
                memcpy(row, p.wa + (size_t)j * nh, sizeof(float) * nh);
                memcpy(row + nh, p.wb + (size_t)j * nh, sizeof(float) * nh);
                memcpy(row + 2 * nh, p.wa1 + (size_t)j * r, sizeof(float) * r);
                memcpy(row + 2 * nh + r, p.wb1 + (size_t)j * r, sizeof(float) * r);
            }
            if ((e = upload(m, &b.wgate, wg.data(), wg.size()))) return e;
        }
        if ((e = upload(m, &b.ba, p.ba, nh))) return e;
        if ((e = upload(m, &b.bb, p.bb, nh))) return e;
        if ((e = upload(m, &b.off, p.off, d))) return e;
        if ((e = upload(m, &b.wa2, p.wa2, (size_t)r * d))) return e;
        if ((e = upload(m, &b.wb2, p.wb2, (size_t)r * d))) return e;
        if (c.value_residual && i > 0) {
            AVA_REQUIRE(p.vres, AVA_ERR_ARG, "model: block %d: value residual needs vres", i);
            if ((e = upload(m, &b.vres, p.vres, 2))) return e;
        }
        if ((e = quantize(m, &b.wo, d, {{p.wo, d}}))) return e;
        if (i == c.eng_block) {
            b.eng = true;
            if ((e = upload(m, &b.eng_norm, p.eng_norm, d))) return e;
            if ((e = quantize(m, &b.eqkv, d, {{p.ewq, de}, {p.ewk, de}, {p.ewv, de}}))) return e;
            if ((e = quantize(m, &b.ewo, de, {{p.ewo, d}}))) return e;
        }
        if ((e = upload(m, &b.mlp_norm, p.mlp_norm, d))) return e;
        if ((e = quantize(m, &b.w1, d, {{p.w1, H}}))) return e;
        if ((e = quantize(m, &b.w2, H, {{p.w2, d}}))) return e;
        if (c.dense) {
            AVA_REQUIRE(p.dense, AVA_ERR_ARG, "model: block %d: dense mix needs its weights", i);
            b.dense.assign(p.dense, p.dense + i + 2);
        }
    }
    return AVA_OK;
}

int ensure_scratch(ava_model *m, size_t rows) {
    if (rows <= m->rows) return AVA_OK;
    AVA_REQUIRE(!m->frozen, AVA_ERR_ARG, "forward: %zu rows need more scratch, and the model's scratch is frozen "
                "(a captured graph uses it)", rows);
    for (void *p : m->scratch) (void)hipFree(p);
    m->scratch.clear();
    m->streams.clear();
    m->scratch_bytes = 0;
    m->rows = 0;
    const ava_config &c = m->cfg;
    const size_t d = c.d, H = c.hidden, de = c.eng_dim, nc = 2 * (d / c.head_size) + 2 * c.gate_rank;
    const size_t ldq = std::max<size_t>(ava::q8_ldk((int)H), std::max<size_t>(ava::q8_ldk((int)d), ava::q8_ldk((int)de)));
    int e = 0;
    auto A = [&](void **p, size_t bytes) {
        if (!e) e = dev_alloc(m, p, bytes, true);
    };
    A((void **)&m->x, rows * d * 4);
    A((void **)&m->h, rows * d * 4);
    A((void **)&m->cur, rows * d * 4);
    A((void **)&m->P, rows * 5 * d * 4);
    A((void **)&m->G, rows * nc * 4);
    A((void **)&m->y, rows * d * 4);
    if (c.value_residual) A((void **)&m->v0, rows * d * 4);
    A((void **)&m->u, rows * H * 4);
    if (c.eng_block >= 0) {
        A((void **)&m->qkv, rows * 3 * de * 4);
        A((void **)&m->eo, rows * de * 4);
    }
    A((void **)&m->xq, (size_t)c.planes * rows * ldq);
    A((void **)&m->xexp, rows * 4);
    A((void **)&m->spk, rows * ava::q8_ldk((int)d));
    A((void **)&m->bad, rows * 4);
    if (c.dense) {
        m->streams.resize(c.layers + 1);
        for (auto &s : m->streams) A((void **)&s, rows * d * 4);
    }
    if (c.cb_units > 0) {
        A((void **)&m->cb_codes, rows * c.cb_units * 4);
        m->cb_lcap = std::min(1024, 2 * (c.cb_units / 32));  // room for ties beyond the k kept
        A((void **)&m->cb_lcnt, rows * 4);
        A((void **)&m->cb_lidx, rows * m->cb_lcap * 4);
        A((void **)&m->cb_lval, rows * m->cb_lcap * 4);
    }
    if (e) return e;
    m->rows = rows;
    return AVA_OK;
}

// Launch timing (ava_model_set_timing).
struct Scope {
    ava_model *m;
    const char *name;
    hipStream_t st;
    hipEvent_t b = nullptr;
    Scope(ava_model *m_, const char *n, hipStream_t s) : m(m_), name(n), st(s) {
        if (!m->timing) return;
        b = ev();
        (void)hipEventRecord(b, st);
    }
    hipEvent_t ev() {
        Timer &t = m->timer;
        if (t.used == t.pool.size()) {
            hipEvent_t e;
            (void)hipEventCreate(&e);
            t.pool.push_back(e);
        }
        return t.pool[t.used++];
    }
    ~Scope() {
        if (!m->timing) return;
        hipEvent_t e = ev();
        (void)hipEventRecord(e, st);
        m->timer.pending.push_back({name, {b, e}});
    }
};

#define AVA_RUN(name, call)                          \
    do {                                             \
        Scope sc_(m, name, st);                      \
        if (int r_ = (call)) return r_;              \
    } while (0)

int collect(ava_model *m) {
    Timer &t = m->timer;
    if (t.pending.empty()) return AVA_OK;
    AVA_HIP(hipStreamSynchronize(m->last_stream));
    for (auto &p : t.pending) {
        float ms = 0.0f;
        AVA_HIP(hipEventElapsedTime(&ms, p.second.first, p.second.second));
        auto it = t.sums.find(p.first);
        if (it == t.sums.end()) it = t.sums.emplace(p.first, Timer::Sum{p.first, 0, 0.0}).first;
        it->second.calls += 1;
        it->second.ms += ms;
    }
    t.pending.clear();
    t.used = 0;
    return AVA_OK;
}

int trace_copy(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t height,
               hipStream_t st) {
    AVA_HIP(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToDevice, st));
    return AVA_OK;
}

// join (nullable): an event the forward waits for before the final norm and the cerebellum (which
// read and overwrite the code, the table and its scale).
int forward(ava_model *m, ava_state *s, const int32_t *ids, int B, int T, float *logits, hipStream_t st,
            hipEvent_t join = nullptr) {
    m->bad_n = 0;  // a forward refused below reports no rows of an earlier one
    const ava_config &c = m->cfg;
    const int d = c.d, nh = d / c.head_size, r = c.gate_rank, H = c.hidden, de = c.eng_dim, L = c.layers;
    const int P = c.planes, N = B * T, ldd = ava::q8_ldk(d), ldh = ava::q8_ldk(H);
    AVA_REQUIRE(s && s->lif_v && s->lif_s && s->lif_a && s->mem_f, AVA_ERR_ARG, "forward: state buffers are NULL");
    AVA_REQUIRE(c.momentum == 0.0f || s->mem_s, AVA_ERR_ARG, "forward: momentum needs state mem_s");
    AVA_REQUIRE(c.eng_block < 0 || (s->eng_k && s->eng_v && s->eng_len >= 0 && s->eng_len + T <= s->eng_cap),
                AVA_ERR_SHAPE, "forward: the engram store holds %d of %d entries, %d more do not fit", s->eng_len,
                s->eng_cap, T);
    const bool tracing = m->tr_spk != nullptr;
    AVA_REQUIRE(!tracing || m->tr_pos + (size_t)N <= m->tr_rows, AVA_ERR_SHAPE,
                "forward: the decision trace holds %zu rows, %zu are used and %d more do not fit", m->tr_rows,
                m->tr_pos, N);
    if (int e = ensure_scratch(m, (size_t)N)) return e;
    if (c.eng_block >= 0) {
        // sized for the fullest store this state can reach, so a decode loop allocates once
        const size_t need = ava::engram_split_floats(B, T, s->eng_cap - T, c.eng_dim, eng_nh(c));
        if (need > m->att_part_floats) {
            AVA_REQUIRE(!m->frozen, AVA_ERR_ARG, "forward: the engram read needs more scratch, and the model's "
                        "scratch is frozen (a captured graph uses it)");
            (void)hipFree(m->att_part);
            m->att_part = nullptr;
            m->att_part_floats = 0;
            AVA_HIP(hipMalloc(&m->att_part, need * sizeof(float)));
            m->att_part_floats = need;
        }
        const size_t need_ml = (s->eng_reads && s->eng_age) ? 2 * (size_t)N * eng_nh(c) : 0;
        if (need_ml > m->eml_floats) {
            AVA_REQUIRE(!m->frozen, AVA_ERR_ARG, "forward: the store's read counts need more scratch, and the "
                        "model's scratch is frozen (a captured graph uses it)");
            (void)hipFree(m->eml);
            m->eml = nullptr;
            m->eml_floats = 0;
            AVA_HIP(hipMalloc(&m->eml, need_ml * sizeof(float)));
            m->eml_floats = need_ml;
        }
    }
    if (m->timing && m->last_stream != st) {
        if (int e = collect(m)) return e;
    }
    m->last_stream = st;

    const bool cb = logits && c.cb_units > 0 && s->cb_code;
    AVA_RUN("zero_ints", ava::zero_ints(m->bad, B, st));
    m->bad_n = B;
    // the embedding and the first block's norm planes in one pass; after each block the dense mix and
    // the next norm's planes in one pass (ready: the planes of the next norm are already in xq)
    AVA_RUN("embed", ava::embed_rms(ids, m->tok_emb, N, d, c.vocab, m->x, c.dense ? m->streams[0] : nullptr,
                                    m->blocks[0].lif_norm, P, m->xq, m->xexp, ldd, st));
    bool ready = true, final_ready = false, advanced = false;
    for (int i = 0; i < L; i++) {
        const Block &b = m->blocks[i];
        const size_t sbd = (size_t)i * B * d;
        // the spiking layer
        if (!ready) AVA_RUN("rms_planes", ava::rms_planes(m->x, N, d, b.lif_norm, P, m->xq, m->xexp, ldd, nullptr, st));
        ready = false;
        if (T == 1 && N <= ava::q8_small_rows()) {
            // one token per stream: the LIF step runs in the Win product's epilogue
            const ava::LifEpi lif{b.ps, s->lif_v + sbd, s->lif_s + sbd, s->lif_a + sbd, m->spk, ava::q8_ldk(d),
                                  c.levels, 1, c.alif};
            AVA_RUN("q8_gemm", ava::q8_gemm_lif(m->xq, m->xexp, P, N, &b.win.w, c.lif_scale ? b.omb : nullptr, lif, st));
        } else {
            AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.win.w, c.lif_scale ? ava::Q8_MUL : ava::Q8_STORE,
                                            m->cur, d, b.omb, st));
            AVA_RUN("lif_scan", ava::lif_scan(m->cur, B, T, d, b.ps, s->lif_v + sbd, s->lif_s + sbd,
                                              s->lif_a + sbd, c.levels, 1, c.alif, m->spk, nullptr, st));
        }
        if (tracing)
            AVA_RUN("trace", trace_copy(m->tr_spk + ((size_t)i * m->tr_rows + m->tr_pos) * d, d, m->spk, ldd, d, N, st));
        AVA_RUN("q8_gemm", ava::q8_gemm(m->spk, nullptr, 1, N, &b.wout.w, ava::Q8_ADD, m->x, d, nullptr, st));
        // the fast-weight memory
        if (ava::rms_gate_fits(N, d, 2 * nh + 2 * r)) {
            AVA_RUN("rms_planes", ava::rms_gate(m->x, N, d, b.mem_norm, P, m->xq, m->xexp, ldd, b.wgate, 2 * nh + 2 * r,
                                                m->G, st));
            AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.wproj.w, ava::Q8_STORE, m->P, 5 * d, nullptr, st));
        } else if (ava::rms_gate_many_fits(N, d, 2 * nh + 2 * r)) {
            AVA_RUN("rms_gate", ava::rms_gate_many(m->x, N, d, b.mem_norm, P, m->xq, m->xexp, ldd, b.wgate,
                                                   2 * nh + 2 * r, m->G, st));
            AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.wproj.w, ava::Q8_STORE, m->P, 5 * d, nullptr, st));
        } else {
            AVA_RUN("rms_planes", ava::rms_planes(m->x, N, d, b.mem_norm, P, m->xq, m->xexp, ldd, m->h, st));
            AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.wproj.w, ava::Q8_STORE, m->P, 5 * d, nullptr, st));
            AVA_RUN("gate_gemm", ava::gate_gemm(m->h, N, d, b.wgate, 2 * nh + 2 * r, m->G, st));
        }
        const bool vr = c.value_residual != 0;
        const size_t sm = (size_t)i * B * nh * 64 * 64;
        AVA_RUN("mem_scan", ava::mem_block(m->P, m->G, B, T, nh, r, b.ba, b.bb, b.off, b.wa2, b.wb2,
                                           vr && i > 0 ? b.vres : nullptr, vr && i > 0 ? m->v0 : nullptr,
                                           vr && i == 0 ? m->v0 : nullptr, c.momentum, c.cap, s->mem_f + sm,
                                           c.momentum != 0.0f ? s->mem_s + sm : nullptr, m->y, m->bad, st));
        AVA_RUN("mem_post", ava::mem_post(m->y, N, d, m->P + 4 * d, 5 * d, P, m->xq, m->xexp, ldd, st));
        AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.wo.w, ava::Q8_ADD, m->x, d, nullptr, st));
        // the engram read
        if (b.eng) {
            AVA_RUN("rms_planes", ava::rms_planes(m->x, N, d, b.eng_norm, P, m->xq, m->xexp, ldd, nullptr, st));
            AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.eqkv.w, ava::Q8_STORE, m->qkv, 3 * de, nullptr, st));
            // the decode form's merge also writes the read's planes and advances the device store length
            ava::PostRead post;
            if (T <= ava::ENGRAM_SPLIT_T && eng_nh(c) == 1) {
                post.xq = m->xq;
                post.xexp = m->xexp;
                post.ldq = ava::q8_ldk(de);
                post.planes = P;
                post.adv = s->eng_len_dev;
                advanced = s->eng_len_dev != nullptr;
            }
            AVA_RUN("attend", ava::engram_read(m->qkv, 3 * de, B, T, de, eng_nh(c), s->eng_k, s->eng_v, c.eng_half, s->eng_cap, s->eng_len,
                                                   s->eng_len_dev, m->eo, m->att_part, m->att_part_floats, st, post));
            if (s->eng_reads && s->eng_age)  // the least-read rule's counts (gpu/memory.rs:700-738)
                AVA_RUN("engram_count", ava::engram_count(m->qkv, 3 * de, s->eng_k, c.eng_half, s->eng_cap, s->eng_len, B,
                                                          T, de, eng_nh(c), m->eml, s->eng_reads, s->eng_age, st));
            if (!post.xq) AVA_RUN("quant_rows", ava::launch_quant_rows(m->eo, N, de, de, P, m->xq, m->xexp, st));
            AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.ewo.w, ava::Q8_ADD, m->x, d, nullptr, st));
        }
        // the sparse MLP
        AVA_RUN("rms_planes", ava::rms_planes(m->x, N, d, b.mlp_norm, P, m->xq, m->xexp, ldd, nullptr, st));
        AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.w1.w, ava::Q8_STORE, m->u, H, nullptr, st));
        AVA_RUN("kwta", ava::kwta_planes(m->u, N, H, c.kwta_k, c.relu2, P, m->xq, m->xexp, ldh,
                                         tracing ? m->tr_kth + (size_t)i * m->tr_rows + m->tr_pos : nullptr, st));
        if (tracing)
            AVA_RUN("trace", trace_copy(m->tr_u + ((size_t)i * m->tr_rows + m->tr_pos) * H, (size_t)H * 4, m->u,
                                        (size_t)H * 4, (size_t)H * 4, N, st));
        AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &b.w2.w, ava::Q8_ADD, m->x, d, nullptr, st));
        if (c.dense) {
            // the block's output becomes stream i + 1 by a buffer exchange; the mix lands in the
            // buffer that stream held (nothing reads a stream or x across forwards)
            std::swap(m->x, m->streams[i + 1]);
            if (i + 1 < L) {
                AVA_RUN("dense_mix", ava::dense_rms(m->x, m->streams.data(), b.dense.data(), i + 2, N, d,
                                                    m->blocks[i + 1].lif_norm, P, m->xq, m->xexp, ldd, nullptr, st));
                ready = true;
            } else if (logits) {
                AVA_RUN("dense_mix", ava::dense_rms(m->x, m->streams.data(), b.dense.data(), i + 2, N, d, m->final_norm,
                                                    P, m->xq, m->xexp, ldd, cb ? m->h : nullptr, st));
                final_ready = true;
            } else {
                AVA_RUN("dense_mix", ava::dense_mix(m->x, m->streams.data(), b.dense.data(), i + 2, (size_t)N * d, st));
            }
        }
    }
    if (tracing) m->tr_pos += (size_t)N;
    if (c.eng_block >= 0) {
        s->eng_len += T;
        if (s->eng_len_dev && !advanced)
            AVA_RUN("store_advance", ava::engram_advance(s->eng_len_dev, T, s->eng_cap, st));
    }
    if (join) AVA_HIP(hipStreamWaitEvent(st, join, 0));
    if (logits) {
        if (!final_ready)
            AVA_RUN("rms_planes", ava::rms_planes(m->x, N, d, m->final_norm, P, m->xq, m->xexp, ldd, cb ? m->h : nullptr,
                                                  st));
        if (cb) {
            // the cerebellum's correction between the final norm and the head (gpu/model/fstep/arch.rs:1045-1047)
            if (ava::cb_head_fits(N, d, c.cb_units, P)) {
                // few rows: the code, the read-out and its planes in one launch
                AVA_RUN("cb_code", ava::cb_head(m->h, ids, m->tok_emb, N, d, c.vocab, m->cb_idx, m->cb_sgn, c.cb_units,
                                                m->cb_k, T, m->cb_codes, s->cb_code, m->cb_lcnt, m->cb_lidx,
                                                m->cb_lval, m->cb_lcap, m->cb_w, s->cb_tab, s->cb_scale, m->y, P,
                                                m->xq, m->xexp, st));
            } else {
                AVA_RUN("cb_code", ava::cb_code(m->h, ids, m->tok_emb, N, d, c.vocab, m->cb_idx, m->cb_sgn, c.cb_units,
                                                m->cb_k, T, m->cb_codes, s->cb_code, m->cb_lcnt, m->cb_lidx,
                                                m->cb_lval, m->cb_lcap, st));
                AVA_RUN("cb_apply", ava::cb_apply_list(m->h, m->cb_codes, N, c.cb_units, d, m->cb_w, s->cb_tab,
                                                       s->cb_scale, T, m->cb_lcnt, m->cb_lidx, m->cb_lval, m->cb_lcap,
                                                       m->y, st));
                AVA_RUN("quant_rows", ava::launch_quant_rows(m->y, N, d, d, P, m->xq, m->xexp, st));
            }
        }
        AVA_RUN("q8_gemm", ava::q8_gemm(m->xq, m->xexp, P, N, &m->head.w, ava::Q8_STORE, logits, c.vocab, nullptr, st));
    }
    return AVA_OK;
}

constexpr int CB_NKS = 32;  // the learning step's delta product: K slices of vocab / 32 each

// The learning step's scratch for B streams (kept; regrown only while the scratch is not frozen).
int ensure_cb(ava_model *m, int B) {
    const ava_config &c = m->cfg;
    if (B <= m->cb_rows) return AVA_OK;
    AVA_REQUIRE(!m->frozen, AVA_ERR_ARG, "cb_learn: %d streams need more scratch, and the model's scratch is "
                "frozen (a captured graph uses it)", B);
    for (void *p : {(void *)m->cb_err, (void *)m->cb_part, (void *)m->cb_delta, (void *)m->cb_fold}) (void)hipFree(p);
    m->cb_err = m->cb_part = m->cb_delta = nullptr;
    m->cb_fold = nullptr;
    m->cb_rows = 0;
    AVA_HIP(hipMalloc(&m->cb_err, (size_t)B * c.vocab * sizeof(float)));
    AVA_HIP(hipMalloc(&m->cb_part, (size_t)CB_NKS * B * c.d * sizeof(float)));
    AVA_HIP(hipMalloc(&m->cb_delta, (size_t)B * c.d * sizeof(float)));
    AVA_HIP(hipMalloc(&m->cb_fold, (size_t)B * sizeof(double)));
    m->cb_rows = B;
    return AVA_OK;
}

}  // namespace

extern "C" int ava_model_new(const ava_config *cfg, const ava_params *params, ava_model **out) {
    AVA_REQUIRE(cfg && params && out, AVA_ERR_ARG, "model_new: NULL argument");
    const ava_config &c = *cfg;
    AVA_REQUIRE(c.head_size == 64, AVA_ERR_UNSUPPORTED, "model_new: head size %d (this build runs 64)", c.head_size);
    AVA_REQUIRE(c.d > 0 && c.d % 128 == 0 && c.d <= 1024, AVA_ERR_SHAPE, "model_new: d=%d (a multiple of 128, <= 1024)",
                c.d);
    AVA_REQUIRE(c.hidden > 0 && c.hidden % 4 == 0 && c.hidden <= 8192 && c.kwta_k > 0, AVA_ERR_SHAPE,
                "model_new: hidden=%d k=%d", c.hidden, c.kwta_k);
    AVA_REQUIRE(c.layers > 0 && c.layers <= 16, AVA_ERR_SHAPE, "model_new: %d layers (1..16)", c.layers);
    AVA_REQUIRE(c.vocab > 0 && c.gate_rank > 0 && c.gate_rank <= 32, AVA_ERR_SHAPE, "model_new: vocab=%d gate_rank=%d",
                c.vocab, c.gate_rank);
    AVA_REQUIRE(c.eng_block < c.layers &&
                    (c.eng_block < 0 || (c.eng_dim == 64 && eng_nh(c) == 1) ||
                     (c.eng_dim % 64 == 0 && c.eng_dim <= 1024 && c.eng_dim == 32 * eng_nh(c))),
                AVA_ERR_UNSUPPORTED, "model_new: engram block %d, %d dims in %d heads (one head of 64, or heads of 32)",
                c.eng_block, c.eng_dim, eng_nh(c));
    AVA_REQUIRE(c.levels == 1 || c.levels == 2, AVA_ERR_ARG, "model_new: levels %d", c.levels);
    AVA_REQUIRE(c.planes >= 1 && c.planes <= 3, AVA_ERR_ARG, "model_new: planes %d (1..3)", c.planes);
    AVA_REQUIRE(c.cb_units == 0 || (c.cb_units > 0 && c.cb_units % 32 == 0 && c.cb_units <= 16384), AVA_ERR_SHAPE,
                "model_new: cb_units %d (0, or a multiple of 32 up to 16384)", c.cb_units);
    ava_model *m = new ava_model();
    m->cfg = c;
    (void)hipGetDevice(&m->device);
    if (int e = build(m, params)) {
        ava_model_free(m);
        return e;
    }
    *out = m;
    return AVA_OK;
}

extern "C" void ava_model_free(ava_model *m) {
    if (!m) return;
    (void)hipDeviceSynchronize();
    for (void *p : m->allocs) (void)hipFree(p);
    for (void *p : m->scratch) (void)hipFree(p);
    for (hipEvent_t e : m->timer.pool) (void)hipEventDestroy(e);
    for (void *p : {(void *)m->cb_err, (void *)m->cb_part, (void *)m->cb_delta, (void *)m->cb_fold}) (void)hipFree(p);
    (void)hipFree(m->att_part);
    (void)hipFree(m->eml);
    if (m->ev_fork) (void)hipEventDestroy(m->ev_fork);
    if (m->ev_join) (void)hipEventDestroy(m->ev_join);
    if (m->side) (void)hipStreamDestroy(m->side);
    delete m;
}

extern "C" int ava_model_forward(ava_model *m, ava_state *st, const int32_t *ids, int B, int T, float *logits,
                                 ava_stream stream) {
    AVA_REQUIRE(m && st && ids, AVA_ERR_ARG, "model_forward: NULL argument");
    AVA_REQUIRE(B > 0 && T > 0 && (long)B * T <= (1L << 24), AVA_ERR_SHAPE, "model_forward: B=%d T=%d", B, T);
    return forward(m, st, ids, B, T, logits, (hipStream_t)stream);
}

extern "C" int ava_model_cb_learn(ava_model *m, ava_state *st, const float *logits, int ld_logits,
                                  const int32_t *next, int B, double *nats, ava_stream stream) {
    AVA_REQUIRE(m && st && logits && next, AVA_ERR_ARG, "cb_learn: NULL argument");
    const ava_config &c = m->cfg;
    AVA_REQUIRE(c.cb_units > 0 && st->cb_tab && st->cb_scale && st->cb_code, AVA_ERR_ARG,
                "cb_learn: the model has no cerebellum head or the state no online table");
    AVA_REQUIRE(B > 0 && ld_logits >= c.vocab, AVA_ERR_SHAPE, "cb_learn: B=%d ld=%d", B, ld_logits);
    if (int e = ensure_cb(m, B)) return e;
    hipStream_t sst = (hipStream_t)stream;
    if (m->timing && m->last_stream != sst) {
        if (int e = collect(m)) return e;
    }
    m->last_stream = sst;
    ava_state *as = st;
    {
        hipStream_t st = sst;  // the stream AVA_RUN times on
        AVA_RUN("cb_learn", ava::cb_learn(logits, ld_logits, c.vocab, next, B, m->tok_emb, c.d, as->cb_code, c.cb_units,
                                          c.cb_lr, m->cb_fade, as->cb_scale, as->cb_tab, m->cb_err, m->cb_part, CB_NKS,
                                          m->cb_delta, m->cb_fold, nats, st));
    }
    return AVA_OK;
}

extern "C" int ava_model_decode_step(ava_model *m, ava_state *st, const int32_t *ids, int B, int T, float *logits,
                                     const float *prev_logits, int ld_prev, const int32_t *prev_next, double *prev_nats,
                                     ava_stream stream) {
    AVA_REQUIRE(m && st && ids, AVA_ERR_ARG, "decode_step: NULL argument");
    AVA_REQUIRE(B > 0 && T > 0 && (long)B * T <= (1L << 24), AVA_ERR_SHAPE, "decode_step: B=%d T=%d", B, T);
    hipStream_t sst = (hipStream_t)stream;
    if (!prev_logits) return forward(m, st, ids, B, T, logits, sst);
    const ava_config &c = m->cfg;
    AVA_REQUIRE(prev_next && c.cb_units > 0 && st->cb_tab && st->cb_scale && st->cb_code && m->side, AVA_ERR_ARG,
                "decode_step: a table step needs the model's cerebellum head, the state's table and prev_next");
    AVA_REQUIRE(ld_prev >= c.vocab, AVA_ERR_SHAPE, "decode_step: ld_prev=%d", ld_prev);
    AVA_REQUIRE(!logits || logits != prev_logits, AVA_ERR_ARG, "decode_step: logits and prev_logits are one buffer");
    if (m->timing) {
        // the launch timer follows one stream: the two parts run one after the other
        if (int e = ava_model_cb_learn(m, st, prev_logits, ld_prev, prev_next, B, prev_nats, stream)) return e;
        return ava_model_forward(m, st, ids, B, T, logits, stream);
    }
    if (int e = ensure_cb(m, B)) return e;
    m->last_stream = sst;
    // fork: the table step of the previous token on the side stream, after everything before it on sst
    AVA_HIP(hipEventRecord(m->ev_fork, sst));
    AVA_HIP(hipStreamWaitEvent(m->side, m->ev_fork, 0));
    if (int e = ava::cb_learn(prev_logits, ld_prev, c.vocab, prev_next, B, m->tok_emb, c.d, st->cb_code, c.cb_units,
                              c.cb_lr, m->cb_fade, st->cb_scale, st->cb_tab, m->cb_err, m->cb_part, CB_NKS, m->cb_delta,
                              m->cb_fold, prev_nats, m->side))
        return e;
    AVA_HIP(hipEventRecord(m->ev_join, m->side));
    // the blocks run meanwhile; the join comes before the final norm and the cerebellum
    return forward(m, st, ids, B, T, logits, sst, m->ev_join);
}

extern "C" size_t ava_model_scratch_bytes(const ava_model *m) { return m ? m->scratch_bytes : 0; }

extern "C" int ava_model_nonfinite(ava_model *m, int32_t *rows, int rows_cap, int *count, ava_stream stream) {
    AVA_REQUIRE(m && count, AVA_ERR_ARG, "model_nonfinite: NULL argument");
    *count = 0;
    AVA_REQUIRE(!rows || rows_cap >= m->bad_n, AVA_ERR_SHAPE,
                "model_nonfinite: rows holds %d entries, the last forward had %d streams", rows_cap, m->bad_n);
    if (m->bad_n == 0) return AVA_OK;
    std::vector<int32_t> h(m->bad_n);
    AVA_HIP(hipSetDevice(m->device));
    AVA_HIP(hipMemcpyAsync(h.data(), m->bad, h.size() * sizeof(int32_t), hipMemcpyDeviceToHost, (hipStream_t)stream));
    AVA_HIP(hipStreamSynchronize((hipStream_t)stream));
    for (int32_t v : h) *count += v != 0;
    if (rows) std::copy(h.begin(), h.end(), rows);
    return AVA_OK;
}

extern "C" int ava_model_freeze(ava_model *m, int on) {
    AVA_REQUIRE(m, AVA_ERR_ARG, "freeze: NULL model");
    m->frozen = on != 0;
    return AVA_OK;
}

extern "C" int ava_model_set_trace(ava_model *m, int8_t *spikes, float *u, float *kth, size_t rows) {
    AVA_REQUIRE(m, AVA_ERR_ARG, "set_trace: NULL model");
    AVA_REQUIRE((spikes && u && kth) || (!spikes && !u && !kth), AVA_ERR_ARG,
                "set_trace: spikes, u and kth are all set or all NULL");
    m->tr_spk = spikes;
    m->tr_u = u;
    m->tr_kth = kth;
    m->tr_rows = spikes ? rows : 0;
    m->tr_pos = 0;
    return AVA_OK;
}

extern "C" int ava_model_set_timing(ava_model *m, int on) {
    AVA_REQUIRE(m, AVA_ERR_ARG, "set_timing: NULL model");
    if (!on && m->timing) {
        if (int e = collect(m)) return e;
    }
    m->timing = on != 0;
    return AVA_OK;
}

extern "C" int ava_model_timing(ava_model *m, const char **names, int *calls, double *ms, int cap, int reset) {
    if (!m) return -1;
    if (collect(m)) return -1;
    int n = 0;
    for (auto &kv : m->timer.sums) {
        if (n < cap) {
            if (names) names[n] = kv.second.name;
            if (calls) calls[n] = kv.second.calls;
            if (ms) ms[n] = kv.second.ms;
        }
        n++;
    }
    if (reset) m->timer.sums.clear();
    return n;
}
