// The float32 training step of the Ava-0.4-shaped block stack (include/ava.h: ava_train_*): one
// teacher-forced batch, its mean cross-entropy loss and the gradient of every parameter, composed the
// way the reference's hand-written step is (gpu/model/fwin.rs:1-40: every forward op a kernel, every
// backward the matching kernel, no autograd). The forward keeps what the backward reads (the
// scans' inputs, the norms' inverse rms, the products' inputs), then the backward walks the blocks in
// reverse:
//   head      logits = rms(x_L) E^T; dlogits = (softmax - onehot) / rows; dE += dlogits^T h; dh = dlogits E
//   dense mix the gradient into each block's raw output and the mixing weights (ava_dense_back)
//   MLP       da = dx W2^T, du = relu2'(u) da (ava_kwta_relu2_bwd), dW1, dW2, the norm's backward
//   engram    causal attention's backward (train.hip), the three projections
//   memory    read-out backward, the scan's backward (ava_mem_scan_bwd), the inputs' preparation backward
//             (unit norms, gates, value residual), the projections and the rank-32 gate read-outs
//   spiking   dS = dx Wout^T, the LIF scan's backward (ava_lif_scan_bwd), the (1 - beta) scale, dWin
// The plain products (x W, dY W^T, X^T dY) are library GEMMs (rocBLAS, f32); the rest is the library's
// own kernels. theta is detached (as in the reference's LIF backward) and the gate offsets are constants,
// so their gradients are zero.
#include <math.h>
#include <string.h>

#include <rocblas/rocblas.h>

#include <string>
#include <vector>

#include "common.h"
#include "train.h"

namespace {

struct Slot {
    std::string name;
    int block;  // -1: a global tensor
    size_t off, n;
};

// per block, in layout order (the dense weights of all blocks sit together at the end, so that they
// form the packed [k (k + 3) / 2 + j] vector ava_dense_back reads)
const char *const BLOCK_NAMES[] = {"lif_norm", "win", "beta_p", "theta", "arho", "again", "wout", "mem_norm",
                                   "wq", "wk", "wv", "we", "wg", "wo", "wa", "ba", "wb", "bb", "off", "wa1",
                                   "wa2", "wb1", "wb2", "vres", "eng_norm", "ewq", "ewk", "ewv", "ewo",
                                   "mlp_norm", "w1", "w2"};

struct Acts {  // one block's saved forward values
    float *inv1, *h1, *z, *cur, *S, *x1, *inv2, *h2, *q, *k, *v, *we, *g, *zab, *z1, *lra, *lrb;
    float *hq, *hk, *he, *hv, *hla, *hb, *y, *o, *x2;
    float *inv3, *h3, *eq, *ek, *ev, *att, *x3;
    float *inv4, *h4, *u, *kth, *a;
    int8_t *spk;
    float *ps, *omb;
    float *lpark = nullptr;  // the LIF state at each segment start (few chains: the backward in segments)
};

}  // namespace

struct ava_trainer {
    ava_config cfg{};
    float slope = 4.0f;
    int reset_grad = 0;
    int device = 0;
    std::vector<Slot> slots;
    size_t nparams = 0, dense_off = 0;
    rocblas_handle blas = nullptr;

    // scratch for N rows
    int N = 0, B = 0, T = 0;
    std::vector<void *> bufs;
    std::vector<Acts> acts;
    float *streams = nullptr, *G = nullptr, *xmix = nullptr;  // [L+1][N d], [L][N d], [L][N d]
    float *hf = nullptr, *invf = nullptr, *logits = nullptr, *lse = nullptr, *lrow = nullptr, *valid = nullptr;
    float *scal = nullptr;
    float *memF = nullptr, *memS = nullptr, *lv = nullptr, *ls = nullptr, *la = nullptr;
    float *dx = nullptr, *dA = nullptr, *dB = nullptr, *dC = nullptr, *dH = nullptr, *dH2 = nullptr;
    float *dq = nullptr, *dk = nullptr, *de = nullptr, *dv = nullptr, *dla = nullptr, *db = nullptr;
    float *dq_raw = nullptr, *dk_raw = nullptr, *dv_raw = nullptr, *dwe = nullptr, *dza = nullptr, *dzb = nullptr;
    float *dzab = nullptr, *dz1 = nullptr, *dvfirst = nullptr, *vres_part = nullptr, *dg = nullptr;
    float *deq = nullptr, *dek = nullptr, *dev = nullptr, *datt = nullptr, *alse = nullptr, *adsum = nullptr;
    float *dI = nullptr, *dv0 = nullptr, *da0 = nullptr, *dbsh = nullptr, *drsh = nullptr, *dgsh = nullptr;
    float *part = nullptr, *dvec = nullptr, *dvec2 = nullptr;
    size_t part_floats = 0;
    void *mwork = nullptr;
    size_t mwork_bytes = 0;
    bool lif_seg = false;  // the LIF backward in parallel segments (few chains)
    float *lws = nullptr;
    size_t lws_floats = 0;
    float *att_part = nullptr;
    size_t att_part_floats = 0;

    ~ava_trainer() { release(); }
    void release() {
        for (void *p : bufs) (void)hipFree(p);
        bufs.clear();
        acts.clear();
        N = 0;
    }
    const Slot *find(const char *name, int block) const {
        for (const Slot &s : slots)
            if (s.block == block && s.name == name) return &s;
        return nullptr;
    }
};

namespace {

int eng_nh(const ava_config &c) { return c.eng_heads > 1 ? c.eng_heads : 1; }

// The LIF backward walks each (stream, channel) chain in one lane; up to this many chains (a quarter of
// the SIMDs at B d = 16,384) and from this many steps, it runs in parallel segments instead
// (ava::lif_scan_bwd_seg).
constexpr size_t LIF_SEG_CHAINS = 16384;
constexpr int LIF_SEG_MIN_T = 128;

size_t block_count(const ava_config &c, int i, const std::string &nm) {
    const size_t d = c.d, nh = c.d / c.head_size, r = c.gate_rank, H = c.hidden, de = c.eng_dim;
    if (nm == "win" || nm == "wout" || nm == "wq" || nm == "wk" || nm == "wv" || nm == "we" || nm == "wg" ||
        nm == "wo")
        return d * d;
    if (nm == "wa" || nm == "wb") return d * nh;
    if (nm == "ba" || nm == "bb") return nh;
    if (nm == "wa1" || nm == "wb1" || nm == "wa2" || nm == "wb2") return d * r;
    if (nm == "vres") return 2;
    if (nm == "ewq" || nm == "ewk" || nm == "ewv" || nm == "ewo") return i == c.eng_block ? d * de : 0;
    if (nm == "eng_norm") return i == c.eng_block ? d : 0;
    if (nm == "w1" || nm == "w2") return d * H;
    return d;  // the norms' gains, beta_p, theta, arho, again, off
}

// row-major C [M][N] (ldc) = alpha op(A) op(B) + beta C, op(A) [M][K] (A stored [M][K], or [K][M] when tA)
int gemm(rocblas_handle h, bool tA, bool tB, int M, int N, int K, float alpha, const float *A, int lda, const float *B,
         int ldb, float beta, float *C, int ldc) {
    if (M == 0 || N == 0) return AVA_OK;
    const rocblas_status s =
        rocblas_sgemm(h, tB ? rocblas_operation_transpose : rocblas_operation_none,
                      tA ? rocblas_operation_transpose : rocblas_operation_none, N, M, K, &alpha, B, ldb, A, lda, &beta,
                      C, ldc);
    AVA_REQUIRE(s == rocblas_status_success, AVA_ERR_HIP, "train: rocblas_sgemm failed (%d) M=%d N=%d K=%d", (int)s, M,
                N, K);
    return AVA_OK;
}

#define TR(call)                         \
    do {                                 \
        if (int r_ = (call)) return r_; \
    } while (0)

int alloc(ava_trainer *t, void **p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) return AVA_OK;
    AVA_HIP(hipMalloc(p, bytes));
    t->bufs.push_back(*p);
    return AVA_OK;
}
#define AF(ptr, nfl) TR(alloc(t, (void **)&(ptr), (size_t)(nfl) * sizeof(float)))

int ensure(ava_trainer *t, int B, int T) {
    if (t->N == B * T && t->B == B && t->T == T) return AVA_OK;
    t->release();
    const ava_config &c = t->cfg;
    const size_t N = (size_t)B * T, d = c.d, H = c.hidden, L = c.layers, nh = d / c.head_size, r = c.gate_rank;
    const size_t de = c.eng_dim, V = c.vocab, Nd = N * d;
    t->acts.resize(L);
    for (size_t i = 0; i < L; i++) {
        Acts &a = t->acts[i];
        AF(a.inv1, N); AF(a.h1, Nd); AF(a.z, Nd); AF(a.cur, Nd); AF(a.S, Nd); AF(a.x1, Nd);
        AF(a.inv2, N); AF(a.h2, Nd); AF(a.q, Nd); AF(a.k, Nd); AF(a.v, Nd); AF(a.we, Nd); AF(a.g, Nd);
        AF(a.zab, N * 2 * nh); AF(a.z1, N * 2 * r); AF(a.lra, Nd); AF(a.lrb, Nd);
        AF(a.hq, Nd); AF(a.hk, Nd); AF(a.he, Nd); AF(a.hv, Nd); AF(a.hla, Nd); AF(a.hb, Nd);
        AF(a.y, Nd); AF(a.o, Nd); AF(a.x2, Nd);
        if ((int)i == c.eng_block) {
            AF(a.inv3, N); AF(a.h3, Nd); AF(a.eq, N * de); AF(a.ek, N * de); AF(a.ev, N * de); AF(a.att, N * de);
            AF(a.x3, Nd);
        } else {
            a.inv3 = a.h3 = a.eq = a.ek = a.ev = a.att = a.x3 = nullptr;
        }
        AF(a.inv4, N); AF(a.h4, Nd); AF(a.u, N * H); AF(a.kth, N); AF(a.a, N * H);
        TR(alloc(t, (void **)&a.spk, Nd));
        AF(a.ps, 4 * d); AF(a.omb, d);
    }
    AF(t->streams, (L + 1) * Nd);
    AF(t->G, L * Nd);
    AF(t->xmix, L * Nd);
    AF(t->hf, Nd); AF(t->invf, N); AF(t->logits, N * V); AF(t->lse, N); AF(t->lrow, N); AF(t->valid, N);
    AF(t->scal, 1);
    AF(t->memF, (size_t)B * nh * 64 * 64); AF(t->memS, (size_t)B * nh * 64 * 64);
    AF(t->lv, B * d); AF(t->ls, B * d); AF(t->la, B * d);
    AF(t->dx, Nd); AF(t->dA, Nd); AF(t->dB, Nd); AF(t->dC, Nd); AF(t->dH, N * H); AF(t->dH2, N * H);
    AF(t->dq, Nd); AF(t->dk, Nd); AF(t->de, Nd); AF(t->dv, Nd); AF(t->dla, Nd); AF(t->db, Nd);
    AF(t->dq_raw, Nd); AF(t->dk_raw, Nd); AF(t->dv_raw, Nd); AF(t->dwe, Nd); AF(t->dza, Nd); AF(t->dzb, Nd);
    AF(t->dzab, N * 2 * nh); AF(t->dz1, N * 2 * r); AF(t->dvfirst, Nd); AF(t->vres_part, N * nh * 2); AF(t->dg, Nd);
    if (c.eng_block >= 0) {
        AF(t->deq, N * de); AF(t->dek, N * de); AF(t->dev, N * de); AF(t->datt, N * de);
        AF(t->alse, N * eng_nh(c)); AF(t->adsum, N * eng_nh(c));
        t->att_part_floats = ava_attend_heads_part_floats(B, T, 0, (int)de, eng_nh(c));
        AF(t->att_part, t->att_part_floats);
    }
    AF(t->dI, Nd); AF(t->dv0, B * d); AF(t->da0, B * d); AF(t->dbsh, B * d); AF(t->drsh, B * d); AF(t->dgsh, B * d);
    size_t pf = ava::train::rms_bwd_part_floats((int)N, (int)d);
    pf = std::max(pf, ava::train::colsum_part_floats((int)(N * nh), (int)std::max<size_t>(d, 2 * nh)));
    pf = std::max(pf, ava::train::dot_part_floats());
    pf = std::max(pf, ava_dense_back_part_floats((long long)Nd, (int)L + 1));
    t->part_floats = pf;
    AF(t->part, pf);
    AF(t->dvec, d); AF(t->dvec2, d);
    t->mwork_bytes = ava_mem_scan_bwd_workspace((int)(B * nh), T, c.momentum != 0.0f);
    TR(alloc(t, &t->mwork, t->mwork_bytes));
    // few LIF chains (B d): the backward in parallel segments, with its workspace
    t->lif_seg = (size_t)B * d <= LIF_SEG_CHAINS && T >= LIF_SEG_MIN_T;
    t->lws_floats = t->lif_seg ? ava::lif_bwd_seg_floats(B, T, (int)d) : 0;
    if (t->lif_seg) {
        AF(t->lws, t->lws_floats);
        for (size_t i = 0; i < L; i++) AF(t->acts[i].lpark, ava::lif_park_floats(B, T, (int)d));
    }
    t->N = (int)N;
    t->B = B;
    t->T = T;
    return AVA_OK;
}

#undef AF

struct P {  // one block's parameter (or gradient) pointers inside a flat buffer
    const ava_trainer *t;
    float *base;
    int blk;
    float *operator()(const char *nm) const {
        const Slot *s = t->find(nm, blk);
        return s && s->n ? base + s->off : nullptr;
    }
};

int step(ava_trainer *t, const float *prm, const int32_t *ids, const int32_t *tgt, int B, int T, float *grads,
         float *loss, hipStream_t st) {
    const ava_config &c = t->cfg;
    const int L = c.layers, d = c.d, H = c.hidden, hs = c.head_size, nh = d / hs, r = c.gate_rank, V = c.vocab;
    const int N = B * T, de = c.eng_dim, enh = eng_nh(c);
    const size_t Nd = (size_t)N * d;
    rocblas_handle hb = t->blas;
    AVA_REQUIRE(rocblas_set_stream(hb, st) == rocblas_status_success, AVA_ERR_HIP, "train: rocblas_set_stream");
    float *pb = const_cast<float *>(prm);
    const float *E = pb + t->find("tok_emb", -1)->off;
    const float *fnorm = pb + t->find("final_norm", -1)->off;
    const float *wdense = pb + t->dense_off;
    AVA_HIP(hipMemsetAsync(grads, 0, t->nparams * sizeof(float), st));

    // ------------------------------------------------------------ forward
    float *x0 = t->streams;  // stream 0: the embedding
    TR(ava::train::embed(ids, E, N, d, V, x0, st));
    float *vfirst = nullptr;
    for (int i = 0; i < L; i++) {
        Acts &a = t->acts[i];
        P w{t, pb, i};
        const float *xin = i == 0 ? x0 : (c.dense ? t->xmix + (size_t)(i - 1) * Nd : t->streams + (size_t)i * Nd);
        // spiking layer: z = rms(x) Win, cur = z (1 - beta), the scan, x1 = x + s Wout
        TR(ava::train::rms_fwd(xin, N, d, w("lif_norm"), a.h1, a.inv1, st));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.h1, d, w("win"), d, 0.0f, a.z, d));
        TR(ava::train::lif_params(w("beta_p"), w("theta"), w("arho"), w("again"), d, c.alif, a.ps, a.omb, st));
        if (c.lif_scale)
            TR(ava::train::scale_cols(a.z, a.omb, N, d, a.cur, st));
        else
            AVA_HIP(hipMemcpyAsync(a.cur, a.z, Nd * 4, hipMemcpyDeviceToDevice, st));
        AVA_HIP(hipMemsetAsync(t->lv, 0, (size_t)B * d * 4, st));
        AVA_HIP(hipMemsetAsync(t->ls, 0, (size_t)B * d * 4, st));
        AVA_HIP(hipMemsetAsync(t->la, 0, (size_t)B * d * 4, st));
        TR(ava::lif_scan(a.cur, B, T, d, a.ps, t->lv, t->ls, t->la, c.levels, 1, c.alif, a.spk, nullptr, st,
                         t->lif_seg ? a.lpark : nullptr));
        TR(ava::train::i8_to_f32(a.spk, Nd, a.S, st));
        AVA_HIP(hipMemcpyAsync(a.x1, xin, Nd * 4, hipMemcpyDeviceToDevice, st));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.S, d, w("wout"), d, 1.0f, a.x1, d));
        // memory
        TR(ava::train::rms_fwd(a.x1, N, d, w("mem_norm"), a.h2, a.inv2, st));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.h2, d, w("wq"), d, 0.0f, a.q, d));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.h2, d, w("wk"), d, 0.0f, a.k, d));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.h2, d, w("wv"), d, 0.0f, a.v, d));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.h2, d, w("we"), d, 0.0f, a.we, d));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.h2, d, w("wg"), d, 0.0f, a.g, d));
        TR(gemm(hb, false, false, N, nh, d, 1.0f, a.h2, d, w("wa"), nh, 0.0f, a.zab, 2 * nh));
        TR(gemm(hb, false, false, N, nh, d, 1.0f, a.h2, d, w("wb"), nh, 0.0f, a.zab + nh, 2 * nh));
        TR(gemm(hb, false, false, N, r, d, 1.0f, a.h2, d, w("wa1"), r, 0.0f, a.z1, 2 * r));
        TR(gemm(hb, false, false, N, r, d, 1.0f, a.h2, d, w("wb1"), r, 0.0f, a.z1 + r, 2 * r));
        TR(gemm(hb, false, false, N, d, r, 1.0f, a.z1, 2 * r, w("wa2"), d, 0.0f, a.lra, d));
        TR(gemm(hb, false, false, N, d, r, 1.0f, a.z1 + r, 2 * r, w("wb2"), d, 0.0f, a.lrb, d));
        if (i == 0) vfirst = a.v;
        TrainPrep pp{a.q, a.k, a.v, a.we, a.zab, a.lra, a.lrb, w("ba"), w("bb"), w("off"),
                     (c.value_residual && i > 0) ? vfirst : nullptr, w("vres"),
                     a.hq, a.hk, a.he, a.hv, a.hla, a.hb, B, T, nh};
        TR(ava::train::prep_fwd(pp, st));
        AVA_HIP(hipMemsetAsync(t->memF, 0, (size_t)B * nh * 64 * 64 * 4, st));
        AVA_HIP(hipMemsetAsync(t->memS, 0, (size_t)B * nh * 64 * 64 * 4, st));
        TR(ava_mem_scan(a.hq, a.hk, a.he, a.hv, a.hla, a.hb, B * nh, T, 64, 64, c.momentum, c.cap, t->memF, t->memS,
                        a.y, st));
        TR(ava::train::readout_fwd(a.y, a.g, B, T, nh, a.o, st));
        AVA_HIP(hipMemcpyAsync(a.x2, a.x1, Nd * 4, hipMemcpyDeviceToDevice, st));
        TR(gemm(hb, false, false, N, d, d, 1.0f, a.o, d, w("wo"), d, 1.0f, a.x2, d));
        const float *x3 = a.x2;
        if (i == c.eng_block) {
            TR(ava::train::rms_fwd(a.x2, N, d, w("eng_norm"), a.h3, a.inv3, st));
            TR(gemm(hb, false, false, N, de, d, 1.0f, a.h3, d, w("ewq"), de, 0.0f, a.eq, de));
            TR(gemm(hb, false, false, N, de, d, 1.0f, a.h3, d, w("ewk"), de, 0.0f, a.ek, de));
            TR(gemm(hb, false, false, N, de, d, 1.0f, a.h3, d, w("ewv"), de, 0.0f, a.ev, de));
            TR(ava_attend_heads(a.eq, de, a.ek, a.ev, 0, T, 0, B, T, de, enh, a.att, t->att_part, t->att_part_floats,
                                st));
            AVA_HIP(hipMemcpyAsync(a.x3, a.x2, Nd * 4, hipMemcpyDeviceToDevice, st));
            TR(gemm(hb, false, false, N, d, de, 1.0f, a.att, de, w("ewo"), d, 1.0f, a.x3, d));
            x3 = a.x3;
        }
        // sparse MLP; the block's raw output is stream i + 1
        float *raw = t->streams + (size_t)(i + 1) * Nd;
        TR(ava::train::rms_fwd(x3, N, d, w("mlp_norm"), a.h4, a.inv4, st));
        TR(gemm(hb, false, false, N, H, d, 1.0f, a.h4, d, w("w1"), H, 0.0f, a.u, H));
        TR(ava_kwta(a.u, N, H, c.kwta_k, 1, a.a, a.kth, st));
        AVA_HIP(hipMemcpyAsync(raw, x3, Nd * 4, hipMemcpyDeviceToDevice, st));
        TR(gemm(hb, false, false, N, d, H, 1.0f, a.a, H, w("w2"), d, 1.0f, raw, d));
        if (c.dense) {
            std::vector<const float *> ss(i + 2);
            for (int j = 0; j <= i + 1; j++) ss[j] = t->streams + (size_t)j * Nd;
            TR(ava::train::mix(t->xmix + (size_t)i * Nd, ss.data(), i + 2, wdense + (size_t)i * (i + 3) / 2, Nd, st));
        }
    }
    const float *xL = c.dense ? t->xmix + (size_t)(L - 1) * Nd : t->streams + (size_t)L * Nd;
    TR(ava::train::rms_fwd(xL, N, d, fnorm, t->hf, t->invf, st));
    TR(gemm(hb, false, true, N, V, d, 1.0f, t->hf, d, E, d, 0.0f, t->logits, V));
    TR(ava::train::cross_entropy(t->logits, tgt, N, V, t->lse, t->lrow, t->valid, loss, t->scal, st));

    // ------------------------------------------------------------ backward
    float *dE = grads + t->find("tok_emb", -1)->off;
    TR(gemm(hb, true, false, V, d, N, 1.0f, t->logits, V, t->hf, d, 0.0f, dE, d));   // dE = dlogits^T h
    TR(gemm(hb, false, false, N, d, V, 1.0f, t->logits, V, E, d, 0.0f, t->dA, d));   // dh = dlogits E
    float *GL = t->G + (size_t)(L - 1) * Nd;
    AVA_HIP(hipMemsetAsync(GL, 0, Nd * 4, st));
    TR(ava::train::rms_bwd(xL, t->invf, fnorm, t->dA, N, d, GL, grads + t->find("final_norm", -1)->off, t->part, st));
    AVA_HIP(hipMemsetAsync(t->dvfirst, 0, Nd * 4, st));
    float *dgd = grads + t->dense_off;
    for (int i = L - 1; i >= 0; i--) {
        Acts &a = t->acts[i];
        P w{t, pb, i}, gw{t, grads, i};
        const float *xin = i == 0 ? x0 : (c.dense ? t->xmix + (size_t)(i - 1) * Nd : t->streams + (size_t)i * Nd);
        float *Gi = t->G + (size_t)i * Nd;
        // the gradient into the block's raw output: dx (running, the residual stream's gradient)
        if (c.dense)
            TR(ava_dense_back(t->streams, t->G, wdense, Gi, t->dx, dgd + (size_t)i * (i + 3) / 2, i + 1, i, L, i + 2,
                              (long long)Nd, t->part, t->part_floats, st));
        else
            AVA_HIP(hipMemcpyAsync(t->dx, Gi, Nd * 4, hipMemcpyDeviceToDevice, st));
        // MLP
        const float *x3 = i == c.eng_block ? a.x3 : a.x2;
        TR(gemm(hb, true, false, H, d, N, 1.0f, a.a, H, t->dx, d, 0.0f, gw("w2"), d));
        TR(gemm(hb, false, true, N, H, d, 1.0f, t->dx, d, w("w2"), d, 0.0f, t->dH, H));
        TR(ava_kwta_relu2_bwd(a.u, a.kth, N, H, t->dH, t->dH2, st));
        TR(gemm(hb, true, false, d, H, N, 1.0f, a.h4, d, t->dH2, H, 0.0f, gw("w1"), H));
        TR(gemm(hb, false, true, N, d, H, 1.0f, t->dH2, H, w("w1"), H, 0.0f, t->dA, d));
        TR(ava::train::rms_bwd(x3, a.inv4, w("mlp_norm"), t->dA, N, d, t->dx, gw("mlp_norm"), t->part, st));
        // engram
        if (i == c.eng_block) {
            TR(gemm(hb, true, false, de, d, N, 1.0f, a.att, de, t->dx, d, 0.0f, gw("ewo"), d));
            TR(gemm(hb, false, true, N, de, d, 1.0f, t->dx, d, w("ewo"), d, 0.0f, t->datt, de));
            TrainAttn at{a.eq, a.ek, a.ev, a.att, t->datt, t->deq, t->dek, t->dev, t->alse, t->adsum,
                         B, T, de, enh, de / enh, (float)(1.0 / sqrt((double)(de / enh)))};
            TR(ava::train::attn_bwd(at, st));
            TR(gemm(hb, true, false, d, de, N, 1.0f, a.h3, d, t->deq, de, 0.0f, gw("ewq"), de));
            TR(gemm(hb, true, false, d, de, N, 1.0f, a.h3, d, t->dek, de, 0.0f, gw("ewk"), de));
            TR(gemm(hb, true, false, d, de, N, 1.0f, a.h3, d, t->dev, de, 0.0f, gw("ewv"), de));
            TR(gemm(hb, false, true, N, d, de, 1.0f, t->deq, de, w("ewq"), de, 0.0f, t->dA, d));
            TR(gemm(hb, false, true, N, d, de, 1.0f, t->dek, de, w("ewk"), de, 1.0f, t->dA, d));
            TR(gemm(hb, false, true, N, d, de, 1.0f, t->dev, de, w("ewv"), de, 1.0f, t->dA, d));
            TR(ava::train::rms_bwd(a.x2, a.inv3, w("eng_norm"), t->dA, N, d, t->dx, gw("eng_norm"), t->part, st));
        }
        // memory: read-out, scan, input preparation, projections
        TR(gemm(hb, true, false, d, d, N, 1.0f, a.o, d, t->dx, d, 0.0f, gw("wo"), d));
        TR(gemm(hb, false, true, N, d, d, 1.0f, t->dx, d, w("wo"), d, 0.0f, t->dA, d));
        TR(ava::train::readout_bwd(a.y, a.g, t->dA, B, T, nh, t->dB, t->dg, st));
        TR(ava_mem_scan_bwd(a.hq, a.hk, a.he, a.hv, a.hla, a.hb, B * nh, T, 64, 64, c.momentum, c.cap, nullptr,
                            nullptr, t->dB, nullptr, nullptr, t->dq, t->dk, t->de, t->dv, t->dla, t->db, nullptr,
                            nullptr, t->mwork, t->mwork_bytes, st));
        const bool res = c.value_residual && i > 0;
        TrainPrep pp{a.q, a.k, a.v, a.we, a.zab, a.lra, a.lrb, w("ba"), w("bb"), w("off"), res ? vfirst : nullptr,
                     w("vres"), a.hq, a.hk, a.he, a.hv, a.hla, a.hb, B, T, nh};
        TrainPrepGrad pg{t->dq, t->dk, t->de, t->dv, t->dla, t->db, t->dq_raw, t->dk_raw, t->dv_raw, t->dwe,
                         t->dza, t->dzb, t->dzab, t->dvfirst, res ? t->vres_part : nullptr};
        TR(ava::train::prep_bwd(pp, pg, st));
        if (res) TR(ava::train::colsum(t->vres_part, N * nh, 2, 2, gw("vres"), 0, t->part, st));
        if (i == 0 && c.value_residual) TR(ava::train::axpy(t->dv_raw, t->dvfirst, 1.0f, Nd, st));
        const float *dps[5] = {t->dq_raw, t->dk_raw, t->dv_raw, t->dwe, t->dg};
        const char *wn[5] = {"wq", "wk", "wv", "we", "wg"};
        for (int p = 0; p < 5; p++) {
            TR(gemm(hb, true, false, d, d, N, 1.0f, a.h2, d, dps[p], d, 0.0f, gw(wn[p]), d));
            TR(gemm(hb, false, true, N, d, d, 1.0f, dps[p], d, w(wn[p]), d, p == 0 ? 0.0f : 1.0f, t->dA, d));
        }
        // the head gates and their biases
        TR(gemm(hb, true, false, d, nh, N, 1.0f, a.h2, d, t->dzab, 2 * nh, 0.0f, gw("wa"), nh));
        TR(gemm(hb, true, false, d, nh, N, 1.0f, a.h2, d, t->dzab + nh, 2 * nh, 0.0f, gw("wb"), nh));
        TR(gemm(hb, false, true, N, d, nh, 1.0f, t->dzab, 2 * nh, w("wa"), nh, 1.0f, t->dA, d));
        TR(gemm(hb, false, true, N, d, nh, 1.0f, t->dzab + nh, 2 * nh, w("wb"), nh, 1.0f, t->dA, d));
        TR(ava::train::colsum(t->dzab, N, nh, 2 * nh, gw("ba"), 0, t->part, st));
        TR(ava::train::colsum(t->dzab + nh, N, nh, 2 * nh, gw("bb"), 0, t->part, st));
        // the rank-r read-outs: lr = (h Wx1) Wx2
        const float *dlr[2] = {t->dza, t->dzb};
        const char *w1n[2] = {"wa1", "wb1"}, *w2n[2] = {"wa2", "wb2"};
        for (int p = 0; p < 2; p++) {
            TR(gemm(hb, true, false, r, d, N, 1.0f, a.z1 + p * r, 2 * r, dlr[p], d, 0.0f, gw(w2n[p]), d));
            TR(gemm(hb, false, true, N, r, d, 1.0f, dlr[p], d, w(w2n[p]), d, 0.0f, t->dz1 + p * r, 2 * r));
            TR(gemm(hb, true, false, d, r, N, 1.0f, a.h2, d, t->dz1 + p * r, 2 * r, 0.0f, gw(w1n[p]), r));
            TR(gemm(hb, false, true, N, d, r, 1.0f, t->dz1 + p * r, 2 * r, w(w1n[p]), r, 1.0f, t->dA, d));
        }
        TR(ava::train::rms_bwd(a.x1, a.inv2, w("mem_norm"), t->dA, N, d, t->dx, gw("mem_norm"), t->part, st));
        // spiking layer
        TR(gemm(hb, true, false, d, d, N, 1.0f, a.S, d, t->dx, d, 0.0f, gw("wout"), d));
        TR(gemm(hb, false, true, N, d, d, 1.0f, t->dx, d, w("wout"), d, 0.0f, t->dA, d));  // dL/dspikes
        AVA_HIP(hipMemsetAsync(t->lv, 0, (size_t)B * d * 4, st));
        if (t->lif_seg)
            TR(ava::lif_scan_bwd_seg(a.cur, B, T, d, a.ps, t->lv, t->lv, t->lv, c.levels, 1, c.alif, t->slope,
                                     t->reset_grad, t->dA, nullptr, nullptr, t->dI, t->dv0, c.alif ? t->da0 : nullptr,
                                     t->dbsh, c.alif ? t->drsh : nullptr, c.alif ? t->dgsh : nullptr, t->lws,
                                     t->lws_floats, a.lpark, st));
        else
            TR(ava_lif_scan_bwd(a.cur, B, T, d, a.ps, t->lv, t->lv, t->lv, c.levels, 1, c.alif, t->slope,
                                t->reset_grad, t->dA, nullptr, nullptr, t->dI, t->dv0, c.alif ? t->da0 : nullptr,
                                t->dbsh, c.alif ? t->drsh : nullptr, c.alif ? t->dgsh : nullptr, st));
        // cur = z (1 - beta): dz = dI (1 - beta); d beta = (the scan's shares over streams) - sum_n dI z
        float *dz = t->dI;
        if (c.lif_scale) {
            TR(ava::train::mul(t->dI, a.z, Nd, t->dB, st));
            TR(ava::train::colsum(t->dB, N, d, d, t->dvec, 0, t->part, st));
            TR(ava::train::scale_cols(t->dI, a.omb, N, d, t->dC, st));
            dz = t->dC;
            TR(ava::train::colsum(t->dbsh, B, d, d, t->dvec2, 0, t->part, st, t->dvec, -1.0f));
        } else {
            TR(ava::train::colsum(t->dbsh, B, d, d, t->dvec2, 0, t->part, st));
        }
        TR(ava::train::sigmoid_chain(w("beta_p"), t->dvec2, d, gw("beta_p"), st));
        if (c.alif) {
            TR(ava::train::colsum(t->drsh, B, d, d, t->dvec, 0, t->part, st));
            TR(ava::train::sigmoid_chain(w("arho"), t->dvec, d, gw("arho"), st));
            TR(ava::train::colsum(t->dgsh, B, d, d, gw("again"), 0, t->part, st));
        }
        TR(gemm(hb, true, false, d, d, N, 1.0f, a.h1, d, dz, d, 0.0f, gw("win"), d));
        TR(gemm(hb, false, true, N, d, d, 1.0f, dz, d, w("win"), d, 0.0f, t->dA, d));
        TR(ava::train::rms_bwd(xin, a.inv1, w("lif_norm"), t->dA, N, d, t->dx, gw("lif_norm"), t->part, st));
        // dx is now dL/d(the block's input) = G_{i-1}
        if (i > 0) AVA_HIP(hipMemcpyAsync(t->G + (size_t)(i - 1) * Nd, t->dx, Nd * 4, hipMemcpyDeviceToDevice, st));
    }
    // the embedding: its direct path into block 0 plus every dense mix that reads stream 0
    if (c.dense)
        TR(ava_dense_back(t->streams, t->G, wdense, t->dx, t->dA, nullptr, 0, 0, L, 0, (long long)Nd, nullptr, 0, st));
    else
        AVA_HIP(hipMemcpyAsync(t->dA, t->dx, Nd * 4, hipMemcpyDeviceToDevice, st));
    TR(ava::train::embed_bwd(ids, t->dA, N, d, V, dE, st));
    return AVA_OK;
}

}  // namespace

extern "C" int ava_train_new(const ava_config *cfg, float slope, int reset_grad, ava_trainer **out) {
    AVA_REQUIRE(cfg && out, AVA_ERR_ARG, "train_new: NULL argument");
    *out = nullptr;
    const ava_config &c = *cfg;
    AVA_REQUIRE(c.head_size == 64 && c.d % 64 == 0 && c.d <= 1024 && c.layers >= 1 && c.layers <= 16, AVA_ERR_SHAPE,
                "train_new: d=%d head_size=%d layers=%d (head size 64, d a multiple of 64 up to 1024, <= 16 blocks)",
                c.d, c.head_size, c.layers);
    AVA_REQUIRE(c.hidden % 4 == 0 && c.hidden <= 8192 && c.kwta_k >= 1 && c.relu2, AVA_ERR_SHAPE,
                "train_new: hidden=%d (a multiple of 4, <= 8192) with relu2", c.hidden);
    AVA_REQUIRE(c.cb_units == 0 && !c.eng_half, AVA_ERR_ARG, "train_new: no cerebellum head, an f32 engram store");
    AVA_REQUIRE(c.gate_rank >= 1 && c.levels >= 1 && c.levels <= 2, AVA_ERR_SHAPE, "train_new: gate_rank=%d levels=%d",
                c.gate_rank, c.levels);
    if (c.eng_block >= 0) {
        const int enh = eng_nh(c);
        AVA_REQUIRE(c.eng_block < c.layers && c.eng_dim % enh == 0 && (c.eng_dim / enh == 64 || c.eng_dim / enh == 32),
                    AVA_ERR_SHAPE, "train_new: engram eng_dim=%d heads=%d (heads of 32 or 64)", c.eng_dim, enh);
    }
    ava_trainer *t = new ava_trainer();
    t->cfg = c;
    t->slope = slope;
    t->reset_grad = reset_grad;
    if (hipGetDevice(&t->device) != hipSuccess) {
        delete t;
        return ava::fail(AVA_ERR_HIP, "train_new: hipGetDevice failed");
    }
    size_t off = 0;
    t->slots.push_back({"tok_emb", -1, off, (size_t)c.vocab * c.d});
    off += (size_t)c.vocab * c.d;
    t->slots.push_back({"final_norm", -1, off, (size_t)c.d});
    off += c.d;
    for (int i = 0; i < c.layers; i++)
        for (const char *nm : BLOCK_NAMES) {
            const size_t n = block_count(c, i, nm);
            t->slots.push_back({nm, i, off, n});
            off += n;
        }
    t->dense_off = off;
    for (int i = 0; i < c.layers; i++) {
        const size_t n = c.dense ? (size_t)i + 2 : 0;
        t->slots.push_back({"dense", i, off, n});
        off += n;
    }
    t->nparams = off;
    if (rocblas_create_handle(&t->blas) != rocblas_status_success) {
        delete t;
        return ava::fail(AVA_ERR_HIP, "train_new: rocblas_create_handle failed");
    }
    *out = t;
    return AVA_OK;
}

extern "C" void ava_train_free(ava_trainer *t) {
    if (!t) return;
    (void)hipSetDevice(t->device);
    if (t->blas) rocblas_destroy_handle(t->blas);
    delete t;
}

extern "C" size_t ava_train_param_floats(const ava_trainer *t) { return t ? t->nparams : 0; }

extern "C" int ava_train_param_slot(const ava_trainer *t, const char *name, int block, size_t *offset,
                                    size_t *count) {
    AVA_REQUIRE(t && name && offset && count, AVA_ERR_ARG, "train_param_slot: NULL argument");
    const Slot *f = t->find(name, block);
    AVA_REQUIRE(f, AVA_ERR_ARG, "train_param_slot: no tensor %s in block %d", name, block);
    *offset = f->off;
    *count = f->n;
    return AVA_OK;
}

extern "C" int ava_train_step(ava_trainer *t, const float *params, const int32_t *ids, const int32_t *targets, int B,
                              int T, float *grads, float *loss, ava_stream stream) {
    AVA_REQUIRE(t && params && ids && targets && grads && loss, AVA_ERR_ARG, "train_step: NULL argument");
    AVA_REQUIRE(B >= 1 && T >= 1 && (size_t)B * T * t->cfg.d % 4 == 0, AVA_ERR_SHAPE, "train_step: B=%d T=%d", B, T);
    AVA_HIP(hipSetDevice(t->device));
    if (int e = ensure(t, B, T)) return e;
    return step(t, params, ids, targets, B, T, grads, loss, (hipStream_t)stream);
}

extern "C" int ava_train_decisions(const ava_trainer *t, int8_t *spikes, float *u, float *kth, ava_stream stream) {
    AVA_REQUIRE(t && t->N > 0, AVA_ERR_ARG, "train_decisions: no step has run");
    const size_t N = t->N, d = t->cfg.d, H = t->cfg.hidden;
    const hipStream_t st = (hipStream_t)stream;
    for (size_t i = 0; i < t->acts.size(); i++) {
        const Acts &a = t->acts[i];
        if (spikes) AVA_HIP(hipMemcpyAsync(spikes + i * N * d, a.spk, N * d, hipMemcpyDeviceToDevice, st));
        if (u) AVA_HIP(hipMemcpyAsync(u + i * N * H, a.u, N * H * 4, hipMemcpyDeviceToDevice, st));
        if (kth) AVA_HIP(hipMemcpyAsync(kth + i * N, a.kth, N * 4, hipMemcpyDeviceToDevice, st));
    }
    return AVA_OK;
}
