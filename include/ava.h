/*
 * ava.h — C ABI of the MI355X-native int8 block forward of Ava (libava_amd.so, gfx950).
 *
 * This header is the drop-in boundary: a host engine (the reference's is Rust, bound through a
 * thin FFI crate) calls these entry points in place of the reference's candle ops and drivers.
 * Each declaration names the reference interface it replaces (paths relative to the reference's
 * design-tests/nn/gpu/src).
 *
 * Conventions (all entry points):
 *   - every buffer is a caller-owned DEVICE pointer unless the comment says "host";
 *   - work is enqueued on `stream` (NULL = the null stream) and nothing synchronises unless stated;
 *   - the return value is an ava_status; a non-zero status leaves a message in ava_last_error()
 *     (per thread). Shape or argument errors are returned, never aborted on (the reference
 *     bail!s on shape/dtype errors: int8.rs:604-613, lif_gen.rs:132-141, mem_gen.rs:179-187);
 *   - row-major layouts; "[a][b]" = a rows of b contiguous elements.
 */
#ifndef AVA_H
#define AVA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *ava_stream; /* == hipStream_t */

enum {
    AVA_OK = 0,
    AVA_ERR_ARG = 1,         /* a NULL pointer, a negative size, an unsupported option */
    AVA_ERR_SHAPE = 2,       /* sizes that do not fit together or exceed a kernel's limits */
    AVA_ERR_HIP = 3,         /* a HIP runtime error (launch, allocation) */
    AVA_ERR_UNSUPPORTED = 4  /* a configuration this build does not run */
};

const char *ava_last_error(void);
const char *ava_version(void);

/* FNV-1a 64 over n host bytes, continuing from h (start: 0xcbf29ce484222325). The model fingerprint a
 * saved state is keyed by hashes the configuration text and sampled weights with it; replaces the
 * Fnv of gpu/state.rs:1095-1107 (Model::fingerprint, gpu/state.rs:1075-1092). */
uint64_t ava_fnv1a64(const void *p, size_t n, uint64_t h);

/* ------------------------------------------------------------------ int8 weights and products */

/* One weight matrix in int8: W [din][dout] (applied x·W), stored transposed as qt [dout][din]
 * (each output column's din weights contiguous: the K-contiguous B operand of the i8 MFMA), one
 * f32 scale per output column. Replaces QW (int8.rs:44-54). */
typedef struct {
    int din, dout;
    int ldk;      /* ava_q8_ldk(din): din padded to a multiple of 128 with zero weights */
    int8_t *qt;   /* [dout][ldk] */
    float *scale; /* [dout] */
} ava_qw;

/* din rounded up to a multiple of 128 (two K steps of the i8 MFMA kernels). */
int ava_q8_ldk(int k);

/* Quantize W [din][dout] f32 into qt [dout][ldk] / scale [dout]: scale_c = max_j |W[j][c]| / 127
 * (1 for an all-zero column), q = clamp(round half away from zero (W / scale_c), +-127), padding 0.
 * Replaces QW::from_rows (int8.rs:59-72) over ava_parts::quant::quantize_int8 (parts/src/quant.rs:18-31). */
int ava_q8_pack(const float *w, int din, int dout, int8_t *qt, float *scale, ava_stream stream);

/* Split-plane activation quantizer (part of the int8 product; the reference keeps f32 activations):
 * per row, e = the smallest exponent with max|x| 2^-e < 127.5, then planes q_p of int8 with
 * x ~= 2^e sum_p q_p 2^(-7p). xq [planes][m][ldk] (ldk = ava_q8_ldk(k), padding 0), xexp [m].
 * planes 1..3. */
int ava_q8_quant_rows(const float *x, int m, int k, int planes, int8_t *xq, int32_t *xexp,
                      ava_stream stream);

/* The raw int32 accumulators acc [planes][m][n] = A_p [m][ldk] · W (i8 MFMA, exact). For checks. */
int ava_q8_gemm_acc(const int8_t *xq, int planes, int m, const ava_qw *w, int32_t *acc,
                    ava_stream stream);

/* y [m][dout] = x [m][din] · W with f32 activations: quantize to `planes` planes (3 = the
 * accurate default), i8 MFMA per plane, combine y = ((float)sum_p acc_p 2^(7(P-1-p))) 2^(e-7(P-1)) scale_c.
 * `ws` is a device workspace of at least ava_q8_workspace(m, din, planes) bytes.
 * Replaces int8::mm / int8::head over Apply "ava-int8-matmul" (int8.rs:592-626, 672-698). */
size_t ava_q8_workspace(int m, int k, int planes);
int ava_q8_matmul(const float *x, int m, const ava_qw *w, int planes, float *y, void *ws,
                  size_t ws_bytes, ava_stream stream);

/* ava_q8_matmul without a workspace argument and without any allocation: no counterpart in the
 * reference. For callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The planes live in a static device array of the library, 32 MiB
 * per GPU, held until the process ends: ava_q8_workspace(m, din, planes) must be at most 32 MiB
 * (AVA_ERR_SHAPE otherwise). Every call on one GPU shares that array, so calls that overlap on one
 * GPU (on different streams, or from different threads) race; calls on one stream are ordered.
 * Nothing in the array needs clearing: each call writes all it reads. Same results as ava_q8_matmul. */
int ava_q8_matmul_noalloc(const float *x, int m, const ava_qw *w, int planes, float *y, ava_stream stream);

/* y [m][dout] from activations already in split-plane form (xq [planes][m][ldk], xexp [m], as
 * ava_q8_quant_rows writes them): the product and combine of ava_q8_matmul without the quantizer.
 * Replaces int8::mm (int8.rs:672-683) where the producer of x writes planes directly. */
int ava_q8_matmul_planes(const int8_t *xq, const int32_t *xexp, int planes, int m, const ava_qw *w,
                         float *y, ava_stream stream);

/* y [m][dout] = s [m][ldk] · W for integer inputs (the LIF's spikes, -2..2; padding columns 0):
 * y = (float)acc · scale_c, the reference's bits exactly (its f32 sum of integer products is
 * exact). Replaces int8::mm on the spikes (arch.rs:1695, fstep/arch.rs:675). */
int ava_q8_matmul_i8(const int8_t *s, int m, const ava_qw *w, float *y, ava_stream stream);

/* ------------------------------------------------------------------ LIF scan */

/* The general LIF scan over cur [B][T][D] (f32): ps = [beta | theta | rho | gain] ([4][D]);
 * v, s, a [B][D]: the carried membrane, last spikes and ALIF trace on entry, the final ones on
 * exit. Per (b, c), sequential in t, each operation rounded alone:
 *   a = a rho + |s| (1 - rho) (alif);  th_t = theta + a gain;  v = (v beta + I) - s th_{t-1};
 *   s = sum_{k=1..levels} [v - k th_t >= 0] - [-v - k th_t >= 0]   (binary: [v - th_t >= 0]).
 * spikes [B][T][D] int8. th_out [B][D] (nullable): the final threshold theta + gain a_T.
 * levels 1..2. Replaces LifGen "lif-gen" (lif_gen.rs:182-237), kernels lifg_fwd_* (lif.cu:3123-3221). */
int ava_lif_scan(const float *cur, int B, int T, int D, const float *ps, float *v, float *s, float *a,
                 int levels, int is_signed, int alif, int8_t *spikes, float *th_out, ava_stream stream);

/* ------------------------------------------------------------------ kWTA */

/* Per row of u [n][h]: kth = the k-th largest value (duplicates counted); keep u_i when
 * u_i - kth >= 0 (ties kept); a = relu(u · mask), squared when relu2. kth_out [n] (nullable).
 * k >= h keeps every unit. h <= 8192. Replaces KwtaMask "kwta-mask" (lif.rs:239-284) /
 * model::kwta_mask (model.rs:504-528) and kwta_relu2 (lif.cu:4629-4680, fwin_ops.rs:133). */
int ava_kwta(const float *u, int n, int h, int k, int relu2, float *a, float *kth_out,
             ava_stream stream);

/* ------------------------------------------------------------------ fast-weight memory */

/* The general fast-weight recurrence per head row-block bh (F [hs][hs], row i = key channel):
 *   r_j = sum_i e_i F_ij;  u_ij = b_i k_i v_j - a_i b_i e_i r_j;  S <- M S + u;
 *   F_ij <- clamp(a_i F_ij + S_ij, +-cap) (M = 0: + u_ij);  y_j = sum_i q_i F_ij.
 * q, k, e, v [BH][T][hs]; la (log alpha), b [BH][T][g] with g = 1 (per head) or hs (per channel);
 * F, S [BH][hs][hs] carried in and out (S ignored when m == 0); y [BH][T][hs]. hs == 64.
 * Replaces MemGen "mem-gen" (mem_gen.rs:248-309) / delta_rec (arch.rs:1091-1136). */
int ava_mem_scan(const float *q, const float *k, const float *e, const float *v, const float *la,
                 const float *b, int BH, int T, int hs, int g, float m, float cap, float *F, float *S,
                 float *y, ava_stream stream);

/* ava_mem_scan's rule (same arguments, layout and result) in its chunked form: chunks of 16 tokens whose
 * contractions with the carried F and S, and the intra-chunk products, run on the fp32 matrix cores; the
 * recalls of a chunk solve one unit lower-triangular system. The bound clamp(F, +-cap) is applied at
 * chunk ends, not per token (equal while no element of F reaches cap inside a chunk). Any T >= 0.
 * Replaces delta_chunk / chunk_core (arch.rs:1151-1164, 1243-1327), the reference's CPU default for
 * per-channel gates and momentum. */
int ava_mem_chunk(const float *q, const float *k, const float *e, const float *v, const float *la,
                  const float *b, int BH, int T, int hs, int g, float m, float cap, float *F, float *S,
                  float *y, ava_stream stream);

/* The gated delta rule F_t = alpha_t (I - beta_t k_t k_t^T) F_{t-1} + beta_t k_t v_t^T, y_t = F_t^T q_t
 * (F = W^T: with alpha = 1 this is W += beta (v - W k) k^T, y = W q) in its chunked (WY/UT) form,
 * chunks of 64 tokens: q, k, v [BH][T][64]; la = log alpha per token and head [BH][T] (NULL: alpha = 1);
 * beta [BH][T]; F [BH][64][64] carried in and out; y [BH][T][64]. T a multiple of 64.
 * Replaces model::delta_rule_from (model.rs:744-799) for per-head gates. */
int ava_delta_chunk(const float *q, const float *k, const float *v, const float *la, const float *beta, int BH,
                    int T, int hs, float *F, float *y, void *work, size_t work_bytes, ava_stream stream);
/* work (nullable): device scratch of ava_delta_chunk_workspace(BH, T) bytes. Without gates (la NULL) and
 * with it, the chunks' triangular inverses are formed for every chunk at once first, and the walk over
 * the chunks is six products per chunk; otherwise one kernel walks the chunks with the solve inside. The
 * results agree to rounding. */
size_t ava_delta_chunk_workspace(int BH, int T);

/* ------------------------------------------------------------------ backward (training step) */

/* The LIF scan's backward: the surrogate gradient of the straight-through spikes (ds/dv per spike edge
 * x = v - k th, -v - k th: 1 / (1 + slope |x|)^2). Inputs as ava_lif_scan's, with the INITIAL state
 * v0, s0, a0 [B][D] (unchanged); g_spk [B][T][D] = dL/d(spikes), g_vT, g_aT [B][D] = dL/d(final v, a)
 * (nullable: 0). reset_grad: the reset v -= s th_{t-1} carries gradient too, its carry capped at
 * 2 beta / (ds/dv) where th ds/dv > 2 beta (the reference's negative slope / rgi = 1). Outputs dI
 * [B][T][D] = dL/dcur, dv0, da0 [B][D], and per (b, c) the shares of dbeta, drho, dgain [B][D] (the
 * parameter gradients are their sums over b; theta is detached). da0, drho, dgain may be NULL without
 * alif. Replaces lifg_bwd_* (gpu/lif.cu:3222-3290, LifGenBwd, gpu/lif_gen.rs:239-361) and the
 * gradient of lif_ref (gpu/arch.rs:964-1071). */
int ava_lif_scan_bwd(const float *cur, int B, int T, int D, const float *ps, const float *v0, const float *s0,
                     const float *a0, int levels, int is_signed, int alif, float slope, int reset_grad,
                     const float *g_spk, const float *g_vT, const float *g_aT, float *dI, float *dv0, float *da0,
                     float *dbeta, float *drho, float *dgain, ava_stream stream);

/* ava_lif_scan_bwd in parallel segments of 32 steps, for few (stream, channel) chains (B D of a few
 * thousand, as at a training batch of 4): the forward is replayed once to park each segment's state,
 * every (chain, segment) then walks its steps back as affine functions of what the later steps carry
 * (the walk is linear in it given the forward), the segments' functions are applied in order, and each
 * segment is walked again with its entering carry to write dI. The same arguments and outputs as
 * ava_lif_scan_bwd, equal up to the association of the backward sums (ava_lif_scan_bwd's walk is the
 * CPU's order), plus a device workspace ws of ava_lif_scan_bwd_segments_workspace(B, T, D) bytes.
 * Replaces lifg_bwd_* (gpu/lif.cu:3222-3290) where its per-chain loop leaves the GPU idle. */
size_t ava_lif_scan_bwd_segments_workspace(int B, int T, int D);
int ava_lif_scan_bwd_segments(const float *cur, int B, int T, int D, const float *ps, const float *v0,
                              const float *s0, const float *a0, int levels, int is_signed, int alif, float slope,
                              int reset_grad, const float *g_spk, const float *g_vT, const float *g_aT, float *dI,
                              float *dv0, float *da0, float *dbeta, float *drho, float *dgain, void *ws,
                              size_t ws_bytes, ava_stream stream);

/* The backward of relu² after kWTA: gu = (u ga) 2 where u - kth >= 0 and u > 0, else 0, for u [n][h]
 * and the row thresholds kth [n] that ava_kwta returned (h a multiple of 4). Replaces relu2_bwd
 * (gpu/lif.cu:4666-4679), whose input a = kwta_relu(u) is u on the kept units. */
int ava_kwta_relu2_bwd(const float *u, const float *kth, int n, int h, const float *ga, float *gu,
                       ava_stream stream);

/* The backward of ava_mem_scan (same layout and gates; hs == 64) from the initial state F0, S0
 * (nullable: zeros) with dy [BH][T][hs] = dL/dy and dF_T, dS_T = dL/d(final F, S) (nullable: zeros):
 * dq, dk, de, dv [BH][T][hs]; dla, db [BH][T][g]; dF0, dS0 [BH][hs][hs] (nullable) = dL/d(F0, S0).
 * The bound clamp(., +-cap) passes no gradient where it holds. work: device memory of
 * ava_mem_scan_bwd_workspace(BH, T, m != 0) bytes (the states the replay keeps and, below 512 heads,
 * where each head's columns are split over four workgroups, their partial row sums). Replaces memg_bwd_* /
 * memg_bwd4_* (gpu/lif.cu:3411-3888; MemGenBwd, gpu/mem_gen.rs:296-470) and the gradient of delta_rec
 * (gpu/arch.rs:1091-1136). */
size_t ava_mem_scan_bwd_workspace(int BH, int T, int momentum);
int ava_mem_scan_bwd(const float *q, const float *k, const float *e, const float *v, const float *la, const float *b,
                     int BH, int T, int hs, int g, float m, float cap, const float *F0, const float *S0,
                     const float *dy, const float *dF_T, const float *dS_T, float *dq, float *dk, float *de,
                     float *dv, float *dla, float *db, float *dF0, float *dS0, void *work, size_t work_bytes,
                     ava_stream stream);

/* The dense (DenseFormer) mix's backward over S [R][M] (the streams: 0 the embedding, j + 1 block j's
 * raw output) and G [L][M] (row k = dL/d(the mix after block k)); wf packs block k's k + 2 weights
 * from k (k + 3) / 2. out [M] = base + sum_{k = i0 .. L-1} w_k[col] G_k (added in k order);
 * dw [nd] = sum_e base_e S_j,e. Block i: base = G_i, col = i + 1, i0 = i, nd = i + 2 gives dL/draw_i
 * and dL/dw_i; the embedding: col 0, i0 0, nd 0. part: ava_dense_back_part_floats(M, nd) floats of
 * device scratch (NULL with nd == 0). M a multiple of 4, nd <= 32. Replaces dense_back
 * (gpu/lif.cu:4922-4971). */
size_t ava_dense_back_part_floats(long long M, int nd);
int ava_dense_back(const float *S, const float *G, const float *wf, const float *base, float *out, float *dw, int col,
                   int i0, int L, int nd, long long M, float *part, size_t part_floats, ava_stream stream);

/* ------------------------------------------------------------------ engram read */

/* The engram's causal single-head read (head size 64) over a store that already holds entries
 * 0..n0+T-1 of each stream: query (b, t), row b*T + t of q (ldq floats apart), reads entries
 * 0..n0+t: softmax(q.k / sqrt(64)) . V, the softmax in its online (running max) form. ks, vs
 * [B][cap][64] of f32, or of fp16 (IEEE binary16) with kv_half; out [B*T][64]. For T <= 4 (decode)
 * the keys are cut into chunks of 1024 read by separate workgroups, whose partials need
 * ava_attend_part_floats(B, T, n0) floats of device scratch in part; for T > 4 part may be NULL.
 * Replaces fstep::attend (model/fstep.rs:303-329) and one head of attention_g (model.rs:543-562) /
 * memory::read. */
size_t ava_attend_part_floats(int B, int T, int n0);
int ava_attend(const float *q, int ldq, const void *ks, const void *vs, int kv_half, int cap, int n0, int B, int T,
               float *out, float *part, size_t part_floats, ava_stream stream);

/* The same read with heads (memory::read, gpu/memory.rs:610-700: heads of 32, scores scaled by
 * 1/sqrt(32)): a row of q, of the store and of out holds de dims, heads h*hd .. h*hd + hd - 1 side
 * by side, hd = de / heads (32 or 64; de a multiple of 64, <= 4096). Each head reads its own slice of
 * the keys and values. ks, vs [B][cap][de]; out [B*T][de]; decode partials as ava_attend's, sized
 * by ava_attend_heads_part_floats. */
size_t ava_attend_heads_part_floats(int B, int T, int n0, int de, int heads);
int ava_attend_heads(const float *q, int ldq, const void *ks, const void *vs, int kv_half, int cap, int n0, int B,
                     int T, int de, int heads, float *out, float *part, size_t part_floats, ava_stream stream);

/* ------------------------------------------------------------------ model */

/* The block options of the path (Ava 0.4's recipe, release/ava-0.4/arch.txt:1). */
typedef struct {
    int vocab, d, layers, hidden, kwta_k, head_size, gate_rank;
    int eng_block;  /* the block with the engram read, -1 for none */
    int eng_dim;    /* the engram's dims: its single head (64), or eng_heads heads of 32 */
    int levels;     /* spike levels each side (2 = int2) */
    int alif, lif_scale, value_residual, dense, relu2;
    float momentum, cap;
    int planes;     /* activation planes of the dense int8 products (3 = accurate) */
    /* The cerebellum head (gpu/v51b.rs:18-32): cb_units granule units (0 = off; a multiple of 32,
     * <= 16384), the top cb_units/32 kept. cb_lr is the online table's rate (Model::cb_rate,
     * gpu/v51b.rs:606-611, gives eta / mean |E_v|^2), cb_half its half-life in tokens (<= 0: it
     * never fades; gpu/v51b.rs:352-367). */
    int cb_units;
    float cb_lr, cb_half;
    /* The engram store's element: 0 = f32 (the reference's store), 1 = fp16, a KV cache of half the
     * bytes (config[4]); the state's eng_k and eng_v then hold IEEE binary16 values. */
    int eng_half;
    /* The engram's heads: 0 or 1 = one head of eng_dim (64); eng_dim / 32 = the reference's heads of
     * 32 (gpu/memory.rs:610-700, HEAD_SIZE 32; eng_dim a multiple of 64 up to 1024, normally d).
     * The store row [eng_dim] holds the heads side by side. */
    int eng_heads;
} ava_config;

/* f32 HOST weights, named as the reference's VarMap (arch.rs:806-860). W [din][dout] as applied x·W. */
typedef struct {
    const float *lif_norm, *win, *beta_p, *theta, *arho, *again, *wout;
    const float *mem_norm, *wq, *wk, *wv, *we, *wg, *wo;
    const float *wa, *ba, *wb, *bb, *off, *wa1, *wa2, *wb1, *wb2, *vres;
    const float *eng_norm, *ewq, *ewk, *ewv, *ewo; /* engram block only */
    const float *mlp_norm, *w1, *w2, *dense;
} ava_block_params;

typedef struct {
    const float *tok_emb;    /* [vocab][d]; the head is its transpose in int8 */
    const float *final_norm; /* [d] */
    const ava_block_params *blocks;
    const float *cb_w;       /* [cb_units][d] the cerebellum's read-out cbh.wo (NULL: zero, as at init) */
} ava_params;

/* The carried state of B streams (caller-owned device buffers). Replaces State's LIF, memory and
 * engram tensors (state.rs:94-116). The engram store is f32, as the reference's key/value store
 * (model/fstep/arch.rs:952-961). mem_s is read and written only when momentum != 0; the engram
 * store only when eng_block >= 0. */
typedef struct {
    float *lif_v, *lif_s, *lif_a; /* [layers][B][d] */
    float *mem_f, *mem_s;         /* [layers][B][d/hs][hs][hs] */
    float *eng_k, *eng_v;         /* [B][eng_cap][eng_dim] (fp16 elements when the config's eng_half) */
    int eng_cap, eng_len;         /* eng_len advances by T per forward */
    /* The cerebellum's online table per stream (gpu/v51b.rs:340-367, CbOnline): cb_tab
     * [B][cb_units][d] (its `delta`; NULL: no table), cb_scale [B] f64 (its `scale`, 1 at the start),
     * and cb_code [B][cb_units], the granule code of each stream's last position, which
     * ava_model_cb_learn uses (CbOnline::last). All NULL when cb_units == 0. */
    float *cb_tab;
    double *cb_scale;
    float *cb_code;
    /* Optional (NULL: unused): the store length on the device, one int32 kept equal to eng_len. With
     * it the engram kernels read the length from the device and each forward advances it there, so a
     * forward captured in a HIP graph stays correct on replay (the host's eng_len only advances on
     * real calls; the caller keeps replays within eng_cap, and the device length saturates there). */
    int32_t *eng_len_dev;
    /* Optional (NULL: not kept), for the least-read cap (Evict::LeastRead, state.rs:37-69, 518-590):
     * per stream and slot [B][eng_cap], the attention mass the slot received from later queries (the
     * mean over heads, each query's own key left out) and how many later queries could see it; each
     * forward advances them as memory::read does with count_reads (memory.rs:700-738). The caller
     * evicts between forwards (ranking slots by reads / age). */
    float *eng_reads, *eng_age;
} ava_state;

typedef struct ava_model ava_model;

/* Build the model: upload and quantize every int8 matrix (Model::new + set_int8, model.rs:805, 949-991). */
int ava_model_new(const ava_config *cfg, const ava_params *params, ava_model **out);
void ava_model_free(ava_model *m);

/* Teacher-forced forward of ids [B][T] (device int32) from the carried state st (updated in place):
 * logits [B*T][vocab] f32 (nullable). Replaces Model::forward_with_state (state.rs:684-865) and,
 * from a zero state, Model::forward (model.rs:1171) / forward_arch (arch.rs:1407-1566).
 * Scratch memory is allocated on first use per (B, T) and kept by the model. */
int ava_model_forward(ava_model *m, ava_state *st, const int32_t *ids, int B, int T, float *logits,
                      ava_stream stream);

/* One online learning step of every stream's cerebellum table (gpu/fast4/cb.rs:25-84, Model::cb_learn):
 * logits [B] rows of ld_logits floats (device; the rows of each stream's last position of the last
 * forward), next [B] the words that followed (device int32; outside [0, vocab): no step for that
 * stream, the reference's IGNORE). Per stream: p = softmax(logits), delta = (p - onehot(next)) . E,
 * the scale fades by 2^(-1/cb_half) (folded into the table below 1e-18), and each unit u of the kept
 * code moves: tab[u] -= (cb_lr c_u / scale) delta. nats [B] (device f64, nullable) = -ln p_next. */
int ava_model_cb_learn(ava_model *m, ava_state *st, const float *logits, int ld_logits, const int32_t *next, int B,
                       double *nats, ava_stream stream);

/* One decode step with the previous token's table step overlapped (no counterpart in the reference,
 * whose talking loop runs Model::cb_learn after each forward: gpu/v51b.rs:590-611). With prev_logits
 * NULL this is ava_model_forward. Otherwise the learning step of ava_model_cb_learn for
 * (prev_logits [B] rows of ld_prev floats, prev_next [B], prev_nats nullable) runs on a second stream
 * of the model's while this step's blocks run on `stream`, and the forward waits for it before its
 * final norm and cerebellum, which read and overwrite the code, the table and its scale. The results
 * are those of ava_model_cb_learn(prev) followed by ava_model_forward(ids), bit for bit. The caller
 * keeps prev_logits and prev_next unchanged until the step completes on `stream` (alternate two
 * buffers for logits and next), and logits may not be prev_logits. Capturable in a HIP graph. */
int ava_model_decode_step(ava_model *m, ava_state *st, const int32_t *ids, int B, int T, float *logits,
                          const float *prev_logits, int ld_prev, const int32_t *prev_next, double *prev_nats,
                          ava_stream stream);

/* Bytes of scratch the model holds after forwards of up to B*T rows. */
size_t ava_model_scratch_bytes(const ava_model *m);

/* While frozen (on != 0) the model never frees or reallocates its scratch: a forward or learning
 * step that would need more fails with AVA_ERR_ARG instead. For callers that capture forwards in HIP
 * graphs, which keep the scratch's addresses (no reference counterpart: the reference has no graphs). */
int ava_model_freeze(ava_model *m, int on);

/* The fused step's non-finite guard (gpu/model/fstep/arch.rs:780-783, 861-864: a non-finite gate, key,
 * query or value refuses the token before anything is committed). Every memory head checks the values
 * it stages (unit q, k and erase key, value, alpha, b k, alpha b e); a head that meets a non-finite one
 * leaves its fast weights F and S as they were and marks its stream. After a forward (this call waits
 * for the stream): count = the streams marked, rows [B of that forward] (nullable, host, rows_cap
 * entries; AVA_ERR_SHAPE when fewer than that forward's B) = 1 for each. A forward that was refused
 * reports no streams. The stream's LIF state and engram store are committed as usual (as the
 * reference's plain path, which then takes the token, commits them). */
int ava_model_nonfinite(ava_model *m, int32_t *rows, int rows_cap, int *count, ava_stream stream);

/* The decision trace, for parity checks (no counterpart in the reference, whose tests compare single
 * ops): with the buffers set (all NULL: off), every forward copies per block i the spikes [B*T][d]
 * int8, the wide layer's values before the kWTA u [B*T][hidden] f32 and each row's k-th largest value
 * kth [B*T] into rows pos .. pos + B*T - 1 of block i's slice of spikes [layers][rows][d],
 * u [layers][rows][hidden] and kth [layers][rows]. pos starts at 0 (each call of this function resets
 * it) and advances by B*T per forward; a forward that would pass `rows` fails with AVA_ERR_SHAPE
 * before it runs. With the spikes and the kWTA's index set (u - kth >= 0) a checker can replay this
 * model's discrete decisions. */
int ava_model_set_trace(ava_model *m, int8_t *spikes, float *u, float *kth, size_t rows);

/* Launch timing by kernel class (the counterpart of int8::set_mm_prof, int8.rs:628-669): with `on`,
 * every launch of ava_model_forward is bracketed by HIP events on its stream. ava_model_timing
 * synchronises the stream of the last forward, then fills up to `cap` entries of names (static
 * strings), launch counts and summed milliseconds since the last reset, and returns the number of
 * classes (or -1 on error). reset clears the sums. */
int ava_model_set_timing(ava_model *m, int on);
int ava_model_timing(ava_model *m, const char **names, int *calls, double *ms, int cap, int reset);

/* The store's cap after a forward (EngramCap / evict, gpu/state.rs:37-69, 518-590), on the device: each
 * of the B streams' stores [B][cap][de] (f32, or fp16 with kv_half) that holds more than eng_max entries
 * keeps eng_max of them, moved to the front in store order. rule 0 (oldest): the last eng_max. rule 1
 * (least-read): every slot ranks by (class, value, index), class 1 for a slot some later query could
 * see (age >= 1; value = reads / age), class 2 for the slots no later query has seen; the last eng_max of
 * the ranking stay. reads, age [B][cap] (rule 1; nullable for rule 0) move with their slots. n: the
 * store length, or len_dev (nullable): the length on the device, read there and set to eng_max (so a
 * captured step may evict). No host synchronisation. */
int ava_engram_evict(void *k, void *v, float *reads, float *age, int B, int cap, int n, int32_t *len_dev, int de,
                     int kv_half, int eng_max, int rule, ava_stream stream);

/* ------------------------------------------------------------------ the training step */

/* The float32 training step of the block stack (the reference's hand-written step, gpu/model/fwin.rs:1-40:
 * every forward op a kernel and every backward the matching one, no autograd): one teacher-forced batch
 * from a zero state, its mean cross-entropy and the gradient of every parameter. The forward is the
 * block of ava_model_forward in f32 (f32 weights, no int8): rms -> Win (1 - beta) -> LIF scan -> Wout;
 * rms -> q, k, v, e, g and the gates -> the memory scan -> read-out -> Wo; the engram read (one block,
 * heads of 32 or 64); rms -> W1 -> kWTA relu^2 -> W2; the dense mix; the final norm and the tied head
 * E^T. slope: the LIF surrogate's slope (the reference's --surrogate-slope, 4 by default); reset_grad:
 * carry the gradient through the reset (--lif-reset-grad). theta is detached and the gate offsets are
 * constants (their gradients are 0). Needs head size 64, relu2, no cerebellum head, an f32 store. */
typedef struct ava_trainer ava_trainer;
int ava_train_new(const ava_config *cfg, float slope, int reset_grad, ava_trainer **out);
void ava_train_free(ava_trainer *t);

/* The parameters (and gradients) are one flat f32 device buffer of ava_train_param_floats floats. A tensor's
 * place: name "tok_emb" or "final_norm" with block -1, or a block tensor named as in ava_block_params
 * ("win", "beta_p", ..., "dense") with its block; shapes as there ([din][dout] for matrices). The dense
 * weights of all blocks are contiguous, block k's k + 2 weights from k (k + 3) / 2 after the first.
 * AVA_ERR_ARG for an unknown name; count 0 for the engram tensors of other blocks. */
size_t ava_train_param_floats(const ava_trainer *t);
int ava_train_param_slot(const ava_trainer *t, const char *name, int block, size_t *offset, size_t *count);

/* One step: ids, targets [B][T] (device int32; a target outside [0, vocab) does not count); params as
 * above; grads (same layout) are overwritten; loss [1] (device f32) = the mean over counted positions of
 * -log softmax(logits)[target]. Scratch for B*T rows is allocated on first use and kept. Replaces the
 * reference's loss_and_grads for the Ava-0.4 recipe (gpu/model/fwin.rs). */
int ava_train_step(ava_trainer *t, const float *params, const int32_t *ids, const int32_t *targets, int B, int T,
                   float *grads, float *loss, ava_stream stream);

/* The last step's discrete decisions (no counterpart in the reference; for parity checks): spikes
 * [layers][B*T][d] int8, the wide layer's u [layers][B*T][hidden] and its k-th values kth [layers][B*T]
 * (device, nullable each). */
int ava_train_decisions(const ava_trainer *t, int8_t *spikes, float *u, float *kth, ava_stream stream);

#ifdef __cplusplus
}
#endif
#endif
