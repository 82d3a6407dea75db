/*
 * ava_oracle.h — CPU oracle for the int8 block forward of Ava (nochallenge/ava).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP kernels are compared against
 * (tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg). The product path
 * (ava_amd/, libava_amd.so) never links, loads or calls it.
 *
 * Every function restates one piece of the reference's CPU engine (Rust, design-tests/nn/):
 * the citation next to each declaration names the file:line it follows. Reference paths are
 * relative to design-tests/nn/ (gpu/ = design-tests/nn/gpu/src).
 *
 * Two int8 product semantics live here:
 *   - the reference's: int8 weights, f32 activations, f32 fused multiply-adds in the order
 *     j = 0, 1, ... from +0, one multiply by the column scale (gpu/int8.rs:301-331);
 *   - the build's split-plane form: activations as P planes of int8 under a power-of-two row
 *     scale, exact int32 accumulators per plane, one combine (no reference counterpart; it is
 *     what the i8 MFMA kernels compute, so their accumulators are checked bit for bit here).
 */
#ifndef AVA_ORACLE_H
#define AVA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- int8 weights */

/* parts/src/quant.rs:18-31. W [din][dout] row-major (applied x·W). scale[c] = max_j |W[j][c]| / 127
 * (1 for an all-zero column); q = clamp(round_half_away(W / scale), -127, 127). */
void orc_quantize_int8(const float *w, int din, int dout, int8_t *q, float *scale);

/* gpu/int8.rs:301-331 (tile_scalar) and :166-211 (matmul_rows_with): y[r][c] = scale[c] *
 * (fma chain over j ascending from +0 of x[r][j] * (float)q[j][c]). Zero inputs are skipped
 * (E2, gpu/int8.rs:10-13: the same bits). q [din][dout] row-major. Rows are split over
 * `threads` OpenMP threads; each output is written by one thread, so any count gives the same bits. */
void orc_q8_matmul_ref(const float *x, int m, int din, const int8_t *q, const float *scale,
                       int dout, float *y, int threads);
/* The two forms orc_q8_matmul_ref chooses between (from 6 rows the blocked one, gpu/int8/block.rs:
 * 6 x 16 register blocks over an f32 copy of each 64-column tile, sparse rows as event sums): the same
 * bits as each other. */
void orc_q8_matmul_rows(const float *x, int m, int din, const int8_t *q, const float *scale, int dout, float *y,
                        int threads);
void orc_q8_matmul_blocked(const float *x, int m, int din, const int8_t *q, const float *scale, int dout,
                           float *y, int threads);

/* The build's split-plane activation quantizer (no reference counterpart). For each row:
 * e = the smallest exponent with max|x| * 2^-e < 127.5 (e = 0 for an all-zero row);
 * t0 = x*2^-e, q0 = rint(t0), r0 = t0 - q0; t1 = r0*128, q1 = rint(t1), r1 = t1 - q1; ...
 * so x ~= 2^e * sum_p q_p * 2^(-7p). xq [planes][m][k], xexp [m]. */
void orc_quant_planes(const float *x, int m, int k, int planes, int8_t *xq, int32_t *xexp);

/* Exact int32 accumulators acc [m][n] = sum_j a[m][j] * q[j][n] for int8 a [m][k], q [k][n]. */
void orc_q8_acc(const int8_t *a, int m, int k, const int8_t *q, int n, int32_t *acc, int threads);

/* The combine shared with the GPU epilogue: A = sum_p acc_p * 2^(7(P-1-p)) (int64, exact);
 * y = (float)A; y = y * 2^(xexp - 7(P-1)) (exact); y = y * scale[n] (one rounding).
 * acc [planes][m][n]; xexp NULL means exponent 0 for every row. */
void orc_q8_combine(const int32_t *acc, int planes, const int32_t *xexp, int m, const float *scale,
                    int n, float *y);

/* Quantize + accumulate + combine: the build's dense int8 product. */
void orc_q8_matmul_planes(const float *x, int m, int k, int planes, const int8_t *q,
                          const float *scale, int n, float *y, int threads);

/* ---------------------------------------------------------------- LIF scan */

/* gpu/lif_gen.rs:151-214 (step + cpu_fwd). cur [B][T][D]; ps = [beta | theta | rho | gain] (each [D]);
 * v, s, a [B][D]: the carried state on entry, the final state on exit. levels 1 or 2; is_signed 0
 * for binary spikes; alif 0/1. spikes [B][T][D] as int8. Each operation rounded on its own. */
void orc_lif_scan(const float *cur, int B, int T, int D, const float *ps, float *v, float *s,
                  float *a, int levels, int is_signed, int alif, int8_t *spikes);

/* ---------------------------------------------------------------- kWTA */

/* gpu/model/fstep.rs:295-299 (kth_largest) and gpu/model/fstep/arch.rs:976-989: per row of u [n][h],
 * kth = the k-th largest (duplicates counted), keep u_i when u_i - kth >= 0 (ties kept), a = relu,
 * squared when relu2. k >= h keeps every unit. kth_out [n] (NaN-free inputs). */
void orc_kwta(const float *u, int n, int h, int k, int relu2, float *a, float *kth_out);

/* ---------------------------------------------------------------- fast-weight memory */

/* gpu/mem_gen.rs:220-273 (cpu_step_h, MemGen::cpu_fwd) = gpu/arch.rs:1091-1136 (delta_rec):
 * per head row-block bh, F [hs][hs] (row i = key channel, column j = value channel):
 *   r_j = sum_i e_i F_ij;  u_ij = b_i k_i v_j - a_i b_i e_i r_j;  S <- M S + u (M != 0);
 *   F_ij <- clamp(a_i F_ij + S_ij (or + u_ij), -cap, cap);  y_j = sum_i q_i F_ij (after the write).
 * q, k, e, v [BH][T][hs]; la (log alpha) and b [BH][T][g], g = 1 (per head) or hs (per channel).
 * F, S [BH][hs][hs] carried in and out (S unused when m == 0). y [BH][T][hs]. */
void orc_mem_rec(const float *q, const float *k, const float *e, const float *v, const float *la,
                 const float *b, int BH, int T, int hs, int g, float m, float cap, float *F,
                 float *S, float *y);

/* The same recurrence in float64 (the brute-force check of orc_mem_rec and of the GPU's chunked form). */
void orc_mem_rec_f64(const float *q, const float *k, const float *e, const float *v,
                     const float *la, const float *b, int BH, int T, int hs, int g, double m,
                     double *F, double *S, double *y);

/* gpu/arch.rs:1151-1164, 1243-1327 (delta_chunk / chunk_core): the same rule in chunks of
 * chunk_len(T, g) tokens (arch.rs:1166-1173), without the bound (the reference's default CPU prefill,
 * state.rs:954). Arguments as orc_mem_rec. */
void orc_mem_chunk(const float *q, const float *k, const float *e, const float *v, const float *la,
                   const float *b, int BH, int T, int hs, int g, float m, float *F, float *S, float *y);

/* The stack memory's form for T > 1: 0 (default) the bounded token loop orc_mem_rec (the reference's
 * GPU kernels; its CPU path under AVA_DELTA_REC=1, arch.rs:1329-1333), 1 orc_mem_chunk (the reference's
 * default CPU prefill, state.rs:954 -> arch.rs:1994, which has no bound). */
void orc_set_mem_chunked(int on);

/* The bounded rule entirely in float64 (inputs, alpha itself rather than its log, state and read-outs):
 * the memory of the float64 reference forward (forward64.py). S NULL without momentum. */
void orc_mem_rec_f64d(const double *q, const double *k, const double *e, const double *v, const double *al,
                      const double *b, int BH, int T, int hs, double m, double cap, double *F, double *S,
                      double *y);

/* ---------------------------------------------------------------- model */

typedef struct {
    const int8_t *q;     /* [din][dout] */
    const float *scale;  /* [dout] */
    int din, dout;
} orc_qw;

typedef struct {
    const float *lif_norm;                 /* [d] */
    orc_qw win;                            /* [d, d] */
    const float *beta_p;                   /* [d] leak logits (beta = sigmoid) */
    const float *theta;                    /* [d] */
    const float *arho;                     /* [d] ALIF decay logits (rho = sigmoid) */
    const float *again;                    /* [d] ALIF gain */
    orc_qw wout;                           /* [d, d] */
    const float *mem_norm;                 /* [d] */
    orc_qw wq, wk, wv, we, wg, wo;         /* [d, d] */
    const float *wa, *ba, *wb, *bb;        /* [d, nh], [nh] */
    const float *off;                      /* [d] */
    const float *wa1, *wa2, *wb1, *wb2;    /* [d, r], [r, d] */
    const float *vres;                     /* [2] */
    const float *eng_norm;                 /* [d] (engram block only) */
    orc_qw ewq, ewk, ewv, ewo;             /* [d, de] x3, [de, d] */
    const float *mlp_norm;                 /* [d] */
    orc_qw w1, w2;                         /* [d, H], [H, d] */
    const float *dense;                    /* [i + 2] */
} orc_block;

typedef struct {
    int vocab, d, layers, hidden, kwta_k, heads, head_size, gate_rank;
    int eng_block;   /* -1: no engram read */
    int eng_dim;
    int levels;      /* spike levels each side (2 = int2) */
    int alif, lif_scale, value_residual, dense, relu2;
    float momentum, cap;
    int eng_half;    /* the engram store keeps keys and values at fp16 precision (config[4]'s KV cache) */
    int eng_heads;   /* 0 or 1: one head of eng_dim; else heads of eng_dim / eng_heads side by side */
} orc_cfg;

typedef struct {
    const float *tok_emb;   /* [V, d] */
    orc_qw head;            /* E^T [d, V] */
    const float *final_norm;
    const orc_block *blocks;
} orc_model;

typedef struct {
    float *lif_v, *lif_s, *lif_a;   /* [layers][B][d] */
    float *mem_f, *mem_s;           /* [layers][B][nh][hs][hs] */
    float *eng_k, *eng_v;           /* [B][eng_cap][de] */
    int eng_cap, eng_len;           /* entries held per stream */
    /* The least-read rule's counts (gpu/memory.rs:592-594, 700-738; NULL: not kept): per stream and
     * slot, the attention mass the slot received from later queries (the mean over heads, the query's
     * own key left out) and how many later queries could see it. [B][eng_cap] each. */
    float *eng_reads, *eng_age;
} orc_state;

/* Optional copies of what each block computed (NULL fields are skipped). Layer-major. */
typedef struct {
    int8_t *spikes;   /* [layers][B*T][d] */
    float *cur;       /* [layers][B*T][d] LIF input currents */
    float *u;         /* [layers][B*T][H] W1 outputs */
    float *kth;       /* [layers][B*T] */
    float *memy;      /* [layers][B*T][d] memory read-outs before the head norm */
    float *x;         /* [layers][B*T][d] stream after each block (after the dense mix) */
    float *hf;        /* [B*T][d] final normed state */
    /* Forced decisions (inputs; NULL: the oracle's own). With force_spikes the spikes that update the
     * LIF state and feed Wout are these ([layers][B*T][d]); `spikes` above still receives the oracle's
     * own decisions. With force_keep the kWTA keeps unit i of a row where force_keep is non-zero
     * ([layers][B*T][H]); `u` and `kth` still receive the oracle's own values. A test feeds the
     * decisions of another implementation here so both follow one trajectory, and checks that every
     * decision where the two differ is a near-tie of the oracle's own values. */
    const int8_t *force_spikes;
    const uint8_t *force_keep;
    float *vm;        /* [layers][B*T][d] the membrane each spike decision compared */
    float *tht;       /* [layers][B*T][d] the threshold it compared with (theta + gain a_t) */
} orc_trace;

/* gpu/arch.rs:1407-1867 (forward_arch / block_arch / mem_arch) with carried state as in
 * gpu/state.rs:684-1071, one op order as gpu/model/fstep/arch.rs:525-1073. ids [B][T].
 * gemm_planes: 0 = the reference's W8A32 products; P >= 1 = the build's split-plane products.
 * logits [B*T][V] (may be NULL). Returns 0 on success. */
int orc_model_forward(const orc_cfg *cfg, const orc_model *mdl, const int32_t *ids, int B, int T,
                      orc_state *st, float *logits, int gemm_planes, int threads, orc_trace *tr);

/* ---------------------------------------------------------------- cerebellum head (CB, CB2) */

/* gpu/v51b.rs:242-265: the fixed granule wiring (idx [g][fan_in] in [0, inputs), sgn +-1/sqrt(fan_in)). */
void orc_cb_wiring(int inputs, int g, int fan_in, uint64_t seed, uint32_t *idx, float *sgn);
/* gpu/model/fstep/arch_f3.rs:225-262: the granule code c [g] of xf [d] and the token's embedding row. */
void orc_cb_code(const float *xf, const float *emb_row, int d, const uint32_t *idx, const float *sgn, int g,
                 int fan_in, int k, float *c);
/* gpu/model/fstep/arch_f3.rs:262-299, gpu/v51b.rs:373-389: out = xf + c.W (+ the online table's share). */
void orc_cb_apply(const float *xf, const float *c, int g, int d, const float *w, const float *tab, double scale,
                  float *out);
/* gpu/fast4/cb.rs:25-84: one online learning step of a stream's table; returns the token's nats. */
double orc_cb_learn(const float *logits, int V, int next, const float *E, int d, const float *c, int g, float lr,
                    double half, double *scale, float *tab);

/* The thread count of the parallel loops (same bits at any count). */
void orc_set_threads(int n);

/* ---------------------------------------------------------------- backward (training) */

/* The LIF scan's backward (lif_ref's surrogate gradient, gpu/arch.rs:964-1071; lifg_bwd, gpu/lif.cu:3228-3290). */
void orc_lif_bwd(const float *cur, int B, int T, int D, const float *ps, const float *v0, const float *s0,
                 const float *a0, int levels, int is_signed, int alif, float slope, int reset_grad, const float *g_spk,
                 const float *g_vT, const float *g_aT, float *dI, float *dv0, float *da0, float *dbeta, float *drho,
                 float *dgain);
/* The fast-weight recurrence's backward (delta_rec's autograd, gpu/arch.rs:1091-1136), float64 inside. */
void orc_mem_rec_bwd(const float *q, const float *k, const float *e, const float *v, const float *la, const float *b,
                     int BH, int T, int hs, int g, float m, float cap, const float *F0, const float *S0, const float *dy,
                     const float *dF_T, const float *dS_T, float *dq, float *dk, float *de, float *dv, float *dla,
                     float *db, float *dF0, float *dS0);

/* The same building blocks exposed for tests. orc_round_half: IEEE binary16 round-to-nearest-even. */
float orc_round_half(float x);
void orc_rmsnorm(const float *x, int n, int d, const float *gain, float *out);
float orc_sigmoid(float x);
float orc_log_sigmoid(float x);

#ifdef __cplusplus
}
#endif
#endif
