// The training step's kernels (train.hip), used by its driver (train.cpp).
#pragma once

#include "common.h"

// The memory's input preparation: raw projections [N][d] row-major (N = B T, rows b-major), outputs
// head-major [B nh][T][64] for ava_mem_scan.
struct TrainPrep {
    const float *q, *k, *v, *we;  // h Wq, h Wk, h Wv, h We
    const float *zab;             // [N][2 nh]: h Wa | h Wb
    const float *lra, *lrb;       // [N][d]: (h Wa1) Wa2, (h Wb1) Wb2
    const float *ba, *bb, *off;   // [nh], [nh], [d]
    const float *vfirst;          // block 0's raw values [N][d] (NULL in block 0: no residual)
    const float *vres;            // [2]: p0, p1
    float *hq, *hk, *he, *hv, *hla, *hb;
    int B, T, nh;
};

struct TrainPrepGrad {
    const float *dq, *dk, *de, *dv, *dla, *db;  // head-major, from ava_mem_scan_bwd
    float *dq_raw, *dk_raw, *dv_raw, *dwe;      // [N][d]
    float *dza, *dzb;                           // [N][d]: per channel (the read-outs' gradients)
    float *dzab;                                // [N][2 nh]: per head
    float *dvfirst;                             // [N][d] += dv p1 (blocks > 0)
    float *vres_part;                           // [N nh][2] (blocks > 0)
};

// Causal self-attention over each stream's T rows (a fresh store): q, k, v, o, dout, dq, dk, dv [B T][de];
// nh heads of hd dims side by side; lse, dsum [B T][nh] scratch.
struct TrainAttn {
    const float *q, *k, *v, *o, *dout;
    float *dq, *dk, *dv, *lse, *dsum;
    int B, T, de, nh, hd;
    float scale;
};

namespace ava {
namespace train {

int rms_fwd(const float *x, int n, int d, const float *g, float *y, float *inv, hipStream_t st);
size_t rms_bwd_part_floats(int n, int d);
// dx += the norm's input gradient; dg = the gain's gradient
int rms_bwd(const float *x, const float *inv, const float *g, const float *dy, int n, int d, float *dx, float *dg,
            float *part, hipStream_t st);
size_t colsum_part_floats(int rows, int cols);
// out[c] (+)= sum_r x[r][c] (+ sign extra[c])
int colsum(const float *x, int rows, int cols, int ld, float *out, int accumulate, float *part, hipStream_t st,
           const float *extra = nullptr, float sign = 0.0f);
size_t dot_part_floats();
int dot(const float *a, const float *b, size_t n, float *out, int accumulate, float *part, hipStream_t st);
int lif_params(const float *beta_p, const float *theta, const float *arho, const float *again, int d, int alif,
               float *ps, float *omb, hipStream_t st);
int scale_cols(const float *x, const float *s, size_t rows, int d, float *y, hipStream_t st);
int i8_to_f32(const int8_t *s, size_t n, float *y, hipStream_t st);
int axpy(float *y, const float *x, float a, size_t n, hipStream_t st);
int sigmoid_chain(const float *p, const float *dq, int n, float *dp, hipStream_t st);
int embed(const int32_t *ids, const float *emb, int n, int d, int V, float *x, hipStream_t st);
int embed_bwd(const int32_t *ids, const float *dx, int n, int d, int V, float *dE, hipStream_t st);
int prep_fwd(const TrainPrep &p, hipStream_t st);
int prep_bwd(const TrainPrep &p, const TrainPrepGrad &g, hipStream_t st);
int readout_fwd(const float *y, const float *g, int B, int T, int nh, float *o, hipStream_t st);
int readout_bwd(const float *y, const float *g, const float *dout, int B, int T, int nh, float *dy, float *dg,
                hipStream_t st);
int attn_bwd(const TrainAttn &a, hipStream_t st);
// out = S_{ns-1} + sum_j w[j] S_j (w on the device), n floats
int mix(float *out, const float *const *streams, int ns, const float *w, size_t n, hipStream_t st);
int mul(const float *a, const float *b, size_t n, float *y, hipStream_t st);
// loss = mean over rows with a target in [0, V) of lse - logit[target]; the logits are overwritten
// with dL/dlogits
int cross_entropy(float *logits, const int32_t *tgt, int n, int V, float *lse, float *loss_row, float *valid,
                  float *loss, float *scal, hipStream_t st);

}  // namespace train
}  // namespace ava
