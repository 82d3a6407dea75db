/*
 * ava_oracle.c — CPU restatement of the reference's int8 block forward (TEST INFRASTRUCTURE ONLY).
 *
 * Checker for the HIP kernels of ava_amd; never part of the product path. Built with
 * -ffp-contract=off so every float operation is rounded on its own unless written as fmaf(),
 * which is used exactly where the reference uses f32::mul_add (its gemm / int8 orders).
 * Citations are relative to the reference's design-tests/nn/ (gpu/ = design-tests/nn/gpu/src).
 *
 * Parity of each function is pinned in tests/test_oracle.py against the reference's own known
 * answers and against independent brute force; see the header for the list.
 */
#include "ava_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NORM_EPS 1e-5f /* gpu/model.rs:36 */

/* The thread count of the oracle's parallel loops (OpenMP's default: OMP_NUM_THREADS, else every
 * CPU). Every parallel loop splits independent units (rows, channels, heads), so any count gives the
 * same bits. */
void orc_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n < 1 ? 1 : n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------ scalar helpers */

/* candle's sigmoid as gpu/model.rs:465-467 builds it: (exp(-x)·1 + 1)^-1 (gpu/model/fstep.rs:260-262). */
/* IEEE binary16 round-to-nearest-even of x, returned as the float it stands for: the subnormal range
 * (below 2^-14) in steps of 2^-24, normals to 10 fraction bits, from 65520 on infinity; NaN stays NaN. */
float orc_round_half(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint32_t sign = u & 0x80000000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return x;
    if (a < 0x38800000u) {
        const float y = rintf(fabsf(x) * 16777216.0f) / 16777216.0f; /* exact: |x| 2^24 < 2^10 */
        return sign ? -y : y;
    }
    a += 0xfffu + ((a >> 13) & 1u);
    a &= ~0x1fffu;
    if (a >= 0x47800000u) a = 0x7f800000u;
    a |= sign;
    float r;
    memcpy(&r, &a, 4);
    return r;
}

float orc_sigmoid(float x) { return 1.0f / (expf(-x) * 1.0f + 1.0f); }

/* gpu/model.rs:618-622 / gpu/model/fstep.rs:265-268: -(relu(-x) + ln(exp(-|x|)·1 + 1)). */
float orc_log_sigmoid(float x) {
    float soft = logf(expf(-fabsf(x)) * 1.0f + 1.0f);
    float r = -x > 0.0f ? -x : 0.0f;
    return -(r + soft);
}

/* (mean(x^2) + eps)^-1/2 as gpu/model/fstep.rs:213-221: sum from 0, the mean's affine, powf. */
static float inv_rms(const float *x, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += x[i] * x[i];
    float ms = s * (float)(1.0 / (double)n) + 0.0f;
    return powf(ms * 1.0f + NORM_EPS, -0.5f);
}

/* gpu/model.rs:458-462 / gpu/model/fstep.rs:207-211: x·inv·gain per row. */
void orc_rmsnorm(const float *x, int n, int d, const float *gain, float *out) {
    for (int r = 0; r < n; r++) {
        const float *xr = x + (size_t)r * d;
        float *o = out + (size_t)r * d;
        float inv = inv_rms(xr, d);
        for (int c = 0; c < d; c++) o[c] = (xr[c] * inv) * gain[c];
    }
}

/* gpu/model.rs:589-592 / gpu/model/fstep.rs:271-282: each head slice times (sum x^2 + 1e-6)^-1/2. */
static void l2_heads(float *x, int n, int hs) {
    for (int h = 0; h < n; h += hs) {
        float s = 0.0f;
        for (int i = 0; i < hs; i++) s += x[h + i] * x[h + i];
        float inv = powf(s * 1.0f + 1e-6f, -0.5f);
        for (int i = 0; i < hs; i++) x[h + i] = x[h + i] * inv;
    }
}

/* gpu/model.rs:583-587 / gpu/model/fstep.rs:285-292: rmsnorm without gain per head. */
static void head_norm(float *y, int n, int hs) {
    for (int h = 0; h < n; h += hs) {
        float inv = inv_rms(y + h, hs);
        for (int i = 0; i < hs; i++) y[h + i] = y[h + i] * inv;
    }
}

/* gpu/model/fstep.rs:223-257: one-row product out[c] = sum_j x[j] w[j][c] in gemm's order
 * (k >= 3: w[0][c]·x[0], then fma over j = 1, 2, ...). */
/* gemv over the first n columns of a matrix whose rows are ld floats apart */
static void gemv_ld(const float *x, int k, const float *w, int ld, int n, float *out) {
    if (k == 0) {
        for (int c = 0; c < n; c++) out[c] = 0.0f;
    } else if (k == 1) {
        for (int c = 0; c < n; c++) out[c] = w[c] * x[0];
    } else if (k == 2) {
        for (int c = 0; c < n; c++) out[c] = w[ld + c] * x[1] + w[c] * x[0];
    } else {
        for (int c = 0; c < n; c++) out[c] = w[c] * x[0];
        for (int j = 1; j < k; j++) {
            const float *wr = w + (size_t)j * ld;
            float xj = x[j];
            for (int c = 0; c < n; c++) out[c] = fmaf(wr[c], xj, out[c]);
        }
    }
}

static void gemv(const float *x, int k, const float *w, int n, float *out) { gemv_ld(x, k, w, n, n, out); }

/* ------------------------------------------------------------------ int8 weights */

void orc_quantize_int8(const float *w, int din, int dout, int8_t *q, float *scale) {
    for (int c = 0; c < dout; c++) scale[c] = 0.0f;
    for (int r = 0; r < din; r++)
        for (int c = 0; c < dout; c++) {
            float a = fabsf(w[(size_t)r * dout + c]);
            if (a > scale[c]) scale[c] = a;
        }
    for (int c = 0; c < dout; c++) scale[c] = scale[c] > 0.0f ? scale[c] / 127.0f : 1.0f;
    for (size_t i = 0; i < (size_t)din * dout; i++) {
        float t = roundf(w[i] / scale[i % dout]); /* round half away from zero, as f32::round */
        if (t > 127.0f) t = 127.0f;
        if (t < -127.0f) t = -127.0f;
        q[i] = (int8_t)t;
    }
}

#define TILE 64

/* One row against one 64-column tile of q [din][dout]: the fma chain of gpu/int8.rs:313-331. */
static void tile_row(const float *x, int din, const int8_t *q, int dout, int c0, int nc,
                     const float *scale, float *y) {
    float acc[TILE];
    for (int c = 0; c < TILE; c++) acc[c] = 0.0f;
    if (nc == TILE) {
        for (int j = 0; j < din; j++) {
            float xj = x[j];
            if (xj == 0.0f) continue; /* E2: fma(0, q, acc) == acc for every acc this chain holds */
            const int8_t *qr = q + (size_t)j * dout + c0;
            for (int c = 0; c < TILE; c++) acc[c] = fmaf(xj, (float)qr[c], acc[c]);
        }
    } else {
        for (int j = 0; j < din; j++) {
            float xj = x[j];
            if (xj == 0.0f) continue;
            const int8_t *qr = q + (size_t)j * dout + c0;
            for (int c = 0; c < nc; c++) acc[c] = fmaf(xj, (float)qr[c], acc[c]);
        }
    }
    for (int c = 0; c < nc; c++) y[c0 + c] = acc[c] * scale[c0 + c];
}

/* The per-row form (gpu/int8.rs:166-211): every row through tile_row, each (row, tile) a unit. */
void orc_q8_matmul_rows(const float *x, int m, int din, const int8_t *q, const float *scale, int dout, float *y,
                        int threads) {
    int tiles = (dout + TILE - 1) / TILE;
    long units = (long)m * tiles;
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (long u = 0; u < units; u++) {
        int t = (int)(u / m), r = (int)(u % m);
        int c0 = t * TILE, nc = dout - c0 < TILE ? dout - c0 : TILE;
        tile_row(x + (size_t)r * din, din, q, dout, c0, nc, scale, y + (size_t)r * dout);
    }
}

/* The row-blocked form of batched products (gpu/int8/block.rs:1-225): a unit is one 64-column tile
 * and up to BLK_CHUNK consecutive rows; the tile is widened to f32 once per unit as four 16-column
 * sub-tiles [4][din][16]; the unit's dense rows go 6 at a time through a 6 x 16 register block (12
 * AVX2 accumulators: two weight loads and six broadcasts per input j), the last 1..5 rows through the
 * same block with fewer rows; rows with at most a tenth of their inputs non-zero keep the per-row
 * event sum. The same bits as tile_row: each output starts at +0 and adds fma(x[j], w[j][c], acc) for
 * j = 0, 1, ...; a zero x[j] leaves acc as it was (acc is never -0: an exact cancellation rounds to
 * +0), so skipping it or not changes nothing; the scale multiplies at the end. */
#define BLK_ROWS 6
#define BLK_SUB 16
#define BLK_CHUNK 48
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
/* NR rows (a compile-time count, so the 2 NR accumulators stay in registers) */
#define BLOCK_ROWS_N(NR)                                                                                       \
    static void block_rows_##NR(const float *x, int din, const float *tf, float *acc) {                       \
        __m256 a[NR][2];                                                                                       \
        for (int r = 0; r < NR; r++) a[r][0] = a[r][1] = _mm256_setzero_ps();                                 \
        for (int j = 0; j < din; j++) {                                                                        \
            const __m256 w0 = _mm256_loadu_ps(tf + (size_t)j * BLK_SUB);                                       \
            const __m256 w1 = _mm256_loadu_ps(tf + (size_t)j * BLK_SUB + 8);                                   \
            for (int r = 0; r < NR; r++) {                                                                     \
                const __m256 xb = _mm256_broadcast_ss(x + (size_t)r * din + j);                                \
                a[r][0] = _mm256_fmadd_ps(xb, w0, a[r][0]);                                                    \
                a[r][1] = _mm256_fmadd_ps(xb, w1, a[r][1]);                                                    \
            }                                                                                                  \
        }                                                                                                      \
        for (int r = 0; r < NR; r++) {                                                                         \
            _mm256_storeu_ps(acc + r * BLK_SUB, a[r][0]);                                                      \
            _mm256_storeu_ps(acc + r * BLK_SUB + 8, a[r][1]);                                                  \
        }                                                                                                      \
    }
BLOCK_ROWS_N(1)
BLOCK_ROWS_N(2)
BLOCK_ROWS_N(3)
BLOCK_ROWS_N(4)
BLOCK_ROWS_N(5)
BLOCK_ROWS_N(6)
static void block_rows(const float *x, int din, const float *tf, int nr, float *acc /* [nr][16] */) {
    switch (nr) {
    case 6: block_rows_6(x, din, tf, acc); break;
    case 5: block_rows_5(x, din, tf, acc); break;
    case 4: block_rows_4(x, din, tf, acc); break;
    case 3: block_rows_3(x, din, tf, acc); break;
    case 2: block_rows_2(x, din, tf, acc); break;
    default: block_rows_1(x, din, tf, acc); break;
    }
}
#else
static void block_rows(const float *x, int din, const float *tf, int nr, float *acc) {
    for (int r = 0; r < nr; r++)
        for (int c = 0; c < BLK_SUB; c++) acc[r * BLK_SUB + c] = 0.0f;
    for (int j = 0; j < din; j++)
        for (int r = 0; r < nr; r++)
            for (int c = 0; c < BLK_SUB; c++)
                acc[r * BLK_SUB + c] = fmaf(x[(size_t)r * din + j], tf[(size_t)j * BLK_SUB + c], acc[r * BLK_SUB + c]);
}
#endif

static void blocked_unit(const float *x, int din, const int8_t *q, int dout, int c0, int nc, int r0, int nr,
                         const unsigned char *dense, const float *scale, float *y, float *tf, float *gath, int *have) {
    /* the tile's f32 copy: sub-tile s holds columns c0 + 16 s .. + 15 (zeros past dout); kept while the
     * thread's next unit reads the same tile */
    if (*have != c0)
        for (int s = 0; s < TILE / BLK_SUB; s++)
        for (int j = 0; j < din; j++)
            for (int c = 0; c < BLK_SUB; c++) {
                const int cc = BLK_SUB * s + c;
                tf[((size_t)s * din + j) * BLK_SUB + c] = cc < nc ? (float)q[(size_t)j * dout + c0 + cc] : 0.0f;
            }
    *have = c0;
    int rows[BLK_CHUNK], nd = 0;
    for (int r = r0; r < r0 + nr; r++) {
        if (dense[r]) rows[nd++] = r;
        else tile_row(x + (size_t)r * din, din, q, dout, c0, nc, scale, y + (size_t)r * dout);
    }
    for (int i = 0; i < nd; i += BLK_ROWS) {
        const int k = nd - i < BLK_ROWS ? nd - i : BLK_ROWS;
        /* consecutive dense rows read x in place; otherwise they are gathered */
        const float *xr = x + (size_t)rows[i] * din;
        int contiguous = rows[i + k - 1] - rows[i] == k - 1;
        if (!contiguous) {
            for (int z = 0; z < k; z++) memcpy(gath + (size_t)z * din, x + (size_t)rows[i + z] * din, sizeof(float) * din);
            xr = gath;
        }
        for (int s = 0; s < TILE / BLK_SUB; s++) {
            const int cs = BLK_SUB * s;
            if (cs >= nc) break;
            float acc[BLK_ROWS * BLK_SUB];
            block_rows(xr, din, tf + (size_t)s * din * BLK_SUB, k, acc);
            for (int z = 0; z < k; z++)
                for (int c = 0; c < BLK_SUB && cs + c < nc; c++)
                    y[(size_t)rows[i + z] * dout + c0 + cs + c] = acc[z * BLK_SUB + c] * scale[c0 + cs + c];
        }
    }
}

void orc_q8_matmul_blocked(const float *x, int m, int din, const int8_t *q, const float *scale, int dout, float *y,
                           int threads) {
    unsigned char *dense = (unsigned char *)malloc((size_t)m);
    for (int r = 0; r < m; r++) {
        int nnz = 0;
        for (int j = 0; j < din; j++) nnz += x[(size_t)r * din + j] != 0.0f;
        dense[r] = (double)nnz > 0.1 * din; /* gpu/int8/block.rs:35 (BLOCK_EVENT_MAX) */
    }
    const int tiles = (dout + TILE - 1) / TILE, nch = (m + BLK_CHUNK - 1) / BLK_CHUNK;
    const long units = (long)tiles * nch;
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        float *tf = (float *)malloc(sizeof(float) * (size_t)din * TILE);
        float *gath = (float *)malloc(sizeof(float) * (size_t)din * BLK_ROWS);
        int have = -1;
#pragma omp for schedule(static)
        for (long u = 0; u < units; u++) {
            const int t = (int)(u / nch), ch = (int)(u % nch);
            const int c0 = t * TILE, nc = dout - c0 < TILE ? dout - c0 : TILE;
            const int r0 = ch * BLK_CHUNK, nr = m - r0 < BLK_CHUNK ? m - r0 : BLK_CHUNK;
            blocked_unit(x, din, q, dout, c0, nc, r0, nr, dense, scale, y, tf, gath, &have);
        }
        free(tf);
        free(gath);
    }
    free(dense);
}

/* y = x W with the reference's CPU int8 product: the blocked form from 6 rows (BLOCK_MIN,
 * gpu/int8/block.rs:33), else the per-row form. Same bits either way. */
void orc_q8_matmul_ref(const float *x, int m, int din, const int8_t *q, const float *scale, int dout, float *y,
                       int threads) {
    if (m >= 6) orc_q8_matmul_blocked(x, m, din, q, scale, dout, y, threads);
    else orc_q8_matmul_rows(x, m, din, q, scale, dout, y, threads);
}

void orc_quant_planes(const float *x, int m, int k, int planes, int8_t *xq, int32_t *xexp) {
    for (int r = 0; r < m; r++) {
        const float *xr = x + (size_t)r * k;
        float amax = 0.0f;
        for (int j = 0; j < k; j++) amax = fmaxf(amax, fabsf(xr[j]));
        int e = 0;
        if (amax > 0.0f) {
            int ex;
            frexpf(amax, &ex);
            e = ex - 7;
            if (ldexpf(amax, -e) >= 127.5f) e += 1;
        }
        xexp[r] = e;
        for (int j = 0; j < k; j++) {
            float t = ldexpf(xr[j], -e);
            for (int p = 0; p < planes; p++) {
                float qv = rintf(t);
                xq[((size_t)p * m + r) * k + j] = (int8_t)qv;
                t = (t - qv) * 128.0f;
            }
        }
    }
}

void orc_q8_acc(const int8_t *a, int m, int k, const int8_t *q, int n, int32_t *acc, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int r = 0; r < m; r++) {
        int32_t *o = acc + (size_t)r * n;
        for (int c = 0; c < n; c++) o[c] = 0;
        const int8_t *ar = a + (size_t)r * k;
        for (int j = 0; j < k; j++) {
            int32_t av = ar[j];
            if (!av) continue;
            const int8_t *qr = q + (size_t)j * n;
            for (int c = 0; c < n; c++) o[c] += av * (int32_t)qr[c];
        }
    }
}

void orc_q8_combine(const int32_t *acc, int planes, const int32_t *xexp, int m, const float *scale,
                    int n, float *y) {
    int sh = 7 * (planes - 1);
    for (int r = 0; r < m; r++) {
        int e = xexp ? xexp[r] : 0;
        for (int c = 0; c < n; c++) {
            int64_t A = 0;
            for (int p = 0; p < planes; p++)
                A += (int64_t)acc[((size_t)p * m + r) * n + c] << (7 * (planes - 1 - p));
            float v = (float)(double)A;
            v = ldexpf(v, e - sh);
            y[(size_t)r * n + c] = v * scale[c];
        }
    }
}

void orc_q8_matmul_planes(const float *x, int m, int k, int planes, const int8_t *q,
                          const float *scale, int n, float *y, int threads) {
    int8_t *xq = (int8_t *)malloc((size_t)planes * m * k);
    int32_t *xe = (int32_t *)malloc(sizeof(int32_t) * (size_t)m);
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)planes * m * n);
    orc_quant_planes(x, m, k, planes, xq, xe);
    for (int p = 0; p < planes; p++)
        orc_q8_acc(xq + (size_t)p * m * k, m, k, q, n, acc + (size_t)p * m * n, threads);
    orc_q8_combine(acc, planes, xe, m, scale, n, y);
    free(xq);
    free(xe);
    free(acc);
}

/* ------------------------------------------------------------------ LIF */

/* gpu/lif_gen.rs:54-64 (Kind::spike). */
static float spike_of(float v, float th, int levels, int is_signed) {
    if (!is_signed) return v - th >= 0.0f ? 1.0f : 0.0f;
    float h = 0.0f;
    for (int k = 1; k <= levels; k++) {
        float kth = th * (float)k;
        h += (v - kth >= 0.0f ? 1.0f : 0.0f) - (-v - kth >= 0.0f ? 1.0f : 0.0f);
    }
    return h;
}

/* The scan with optional forced spikes: spikes[j] gets the scan's own decision; the state (the reset
 * and the ALIF trace) follows force[j] when force is given. vm/tho (nullable) get the membrane and the
 * threshold each decision compared. Each (b, c) is its own sequential scan, so the units run in
 * parallel with the same bits at any thread count. */
static void lif_scan_ex(const float *cur, int B, int T, int D, const float *ps, float *v, float *s, float *a,
                        int levels, int is_signed, int alif, int8_t *spikes, const int8_t *force, float *vm,
                        float *tho) {
#pragma omp parallel for schedule(static)
    for (long i_ = 0; i_ < (long)B * D; i_++) {
        {
            const int bi = (int)(i_ / D), c = (int)(i_ % D);
            int i = bi * D + c;
            float bt = ps[c], th0 = ps[D + c], rho = ps[2 * D + c], gain = ps[3 * D + c];
            float omr = 1.0f - rho;
            float vv = v[i], sp = s[i], aa = a[i];
            float thp = alif ? th0 + aa * gain : th0;
            for (int t = 0; t < T; t++) {
                size_t j = ((size_t)bi * T + t) * D + c;
                float tht = th0;
                if (alif) {
                    aa = aa * rho + fabsf(sp) * omr;
                    tht = th0 + aa * gain;
                }
                vv = (vv * bt + cur[j]) - sp * thp;
                sp = spike_of(vv, tht, levels, is_signed);
                spikes[j] = (int8_t)sp;
                if (vm) vm[j] = vv;
                if (tho) tho[j] = tht;
                if (force) sp = (float)force[j];
                thp = tht;
            }
            v[i] = vv;
            s[i] = sp;
            a[i] = aa;
        }
    }
}

void orc_lif_scan(const float *cur, int B, int T, int D, const float *ps, float *v, float *s,
                  float *a, int levels, int is_signed, int alif, int8_t *spikes) {
    lif_scan_ex(cur, B, T, D, ps, v, s, a, levels, is_signed, alif, spikes, NULL, NULL, NULL);
}

/* ------------------------------------------------------------------ kWTA */

static int cmp_desc(const void *pa, const void *pb) {
    float a = *(const float *)pa, b = *(const float *)pb;
    return (a < b) - (a > b);
}

void orc_kwta(const float *u, int n, int h, int k, int relu2, float *a, float *kth_out) {
#pragma omp parallel
    {
    float *buf = (float *)malloc(sizeof(float) * (size_t)h);
#pragma omp for schedule(static)
    for (int r = 0; r < n; r++) {
        const float *ur = u + (size_t)r * h;
        float *ar = a + (size_t)r * h;
        int keep_all = k >= h;
        float kth = 0.0f;
        if (!keep_all) {
            memcpy(buf, ur, sizeof(float) * (size_t)h);
            qsort(buf, (size_t)h, sizeof(float), cmp_desc);
            kth = buf[k - 1];
        }
        if (kth_out) kth_out[r] = keep_all ? -INFINITY : kth;
        for (int i = 0; i < h; i++) {
            float x = ur[i];
            float keep = keep_all ? 1.0f : (x - kth >= 0.0f ? 1.0f : 0.0f);
            float y = x * keep;
            y = y > 0.0f ? y : 0.0f;
            ar[i] = relu2 ? y * y : y;
        }
    }
    free(buf);
    }
}

/* ------------------------------------------------------------------ fast-weight memory */

void orc_mem_rec(const float *q, const float *k, const float *e, const float *v, const float *la,
                 const float *b, int BH, int T, int hs, int g, float m, float cap, float *F,
                 float *S, float *y) {
#pragma omp parallel
    {
    float *r = (float *)malloc(sizeof(float) * (size_t)hs);
    float *al = (float *)malloc(sizeof(float) * (size_t)hs);
    float *bb = (float *)malloc(sizeof(float) * (size_t)hs);
#pragma omp for schedule(dynamic)
    for (int bh = 0; bh < BH; bh++) {
        float *f = F + (size_t)bh * hs * hs;
        float *sm = S ? S + (size_t)bh * hs * hs : NULL;
        for (int t = 0; t < T; t++) {
            size_t o = ((size_t)bh * T + t) * hs, og = ((size_t)bh * T + t) * g;
            const float *qt = q + o, *kt = k + o, *et = e + o, *vt = v + o;
            for (int i = 0; i < hs; i++) {
                al[i] = expf(la[og + (g > 1 ? i : 0)]);
                bb[i] = b[og + (g > 1 ? i : 0)];
            }
            for (int j = 0; j < hs; j++) {
                float sacc = 0.0f;
                for (int i = 0; i < hs; i++) sacc += et[i] * f[i * hs + j];
                r[j] = sacc;
            }
            for (int i = 0; i < hs; i++)
                for (int j = 0; j < hs; j++) {
                    float u = ((bb[i] * kt[i]) * vt[j]) - (((al[i] * bb[i]) * et[i]) * r[j]);
                    int p = i * hs + j;
                    float fp;
                    if (m != 0.0f) {
                        sm[p] = m * sm[p] + u;
                        fp = al[i] * f[p] + sm[p];
                    } else {
                        fp = al[i] * f[p] + u;
                    }
                    f[p] = fp < -cap ? -cap : (fp > cap ? cap : fp);
                }
            float *yt = y + o;
            for (int j = 0; j < hs; j++) {
                float sacc = 0.0f;
                for (int i = 0; i < hs; i++) sacc += qt[i] * f[i * hs + j];
                yt[j] = sacc;
            }
        }
    }
    free(r);
    free(al);
    free(bb);
    }
}

void orc_mem_rec_f64(const float *q, const float *k, const float *e, const float *v,
                     const float *la, const float *b, int BH, int T, int hs, int g, double m,
                     double *F, double *S, double *y) {
#pragma omp parallel
    {
    double *r = (double *)malloc(sizeof(double) * (size_t)hs);
#pragma omp for schedule(dynamic)
    for (int bh = 0; bh < BH; bh++) {
        double *f = F + (size_t)bh * hs * hs;
        double *sm = S ? S + (size_t)bh * hs * hs : NULL;
        for (int t = 0; t < T; t++) {
            size_t o = ((size_t)bh * T + t) * hs, og = ((size_t)bh * T + t) * g;
            for (int j = 0; j < hs; j++) {
                double sacc = 0.0;
                for (int i = 0; i < hs; i++) sacc += (double)e[o + i] * f[i * hs + j];
                r[j] = sacc;
            }
            for (int i = 0; i < hs; i++) {
                double al = exp((double)la[og + (g > 1 ? i : 0)]), bi = b[og + (g > 1 ? i : 0)];
                for (int j = 0; j < hs; j++) {
                    double u = bi * k[o + i] * v[o + j] - al * bi * e[o + i] * r[j];
                    int p = i * hs + j;
                    if (m != 0.0) {
                        sm[p] = m * sm[p] + u;
                        f[p] = al * f[p] + sm[p];
                    } else {
                        f[p] = al * f[p] + u;
                    }
                }
            }
            for (int j = 0; j < hs; j++) {
                double sacc = 0.0;
                for (int i = 0; i < hs; i++) sacc += (double)q[o + i] * f[i * hs + j];
                y[o + j] = sacc;
            }
        }
    }
    free(r);
    }
}

/* The bounded rule (gpu/arch.rs:1091-1136 with the +-cap bound of mem_gen.rs:20-28) entirely in float64,
 * inputs included: q, k, e, v, al (alpha itself, not its log) and b [BH][T][hs], F, S [BH][hs][hs]
 * in/out (S NULL with m = 0), y [BH][T][hs]. The float64 reference forward's memory (forward64.py). */
void orc_mem_rec_f64d(const double *q, const double *k, const double *e, const double *v, const double *al,
                      const double *b, int BH, int T, int hs, double m, double cap, double *F, double *S,
                      double *y) {
#pragma omp parallel
    {
    double *r = (double *)malloc(sizeof(double) * (size_t)hs);
#pragma omp for schedule(dynamic)
    for (int bh = 0; bh < BH; bh++) {
        double *f = F + (size_t)bh * hs * hs;
        double *sm = S ? S + (size_t)bh * hs * hs : NULL;
        for (int t = 0; t < T; t++) {
            size_t o = ((size_t)bh * T + t) * hs;
            for (int j = 0; j < hs; j++) {
                double sacc = 0.0;
                for (int i = 0; i < hs; i++) sacc += e[o + i] * f[i * hs + j];
                r[j] = sacc;
            }
            for (int i = 0; i < hs; i++) {
                const double a = al[o + i], bk = b[o + i] * k[o + i], abe = a * b[o + i] * e[o + i];
                for (int j = 0; j < hs; j++) {
                    const double u = bk * v[o + j] - abe * r[j];
                    const int p = i * hs + j;
                    double fp;
                    if (sm) {
                        sm[p] = m * sm[p] + u;
                        fp = a * f[p] + sm[p];
                    } else {
                        fp = a * f[p] + u;
                    }
                    f[p] = fp < -cap ? -cap : (fp > cap ? cap : fp);
                }
            }
            for (int j = 0; j < hs; j++) {
                double sacc = 0.0;
                for (int i = 0; i < hs; i++) sacc += q[o + i] * f[i * hs + j];
                y[o + j] = sacc;
            }
        }
    }
    free(r);
    }
}

/* The form of the stack's memory for T > 1: 0 (default) = the token loop delta_rec with the bound at
 * every token (the reference's GPU kernels and its CPU path under AVA_DELTA_REC=1, arch.rs:1329-1333),
 * 1 = delta_chunk (the reference's default CPU prefill, no bound). The two agree to rounding until a
 * head's fast weights reach the bound. */
static int g_mem_chunked = 0;
void orc_set_mem_chunked(int on) { g_mem_chunked = on != 0; }

/* gpu/arch.rs:1166-1173 (chunk_len): 64 tokens for per-head gates, 16 per channel, halved until the
 * length divides T. */
static int chunk_len(int T, int g) {
    int c = g == 1 ? 64 : 16;
    while (c > 1 && T % c != 0) c /= 2;
    return c;
}

/* gpu/arch.rs:1151-1164 (delta_chunk) with 1243-1327 (chunk_core): the recurrence of orc_mem_rec in chunks
 * of c = chunk_len(T, g) tokens, without the bound (the chunked form has none). Inside a chunk, per key
 * channel: D_im = prod_{t=m+1..i} alpha_t (the decay ratio <= 1, formed pair by pair), Gamma_i = D_i0
 * alpha_0, K_ij = sum_{m=j..i} M^(m-j) D_im (as K_ij = D_ij + M K_i,j+1); with w = b k, ah = alpha b e:
 *   Qw_ij = sum_ch q_i K_ij w_j, Qa_ij = sum_ch q_i K_ij ah_j (j <= i); Ke, Ae the same with e_i and
 *   K_{i-1,j} (j < i);
 *   (I + Ae) R = (e Gamma_{i-1}) F0 + (e M K_{i-1,0}) S0 + Ke V   (forward substitution);
 *   Y = (q Gamma) F0 + (q M K_{i,0}) S0 + Qw V - Qa R;
 *   F' = Gamma_{c-1} F0 + M K_{c-1,0} S0 + sum_j K_{c-1,j} (w_j v_j^T - ah_j r_j^T);
 *   S' = M^c S0 + sum_j M^(c-1-j) (w_j v_j^T - ah_j r_j^T)   (M^p in double, rounded once).
 * Arguments as orc_mem_rec (no cap). */
void orc_mem_chunk(const float *q, const float *k, const float *e, const float *v, const float *la,
                   const float *b, int BH, int T, int hs, int g, float m, float *F, float *S, float *y) {
    const int c = chunk_len(T, g);
    const int mom = m != 0.0f;
#pragma omp parallel
    {
    const size_t cv = (size_t)c * hs, cc = (size_t)c * c;
    float *al = (float *)malloc(sizeof(float) * cv), *w = (float *)malloc(sizeof(float) * cv);
    float *ah = (float *)malloc(sizeof(float) * cv), *gm = (float *)malloc(sizeof(float) * cv);
    float *mk = (float *)malloc(sizeof(float) * cv), *kl = (float *)malloc(sizeof(float) * cv);
    float *R = (float *)malloc(sizeof(float) * cv);
    float *qw = (float *)calloc(cc, sizeof(float)), *qa = (float *)calloc(cc, sizeof(float));
    float *ke = (float *)calloc(cc, sizeof(float)), *ae = (float *)calloc(cc, sizeof(float));
    float *D = (float *)malloc(sizeof(float) * hs), *K = (float *)malloc(sizeof(float) * hs);
    float *F2 = (float *)malloc(sizeof(float) * hs * hs), *S2 = (float *)malloc(sizeof(float) * hs * hs);
    float *mu = (float *)malloc(sizeof(float) * c);
    double pw = 1.0;
    for (int p = 0; p < c; p++) pw *= (double)m;
    const float mc = (float)pw;
    for (int j = 0; j < c; j++) {
        double x = 1.0;
        for (int p = 0; p < c - 1 - j; p++) x *= (double)m;
        mu[j] = (float)x;
    }
#pragma omp for schedule(dynamic)
    for (int bh = 0; bh < BH; bh++) {
        float *f = F + (size_t)bh * hs * hs;
        float *sm = mom ? S + (size_t)bh * hs * hs : NULL;
        for (int t0 = 0; t0 < T; t0 += c) {
            const size_t o0 = ((size_t)bh * T + t0) * hs, og0 = ((size_t)bh * T + t0) * g;
            const float *qc = q + o0, *kc = k + o0, *ec = e + o0, *vc = v + o0;
            for (int p = 0; p < c; p++)
                for (int ch = 0; ch < hs; ch++) {
                    const size_t og = og0 + (size_t)p * g + (g > 1 ? ch : 0);
                    const float a = expf(la[og]), bw = b[og];
                    al[p * hs + ch] = a;
                    w[p * hs + ch] = bw * kc[p * hs + ch];
                    ah[p * hs + ch] = (a * bw) * ec[p * hs + ch];
                }
            memset(qw, 0, sizeof(float) * cc);
            memset(qa, 0, sizeof(float) * cc);
            memset(ke, 0, sizeof(float) * cc);
            memset(ae, 0, sizeof(float) * cc);
            for (int i = 0; i < c; i++) {
                for (int ch = 0; ch < hs; ch++) D[ch] = K[ch] = 0.0f;
                for (int j = i; j >= 0; j--) {
                    for (int ch = 0; ch < hs; ch++) {
                        D[ch] = j == i ? 1.0f : D[ch] * al[(j + 1) * hs + ch];
                        K[ch] = mom ? fmaf(m, K[ch], D[ch]) : D[ch];
                    }
                    float sw = 0.0f, sa = 0.0f, tw = 0.0f, ta = 0.0f;
                    for (int ch = 0; ch < hs; ch++) {
                        const float kw = K[ch] * w[j * hs + ch], ka = K[ch] * ah[j * hs + ch];
                        sw = fmaf(qc[i * hs + ch], kw, sw);
                        sa = fmaf(qc[i * hs + ch], ka, sa);
                        if (i + 1 < c) {
                            tw = fmaf(ec[(i + 1) * hs + ch], kw, tw);
                            ta = fmaf(ec[(i + 1) * hs + ch], ka, ta);
                        }
                    }
                    qw[i * c + j] = sw;
                    qa[i * c + j] = sa;
                    if (i + 1 < c) {
                        ke[(i + 1) * c + j] = tw;
                        ae[(i + 1) * c + j] = ta;
                    }
                    if (i == c - 1)
                        for (int ch = 0; ch < hs; ch++) kl[j * hs + ch] = K[ch];
                }
                for (int ch = 0; ch < hs; ch++) {
                    gm[i * hs + ch] = D[ch] * al[ch];
                    mk[i * hs + ch] = m * K[ch];
                }
            }
            /* recalls, then read-outs, column by column */
            for (int col = 0; col < hs; col++) {
                for (int i = 0; i < c; i++) {
                    float x = 0.0f;
                    for (int ch = 0; ch < hs; ch++) {
                        const float ea = i == 0 ? ec[ch] : ec[i * hs + ch] * gm[(i - 1) * hs + ch];
                        x = fmaf(ea, f[ch * hs + col], x);
                        if (mom && i > 0) x = fmaf(ec[i * hs + ch] * mk[(i - 1) * hs + ch], sm[ch * hs + col], x);
                    }
                    for (int j = 0; j < i; j++) x = fmaf(ke[i * c + j], vc[j * hs + col], x);
                    for (int j = 0; j < i; j++) x = fmaf(-ae[i * c + j], R[j * hs + col], x);
                    R[i * hs + col] = x;
                }
                for (int i = 0; i < c; i++) {
                    float x = 0.0f;
                    for (int ch = 0; ch < hs; ch++) {
                        x = fmaf(qc[i * hs + ch] * gm[i * hs + ch], f[ch * hs + col], x);
                        if (mom) x = fmaf(qc[i * hs + ch] * mk[i * hs + ch], sm[ch * hs + col], x);
                    }
                    for (int j = 0; j <= i; j++) {
                        x = fmaf(qw[i * c + j], vc[j * hs + col], x);
                        x = fmaf(-qa[i * c + j], R[j * hs + col], x);
                    }
                    y[o0 + (size_t)i * hs + col] = x;
                }
            }
            /* the state at the chunk's end */
            for (int row = 0; row < hs; row++)
                for (int col = 0; col < hs; col++) {
                    const int pq = row * hs + col;
                    float x = gm[(c - 1) * hs + row] * f[pq];
                    if (mom) x = fmaf(mk[(c - 1) * hs + row], sm[pq], x);
                    float z = mom ? mc * sm[pq] : 0.0f;
                    for (int j = 0; j < c; j++) {
                        const float wv = w[j * hs + row], av = ah[j * hs + row], kj = kl[j * hs + row];
                        x = fmaf(wv * kj, vc[j * hs + col], x);
                        x = fmaf(-(av * kj), R[j * hs + col], x);
                        if (mom) {
                            z = fmaf(wv * mu[j], vc[j * hs + col], z);
                            z = fmaf(-(av * mu[j]), R[j * hs + col], z);
                        }
                    }
                    F2[pq] = x;
                    S2[pq] = z;
                }
            memcpy(f, F2, sizeof(float) * hs * hs);
            if (mom) memcpy(sm, S2, sizeof(float) * hs * hs);
        }
    }
    free(al); free(w); free(ah); free(gm); free(mk); free(kl); free(R);
    free(qw); free(qa); free(ke); free(ae); free(D); free(K); free(F2); free(S2); free(mu);
    }
}

/* ------------------------------------------------------------------ model */

/* x [m, din] · W: the reference's W8A32 product (planes == 0) or the build's split planes. */
static void mm(const float *x, int m, const orc_qw *w, float *y, int planes, int threads) {
    if (planes <= 0)
        orc_q8_matmul_ref(x, m, w->din, w->q, w->scale, w->dout, y, threads);
    else
        orc_q8_matmul_planes(x, m, w->din, planes, w->q, w->scale, w->dout, y, threads);
}

/* Integer inputs (the spikes): both semantics agree exactly; the exact integer sum, times the scale. */
static void mm_int(const int8_t *s, int m, const orc_qw *w, float *y, int threads) {
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)m * w->dout);
    orc_q8_acc(s, m, w->din, w->q, w->dout, acc, threads);
    orc_q8_combine(acc, 1, NULL, m, w->scale, w->dout, y);
    free(acc);
}

/* One head's causal read (gpu/model/fstep.rs:303-329: scores in gemm's order, softmax, p·V). The
 * head's hs key and value dims sit in store rows ld floats apart (ld = hs for one head). */
static void attend(const float *q, const float *kc, const float *vc, int n, int hs, int ld, float scale,
                   float *sc, float *out) {
    for (int j = 0; j < n; j++) {
        const float *kr = kc + (size_t)j * ld;
        float s = kr[0] * q[0];
        for (int a = 1; a < hs; a++) s = fmaf(kr[a], q[a], s);
        sc[j] = s * scale + 0.0f;
    }
    float mx = sc[0];
    for (int j = 0; j < n; j++)
        if (mx < sc[j]) mx = sc[j];
    float den = 0.0f;
    for (int j = 0; j < n; j++) {
        sc[j] = expf(sc[j] - mx);
        den += sc[j];
    }
    for (int j = 0; j < n; j++) sc[j] = sc[j] / den;
    gemv_ld(sc, n, vc, ld, hs, out);
}

#define ALLOC(T_, n) ((T_ *)malloc(sizeof(T_) * (size_t)(n)))

int orc_model_forward(const orc_cfg *cfg, const orc_model *mdl, const int32_t *ids, int B, int T,
                      orc_state *st, float *logits, int planes, int threads, orc_trace *tr) {
    const int d = cfg->d, H = cfg->hidden, hs = cfg->head_size, nh = d / hs, rk = cfg->gate_rank;
    const int de = cfg->eng_dim, L = cfg->layers;
    const size_t N = (size_t)B * T;
    if (d % hs || B < 1 || T < 1) return 1;
    if (cfg->eng_block >= 0 && st->eng_len + T > st->eng_cap) return 2;

    float *x = ALLOC(float, N * d), *h = ALLOC(float, N * d), *y = ALLOC(float, N * d);
    float *cur = ALLOC(float, N * d);
    int8_t *spk = ALLOC(int8_t, N * d);
    float *q = ALLOC(float, N * d), *kr = ALLOC(float, N * d), *k = ALLOC(float, N * d);
    float *v = ALLOC(float, N * d), *weo = ALLOC(float, N * d), *gq = ALLOC(float, N * d);
    float *ek = ALLOC(float, N * d), *la = ALLOC(float, N * d), *bw = ALLOC(float, N * d);
    float *vfirst = ALLOC(float, N * d);
    float *u = ALLOC(float, N * H), *act = ALLOC(float, N * H);
    float *za = ALLOC(float, nh), *zb = ALLOC(float, nh), *z1 = ALLOC(float, rk);
    float *lra = ALLOC(float, d), *lrb = ALLOC(float, d);
    float *ps = ALLOC(float, 4 * d);
    /* head-major copies for the recurrence: [B][nh][T][hs] */
    float *hq = ALLOC(float, N * d), *hk = ALLOC(float, N * d), *he = ALLOC(float, N * d);
    float *hv = ALLOC(float, N * d), *hla = ALLOC(float, N * d), *hb = ALLOC(float, N * d);
    float *hy = ALLOC(float, N * d);
    float **streams = NULL;
    if (cfg->dense) {
        streams = ALLOC(float *, L + 1);
        for (int i = 0; i <= L; i++) streams[i] = ALLOC(float, N * d);
    }

    for (size_t n = 0; n < N; n++)
        memcpy(x + n * d, mdl->tok_emb + (size_t)ids[n] * d, sizeof(float) * d);
    if (cfg->dense) memcpy(streams[0], x, sizeof(float) * N * d);

    for (int i = 0; i < L; i++) {
        const orc_block *bk = &mdl->blocks[i];
        /* ---- the spiking layer (gpu/arch.rs:1632-1695; gpu/model/fstep/arch.rs:636-681) */
        orc_rmsnorm(x, (int)N, d, bk->lif_norm, h);
        mm(h, (int)N, &bk->win, cur, planes, threads);
        for (int c = 0; c < d; c++) {
            float beta = orc_sigmoid(bk->beta_p[c]);
            ps[c] = beta;
            ps[d + c] = bk->theta[c];
            ps[2 * d + c] = cfg->alif ? orc_sigmoid(bk->arho[c]) : 0.0f;
            ps[3 * d + c] = cfg->alif ? bk->again[c] : 0.0f;
        }
        if (cfg->lif_scale)
            for (size_t n = 0; n < N; n++)
                for (int c = 0; c < d; c++) cur[n * d + c] = cur[n * d + c] * (ps[c] * -1.0f + 1.0f);
        if (tr && tr->cur) memcpy(tr->cur + (size_t)i * N * d, cur, sizeof(float) * N * d);
        const int8_t *fsp = tr && tr->force_spikes ? tr->force_spikes + (size_t)i * N * d : NULL;
        lif_scan_ex(cur, B, T, d, ps, st->lif_v + (size_t)i * B * d, st->lif_s + (size_t)i * B * d,
                    st->lif_a + (size_t)i * B * d, cfg->levels, 1, cfg->alif, spk, fsp,
                    tr && tr->vm ? tr->vm + (size_t)i * N * d : NULL, tr && tr->tht ? tr->tht + (size_t)i * N * d : NULL);
        if (tr && tr->spikes) memcpy(tr->spikes + (size_t)i * N * d, spk, N * d);
        mm_int(fsp ? fsp : spk, (int)N, &bk->wout, y, threads);
        for (size_t j = 0; j < N * d; j++) x[j] = x[j] + y[j];

        /* ---- the fast-weight memory (gpu/arch.rs:1873-2020; gpu/model/fstep/arch.rs:683-896) */
        orc_rmsnorm(x, (int)N, d, bk->mem_norm, h);
        mm(h, (int)N, &bk->wq, q, planes, threads);
        mm(h, (int)N, &bk->wk, kr, planes, threads);
        mm(h, (int)N, &bk->wv, v, planes, threads);
        mm(h, (int)N, &bk->we, weo, planes, threads);
        mm(h, (int)N, &bk->wg, gq, planes, threads);
        memcpy(k, kr, sizeof(float) * N * d);
        l2_heads(q, (int)(N * d), hs);
        l2_heads(k, (int)(N * d), hs);
        if (cfg->value_residual) {
            if (i == 0) {
                memcpy(vfirst, v, sizeof(float) * N * d);
            } else {
                float p0 = bk->vres[0] * 1.0f + 1.0f, p1 = bk->vres[1];
                for (size_t j = 0; j < N * d; j++) v[j] = v[j] * p0 + vfirst[j] * p1;
            }
        }
        for (size_t n = 0; n < N; n++) {
            const float *hr = h + n * d;
            gemv(hr, d, bk->wa, nh, za);
            gemv(hr, d, bk->wb, nh, zb);
            for (int e = 0; e < nh; e++) {
                za[e] = za[e] + bk->ba[e];
                zb[e] = zb[e] + bk->bb[e];
            }
            gemv(hr, d, bk->wa1, rk, z1);
            gemv(z1, rk, bk->wa2, d, lra);
            gemv(hr, d, bk->wb1, rk, z1);
            gemv(z1, rk, bk->wb2, d, lrb);
            for (int c = 0; c < d; c++) {
                int e = c / hs;
                la[n * d + c] = orc_log_sigmoid((za[e] + bk->off[c]) + lra[c]);
                bw[n * d + c] = orc_sigmoid(zb[e] + lrb[c]) * 2.0f + 0.0f;
                ek[n * d + c] = kr[n * d + c] + weo[n * d + c];
            }
        }
        l2_heads(ek, (int)(N * d), hs);
        /* [B*T][nh][hs] -> [B][nh][T][hs] */
        for (int bi = 0; bi < B; bi++)
            for (int t = 0; t < T; t++)
                for (int e = 0; e < nh; e++) {
                    size_t src = ((size_t)bi * T + t) * d + (size_t)e * hs;
                    size_t dst = (((size_t)bi * nh + e) * T + t) * hs;
                    memcpy(hq + dst, q + src, sizeof(float) * hs);
                    memcpy(hk + dst, k + src, sizeof(float) * hs);
                    memcpy(he + dst, ek + src, sizeof(float) * hs);
                    memcpy(hv + dst, v + src, sizeof(float) * hs);
                    memcpy(hla + dst, la + src, sizeof(float) * hs);
                    memcpy(hb + dst, bw + src, sizeof(float) * hs);
                }
        /* the State path's memory (gpu/state.rs:954 -> arch.rs:1994): the bounded token loop, or with
         * orc_set_mem_chunked(1) delta_chunk over T > 1 tokens (one token is always the fused step's
         * bounded recurrence, gpu/model/fstep/arch.rs:256-337) */
        if (T > 1 && g_mem_chunked)
            orc_mem_chunk(hq, hk, he, hv, hla, hb, B * nh, T, hs, hs, cfg->momentum,
                          st->mem_f + (size_t)i * B * nh * hs * hs,
                          cfg->momentum != 0.0f ? st->mem_s + (size_t)i * B * nh * hs * hs : NULL, hy);
        else
            orc_mem_rec(hq, hk, he, hv, hla, hb, B * nh, T, hs, hs, cfg->momentum, cfg->cap,
                        st->mem_f + (size_t)i * B * nh * hs * hs,
                        cfg->momentum != 0.0f ? st->mem_s + (size_t)i * B * nh * hs * hs : NULL, hy);
        for (int bi = 0; bi < B; bi++)
            for (int t = 0; t < T; t++)
                for (int e = 0; e < nh; e++)
                    memcpy(y + ((size_t)bi * T + t) * d + (size_t)e * hs,
                           hy + (((size_t)bi * nh + e) * T + t) * hs, sizeof(float) * hs);
        if (tr && tr->memy) memcpy(tr->memy + (size_t)i * N * d, y, sizeof(float) * N * d);
        head_norm(y, (int)(N * d), hs);
        for (size_t j = 0; j < N * d; j++) {
            float g = gq[j];
            y[j] = y[j] * (g / (1.0f + expf(-g)));
        }
        mm(y, (int)N, &bk->wo, h, planes, threads);
        for (size_t j = 0; j < N * d; j++) x[j] = x[j] + h[j];

        /* ---- the engram read (gpu/arch.rs:1706-1738; gpu/model/fstep/arch.rs:898-974): one head of
         * eng_dim, or eng_heads heads side by side in each row (memory::read, gpu/memory.rs:610-700) */
        if (i == cfg->eng_block) {
            float *eq = ALLOC(float, N * de), *ekk = ALLOC(float, N * de), *evv = ALLOC(float, N * de);
            float *eo = ALLOC(float, N * de), *sc = ALLOC(float, st->eng_len + T);
            orc_rmsnorm(x, (int)N, d, bk->eng_norm, h);
            mm(h, (int)N, &bk->ewq, eq, planes, threads);
            mm(h, (int)N, &bk->ewk, ekk, planes, threads);
            mm(h, (int)N, &bk->ewv, evv, planes, threads);
            int n0 = st->eng_len;
            for (int bi = 0; bi < B; bi++)
                for (int t = 0; t < T; t++) {
                    size_t dst = ((size_t)bi * st->eng_cap + n0 + t) * de;
                    memcpy(st->eng_k + dst, ekk + ((size_t)bi * T + t) * de, sizeof(float) * de);
                    memcpy(st->eng_v + dst, evv + ((size_t)bi * T + t) * de, sizeof(float) * de);
                    if (cfg->eng_half)
                        for (int c = 0; c < de; c++) {
                            st->eng_k[dst + c] = orc_round_half(st->eng_k[dst + c]);
                            st->eng_v[dst + c] = orc_round_half(st->eng_v[dst + c]);
                        }
                }
            const int enh = cfg->eng_heads > 1 ? cfg->eng_heads : 1, hd = de / enh;
            float scale = (float)(1.0 / sqrt((double)hd));
            const int counts = st->eng_reads && st->eng_age;
            float *hsum = counts ? ALLOC(float, n0 + T) : NULL, *got = counts ? ALLOC(float, n0 + T) : NULL;
            for (int bi = 0; bi < B; bi++) {
                if (counts)
                    for (int j = 0; j < n0 + T; j++) got[j] = 0.0f;
                for (int t = 0; t < T; t++) {
                    if (counts)
                        for (int j = 0; j < n0 + t; j++) hsum[j] = 0.0f;
                    for (int hh = 0; hh < enh; hh++) {
                        size_t base = (size_t)bi * st->eng_cap * de + (size_t)hh * hd;
                        size_t row = ((size_t)bi * T + t) * de + (size_t)hh * hd;
                        attend(eq + row, st->eng_k + base, st->eng_v + base, n0 + t + 1, hd, de, scale, sc, eo + row);
                        if (counts)
                            for (int j = 0; j < n0 + t; j++) hsum[j] += sc[j];
                    }
                    /* gpu/memory.rs:709-714: the mean over heads of the mass each slot got from this
                     * query, for the slots it sees before its own (the old ones and the earlier new ones) */
                    if (counts)
                        for (int j = 0; j < n0 + t; j++) got[j] += hsum[j] * (1.0f / (float)enh);
                }
                if (counts) {
                    /* gpu/memory.rs:716-736: old slots add their mass and age by T; new slot j is seen
                     * by the T - 1 - j later queries of this call */
                    float *rd = st->eng_reads + (size_t)bi * st->eng_cap, *ag = st->eng_age + (size_t)bi * st->eng_cap;
                    for (int j = 0; j < n0; j++) {
                        rd[j] = rd[j] + got[j];
                        ag[j] = ag[j] + (float)T;
                    }
                    for (int j = n0; j < n0 + T; j++) {
                        rd[j] = 0.0f + got[j];
                        ag[j] = (float)(T - 1 - (j - n0));
                    }
                }
            }
            free(hsum);
            free(got);
            st->eng_len = n0 + T;
            mm(eo, (int)N, &bk->ewo, h, planes, threads);
            for (size_t j = 0; j < N * d; j++) x[j] = x[j] + h[j];
            free(eq);
            free(ekk);
            free(evv);
            free(eo);
            free(sc);
        }

        /* ---- the sparse MLP (gpu/arch.rs:1814-1855; gpu/model/fstep/arch.rs:976-996) */
        orc_rmsnorm(x, (int)N, d, bk->mlp_norm, h);
        mm(h, (int)N, &bk->w1, u, planes, threads);
        if (tr && tr->u) memcpy(tr->u + (size_t)i * N * H, u, sizeof(float) * N * H);
        orc_kwta(u, (int)N, H, cfg->kwta_k, cfg->relu2, act, tr && tr->kth ? tr->kth + (size_t)i * N : NULL);
        if (tr && tr->force_keep) {
            /* the forced index set in the same formula: relu(u mask), squared with relu2 */
            const uint8_t *fk = tr->force_keep + (size_t)i * N * H;
            for (size_t z = 0; z < N * (size_t)H; z++) {
                float yv = u[z] * (fk[z] ? 1.0f : 0.0f);
                yv = yv > 0.0f ? yv : 0.0f;
                act[z] = cfg->relu2 ? yv * yv : yv;
            }
        }
        mm(act, (int)N, &bk->w2, h, planes, threads);
        for (size_t j = 0; j < N * d; j++) x[j] = x[j] + h[j];

        /* ---- the dense residual (gpu/arch.rs:1492-1500; gpu/model/fstep/arch.rs:1010-1024) */
        if (cfg->dense) {
            memcpy(streams[i + 1], x, sizeof(float) * N * d);
            for (int j = 0; j <= i + 1; j++) {
                float w = bk->dense[j];
                const float *sj = streams[j];
                for (size_t z = 0; z < N * d; z++) x[z] = x[z] + sj[z] * w;
            }
        }
        if (tr && tr->x) memcpy(tr->x + (size_t)i * N * d, x, sizeof(float) * N * d);
    }

    orc_rmsnorm(x, (int)N, d, mdl->final_norm, h);
    if (tr && tr->hf) memcpy(tr->hf, h, sizeof(float) * N * d);
    if (logits) mm(h, (int)N, &mdl->head, logits, planes, threads);

    free(x); free(h); free(y); free(cur); free(spk); free(q); free(kr); free(k); free(v);
    free(weo); free(gq); free(ek); free(la); free(bw); free(vfirst); free(u); free(act);
    free(za); free(zb); free(z1); free(lra); free(lrb); free(ps);
    free(hq); free(hk); free(he); free(hv); free(hla); free(hb); free(hy);
    if (streams) {
        for (int i = 0; i <= L; i++) free(streams[i]);
        free(streams);
    }
    return 0;
}

/* ------------------------------------------------------------------ cerebellum head (CB) */

/* gpu/v51b.rs:242-265 (cb_wiring): xorshift64 from seed | 1; per unit, fan_in distinct inputs
 * next() % inputs, then one sign per input from next() & 1, amplitude 1/sqrt(fan_in). */
void orc_cb_wiring(int inputs, int g, int fan_in, uint64_t seed, uint32_t *idx, float *sgn) {
    uint64_t s = seed | 1u;
    const float amp = 1.0f / sqrtf((float)fan_in);
    const int want = fan_in < inputs ? fan_in : inputs;
    for (int j = 0; j < g; j++) {
        uint32_t picked[64];
        int np = 0;
        while (np < want) {
            s ^= s << 13;
            s ^= s >> 7;
            s ^= s << 17;
            uint32_t r = (uint32_t)(s % (uint64_t)inputs);
            int seen = 0;
            for (int a = 0; a < np; a++) seen |= picked[a] == r;
            if (!seen) picked[np++] = r;
        }
        for (int a = 0; a < np; a++) {
            s ^= s << 13;
            s ^= s >> 7;
            s ^= s << 17;
            idx[(size_t)j * fan_in + a] = picked[a];
            sgn[(size_t)j * fan_in + a] = (s & 1u) == 0 ? amp : -amp;
        }
    }
}

/* gpu/model/fstep/arch_f3.rs:225-262 (cb_parts, the code) = gpu/v51b.rs:329-337 (cb_code):
 * u = [xf, rmsnorm(emb_row, 1)] (2d); h_j = sum over the unit's fan-in of u[idx] * sgn, from 0 in
 * order; the k-th largest of h kept (v - kth >= 0, ties kept), relu; c = a / (sqrt(sum a^2) + 1e-6),
 * the sum from 0 in unit order. c [g]. */
void orc_cb_code(const float *xf, const float *emb_row, int d, const uint32_t *idx, const float *sgn, int g,
                 int fan_in, int k, float *c) {
    float *u = (float *)malloc(sizeof(float) * 2 * (size_t)d);
    float *ones = (float *)malloc(sizeof(float) * (size_t)d);
    for (int i = 0; i < d; i++) ones[i] = 1.0f;
    memcpy(u, xf, sizeof(float) * (size_t)d);
    orc_rmsnorm(emb_row, 1, d, ones, u + d);
    float *h = (float *)malloc(sizeof(float) * (size_t)g);
    for (int j = 0; j < g; j++) {
        float acc = 0.0f;
        for (int a = 0; a < fan_in; a++) acc += u[idx[(size_t)j * fan_in + a]] * sgn[(size_t)j * fan_in + a];
        h[j] = acc;
    }
    orc_kwta(h, 1, g, k, 0, c, NULL);
    float s2 = 0.0f;
    for (int j = 0; j < g; j++) s2 += c[j] * c[j];
    const float len = sqrtf(s2) * 1.0f + (float)1e-6;
    for (int j = 0; j < g; j++) c[j] = c[j] / len;
    free(u);
    free(ones);
    free(h);
}

/* gpu/model/fstep/arch_f3.rs:262-299 (cb_parts, the read-out and the online table's share) with
 * gpu/v51b.rs:373-389 (CbOnline::add): corr = sum over the non-zero units j in order of W[j] * c_j
 * (W NULL: a zero read-out, corr = 0); out = xf + corr; with a table, out += sum over the same units
 * of x_j * tab[j] where x_j = c_j, or (float)((double)c_j * scale) when scale != 1. */
void orc_cb_apply(const float *xf, const float *c, int g, int d, const float *w, const float *tab, double scale,
                  float *out) {
    float *acc = (float *)calloc((size_t)d, sizeof(float));
    if (w)
        for (int j = 0; j < g; j++) {
            if (c[j] == 0.0f) continue;
            const float *wr = w + (size_t)j * d;
            for (int i = 0; i < d; i++) acc[i] += wr[i] * c[j];
        }
    for (int i = 0; i < d; i++) out[i] = xf[i] + acc[i];
    if (tab) {
        memset(acc, 0, sizeof(float) * (size_t)d);
        for (int j = 0; j < g; j++) {
            if (c[j] == 0.0f) continue;
            const float x = scale == 1.0 ? c[j] : (float)((double)c[j] * scale);
            const float *tr = tab + (size_t)j * d;
            for (int i = 0; i < d; i++) acc[i] += x * tr[i];
        }
        for (int i = 0; i < d; i++) out[i] = out[i] + acc[i];
    }
    free(acc);
}

/* gpu/fast4/cb.rs:25-84 (fast4_cb_learn_sized): p = softmax(logits) (max, exp(z - max), the sum
 * from 0 in order, p / sum); err = p - onehot(next); delta = err . E (E [V][d], each output summed
 * over v in order); the scale fades by 2^(-1/half) when half is finite (> 0 here) and the table
 * folds (tab * scale in double, scale back to 1) below 1e-18; then for each non-zero unit u of the
 * kept code c: s = lr * c_u, divided by the scale in double when it is not 1, tab[u] -= s * delta.
 * Returns -ln max(p_next, 1e-30); a next outside [0, V) (the reference's IGNORE) changes nothing
 * and returns NaN. */
double orc_cb_learn(const float *logits, int V, int next, const float *E, int d, const float *c, int g, float lr,
                    double half, double *scale, float *tab) {
    if (V <= 0 || next < 0 || next >= V) return NAN; /* IGNORE (u32::MAX): no step, fast4/cb.rs:45-47 */
    float *p = (float *)malloc(sizeof(float) * (size_t)V);
    float mx = logits[0];
    for (int j = 0; j < V; j++)
        if (mx < logits[j]) mx = logits[j];
    float den = 0.0f;
    for (int j = 0; j < V; j++) {
        p[j] = expf(logits[j] - mx);
        den += p[j];
    }
    for (int j = 0; j < V; j++) p[j] = p[j] / den;
    const double ce = -log((double)(p[next] > 1e-30f ? p[next] : 1e-30f));
    for (int j = 0; j < V; j++) p[j] = p[j] - (j == next ? 1.0f : 0.0f);
    float *delta = (float *)calloc((size_t)d, sizeof(float));
    for (int i = 0; i < d; i++) {
        float acc = 0.0f;
        for (int j = 0; j < V; j++) acc = fmaf(p[j], E[(size_t)j * d + i], acc);
        delta[i] = acc;
    }
    if (half > 0.0 && isfinite(half)) {
        *scale *= exp2(-1.0 / half);
        if (*scale < 1e-18) {
            for (size_t z = 0; z < (size_t)g * d; z++) tab[z] = (float)((double)tab[z] * *scale);
            *scale = 1.0;
        }
    }
    const double sc = *scale;
    for (int u = 0; u < g; u++) {
        if (c[u] == 0.0f) continue;
        float s = lr * c[u];
        if (sc != 1.0) s = (float)((double)s / sc);
        float *wr = tab + (size_t)u * d;
        for (int i = 0; i < d; i++) wr[i] -= s * delta[i];
    }
    free(p);
    free(delta);
    return ce;
}

/* ------------------------------------------------------------------ backward (training) */

/* The surrogate derivative of one spike edge, 1 / (1 + S |x|)^2 (the slope of the fast sigmoid
 * x / (1 + S |x|) that lif_ref's straight-through spikes carry, gpu/arch.rs:953-956). */
static float sur(float x, float slope) {
    const float a = 1.0f + slope * fabsf(x);
    return 1.0f / (a * a);
}

/* d s / d v and d s / d theta_t of a step's surrogate spike (the soft sum of gpu/arch.rs:1006-1034). */
static void dspike(float v, float th, int levels, int is_signed, float slope, float *dv, float *dth) {
    if (!is_signed) {
        const float g = sur(v - th, slope);
        *dv = g;
        *dth = -g;
        return;
    }
    float a = 0.0f, b = 0.0f;
    for (int k = 1; k <= levels; k++) {
        const float kth = th * (float)k;
        const float gu = sur(v - kth, slope), gd = sur(-v - kth, slope);
        a += gu + gd;
        b += (float)k * (gd - gu);
    }
    *dv = a;
    *dth = b;
}

/* The backward of the LIF scan (the gradient lif_ref's autograd gives, gpu/arch.rs:964-1071; the CUDA
 * form lifg_bwd, gpu/lif.cu:3228-3290). Per (b, c): the forward is replayed from (v0, s0, a0) keeping
 * v_t and a_t, then walked back: G_t = dL/dv_t = gs_t ds_t/dv_t + beta G_{t+1} (G_T's carry = g_vT);
 * dbeta += G_t v_{t-1}. With ALIF: dL/dth_t = gs_t ds_t/dth_t, da_t = dth_t gain + rho da_{t+1},
 * dgain += dth_t a_t, drho += da_t (a_{t-1} - |s_{t-1}|) (the trace's spikes detached). With reset_grad
 * the reset v_{t+1} -= s_t th_t also carries gradient: gs_t -= te_t G_{t+1} with te_t = th_t, or
 * 2 beta / (ds/dv) where th_t ds/dv > 2 beta; dL/dth_t -= s_t G_{t+1} (and the first step's reset with
 * th_{-1} = theta + a0 gain). Outputs: dI [B][T][D], dv0, da0 and this row's shares of dbeta, drho and
 * dgain ([B][D] each; the caller sums over b). g_aT nullable (0). */
void orc_lif_bwd(const float *cur, int B, int T, int D, const float *ps, const float *v0, const float *s0,
                 const float *a0, int levels, int is_signed, int alif, float slope, int reset_grad, const float *g_spk,
                 const float *g_vT, const float *g_aT, float *dI, float *dv0, float *da0, float *dbeta, float *drho,
                 float *dgain) {
#pragma omp parallel
    {
        float *vs = (float *)malloc(sizeof(float) * (size_t)T);
        float *as = (float *)malloc(sizeof(float) * (size_t)T);
        float *ss = (float *)malloc(sizeof(float) * (size_t)T);
#pragma omp for schedule(static)
        for (long i_ = 0; i_ < (long)B * D; i_++) {
            const int bi = (int)(i_ / D), c = (int)(i_ % D);
            const int i = bi * D + c;
            const float bt = ps[c], th0 = ps[D + c], rho = ps[2 * D + c], gain = ps[3 * D + c];
            const float omr = 1.0f - rho;
            float vv = v0[i], sp = s0[i], aa = a0[i];
            float thp = alif ? th0 + aa * gain : th0;
            for (int t = 0; t < T; t++) {
                float tht = th0;
                if (alif) {
                    aa = aa * rho + fabsf(sp) * omr;
                    tht = th0 + aa * gain;
                }
                vv = (vv * bt + cur[((size_t)bi * T + t) * D + c]) - sp * thp;
                sp = spike_of(vv, tht, levels, is_signed);
                thp = tht;
                vs[t] = vv;
                as[t] = aa;
                ss[t] = sp;
            }
            float cv = g_vT ? g_vT[i] : 0.0f, ca = (alif && g_aT) ? g_aT[i] : 0.0f;
            float gb = 0.0f, gr = 0.0f, gg = 0.0f, Gn = 0.0f; /* Gn = G_{t+1} */
            for (int t = T - 1; t >= 0; t--) {
                const float vt = vs[t], at = alif ? as[t] : 0.0f;
                const float tht = alif ? th0 + at * gain : th0;
                float dv, dth;
                dspike(vt, tht, levels, is_signed, slope, &dv, &dth);
                float gs = g_spk[((size_t)bi * T + t) * D + c];
                if (reset_grad) {
                    const float q = tht * dv, cap = 2.0f * bt;
                    gs -= (q > cap ? cap / dv : tht) * Gn;
                }
                const float G = gs * dv + cv;
                gb += G * (t > 0 ? vs[t - 1] : v0[i]);
                if (alif) {
                    float gth = gs * dth;
                    if (reset_grad) gth -= ss[t] * Gn;
                    const float ga = gth * gain + ca;
                    gg += gth * at;
                    const float ap = t > 0 ? as[t - 1] : a0[i];
                    const float sprev = t > 0 ? ss[t - 1] : s0[i];
                    gr += ga * (ap - fabsf(sprev));
                    ca = rho * ga;
                }
                dI[((size_t)bi * T + t) * D + c] = G;
                Gn = G;
                cv = bt * G;
            }
            if (alif && reset_grad) {
                const float g0 = -s0[i] * Gn; /* the first step's reset threshold theta + a0 gain */
                gg += g0 * a0[i];
                ca += g0 * gain;
            }
            dv0[i] = cv;
            da0[i] = ca;
            dbeta[i] = gb;
            drho[i] = alif ? gr : 0.0f;
            dgain[i] = alif ? gg : 0.0f;
        }
        free(vs);
        free(as);
        free(ss);
    }
}

/* The backward of the fast-weight recurrence (orc_mem_rec; gpu/arch.rs:1091-1136 delta_rec's autograd,
 * the CUDA forms memg_bwd / memg_bwd4, gpu/lif.cu:3413-3890), in float64 over float32 inputs. Per head,
 * the forward is replayed keeping F_{t-1} and S_{t-1}; then from t = T-1 down, with F' = clamp(P) and
 * P = alpha F + S' (or + u without momentum), S' = M S + u, u_ij = b_i k_i v_j - alpha_i b_i e_i r_j,
 * r = F^T e, y = F'^T q:
 *   dq_i = sum_j dy_j F'_ij;  dF' += q dy^T;  gP = dF' where |P| < cap (else 0);
 *   dalpha_i += sum_j gP_ij F_ij;  dF = alpha gP (+ e dr^T below);  du = gP + dS' (momentum) ;  dS = M du;
 *   db_i += sum_j du_ij (k_i v_j - alpha_i e_i r_j); dk_i += b_i sum_j du_ij v_j; dv_j += sum_i du_ij b_i k_i;
 *   dalpha_i -= b_i e_i sum_j du_ij r_j; de_i -= alpha_i b_i sum_j du_ij r_j; dr_j = -sum_i du_ij alpha_i b_i e_i;
 *   de_i += sum_j dr_j F_ij;  dF += e dr^T;  dla = dalpha alpha.
 * With g = 1 (one gate per head) dla and db are the sums over the head's rows. dF_T, dS_T: the carried
 * gradients at the end (nullable: 0); dF0, dS0 out (dS0 only with momentum; nullable). */
void orc_mem_rec_bwd(const float *q, const float *k, const float *e, const float *v, const float *la, const float *b,
                     int BH, int T, int hs, int g, float m, float cap, const float *F0, const float *S0, const float *dy,
                     const float *dF_T, const float *dS_T, float *dq, float *dk, float *de, float *dv, float *dla,
                     float *db, float *dF0, float *dS0) {
#pragma omp parallel
    {
        const size_t hh = (size_t)hs * hs;
        double *Fs = (double *)malloc(sizeof(double) * hh * (size_t)(T + 1));
        double *Ss = (double *)malloc(sizeof(double) * hh * (size_t)(T + 1));
        double *r = (double *)malloc(sizeof(double) * (size_t)hs);
        double *dF = (double *)malloc(sizeof(double) * hh), *dS = (double *)malloc(sizeof(double) * hh);
        double *du = (double *)malloc(sizeof(double) * hh), *dr = (double *)malloc(sizeof(double) * (size_t)hs);
        double *al = (double *)malloc(sizeof(double) * (size_t)hs), *bb = (double *)malloc(sizeof(double) * (size_t)hs);
        double *dal = (double *)malloc(sizeof(double) * (size_t)hs), *dbb = (double *)malloc(sizeof(double) * (size_t)hs);
#pragma omp for schedule(dynamic)
        for (int bh = 0; bh < BH; bh++) {
            for (size_t z = 0; z < hh; z++) {
                Fs[z] = F0 ? F0[(size_t)bh * hh + z] : 0.0;
                Ss[z] = (m != 0.0f && S0) ? S0[(size_t)bh * hh + z] : 0.0;
            }
            for (int t = 0; t < T; t++) { /* F_t, S_t into slot t + 1 */
                const size_t o = ((size_t)bh * T + t) * hs, og = ((size_t)bh * T + t) * g;
                const double *F = Fs + hh * t, *S = Ss + hh * t;
                double *Fn = Fs + hh * (t + 1), *Sn = Ss + hh * (t + 1);
                for (int j = 0; j < hs; j++) {
                    double a = 0.0;
                    for (int i = 0; i < hs; i++) a += (double)e[o + i] * F[i * hs + j];
                    r[j] = a;
                }
                for (int i = 0; i < hs; i++) {
                    const double a = exp((double)la[og + (g > 1 ? i : 0)]), bi = b[og + (g > 1 ? i : 0)];
                    for (int j = 0; j < hs; j++) {
                        const double u = bi * k[o + i] * v[o + j] - a * bi * e[o + i] * r[j];
                        const int p = i * hs + j;
                        double P;
                        if (m != 0.0f) {
                            Sn[p] = m * S[p] + u;
                            P = a * F[p] + Sn[p];
                        } else {
                            Sn[p] = 0.0;
                            P = a * F[p] + u;
                        }
                        Fn[p] = P < -cap ? -cap : (P > cap ? cap : P);
                    }
                }
            }
            for (size_t z = 0; z < hh; z++) {
                dF[z] = dF_T ? dF_T[(size_t)bh * hh + z] : 0.0;
                dS[z] = (m != 0.0f && dS_T) ? dS_T[(size_t)bh * hh + z] : 0.0;
            }
            for (int i = 0; i < hs; i++) {
                dal[i] = 0.0;
                dbb[i] = 0.0;
            }
            for (int t = T - 1; t >= 0; t--) {
                const size_t o = ((size_t)bh * T + t) * hs, og = ((size_t)bh * T + t) * g;
                const double *F = Fs + hh * t, *S = Ss + hh * t, *Fn = Fs + hh * (t + 1);
                for (int i = 0; i < hs; i++) {
                    al[i] = exp((double)la[og + (g > 1 ? i : 0)]);
                    bb[i] = b[og + (g > 1 ? i : 0)];
                }
                for (int j = 0; j < hs; j++) {
                    double a = 0.0;
                    for (int i = 0; i < hs; i++) a += (double)e[o + i] * F[i * hs + j];
                    r[j] = a;
                }
                for (int i = 0; i < hs; i++) {
                    double a = 0.0;
                    for (int j = 0; j < hs; j++) a += (double)dy[o + j] * Fn[i * hs + j];
                    dq[o + i] = (float)a;
                }
                /* gP, dalpha from alpha F, du, dS */
                for (int i = 0; i < hs; i++)
                    for (int j = 0; j < hs; j++) {
                        const int p = i * hs + j;
                        const double u = bb[i] * k[o + i] * v[o + j] - al[i] * bb[i] * e[o + i] * r[j];
                        const double P = al[i] * F[p] + (m != 0.0f ? m * S[p] + u : u);
                        const double gP = (dF[p] + (double)q[o + i] * dy[o + j]) * ((P > -cap && P < cap) ? 1.0 : 0.0);
                        dal[i] += gP * F[p];
                        du[p] = gP + (m != 0.0f ? dS[p] : 0.0);
                        dF[p] = al[i] * gP;
                        dS[p] = m * du[p];
                    }
                for (int j = 0; j < hs; j++) dr[j] = 0.0;
                for (int i = 0; i < hs; i++) {
                    double sdv = 0.0, sdr = 0.0, sdkv = 0.0;
                    for (int j = 0; j < hs; j++) {
                        const double d = du[i * hs + j];
                        sdv += d * v[o + j];
                        sdr += d * r[j];
                        dr[j] -= d * al[i] * bb[i] * e[o + i];
                    }
                    dbb[i] += k[o + i] * sdv - al[i] * e[o + i] * sdr;
                    sdkv = bb[i] * sdv;
                    dk[o + i] = (float)sdkv;
                    dal[i] -= bb[i] * e[o + i] * sdr;
                    de[o + i] = (float)(-al[i] * bb[i] * sdr);
                }
                for (int j = 0; j < hs; j++) {
                    double a = 0.0;
                    for (int i = 0; i < hs; i++) a += du[i * hs + j] * bb[i] * k[o + i];
                    dv[o + j] = (float)a;
                }
                for (int i = 0; i < hs; i++) {
                    double a = 0.0;
                    for (int j = 0; j < hs; j++) a += dr[j] * F[i * hs + j];
                    de[o + i] = (float)(de[o + i] + a);
                    for (int j = 0; j < hs; j++) dF[i * hs + j] += (double)e[o + i] * dr[j];
                }
                if (g > 1) {
                    for (int i = 0; i < hs; i++) {
                        dla[og + i] = (float)(dal[i] * al[i]);
                        db[og + i] = (float)dbb[i];
                        dal[i] = 0.0;
                        dbb[i] = 0.0;
                    }
                } else {
                    double sa = 0.0, sb = 0.0;
                    for (int i = 0; i < hs; i++) {
                        sa += dal[i] * al[i];
                        sb += dbb[i];
                        dal[i] = 0.0;
                        dbb[i] = 0.0;
                    }
                    dla[og] = (float)sa;
                    db[og] = (float)sb;
                }
            }
            if (dF0)
                for (size_t z = 0; z < hh; z++) dF0[(size_t)bh * hh + z] = (float)dF[z];
            if (dS0 && m != 0.0f)
                for (size_t z = 0; z < hh; z++) dS0[(size_t)bh * hh + z] = (float)dS[z];
        }
        free(Fs); free(Ss); free(r); free(dF); free(dS); free(du); free(dr); free(al); free(bb); free(dal); free(dbb);
    }
}
