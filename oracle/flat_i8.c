/*
 * CPU restatement of the flat-HTRC INT8 attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker.  The product
 * path (htrc_amd/) never links or calls it.
 *
 * Every function restates one step of the reference operator
 *   h3/htrc_flat.py            (_tiles :142-156, K int8 pack :213-219, top-k :250-265)
 *   h3/htrc_flat_triton.py     (_stats_kernel :41-85, _tile_kernel :88-211,
 *                               _rowmax_kernel :214-254, _merge_kernel :257-273,
 *                               _split :297-299)
 * in plain IEEE fp32 (built with -ffp-contract=off, no fast-math).  Where the
 * reference leaves an order open (sums inside tl.dot / tl.sum / torch.mean), this
 * file fixes one and the HIP kernels follow the same order wherever a boundary is
 * required to be bit-exact (pack, select, top-k).
 *
 * Layouts (per head; the Python wrapper loops over heads):
 *   q      fp32 [n, d]                 k, v  bf16 bits [nk, d]
 *   mu     fp32 [ng, d]                q8/dq8 int8 [nt*tile, d], sq/sdq fp32 [nt*tile]
 *   k8     int8 [nk, d], ks fp32 [nk]
 *   g8     int8 [ng, nb, d], sg/lz fp32 [ng, nb], vb bf16 bits [ng, nb, d]
 *   sel    fp32 [ng, nb]; idx int32 [ng, kx] (ascending); excl int8 [ng, nb]
 *   pm/pl  fp32 [nt, ns, tile]; pacc fp32 [nt, ns, tile, d]
 *   out    fp32 [nt*tile, d]; logz fp32 [nt*tile]
 * ng = nt, or ceil(nt / G) when G consecutive tiles share one centre, one state and one near
 * set (kern["group"], h3/htrc_flat.py:223-231; the tile kernel's gt = t // GR).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* fp32(1/127) = 0x3C010204: the constant the reference multiplies by
 * (h3/htrc_flat.py:217, h3/htrc_flat_triton.py:76,112,115,231). */
static const float R127 = 1.0f / 127.0f;

int oracle_abi_version(void) { return 6; }

float oracle_r127(void) { return R127; }

static inline float bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fp32 -> bf16 round-to-nearest-even (torch .to(bfloat16), Triton .to(tl.bfloat16)). */
static inline uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

uint16_t oracle_f2bf(float f) { return f2bf(f); }

/* In-kernel int8 rounding of the reference: where(x >= 0, x + 0.5, x - 0.5).to(int8),
 * i.e. an fp32 add followed by truncation toward zero
 * (h3/htrc_flat_triton.py:78-79, 114, 117, 233). */
static inline int8_t round_away(float x) {
    float y = x >= 0.0f ? x + 0.5f : x - 0.5f;
    return (int8_t)(int)truncf(y);
}

/* K pack rounding: (k / ks).round_().clamp_(-127, 127) -- round half to even
 * (h3/htrc_flat.py:218). */
static inline int8_t round_even_clamp(float x) {
    float y = rintf(x);
    if (y > 127.0f) y = 127.0f;
    if (y < -127.0f) y = -127.0f;
    return (int8_t)(int)y;
}

/* Per-row symmetric scale max(amax * fp32(1/127), floor); NaN propagates like
 * torch.clamp_min / tl.maximum do not matter here (inputs are finite). */
static inline float row_scale(float amax, float floor_) {
    float s = amax * R127;
    return s < floor_ ? floor_ : s;
}

/* K int8 pack, h3/htrc_flat.py:216-218:
 *   ks = clamp_min(amax_i |k| * fp32(1/127), 1e-20); k8 = clamp(rne(k / ks), +-127). */
void oracle_pack_k(const uint16_t *k, int64_t nk, int d, int8_t *k8, float *ks) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < nk; ++j) {
        const uint16_t *row = k + j * d;
        float amax = 0.0f;
        for (int i = 0; i < d; ++i) {
            float a = fabsf(bf2f(row[i]));
            if (a > amax) amax = a;
        }
        float s = row_scale(amax, 1e-20f);
        ks[j] = s;
        for (int i = 0; i < d; ++i) k8[j * d + i] = round_even_clamp(bf2f(row[i]) / s);
    }
}

/* Tile centres, h3/htrc_flat.py:142-156: mu[t] = mean of the tile's real rows.
 * Order fixed here: sequential fp32 sum over rows r = 0..nr-1, then IEEE division
 * by nr (the HIP pack kernel sums in the same order). */
void oracle_tile_centres(const float *q, int64_t n, int d, int tile, float *mu) {
    int64_t nt = (n + tile - 1) / tile;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < nt; ++t) {
        int64_t r0 = t * tile;
        int nr = (int)((n - r0) < tile ? (n - r0) : tile);
        for (int i = 0; i < d; ++i) {
            float s = 0.0f;
            for (int r = 0; r < nr; ++r) s += q[(r0 + r) * d + i];
            mu[t * d + i] = s / (float)nr;
        }
    }
}

/* Shared centres of groups of G tiles, h3/htrc_flat.py:223-229: the tiles are padded to a
 * multiple of G with repeats of the last tile (itself padded with repeats of the last row),
 * and mu[g] is the mean of the G * tile rows of tiles gG .. gG + G - 1.
 * Order fixed here: sequential fp32 sum over the group's rows j = 0 .. G*tile - 1, then IEEE
 * division by G*tile (the HIP group_centres kernel sums in the same order). */
void oracle_group_centres(const float *q, int64_t n, int d, int tile, int group, float *mu) {
    int64_t nt = (n + tile - 1) / tile;
    int64_t ng = (nt + group - 1) / group;
    int rows = group * tile;
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < ng; ++g) {
        for (int i = 0; i < d; ++i) {
            float s = 0.0f;
            for (int j = 0; j < rows; ++j) {
                int64_t t = g * group + j / tile;
                if (t > nt - 1) t = nt - 1;
                int64_t p = t * tile + j % tile;
                if (p > n - 1) p = n - 1;
                s += q[p * d + i];
            }
            mu[g * d + i] = s / (float)rows;
        }
    }
}

/* Row quantisation of q and dq = q - mu, h3/htrc_flat_triton.py:104-117 (tile kernel)
 * and :225-233 (rowmax kernel).  Rows are the padded tile rows: row p of tile t reads
 * query min(p, n-1) (the reference pads by repeating the last row, h3/htrc_flat.py:150-151).
 * The centre of tile t is mu[t / group] (the tile kernel's gt = t // GR, :96). */
void oracle_pack_q(const float *q, int64_t n, int d, int tile, int group, const float *mu,
                   int8_t *q8, float *sq, int8_t *dq8, float *sdq) {
    int64_t nt = (n + tile - 1) / tile;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < nt * tile; ++p) {
        int64_t src = p < n ? p : n - 1;
        const float *row = q + src * d;
        const float *m = mu + (p / tile / group) * d;
        float aq = 0.0f, adq = 0.0f;
        for (int i = 0; i < d; ++i) {
            float a = fabsf(row[i]);
            float b = fabsf(row[i] - m[i]);
            if (a > aq) aq = a;
            if (b > adq) adq = b;
        }
        float s1 = row_scale(aq, 1e-20f), s2 = row_scale(adq, 1e-20f);
        sq[p] = s1;
        sdq[p] = s2;
        for (int i = 0; i < d; ++i) {
            q8[p * d + i] = round_away(row[i] / s1);
            dq8[p * d + i] = round_away((row[i] - m[i]) / s2);
        }
    }
}

/* Leaf statistics at the tile centres, h3/htrc_flat_triton.py:55-85 (I8 store):
 *   a_s = (mu_t . k_s) * scale; m = max a; w = exp(a - m); z = sum w; w = w / z
 *   g = (w . K_l) * scale; vb = w . V_l; lz = m + log z
 *   am = max(max|g|, 1e-30); sg = am * fp32(1/127); g8 = round_away(g * (127 / am))
 *   vb stored as bf16 (RNE).
 * Dots are sequential fp32 sums (dims for a, leaf tokens for g / vb). */
/* TF32 operand (h3/htrc_flat_triton.py's dots with input_precision="tf32"): 10 explicit mantissa
 * bits, to nearest with ties away from zero; infinities and NaN unchanged. */
static inline float tf32_rna(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) != 0x7f800000u) u = (u + 0x1000u) & 0xffffe000u;
    memcpy(&x, &u, 4);
    return x;
}

/* The fp32 leaf state of centre m_ and leaf rows K, V (bf16): g (scaled) in gs, vb in vs,
 * returning max a and z through mx, z.  a, kf are work arrays of leaf and leaf * d floats.
 * tf32: the dots take TF32 operands (PREC "tf32"): the centre and the normalised weights are
 * rounded first (k and v, bf16, are TF32 values already). */
static void leaf_state(const float *m_, const uint16_t *K, const uint16_t *V, int leaf, int d, float scale,
                       int tf32, float *a, float *kf, float *gs, float *vs, float *mx_out, float *z_out) {
    for (int s = 0; s < leaf * d; ++s) kf[s] = bf2f(K[s]);
    for (int s = 0; s < leaf; ++s) a[s] = 0.0f;
    for (int i = 0; i < d; ++i) {        /* a[s] summed over i in order, vectorised over s */
        const float mi = tf32 ? tf32_rna(m_[i]) : m_[i];
        for (int s = 0; s < leaf; ++s) a[s] += mi * kf[s * d + i];
    }
    float mx = -INFINITY;
    for (int s = 0; s < leaf; ++s) {
        a[s] = a[s] * scale;
        if (a[s] > mx) mx = a[s];
    }
    float z = 0.0f;
    for (int s = 0; s < leaf; ++s) {
        a[s] = expf(a[s] - mx);
        z += a[s];
    }
    for (int s = 0; s < leaf; ++s) a[s] = tf32 ? tf32_rna(a[s] / z) : a[s] / z;
    for (int i = 0; i < d; ++i) gs[i] = vs[i] = 0.0f;
    for (int s = 0; s < leaf; ++s)       /* summed over tokens in order, vectorised over dims */
        for (int i = 0; i < d; ++i) {
            gs[i] += a[s] * kf[s * d + i];
            vs[i] += a[s] * bf2f(V[s * d + i]);
        }
    for (int i = 0; i < d; ++i) gs[i] = gs[i] * scale;
    *mx_out = mx;
    *z_out = z;
}

void oracle_stats(const float *mu, int64_t nt, const uint16_t *k, const uint16_t *v,
                  int64_t nb, int leaf, int d, float scale, int tf32,
                  int8_t *g8, float *sg, uint16_t *vb, float *lz) {
#pragma omp parallel
    {
        float *a = (float *)malloc(sizeof(float) * (size_t)leaf);
        float *kf = (float *)malloc(sizeof(float) * (size_t)leaf * d);
        float *gs = (float *)malloc(sizeof(float) * (size_t)d);
        float *vs = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t tl_ = 0; tl_ < nt * nb; ++tl_) {
            int64_t t = tl_ / nb, l = tl_ % nb;
            float mx, z;
            leaf_state(mu + t * d, k + l * leaf * d, v + l * leaf * d, leaf, d, scale, tf32, a, kf, gs, vs, &mx, &z);
            float am = 0.0f;
            for (int i = 0; i < d; ++i) {
                float x = fabsf(gs[i]);
                if (x > am) am = x;
            }
            if (am < 1e-30f) am = 1e-30f;
            float c = 127.0f / am;
            int8_t *go = g8 + (t * nb + l) * d;
            uint16_t *vo = vb + (t * nb + l) * d;
            for (int i = 0; i < d; ++i) {
                go[i] = round_away(gs[i] * c);
                vo[i] = f2bf(vs[i]);
            }
            sg[t * nb + l] = am * R127;
            lz[t * nb + l] = mx + logf(z);
        }
        free(a);
        free(kf);
        free(gs);
        free(vs);
    }
}

/* e4m3fn (OCP fp8, bias 7, no infinities) code of x, round to nearest even; |x| above 448 (the
 * largest finite value) saturates to 448 (Triton's satfinite conversion; the state scales keep
 * |x| <= 448). */
uint8_t oracle_f32_to_e4m3(float x) {
    uint8_t sgn = (uint8_t)(signbit(x) ? 0x80 : 0);
    float a = fabsf(x);
    if (!(a <= 448.0f)) a = 448.0f;
    if (a < 0.015625f) return sgn | (uint8_t)nearbyintf(a * 512.0f);   /* subnormal grid m * 2^-9 */
    int e;
    float f = frexpf(a, &e);                    /* a = f * 2^e, f in [0.5, 1) */
    float m = nearbyintf(f * 16.0f);            /* 4 significant bits: 8 .. 16 */
    if (m == 16.0f) {
        m = 8.0f;
        e += 1;
    }
    int ex = e - 1 + 7;                         /* biased exponent of 1.mmm * 2^(e-1) */
    return sgn | (uint8_t)((ex << 3) | ((int)m - 8));
}

float oracle_e4m3_to_f32(uint8_t b) {
    int e = (b >> 3) & 15, m = b & 7;
    float v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
    if (e == 15 && m == 7) v = NAN;
    return (b & 0x80) ? -v : v;
}

/* Leaf statistics with the fp8 state store, h3/htrc_flat_triton.py:65-72:
 *   sg = max(max|g| * fp32(1/448), 1e-30), g code = e4m3(g / sg); sv, vb code likewise. */
void oracle_stats_fp8(const float *mu, int64_t nt, const uint16_t *k, const uint16_t *v,
                      int64_t nb, int leaf, int d, float scale, int tf32,
                      uint8_t *g8, float *sg, uint8_t *vb8, float *sv, float *lz) {
    const float r448 = 1.0f / 448.0f;
#pragma omp parallel
    {
        float *a = (float *)malloc(sizeof(float) * (size_t)leaf);
        float *kf = (float *)malloc(sizeof(float) * (size_t)leaf * d);
        float *gs = (float *)malloc(sizeof(float) * (size_t)d);
        float *vs = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t tl_ = 0; tl_ < nt * nb; ++tl_) {
            int64_t t = tl_ / nb, l = tl_ % nb;
            float mx, z;
            leaf_state(mu + t * d, k + l * leaf * d, v + l * leaf * d, leaf, d, scale, tf32, a, kf, gs, vs, &mx, &z);
            float ag = 0.0f, av = 0.0f;
            for (int i = 0; i < d; ++i) {
                if (fabsf(gs[i]) > ag) ag = fabsf(gs[i]);
                if (fabsf(vs[i]) > av) av = fabsf(vs[i]);
            }
            float sgv = ag * r448, svv = av * r448;
            if (sgv < 1e-30f) sgv = 1e-30f;
            if (svv < 1e-30f) svv = 1e-30f;
            for (int i = 0; i < d; ++i) {
                g8[(t * nb + l) * d + i] = oracle_f32_to_e4m3(gs[i] / sgv);
                vb8[(t * nb + l) * d + i] = oracle_f32_to_e4m3(vs[i] / svv);
            }
            sg[tl_] = sgv;
            sv[tl_] = svv;
            lz[tl_] = mx + logf(z);
        }
        free(a);
        free(kf);
        free(gs);
        free(vs);
    }
}

static inline int32_t dot_i8(const int8_t *x, const int8_t *y, int d) {
    int32_t s = 0;
    for (int i = 0; i < d; ++i) s += (int32_t)x[i] * (int32_t)y[i];
    return s;
}

/* Row-max routing score, h3/htrc_flat_triton.py:214-254 (I8), per group of G tiles over the
 * group's G * tile rows (h3/htrc_flat.py:244-252 passes them as one row block):
 *   SEL[g,l] = max_{r = 0, stride, ..} ( float(dq8_r . g8_gl) * (sdq_r * sg_gl) ) + lz_gl
 * Rows of padded tiles (past the nt real ones) are those of the last tile. */
void oracle_select(const int8_t *dq8, const float *sdq, int tile, int stride, int group, int64_t nt,
                   const int8_t *g8, const float *sg, const float *lz,
                   int64_t ng, int64_t nb, int d, float *sel) {
    int ts = group * tile / stride;
#pragma omp parallel for schedule(static)
    for (int64_t tl_ = 0; tl_ < ng * nb; ++tl_) {
        int64_t gi = tl_ / nb;
        const int8_t *g = g8 + tl_ * d;
        float best = -INFINITY;
        for (int rr = 0; rr < ts; ++rr) {
            int64_t j = (int64_t)rr * stride;
            int64_t t = gi * group + j / tile;
            if (t > nt - 1) t = nt - 1;
            int64_t p = t * tile + j % tile;
            float x = (float)dot_i8(dq8 + p * d, g, d) * (sdq[p] * sg[tl_]);
            if (x > best) best = x;
        }
        sel[tl_] = best + lz[tl_];
    }
}

typedef struct {
    float v;
    int32_t i;
} vi_t;

static int cmp_desc(const void *a, const void *b) {
    const vi_t *x = (const vi_t *)a, *y = (const vi_t *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->i > y->i) - (x->i < y->i);
}

static int cmp_i32(const void *a, const void *b) {
    int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return (x > y) - (x < y);
}

/* Near-leaf selection, h3/htrc_flat.py:262-265: sink leaves forced to +inf, then the
 * kx largest SEL per tile; excl[t, idx] = 1.  torch.topk(sorted=False) fixes neither the
 * order nor ties: here ties go to the lower leaf index and idx is written ascending. */
void oracle_topk(const float *sel, int64_t nt, int64_t nb, int kx, int sink,
                 int32_t *idx, int8_t *excl) {
#pragma omp parallel
    {
        vi_t *buf = (vi_t *)malloc(sizeof(vi_t) * (size_t)nb);
#pragma omp for schedule(static)
        for (int64_t t = 0; t < nt; ++t) {
            for (int64_t l = 0; l < nb; ++l) {
                buf[l].v = l < sink ? INFINITY : sel[t * nb + l];
                buf[l].i = (int32_t)l;
            }
            qsort(buf, (size_t)nb, sizeof(vi_t), cmp_desc);
            int32_t *o = idx + t * kx;
            for (int j = 0; j < kx; ++j) o[j] = buf[j].i;
            qsort(o, (size_t)kx, sizeof(int32_t), cmp_i32);
            memset(excl + t * nb, 0, (size_t)nb);
            for (int j = 0; j < kx; ++j) excl[t * nb + o[j]] = 1;
        }
        free(buf);
    }
}

/* _split, h3/htrc_flat_triton.py:297-299. */
int64_t oracle_split(int64_t n, int64_t ns, int64_t bn) {
    int64_t per = (n + ns - 1) / ns;
    int64_t r = (per + bn - 1) / bn * bn;
    return r > bn ? r : bn;
}

/* One online-softmax block update, h3/htrc_flat_triton.py:143-157 / :177-186:
 *   m_new = max(m, max sc); m_s = m_new == -inf ? 0 : m_new; p = exp(sc - m_s)
 *   alpha = exp(m - m_s); l = l * alpha + sum p; acc = acc * alpha + bf16(p) . V. */
static void block_update(const float *sc, const uint16_t *const *vals, int nc, int d,
                         float *m, float *l, float *acc, float *dacc) {
    float bm = -INFINITY;
    for (int c = 0; c < nc; ++c)
        if (sc[c] > bm) bm = sc[c];
    float m_new = *m > bm ? *m : bm;
    float m_s = (m_new == -INFINITY) ? 0.0f : m_new;
    float psum = 0.0f;
    for (int i = 0; i < d; ++i) dacc[i] = 0.0f;
    for (int c = 0; c < nc; ++c) {
        float p = expf(sc[c] - m_s);
        psum += p;
        if (vals[c] == NULL) continue;
        float pb = bf2f(f2bf(p));
        for (int i = 0; i < d; ++i) dacc[i] += pb * bf2f(vals[c][i]);
    }
    float alpha = expf(*m - m_s);
    *l = *l * alpha + psum;
    for (int i = 0; i < d; ++i) acc[i] = acc[i] * alpha + dacc[i];
    *m = m_new;
}

/* Split-K tile kernel, h3/htrc_flat_triton.py:95-211 (DOT=1, I8=1, GR=1, no tail):
 * program (t, sp) covers far leaves [sp*lps, +lps) not excluded and exact tokens
 * [sp*eps, +eps) of the tile's kx selected leaves (tok = idx[t, j / leaf] * leaf + j % leaf).
 *   far  score  float(dq8 . g8) * (sdq * sg) + lz,  value vb (bf16)
 *   near score  float(q8 . k8)  * ((sq * ks) * scale), value v (bf16)
 * Writes the partial (m, l, acc) of every (tile, split, row). */
void oracle_tile(int64_t nt, int tile, int d, int64_t nb, int leaf, int kx, int group,
                 const int32_t *idx, const int8_t *excl,
                 const int8_t *q8, const float *sq, const int8_t *dq8, const float *sdq,
                 const int8_t *g8, const float *sg, const float *lz, const uint16_t *vb,
                 const int8_t *k8, const float *ks, const uint16_t *v,
                 float scale, int ns, int bn, float *pm, float *pl, float *pacc) {
    int64_t lps = oracle_split(nb, ns, bn);
    int64_t eps = oracle_split((int64_t)kx * leaf, ns, bn);
#pragma omp parallel
    {
        float *sc = (float *)malloc(sizeof(float) * (size_t)bn);
        const uint16_t **vals = (const uint16_t **)malloc(sizeof(void *) * (size_t)bn);
        float *acc = (float *)malloc(sizeof(float) * (size_t)d);
        float *dacc = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t job = 0; job < nt * ns * tile; ++job) {
            int64_t t = job / ((int64_t)ns * tile);
            int sp = (int)((job / tile) % ns);
            int r = (int)(job % tile);
            int64_t p = t * tile + r;
            int64_t gs = t / group;          /* the group's state and near set (gt = t // GR) */
            float m = -INFINITY, l = 0.0f;
            for (int i = 0; i < d; ++i) acc[i] = 0.0f;
            int64_t lo = sp * lps, hi = lo + lps < nb ? lo + lps : nb;
            for (int64_t n0 = lo; n0 < hi; n0 += bn) {
                for (int c = 0; c < bn; ++c) {
                    int64_t cc = n0 + c;
                    if (cc < hi && excl[gs * nb + cc] == 0) {
                        int64_t s = gs * nb + cc;
                        sc[c] = (float)dot_i8(dq8 + p * d, g8 + s * d, d) * (sdq[p] * sg[s]) + lz[s];
                        vals[c] = vb + s * d;
                    } else {
                        sc[c] = -INFINITY;
                        vals[c] = NULL;
                    }
                }
                block_update(sc, vals, bn, d, &m, &l, acc, dacc);
            }
            int64_t e_n = (int64_t)kx * leaf;
            int64_t e_lo = sp * eps, e_hi = e_lo + eps < e_n ? e_lo + eps : e_n;
            for (int64_t e0 = e_lo; e0 < e_hi; e0 += bn) {
                for (int c = 0; c < bn; ++c) {
                    int64_t j = e0 + c;
                    if (j < e_hi) {
                        int64_t tok = (int64_t)idx[gs * kx + j / leaf] * leaf + j % leaf;
                        sc[c] = (float)dot_i8(q8 + p * d, k8 + tok * d, d) * ((sq[p] * ks[tok]) * scale);
                        vals[c] = v + tok * d;
                    } else {
                        sc[c] = -INFINITY;
                        vals[c] = NULL;
                    }
                }
                block_update(sc, vals, bn, d, &m, &l, acc, dacc);
            }
            int64_t base = (t * ns + sp) * tile + r;
            pm[base] = m;
            pl[base] = l;
            memcpy(pacc + base * d, acc, sizeof(float) * (size_t)d);
        }
        free(sc);
        free(vals);
        free(acc);
        free(dacc);
    }
}

/* fp16 <-> fp32 (IEEE binary16, round to nearest even). */
static float f16_to_f32(uint16_t h) {
    int e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + m), e - 25);
    return (h & 0x8000) ? -v : v;
}

uint16_t oracle_f32_to_f16(float x) {
    uint16_t sgn = (uint16_t)(signbit(x) ? 0x8000 : 0);
    float a = fabsf(x);
    if (isnan(a)) return sgn | 0x7e00;
    if (a >= 65520.0f) return sgn | 0x7c00;                     /* rounds to infinity */
    if (a < 6.103515625e-05f) return sgn | (uint16_t)nearbyintf(a * 16777216.0f);   /* subnormal: m * 2^-24 */
    int e;
    float f = frexpf(a, &e);
    float m = nearbyintf(f * 2048.0f);                          /* 11 significant bits */
    if (m == 2048.0f) {
        m = 1024.0f;
        e += 1;
    }
    return sgn | (uint16_t)(((e - 1 + 15) << 10) | ((int)m - 1024));
}

/* fp8 state store select, h3/htrc_flat_triton.py:214-254 with FP8 = 1:
 *   SEL[g,l] = max_r (sum_i dq_ri * g_li) * sg_gl + lz_gl, dq in fp16, g the e4m3 value
 *   (every product exact in fp32; summed over the dims in order). */
void oracle_select_fp8(const uint16_t *dq16, int tile, int stride, int group, int64_t nt,
                       const uint8_t *g8, const float *sg, const float *lz, int64_t ng, int64_t nb, int d,
                       float *sel) {
    int ts = group * tile / stride;
#pragma omp parallel for schedule(static)
    for (int64_t tl_ = 0; tl_ < ng * nb; ++tl_) {
        int64_t gi = tl_ / nb;
        const uint8_t *g = g8 + tl_ * d;
        float best = -INFINITY;
        for (int rr = 0; rr < ts; ++rr) {
            int64_t j = (int64_t)rr * stride;
            int64_t t = gi * group + j / tile;
            if (t > nt - 1) t = nt - 1;
            int64_t p = t * tile + j % tile;
            float acc = 0.0f;
            for (int i = 0; i < d; ++i) acc += f16_to_f32(dq16[p * d + i]) * oracle_e4m3_to_f32(g[i]);
            float x = acc * sg[tl_];
            if (x > best) best = x;
        }
        sel[tl_] = best + lz[tl_];
    }
}

/* Online update whose PV operand is fp16: P = fp16(p * pscale[c]), values e4m3 rows. */
static void block_update_f16(const float *sc, const uint8_t *const *vals, const float *pscale, int nc, int d,
                             float *m, float *l, float *acc, float *dacc) {
    float bm = -INFINITY;
    for (int c = 0; c < nc; ++c)
        if (sc[c] > bm) bm = sc[c];
    float m_new = *m > bm ? *m : bm;
    float m_s = (m_new == -INFINITY) ? 0.0f : m_new;
    float psum = 0.0f;
    for (int i = 0; i < d; ++i) dacc[i] = 0.0f;
    for (int c = 0; c < nc; ++c) {
        float p = expf(sc[c] - m_s);
        psum += p;
        if (vals[c] == NULL) continue;
        float ph = f16_to_f32(oracle_f32_to_f16(p * pscale[c]));
        for (int i = 0; i < d; ++i) dacc[i] += ph * oracle_e4m3_to_f32(vals[c][i]);
    }
    float alpha = expf(*m - m_s);
    *l = *l * alpha + psum;
    for (int i = 0; i < d; ++i) acc[i] = acc[i] * alpha + dacc[i];
    *m = m_new;
}

/* Split-K tile kernel with the fp8 state store, h3/htrc_flat_triton.py:95-211 (DOT=1, FP8=1):
 *   far  score (sum dq16 . g) * sg + lz,  PV fp16(p * sv) . vb (e4m3)
 *   near score (sum q(bf16) . k(bf16)) * scale, PV bf16(p) . v (bf16)
 * Tile t uses the state and near set of its group t / group. */
void oracle_tile_fp8(int64_t nt, int tile, int d, int64_t nb, int leaf, int kx, int group,
                     const int32_t *idx, const int8_t *excl, const uint16_t *q16, const uint16_t *dq16,
                     const uint8_t *g8, const float *sg, const float *lz, const uint8_t *vb8, const float *sv,
                     const uint16_t *k, const uint16_t *v, float scale, int ns, int bn,
                     float *pm, float *pl, float *pacc) {
    int64_t lps = oracle_split(nb, ns, bn);
    int64_t eps = oracle_split((int64_t)kx * leaf, ns, bn);
#pragma omp parallel
    {
        float *sc = (float *)malloc(sizeof(float) * (size_t)bn);
        float *ps = (float *)malloc(sizeof(float) * (size_t)bn);
        const uint8_t **v8 = (const uint8_t **)malloc(sizeof(void *) * (size_t)bn);
        const uint16_t **vals = (const uint16_t **)malloc(sizeof(void *) * (size_t)bn);
        float *acc = (float *)malloc(sizeof(float) * (size_t)d);
        float *dacc = (float *)malloc(sizeof(float) * (size_t)d);
        float *qf = (float *)malloc(sizeof(float) * (size_t)d);
        float *dqf = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t job = 0; job < nt * ns * tile; ++job) {
            int64_t t = job / ((int64_t)ns * tile);
            int sp = (int)((job / tile) % ns);
            int r = (int)(job % tile);
            int64_t p = t * tile + r;
            int64_t gs = t / group;
            for (int i = 0; i < d; ++i) {
                qf[i] = bf2f(q16[p * d + i]);
                dqf[i] = f16_to_f32(dq16[p * d + i]);
            }
            float m = -INFINITY, l = 0.0f;
            for (int i = 0; i < d; ++i) acc[i] = 0.0f;
            int64_t lo = sp * lps, hi = lo + lps < nb ? lo + lps : nb;
            for (int64_t n0 = lo; n0 < hi; n0 += bn) {
                for (int c = 0; c < bn; ++c) {
                    int64_t cc = n0 + c;
                    if (cc < hi && excl[gs * nb + cc] == 0) {
                        int64_t s_ = gs * nb + cc;
                        float a = 0.0f;
                        for (int i = 0; i < d; ++i) a += dqf[i] * oracle_e4m3_to_f32(g8[s_ * d + i]);
                        sc[c] = a * sg[s_] + lz[s_];
                        v8[c] = vb8 + s_ * d;
                        ps[c] = sv[s_];
                    } else {
                        sc[c] = -INFINITY;
                        v8[c] = NULL;
                        ps[c] = 0.0f;
                    }
                }
                block_update_f16(sc, v8, ps, bn, d, &m, &l, acc, dacc);
            }
            int64_t e_n = (int64_t)kx * leaf;
            int64_t e_lo = sp * eps, e_hi = e_lo + eps < e_n ? e_lo + eps : e_n;
            for (int64_t e0 = e_lo; e0 < e_hi; e0 += bn) {
                for (int c = 0; c < bn; ++c) {
                    int64_t j = e0 + c;
                    if (j < e_hi) {
                        int64_t tok = (int64_t)idx[gs * kx + j / leaf] * leaf + j % leaf;
                        float a = 0.0f;
                        for (int i = 0; i < d; ++i) a += qf[i] * bf2f(k[tok * d + i]);
                        sc[c] = a * scale;
                        vals[c] = v + tok * d;
                    } else {
                        sc[c] = -INFINITY;
                        vals[c] = NULL;
                    }
                }
                block_update(sc, vals, bn, d, &m, &l, acc, dacc);
            }
            int64_t base = (t * ns + sp) * tile + r;
            pm[base] = m;
            pl[base] = l;
            memcpy(pacc + base * d, acc, sizeof(float) * (size_t)d);
        }
        free(sc);
        free(ps);
        free(v8);
        free(vals);
        free(acc);
        free(dacc);
        free(qf);
        free(dqf);
    }
}

/* Leaf statistics with the bf16 state store (store="bf16"): g (scaled) and vb rounded to bf16. */
void oracle_stats_bf16(const float *mu, int64_t nt, const uint16_t *k, const uint16_t *v,
                       int64_t nb, int leaf, int d, float scale, int tf32, uint16_t *g16, uint16_t *vb16, float *lz) {
#pragma omp parallel
    {
        float *a = (float *)malloc(sizeof(float) * (size_t)leaf);
        float *kf = (float *)malloc(sizeof(float) * (size_t)leaf * d);
        float *gs = (float *)malloc(sizeof(float) * (size_t)d);
        float *vs = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t tl_ = 0; tl_ < nt * nb; ++tl_) {
            int64_t t = tl_ / nb, l = tl_ % nb;
            float mx, z;
            leaf_state(mu + t * d, k + l * leaf * d, v + l * leaf * d, leaf, d, scale, tf32, a, kf, gs, vs, &mx, &z);
            for (int i = 0; i < d; ++i) {
                g16[tl_ * d + i] = f2bf(gs[i]);
                vb16[tl_ * d + i] = f2bf(vs[i]);
            }
            lz[tl_] = mx + logf(z);
        }
        free(a);
        free(kf);
        free(gs);
        free(vs);
    }
}

/* bf16 state store select: SEL[g,l] = max_r (sum_i bf16(dq)_ri * g_li) + lz_gl (products exact). */
void oracle_select_bf16(const uint16_t *dq16, int tile, int stride, int group, int64_t nt,
                        const uint16_t *g16, const float *lz, int64_t ng, int64_t nb, int d, float *sel) {
    int ts = group * tile / stride;
#pragma omp parallel for schedule(static)
    for (int64_t tl_ = 0; tl_ < ng * nb; ++tl_) {
        int64_t gi = tl_ / nb;
        const uint16_t *g = g16 + tl_ * d;
        float best = -INFINITY;
        for (int rr = 0; rr < ts; ++rr) {
            int64_t j = (int64_t)rr * stride;
            int64_t t = gi * group + j / tile;
            if (t > nt - 1) t = nt - 1;
            int64_t p = t * tile + j % tile;
            float acc = 0.0f;
            for (int i = 0; i < d; ++i) acc += bf2f(dq16[p * d + i]) * bf2f(g[i]);
            if (acc > best) best = acc;
        }
        sel[tl_] = best + lz[tl_];
    }
}

/* Split-K tile kernel with the bf16 state store: far score (sum bf16 dq . g) + lz, PV bf16(p) . vb;
 * near as oracle_tile_fp8. */
void oracle_tile_bf16(int64_t nt, int tile, int d, int64_t nb, int leaf, int kx, int group,
                      const int32_t *idx, const int8_t *excl, const uint16_t *q16, const uint16_t *dq16,
                      const uint16_t *g16, const float *lz, const uint16_t *vb16, const uint16_t *k, const uint16_t *v,
                      float scale, int ns, int bn, float *pm, float *pl, float *pacc) {
    int64_t lps = oracle_split(nb, ns, bn);
    int64_t eps = oracle_split((int64_t)kx * leaf, ns, bn);
#pragma omp parallel
    {
        float *sc = (float *)malloc(sizeof(float) * (size_t)bn);
        const uint16_t **vals = (const uint16_t **)malloc(sizeof(void *) * (size_t)bn);
        float *acc = (float *)malloc(sizeof(float) * (size_t)d);
        float *dacc = (float *)malloc(sizeof(float) * (size_t)d);
        float *qf = (float *)malloc(sizeof(float) * (size_t)d);
        float *dqf = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t job = 0; job < nt * ns * tile; ++job) {
            int64_t t = job / ((int64_t)ns * tile);
            int sp = (int)((job / tile) % ns);
            int r = (int)(job % tile);
            int64_t p = t * tile + r;
            int64_t gs = t / group;
            for (int i = 0; i < d; ++i) {
                qf[i] = bf2f(q16[p * d + i]);
                dqf[i] = bf2f(dq16[p * d + i]);
            }
            float m = -INFINITY, l = 0.0f;
            for (int i = 0; i < d; ++i) acc[i] = 0.0f;
            int64_t lo = sp * lps, hi = lo + lps < nb ? lo + lps : nb;
            for (int64_t n0 = lo; n0 < hi; n0 += bn) {
                for (int c = 0; c < bn; ++c) {
                    int64_t cc = n0 + c;
                    if (cc < hi && excl[gs * nb + cc] == 0) {
                        int64_t s_ = gs * nb + cc;
                        float a = 0.0f;
                        for (int i = 0; i < d; ++i) a += dqf[i] * bf2f(g16[s_ * d + i]);
                        sc[c] = a + lz[s_];
                        vals[c] = vb16 + s_ * d;
                    } else {
                        sc[c] = -INFINITY;
                        vals[c] = NULL;
                    }
                }
                block_update(sc, vals, bn, d, &m, &l, acc, dacc);
            }
            int64_t e_n = (int64_t)kx * leaf;
            int64_t e_lo = sp * eps, e_hi = e_lo + eps < e_n ? e_lo + eps : e_n;
            for (int64_t e0 = e_lo; e0 < e_hi; e0 += bn) {
                for (int c = 0; c < bn; ++c) {
                    int64_t j = e0 + c;
                    if (j < e_hi) {
                        int64_t tok = (int64_t)idx[gs * kx + j / leaf] * leaf + j % leaf;
                        float a = 0.0f;
                        for (int i = 0; i < d; ++i) a += qf[i] * bf2f(k[tok * d + i]);
                        sc[c] = a * scale;
                        vals[c] = v + tok * d;
                    } else {
                        sc[c] = -INFINITY;
                        vals[c] = NULL;
                    }
                }
                block_update(sc, vals, bn, d, &m, &l, acc, dacc);
            }
            int64_t base = (t * ns + sp) * tile + r;
            pm[base] = m;
            pl[base] = l;
            memcpy(pacc + base * d, acc, sizeof(float) * (size_t)d);
        }
        free(sc);
        free(vals);
        free(acc);
        free(dacc);
        free(qf);
        free(dqf);
    }
}

/* Split merge, h3/htrc_flat_triton.py:257-273, plus the log-partition of the row
 * (logz = mm + log den), which the reference computes but discards. */
void oracle_merge(const float *pm, const float *pl, const float *pacc, int64_t nt, int ns,
                  int tile, int d, float *out, float *logz) {
#pragma omp parallel
    {
        float *num = (float *)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
        for (int64_t tr = 0; tr < nt * tile; ++tr) {
            int64_t t = tr / tile;
            int r = (int)(tr % tile);
            float mm = -INFINITY;
            for (int s = 0; s < ns; ++s) {
                float x = pm[(t * ns + s) * tile + r];
                if (x > mm) mm = x;
            }
            if (mm == -INFINITY) mm = 0.0f;
            float den = 0.0f;
            for (int i = 0; i < d; ++i) num[i] = 0.0f;
            for (int s = 0; s < ns; ++s) {
                int64_t b = (t * ns + s) * tile + r;
                float w = expf(pm[b] - mm);
                den += pl[b] * w;
                for (int i = 0; i < d; ++i) num[i] += pacc[b * d + i] * w;
            }
            float dd = den < 1e-30f ? 1e-30f : den;
            for (int i = 0; i < d; ++i) out[tr * d + i] = num[i] / dd;
            logz[tr] = mm + logf(den);
        }
        free(num);
    }
}

/* k-means query order, h3/htrc_flat.py:47-61, in the arithmetic the HIP kernels fix:
 *   sample i: query round(linspace(0, n-1, m)[i]), m = min(sample, n), with torch's float32
 *   device linspace (step = (n-1)/(m-1); i < m/2: step*i, else fma(-step, m-1-i, n-1), one
 *   rounding) rounded to nearest even; initial centre j: sample round(linspace(0, m-1, C)[j]);
 *   nearest centre: squared distance as a sequential fp32 sum over the dims, the lowest centre
 *   on ties (none finite: centre 0);
 *   Lloyd update: per centre the sequential fp32 sum of its samples in sample order / count,
 *   a centre without samples keeps its position;
 *   perm: the queries ordered by centre, stable (torch.argsort(stable=True)). */
int64_t oracle_linspace_round(int64_t hi, int64_t steps, int64_t i) {
    if (steps <= 1) return 0;
    float step = (float)hi / (float)(steps - 1);
    /* upper half in one fused multiply-add, as torch's device linspace computes it */
    float v = i < steps / 2 ? step * (float)i : fmaf(-step, (float)(steps - 1 - i), (float)hi);
    int64_t r = (int64_t)nearbyintf(v);
    return r < 0 ? 0 : (r > hi ? hi : r);      /* (float)hi may round above hi for hi >= 2^24 */
}

static int nearest_centre(const float *x, const float *c, int clusters, int d) {
    float best = INFINITY;
    int bj = clusters;
    for (int j = 0; j < clusters; ++j) {
        float acc = 0.0f;
        for (int i = 0; i < d; ++i) {
            float df = x[i] - c[(int64_t)j * d + i];
            acc += df * df;
        }
        if (acc < best) {
            best = acc;
            bj = j;
        }
    }
    return bj < clusters ? bj : 0;
}

void oracle_kmeans_order(const float *q, int64_t n, int d, int clusters, int sample, int iters, int32_t *perm) {
    int64_t m = sample < n ? sample : n;
    float *c = (float *)malloc(sizeof(float) * (size_t)clusters * (size_t)d);
    float *acc = (float *)malloc(sizeof(float) * (size_t)d);
    int32_t *a = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    int64_t *cnt = (int64_t *)calloc((size_t)clusters + 1, sizeof(int64_t));
    for (int j = 0; j < clusters; ++j) {
        int64_t row = oracle_linspace_round(n - 1, m, oracle_linspace_round(m - 1, clusters, j));
        memcpy(c + (int64_t)j * d, q + row * d, sizeof(float) * (size_t)d);
    }
    for (int it = 0; it < iters; ++it) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i)
            a[i] = nearest_centre(q + oracle_linspace_round(n - 1, m, i) * d, c, clusters, d);
        for (int j = 0; j < clusters; ++j) {
            int64_t k = 0;
            for (int e = 0; e < d; ++e) acc[e] = 0.0f;
            for (int64_t i = 0; i < m; ++i) {
                if (a[i] != j) continue;
                const float *x = q + oracle_linspace_round(n - 1, m, i) * d;
                for (int e = 0; e < d; ++e) acc[e] += x[e];
                ++k;
            }
            if (k > 0)
                for (int e = 0; e < d; ++e) c[(int64_t)j * d + e] = acc[e] / (float)k;
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < n; ++p) a[p] = nearest_centre(q + p * d, c, clusters, d);
    for (int64_t p = 0; p < n; ++p) cnt[a[p] + 1]++;
    for (int j = 0; j < clusters; ++j) cnt[j + 1] += cnt[j];
    for (int64_t p = 0; p < n; ++p) perm[cnt[a[p]]++] = (int32_t)p;
    free(c);
    free(acc);
    free(a);
    free(cnt);
}
