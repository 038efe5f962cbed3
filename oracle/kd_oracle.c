/*
 * kd_oracle.c - CPU oracle for the CrossDiT flash-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY (what results are checked against, never the
 * thing measured or shipped).  Loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py; the product library never links it.
 *
 * Built with -ffp-contract=off so that every a*b+c written below rounds
 * twice, like the separate ggml ops of rope::apply; fused multiply-adds
 * are written explicitly (fmaf) where the restated algorithm uses them.
 */
#define _GNU_SOURCE
#include "kd_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 conversions (round to nearest even).       */
/* ------------------------------------------------------------------ */

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float f16_decode(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in float */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

static float g_f16_table[65536];
static pthread_once_t g_f16_once = PTHREAD_ONCE_INIT;
static void f16_table_init(void) {
    for (uint32_t i = 0; i < 65536; ++i) g_f16_table[i] = f16_decode((uint16_t)i);
}
static inline float f16_to_f32(uint16_t h) { return g_f16_table[h]; }

float kdo_f16_to_f32(uint16_t h) {
    pthread_once(&g_f16_once, f16_table_init);
    return f16_to_f32(h);
}

uint16_t kdo_f32_to_f16(float f) {
    const uint32_t x = f32_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: inf */
    if (ax < 0x38800000u) {
        /* result is a binary16 subnormal (or rounds up to the smallest
         * normal): scale by 2^24 (exact) and round to an integer. */
        const float scaled = bits_f32(ax) * 16777216.0f;
        return (uint16_t)(sign | (uint16_t)rintf(scaled));
    }
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t h = ((((ax >> 23) - 112u) << 10) | (mant >> 13));
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float kdo_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t kdo_f32_to_bf16(float f) {
    const uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

float kdo_round_to(float f, int type) {
    switch (type) {
    case KD_FA_TYPE_F16:  return f16_decode(kdo_f32_to_f16(f));
    case KD_FA_TYPE_BF16: return kdo_bf16_to_f32(kdo_f32_to_bf16(f));
    default:              return f;
    }
}

void kdo_f32_to_f16_n(const float *s, uint16_t *d, int64_t n) {
    for (int64_t i = 0; i < n; ++i) d[i] = kdo_f32_to_f16(s[i]);
}
void kdo_f32_to_bf16_n(const float *s, uint16_t *d, int64_t n) {
    for (int64_t i = 0; i < n; ++i) d[i] = kdo_f32_to_bf16(s[i]);
}
void kdo_f16_to_f32_n(const uint16_t *s, float *d, int64_t n) {
    pthread_once(&g_f16_once, f16_table_init);
    for (int64_t i = 0; i < n; ++i) d[i] = f16_to_f32(s[i]);
}
void kdo_bf16_to_f32_n(const uint16_t *s, float *d, int64_t n) {
    for (int64_t i = 0; i < n; ++i) d[i] = kdo_bf16_to_f32(s[i]);
}

/* The same two conversions by the F16C instructions (VCVTPS2PH with
 * round-to-nearest-even, VCVTPH2PS), eight lanes at a time, as ggml's SIMD
 * paths convert; pinned bitwise against the software codec above
 * (kdo_f16_codec_mismatches). */
void kdo_f32_to_f16_hw_n(const float *s, uint16_t *d, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        _mm_storeu_si128((__m128i *)(d + i),
                         _mm256_cvtps_ph(_mm256_loadu_ps(s + i), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
    for (; i < n; ++i)
        d[i] = (uint16_t)_mm_extract_epi16(_mm_cvtps_ph(_mm_set_ss(s[i]), _MM_FROUND_TO_NEAREST_INT), 0);
}
void kdo_f16_to_f32_hw_n(const uint16_t *s, float *d, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) _mm256_storeu_ps(d + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(s + i))));
    for (; i < n; ++i) d[i] = _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(s[i])));
}

/* Mismatches between the F16C and the software conversions: every F16 bit
 * pattern decoded, and `count` F32 bit patterns start, start + stride, ...
 * encoded (NaN payloads included; VCVTPH2PS quiets a signalling NaN, so a
 * decoded NaN is compared with its quiet bit set). */
int64_t kdo_f16_codec_mismatches(uint32_t start, uint32_t stride, int64_t count) {
    pthread_once(&g_f16_once, f16_table_init);
    int64_t bad = 0;
    uint16_t h[8];
    float f[8];
    for (uint32_t i = 0; i < 65536; i += 8) {
        for (int l = 0; l < 8; ++l) h[l] = (uint16_t)(i + l);
        kdo_f16_to_f32_hw_n(h, f, 8);
        for (int l = 0; l < 8; ++l) {
            const uint32_t hw = f32_bits(f[l]), sw = f32_bits(f16_decode(h[l]));
            const int nan = (sw & 0x7fffffffu) > 0x7f800000u;
            bad += nan ? hw != (sw | 0x00400000u) : hw != sw;
        }
    }
    uint32_t x = start;
    for (int64_t i = 0; i < count; i += 8) {
        const int m = count - i < 8 ? (int)(count - i) : 8;
        uint32_t u[8];
        for (int l = 0; l < m; ++l, x += stride) {
            u[l] = x;
            f[l] = bits_f32(x);
        }
        kdo_f32_to_f16_hw_n(f, h, m);
        for (int l = 0; l < m; ++l) bad += h[l] != kdo_f32_to_f16(bits_f32(u[l]));
    }
    return bad;
}

static inline float load_elem(const char *p, int type) {
    switch (type) {
    case KD_FA_TYPE_F32:  { float f; memcpy(&f, p, 4); return f; }
    case KD_FA_TYPE_F16:  { uint16_t h; memcpy(&h, p, 2); return f16_to_f32(h); }
    default:              { uint16_t h; memcpy(&h, p, 2); return kdo_bf16_to_f32(h); }
    }
}

static inline size_t type_size(int type) { return type == KD_FA_TYPE_F32 ? 4 : 2; }

/* ------------------------------------------------------------------ */
/* RoPE (src/rope.hpp).                                                */
/* ------------------------------------------------------------------ */

/* rope::get_freqs (src/rope.hpp:23-29): exp(-log(max_period) * i / dim),
 * evaluated in float in the same order. */
void kdo_rope_freqs(int dim, float max_period, float *out) {
    for (int i = 0; i < dim; i++)
        out[i] = expf(-logf(max_period) * (float)i / (float)dim);
}

/* rope::compute_text_rope (src/rope.hpp:36-49). */
void kdo_rope_text_table(int L, int D, float theta, float *out) {
    const int half = D / 2;
    float *f = (float *)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    kdo_rope_freqs(half, theta, f);
    for (int pos = 0; pos < L; pos++)
        for (int d = 0; d < half; d++) {
            const float angle = (float)pos * f[d];
            out[(size_t)pos * D + 2 * d + 0] = cosf(angle);
            out[(size_t)pos * D + 2 * d + 1] = sinf(angle);
        }
    free(f);
}

/* rope::compute_visual_rope (src/rope.hpp:56-102): row (t*Hp + h)*Wp + w,
 * column blocks t | h | w of axes[0] | axes[1] | axes[2] interleaved
 * (cos, sin) pairs of pos * freq_i / scale_factor[axis]. */
void kdo_rope_visual_table(int T, int Hp, int Wp, const int axes[3],
                           const float sf[3], float theta, float *out) {
    const int D = axes[0] + axes[1] + axes[2];
    const int half[3] = {axes[0] / 2, axes[1] / 2, axes[2] / 2};
    float *f[3];
    for (int a = 0; a < 3; ++a) {
        f[a] = (float *)malloc(sizeof(float) * (size_t)(half[a] > 0 ? half[a] : 1));
        kdo_rope_freqs(half[a], theta, f[a]);
    }
    for (int t = 0; t < T; t++)
        for (int h = 0; h < Hp; h++)
            for (int w = 0; w < Wp; w++) {
                float *row = out + (size_t)((t * Hp + h) * Wp + w) * D;
                const int pos[3] = {t, h, w};
                int off = 0;
                for (int a = 0; a < 3; ++a) {
                    for (int d = 0; d < half[a]; d++) {
                        const float angle = (float)pos[a] * f[a][d] / sf[a];
                        row[off + 2 * d + 0] = cosf(angle);
                        row[off + 2 * d + 1] = sinf(angle);
                    }
                    off += axes[a];
                }
            }
    for (int a = 0; a < 3; ++a) free(f[a]);
}

/* rope::apply (src/rope.hpp:109-155): per pair, out0 = x0*c - x1*s and
 * out1 = x0*s + x1*c, each product and sum rounded to F32 (separate ggml
 * mul / sub / add ops).  x is [B][L][H][D] (ggml [D, H, L, B]); the table
 * row is shared by all heads. */
void kdo_rope_apply_f32(const float *x, int64_t D, int64_t H, int64_t L,
                        int64_t B, const float *table, float *out) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t l = 0; l < L; ++l)
            for (int64_t h = 0; h < H; ++h) {
                const float *xr = x + ((b * L + l) * H + h) * D;
                float *orow = out + ((b * L + l) * H + h) * D;
                const float *cs = table + l * D;
                for (int64_t i = 0; i < D / 2; ++i) {
                    const float x0 = xr[2 * i], x1 = xr[2 * i + 1];
                    const float c = cs[2 * i], s = cs[2 * i + 1];
                    const float a = x0 * c, bb = x1 * s, e = x0 * s, g = x1 * c;
                    orow[2 * i] = a - bb;
                    orow[2 * i + 1] = e + g;
                }
            }
}

/* ggml_rms_norm followed by ggml_mul with the weight (ops::rms_norm,
 * src/core/ops.hpp:76-80, of the RMSNorm module src/core/module.hpp:163-180
 * that normalises each head row of Q and K, src/models/crossdit.hpp:135-136
 * and 192-193, eps 1e-6).  Per row of D elements: the squares, each rounded
 * to F32, summed in double; mean = (float)(sum / D); scale =
 * 1.0f / sqrtf(mean + eps); y = x * scale, then z = y * w, each an F32
 * operation as the two separate ggml ops round.  w == NULL skips the
 * multiply.  Rows are contiguous ([rows][D]); out may alias x. */
void kdo_rms_norm_mul(const float *x, int64_t rows, int64_t D, const float *w,
                      float eps, float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * D;
        float *orow = out + r * D;
        double sum = 0.0;
        for (int64_t i = 0; i < D; ++i) {
            const float sq = xr[i] * xr[i];
            sum += (double)sq;
        }
        const float mean = (float)(sum / (double)D);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < D; ++i) {
            const float y = xr[i] * scale;
            orow[i] = w ? y * w[i] : y;
        }
    }
}

/* (cos, sin) of pair i for token idx under a RoPE descriptor whose data
 * pointers are host-readable. */
static inline void rope_pair(const kd_fa_rope *r, int64_t idx, int64_t i,
                             float *c, float *s) {
    const int64_t d = 2 * i;
    if (r->mode == KD_FA_ROPE_TABLE) {
        const float *row = (const float *)((const char *)r->table.data + idx * (int64_t)r->table.nb[1]);
        *c = row[d];
        *s = row[d + 1];
        return;
    }
    const int64_t T = r->grid[0], Hp = r->grid[1], Wp = r->grid[2];
    (void)T;
    const int64_t t = idx / (Hp * Wp), h = (idx / Wp) % Hp, w = idx % Wp;
    const int64_t a0 = r->axes[0], a1 = r->axes[1], a2 = r->axes[2];
    const float *p;
    if (d < a0)           p = r->axes_data + t * a0 + d;
    else if (d < a0 + a1) p = r->axes_data + T * a0 + h * a1 + (d - a0);
    else                  p = r->axes_data + T * a0 + Hp * a1 + w * a2 + (d - a0 - a1);
    *c = p[0];
    *s = p[1];
}

/* Rotate one F32 row in place (rope.hpp:137-138 arithmetic). */
static void rope_row(const kd_fa_rope *r, int64_t idx, float *x, int64_t D) {
    for (int64_t i = 0; i < D / 2; ++i) {
        float c, s;
        rope_pair(r, idx, i, &c, &s);
        const float x0 = x[2 * i], x1 = x[2 * i + 1];
        const float a = x0 * c, b = x1 * s, e = x0 * s, g = x1 * c;
        x[2 * i] = a - b;
        x[2 * i + 1] = e + g;
    }
}

/* ------------------------------------------------------------------ */
/* Flash attention (ggml GGML_OP_FLASH_ATTN_EXT semantics).            */
/* ------------------------------------------------------------------ */

static int check_desc(const kd_fa_desc *d, const kd_fa_rope *r, int need_dst) {
    if (!d || !d->q.data || !d->k.data || !d->v.data || (need_dst && !d->dst.data)) return KD_FA_ERR_NULL;
    const int kt = d->k.type;
    if (kt != KD_FA_TYPE_F16 && kt != KD_FA_TYPE_BF16 && kt != KD_FA_TYPE_F32) return KD_FA_ERR_TYPE;
    if (d->v.type != KD_FA_TYPE_F16 && d->v.type != KD_FA_TYPE_BF16 && d->v.type != KD_FA_TYPE_F32) return KD_FA_ERR_TYPE;
    if (d->q.type != KD_FA_TYPE_F16 && d->q.type != KD_FA_TYPE_BF16 && d->q.type != KD_FA_TYPE_F32) return KD_FA_ERR_TYPE;
    if (need_dst && d->dst.type != KD_FA_TYPE_F32) return KD_FA_ERR_TYPE;
    /* ALiBi (max_bias > 0) is not restated: the op is only built with 0. */
    if (d->max_bias != 0.0f) return KD_FA_ERR_PARAM;
    /* Attention sinks (newer ggml's src[4]) are not restated either: the
       reference never sets them (ops.hpp:176). */
    if (d->sinks.data) return KD_FA_ERR_PARAM;
    if (d->k.ne[0] != d->q.ne[0] || d->k.ne[1] != d->v.ne[1]) return KD_FA_ERR_SHAPE;
    if (d->k.ne[2] <= 0 || d->q.ne[2] % d->k.ne[2] || d->k.ne[3] <= 0 || d->q.ne[3] % d->k.ne[3]) return KD_FA_ERR_SHAPE;
    if (d->v.ne[2] <= 0 || d->q.ne[2] % d->v.ne[2] || d->v.ne[3] <= 0 || d->q.ne[3] % d->v.ne[3]) return KD_FA_ERR_SHAPE;
    if (need_dst && (d->dst.ne[0] != d->v.ne[0] || d->dst.ne[1] != d->q.ne[2] || d->dst.ne[2] != d->q.ne[1] || d->dst.ne[3] != d->q.ne[3])) return KD_FA_ERR_SHAPE;
    if (d->mask.data) {
        if (d->mask.type != KD_FA_TYPE_F16) return KD_FA_ERR_TYPE;
        if (d->mask.ne[0] < d->k.ne[1] || d->mask.ne[1] < d->q.ne[1]) return KD_FA_ERR_SHAPE;
        if (d->mask.ne[2] <= 0 || d->q.ne[2] % d->mask.ne[2] || d->mask.ne[3] <= 0 || d->q.ne[3] % d->mask.ne[3]) return KD_FA_ERR_SHAPE;
    }
    if (r && r->mode != KD_FA_ROPE_NONE) {
        const int64_t D = d->q.ne[0], L = d->q.ne[1] > d->k.ne[1] ? d->q.ne[1] : d->k.ne[1];
        if (D % 2) return KD_FA_ERR_ROPE;
        if (r->mode == KD_FA_ROPE_TABLE) {
            if (!r->table.data || r->table.type != KD_FA_TYPE_F32 || r->table.ne[0] != D || r->table.ne[1] < L) return KD_FA_ERR_ROPE;
        } else if (r->mode == KD_FA_ROPE_AXES) {
            if (!r->axes_data || r->axes[0] + r->axes[1] + r->axes[2] != D) return KD_FA_ERR_ROPE;
            if ((r->axes[0] | r->axes[1] | r->axes[2]) & 1) return KD_FA_ERR_ROPE;
            if ((int64_t)r->grid[0] * r->grid[1] * r->grid[2] < L) return KD_FA_ERR_ROPE;
        } else {
            return KD_FA_ERR_ROPE;
        }
    }
    return KD_FA_OK;
}

/* Worker threads when the caller asks for the default: the CPU share the
   environment grants (OMP_NUM_THREADS, as a one-GPU job is given), else
   every online core. */
static int default_threads(void) {
    const char *e = getenv("OMP_NUM_THREADS");
    if (e) {
        const int n = atoi(e);
        if (n > 0) return n;
    }
    return (int)sysconf(_SC_NPROCESSORS_ONLN);
}

typedef struct {
    const kd_fa_desc *d;
    const kd_fa_rope *r;     /* NULL or mode NONE: no rotation */
    int f16_vacc;
    int f64;
    const int64_t *order;    /* row ids, sorted by (b_kv, h_kv)    */
    const int64_t *slot;     /* output slot of order[i] (f64 mode)  */
    int64_t n;
    double *out;
    int n_threads;
} fa_job;

typedef struct {
    fa_job *job;
    int tid;
} fa_arg;

static inline void row_coords(const kd_fa_desc *d, int64_t ir, int64_t *b, int64_t *h, int64_t *i) {
    const int64_t Lq = d->q.ne[1], H = d->q.ne[2];
    *b = ir / (H * Lq);
    *h = (ir - *b * H * Lq) / Lq;
    *i = ir - *b * H * Lq - *h * Lq;
}

/* K of one (b_k, h_k) head and V of one (b_v, h_v) head converted to
 * float once (ggml broadcasts K and V separately: h_k = h / (H / Hk),
 * h_v = h / (H / Hv)); K rotated and rounded to its own type when RoPE is
 * on. */
typedef struct {
    int64_t bk, hk, bv, hv;
    float *kf, *vf;
} kv_cache;

static void load_kv(const fa_job *j, kv_cache *c, int64_t bk, int64_t hk, int64_t bv, int64_t hv) {
    const kd_fa_desc *d = j->d;
    const int64_t Dk = d->k.ne[0], Dv = d->v.ne[0], Lk = d->k.ne[1];
    const int rope = j->r && j->r->mode != KD_FA_ROPE_NONE;
    for (int64_t jx = 0; jx < Lk; ++jx) {
        const char *kp = (const char *)d->k.data + jx * d->k.nb[1] + hk * d->k.nb[2] + bk * d->k.nb[3];
        float *kr = c->kf + jx * Dk;
        for (int64_t e = 0; e < Dk; ++e) kr[e] = load_elem(kp + e * d->k.nb[0], d->k.type);
        if (rope) {
            rope_row(j->r, jx, kr, Dk);
            for (int64_t e = 0; e < Dk; ++e) kr[e] = kdo_round_to(kr[e], d->k.type);
        }
        const char *vp = (const char *)d->v.data + jx * d->v.nb[1] + hv * d->v.nb[2] + bv * d->v.nb[3];
        float *vr = c->vf + jx * Dv;
        for (int64_t e = 0; e < Dv; ++e) vr[e] = load_elem(vp + e * d->v.nb[0], d->v.type);
    }
    c->bk = bk;
    c->hk = hk;
    c->bv = bv;
    c->hv = hv;
}

/* ggml_vec_dot_{f16,bf16} with F32 lanes: 32 running FMA sums, combined
 * pairwise. */
static inline float dot_f32(const float *a, const float *b, int64_t n) {
    float acc[32];
    for (int l = 0; l < 32; ++l) acc[l] = 0.0f;
    int64_t e = 0;
    for (; e + 32 <= n; e += 32)
        for (int l = 0; l < 32; ++l) acc[l] = fmaf(a[e + l], b[e + l], acc[l]);
    for (int l = 0; e < n; ++e, ++l) acc[l] = fmaf(a[e], b[e], acc[l]);
    for (int w = 16; w >= 1; w >>= 1)
        for (int l = 0; l < w; ++l) acc[l] += acc[l + w];
    return acc[0];
}

static void run_rows(fa_job *j, int64_t r0, int64_t r1) {
    const kd_fa_desc *d = j->d;
    const int64_t Dk = d->k.ne[0], Dv = d->v.ne[0], Lk = d->k.ne[1];
    const int64_t H = d->q.ne[2], B = d->q.ne[3];
    const int64_t rk2 = H / d->k.ne[2], rk3 = B / d->k.ne[3];
    const int64_t rv2 = H / d->v.ne[2], rv3 = B / d->v.ne[3];
    const int vt = d->v.type;
    const float scale = d->scale, softcap = d->logit_softcap;
    const int rope = j->r && j->r->mode != KD_FA_ROPE_NONE;

    kv_cache c;
    c.bk = c.hk = c.bv = c.hv = -1;
    c.kf = (float *)malloc(sizeof(float) * (size_t)(Lk * Dk + 1));
    c.vf = (float *)malloc(sizeof(float) * (size_t)(Lk * Dv + 1));
    float *q = (float *)malloc(sizeof(float) * (size_t)Dk);
    float *vkq32 = (float *)malloc(sizeof(float) * (size_t)Dv);
    uint16_t *vkq16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)Dv);
    double *sc = (double *)malloc(sizeof(double) * (size_t)(Lk + 1));
    double *acc = (double *)malloc(sizeof(double) * (size_t)Dv);

    for (int64_t x = r0; x < r1; ++x) {
        const int64_t ir = j->order[x];
        int64_t b, h, i;
        row_coords(d, ir, &b, &h, &i);
        const int64_t bk = b / rk3, hk = h / rk2, bv = b / rv3, hv = h / rv2;
        if (bk != c.bk || hk != c.hk || bv != c.bv || hv != c.hv) load_kv(j, &c, bk, hk, bv, hv);

        /* Q row -> F32 -> (RoPE) -> K's dot type. */
        const char *qp = (const char *)d->q.data + i * d->q.nb[1] + h * d->q.nb[2] + b * d->q.nb[3];
        for (int64_t e = 0; e < Dk; ++e) q[e] = load_elem(qp + e * d->q.nb[0], d->q.type);
        if (rope) rope_row(j->r, i, q, Dk);
        for (int64_t e = 0; e < Dk; ++e) q[e] = kdo_round_to(q[e], d->k.type);

        const uint16_t *mp = NULL;
        if (d->mask.data)
            mp = (const uint16_t *)((const char *)d->mask.data + i * d->mask.nb[1] +
                                    (h % d->mask.ne[2]) * d->mask.nb[2] + (b % d->mask.ne[3]) * d->mask.nb[3]);
        const float slope = 1.0f; /* max_bias == 0 */

        if (!j->f64) {
            /* ggml_compute_forward_flash_attn_ext_f16, one query row. */
            const int f16acc = j->f16_vacc && vt == KD_FA_TYPE_F16;
            float S = 0.0f, M = -INFINITY;
            if (f16acc) memset(vkq16, 0, sizeof(uint16_t) * (size_t)Dv);
            else        memset(vkq32, 0, sizeof(float) * (size_t)Dv);
            for (int64_t jx = 0; jx < Lk; ++jx) {
                const float mv = mp ? slope * f16_to_f32(mp[jx]) : 0.0f;
                if (mv == -INFINITY) continue;
                float s = dot_f32(c.kf + jx * Dk, q, Dk);
                s = s * scale;
                if (softcap != 0.0f) s = softcap * tanhf(s);
                s += mv;
                const float Mold = M;
                float ms = 1.0f, vs = 1.0f;
                const float *v = c.vf + jx * Dv;
                if (s > M) {
                    M = s;
                    ms = expf(Mold - M);
                    if (f16acc) {
                        /* ggml_vec_scale_f16: F16 -> F32, product, -> F16 */
                        int64_t e = 0;
                        const __m256 vm = _mm256_set1_ps(ms);
                        for (; e + 8 <= Dv; e += 8) {
                            const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(vkq16 + e)));
                            _mm_storeu_si128((__m128i *)(vkq16 + e),
                                             _mm256_cvtps_ph(_mm256_mul_ps(a, vm), _MM_FROUND_TO_NEAREST_INT));
                        }
                        for (; e < Dv; ++e) vkq16[e] = kdo_f32_to_f16(f16_to_f32(vkq16[e]) * ms);
                    } else {
                        for (int64_t e = 0; e < Dv; ++e) vkq32[e] *= ms;
                    }
                } else {
                    vs = expf(s - M);
                }
                if (f16acc) {
                    /* ggml_vec_mad_f16: one fused multiply-add per element,
                     * the F16 accumulator converted by F16C both ways */
                    int64_t e = 0;
                    const __m256 vv = _mm256_set1_ps(vs);
                    for (; e + 8 <= Dv; e += 8) {
                        const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(vkq16 + e)));
                        const __m256 r = _mm256_fmadd_ps(_mm256_loadu_ps(v + e), vv, a);
                        _mm_storeu_si128((__m128i *)(vkq16 + e), _mm256_cvtps_ph(r, _MM_FROUND_TO_NEAREST_INT));
                    }
                    for (; e < Dv; ++e) vkq16[e] = kdo_f32_to_f16(fmaf(v[e], vs, f16_to_f32(vkq16[e])));
                } else {
                    for (int64_t e = 0; e < Dv; ++e) vkq32[e] = fmaf(v[e], vs, vkq32[e]);
                }
                S = S * ms + vs;
            }
            if (f16acc)
                for (int64_t e = 0; e < Dv; ++e) vkq32[e] = f16_to_f32(vkq16[e]);
            const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
            float *o = (float *)((char *)d->dst.data + i * d->dst.nb[2] + h * d->dst.nb[1] + b * d->dst.nb[3]);
            for (int64_t e = 0; e < Dv; ++e) o[e] = vkq32[e] * S_inv;
        } else {
            /* Textbook softmax(scale*q.k + mask) v in double. */
            double mx = -INFINITY;
            for (int64_t jx = 0; jx < Lk; ++jx) {
                const double mv = mp ? (double)slope * (double)f16_to_f32(mp[jx]) : 0.0;
                if (mv == -INFINITY) { sc[jx] = -INFINITY; continue; }
                const float *kr = c.kf + jx * Dk;
                double s = 0.0;
                for (int64_t e = 0; e < Dk; ++e) s += (double)kr[e] * (double)q[e];
                s *= (double)scale;
                if (softcap != 0.0f) s = (double)softcap * tanh(s);
                s += mv;
                sc[jx] = s;
                if (s > mx) mx = s;
            }
            double *o = j->out + j->slot[x] * Dv;
            for (int64_t e = 0; e < Dv; ++e) acc[e] = 0.0;
            double sum = 0.0;
            if (mx != -INFINITY) {
                for (int64_t jx = 0; jx < Lk; ++jx) {
                    if (sc[jx] == -INFINITY) continue;
                    const double p = exp(sc[jx] - mx);
                    sum += p;
                    const float *v = c.vf + jx * Dv;
                    for (int64_t e = 0; e < Dv; ++e) acc[e] += p * (double)v[e];
                }
            }
            for (int64_t e = 0; e < Dv; ++e) o[e] = sum > 0.0 ? acc[e] / sum : 0.0;
        }
    }
    free(c.kf); free(c.vf); free(q); free(vkq32); free(vkq16); free(sc); free(acc);
}

static void *worker(void *p) {
    fa_arg *a = (fa_arg *)p;
    fa_job *j = a->job;
    const int64_t r0 = j->n * a->tid / j->n_threads;
    const int64_t r1 = j->n * (a->tid + 1) / j->n_threads;
    if (r1 > r0) run_rows(j, r0, r1);
    return NULL;
}

typedef struct { int64_t key, ir, slot; } sort_ent;
static int cmp_ent(const void *a, const void *b) {
    const sort_ent *x = (const sort_ent *)a, *y = (const sort_ent *)b;
    if (x->key != y->key) return x->key < y->key ? -1 : 1;
    if (x->ir != y->ir) return x->ir < y->ir ? -1 : 1;
    return 0;
}

static int run(const kd_fa_desc *d, const kd_fa_rope *r, int f16_vacc, int f64,
               const int64_t *rows, int64_t n_rows, double *out, int n_threads) {
    pthread_once(&g_f16_once, f16_table_init);
    int st = check_desc(d, r, !f64);
    if (st != KD_FA_OK) return st;
    const int64_t Lq = d->q.ne[1], H = d->q.ne[2], B = d->q.ne[3];
    const int64_t total = Lq * H * B;
    const int64_t n = rows ? n_rows : total;
    if (n <= 0) return 1;
    const int64_t rk2 = H / d->k.ne[2], rk3 = B / d->k.ne[3];
    sort_ent *ents = (sort_ent *)malloc(sizeof(sort_ent) * (size_t)n);
    for (int64_t x = 0; x < n; ++x) {
        const int64_t ir = rows ? rows[x] : x;
        if (ir < 0 || ir >= total) { free(ents); return KD_FA_ERR_SHAPE; }
        int64_t b, h, i;
        row_coords(d, ir, &b, &h, &i);
        ents[x].key = (b / rk3) * d->k.ne[2] + h / rk2;
        ents[x].ir = ir;
        ents[x].slot = x;
    }
    qsort(ents, (size_t)n, sizeof(sort_ent), cmp_ent);
    int64_t *order = (int64_t *)malloc(sizeof(int64_t) * (size_t)n);
    int64_t *slot = (int64_t *)malloc(sizeof(int64_t) * (size_t)n);
    for (int64_t x = 0; x < n; ++x) { order[x] = ents[x].ir; slot[x] = ents[x].slot; }
    free(ents);

    if (n_threads <= 0) n_threads = default_threads();
    if (n_threads < 1) n_threads = 1;
    if (n_threads > n) n_threads = (int)n;

    fa_job job = {d, r, f16_vacc, f64, order, slot, n, out, n_threads};
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
    fa_arg *args = (fa_arg *)malloc(sizeof(fa_arg) * (size_t)n_threads);
    for (int t = 0; t < n_threads; ++t) {
        args[t].job = &job;
        args[t].tid = t;
        if (t > 0) pthread_create(&th[t], NULL, worker, &args[t]);
    }
    worker(&args[0]);
    for (int t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
    free(th); free(args); free(order); free(slot);
    return n_threads;
}

int kdo_fa_ggml(const kd_fa_desc *desc, const kd_fa_rope *rope, int f16_vacc,
                const int64_t *rows, int64_t n_rows, int n_threads) {
    return run(desc, rope, f16_vacc, 0, rows, n_rows, NULL, n_threads);
}

int kdo_fa_f64(const kd_fa_desc *desc, const kd_fa_rope *rope, const int64_t *rows,
               int64_t n_rows, double *out, int n_threads) {
    if (!out) return KD_FA_ERR_NULL;
    return run(desc, rope, 0, 1, rows, n_rows, out, n_threads);
}
