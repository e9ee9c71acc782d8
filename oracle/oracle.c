/*
 * CPU oracle for the Inferno paged-KV attention path -- TEST INFRASTRUCTURE.
 *
 * This file restates the reference's Mojo kernels in plain C.  It is loaded
 * only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, and
 * only as the checker or the timed CPU baseline.  The HIP product never calls
 * it.  Every function cites the reference file:line it follows (paths are
 * relative to the reference repository root).
 *
 * What pins each function (checked in tests/test_oracle_*.py):
 *   ifo_fexp            closed form of exponential.mojo:177-194 evaluated in
 *                       float64 on the same integer bit path; error envelope
 *                       vs exp() on [-30, 0]; values at 0 and -87.
 *   ifo_splitmix64      published SplitMix64 finalizer test vectors.
 *   ifo_f32_to_bf16     RNE identities (ties to even, exact values, +-0).
 *   ifo_plan_run_splits brute-force re-derivation of the greedy rule and its
 *                       invariants (sum of splits == cap or saturation,
 *                       ceiling per run, split_base prefix sums).
 *   ifo_worker_range    partition identities (disjoint, covering, ordered).
 *   ifo_paged_slot      hand-computed slots for the reference test's ring
 *                       pages (tests/test_sliding_attention_degree_parity
 *                       .mojo:83-86 ring_slot).
 *   ifo_attention       the q = 0 closed form on every dispatch route (tile
 *                       and split structure); with a one-split plan and a
 *                       single tile, textbook softmax within the fexp error
 *                       bound.
 *   ifo_flash_partial   a float64 model of the tile-wise online softmax (the
 *                       same tiles and biased exp, exact dots) on profiles
 *                       with a dominant score in an early tile and a later
 *                       new maximum, where a missing max carry, a rescale
 *                       after the add or l without corr each move the
 *                       partials far beyond the tolerance
 *                       (tests/test_oracle_pins.py).
 *   ifo_finalize_head   a float64 model of merge_segments on the oracle's own
 *                       partials with spread maxima and empty stripes.
 *   ifo_rope_cache_write identity tables (cos=1, sin=0) make it a copy;
 *                       90-degree tables (cos=0, sin=1) swap pairs with sign.
 *   ifo_copy_jobs / ifo_gather_rows  byte-exact closed forms (memcpy/index).
 *   ifo_fwht            Sylvester Hadamard matrix product in float64 and the
 *                       impulse/constant special cases.
 *   ifo_absmax_quantize definition (butterquant.md:15-21): max code 127,
 *                       |code| <= 128, dequantized error <= amax/254.
 *   ifo_rms_norm_qkv_heads closed forms on constant rows, exact power-of-two
 *                       scale invariance, unit RMS of the output, gains on q
 *                       and k only, float64 RMS norm to one bf16 rounding.
 *   ifo_gemm_cols       integer-valued operands (exact sums, so the bf16
 *                       result is the rounded integer matmul), the identity
 *                       weight, and float64 matmul within one bf16 rounding
 *                       on random operands, with and without a k tail.
 *   ifo_bq_block_quant  known answers with exact scales (amax 127 and 254 give
 *                       inv 1 and 0.5, so ties land on .5 and must go to
 *                       even), the all-zero block (codes 0, scale 0), the
 *                       amax element's code +-127, the half-step error bound,
 *                       and blocks that do not see each other's values.
 *   ifo_bq_attention    the reference's own scalar reference_head with exact
 *                       exp (tests/test_sliding_attention_degree_parity.mojo:
 *                       93-141) on the reference test's 10-step schedule at
 *                       its tolerance 0.05.
 *
 * Parity left unpinned (no way to run Mojo here): the lane order of Mojo's
 * SIMD.reduce_add (taken as the halving tree of SIMD.reduce), FMA contraction
 * of `a*b - c*d` in RoPE, of `l*corr + sum` and of fexp's `a_magic*x + bias_f`
 * (all taken as not contracted; the fexp tests build the same choice in), the
 * f32->bf16 cast (taken as RNE, butterquant/convert.mojo:14-17), the order of
 * the sum of squares in the head RMS norm (VDPBF16PS pairs into port_unroll
 * accumulators, below float64 agreement) and fptosi in
 * the fast exp (taken as truncation toward zero).
 *
 * The reference targets AVX-512, so its f32 SIMD width W, and with it the
 * attention TILE (kernels/attention_ops.mojo:10), is 16.
 */
#include "oracle.h"

#if defined(__AVX512F__)
#include <immintrin.h>
#endif
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define W 16
#define TILE W
#define NEG_BIG (-1e30f)

/* ------------------------------------------------------------------------ */
/* numeric primitives                                                        */
/* ------------------------------------------------------------------------ */

float ifo_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even f32 -> bf16 (butterquant/convert.mojo:14-17). */
uint16_t ifo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t rne = u + ((u >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)(rne >> 16);
}

static inline float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fast_exp_softmax_biased (simd_math/exponential.mojo:177-194). */
float ifo_fexp(float x) {
    const float a_magic = 12102203.16156148f;
    const float bias_f = 1059208216.0f;
    const float inv_two23 = 1.0f / (float)(1 << 23);
    const float qc_a = 1.6501418352127075f;
    const float qc_b = -0.37554836273193359f;
    const float qc_c = 0.38696467876434326f;
    float t = a_magic * x;
    t = t + bias_f;
    int32_t i = (int32_t)t;
    uint32_t u = (uint32_t)i;
    float k = bits_to_f32(u);
    float f = (float)(u & 0x7FFFFFu) * inv_two23;
    float p = f * qc_c;
    p = qc_b + p;
    p = f * p;
    p = qc_a + p;
    return k * p;
}

void ifo_fexp_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ifo_fexp(x[i]);
}

/* splitmix64 finalizer (simd_math/sampling_rng.mojo:10-19). */
uint64_t ifo_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* rng_uniform (simd_math/sampling_rng.mojo:30-35): open interval (0, 1). */
float ifo_rng_uniform(uint64_t seed, uint64_t counter) {
    uint64_t h = ifo_splitmix64(seed ^ ifo_splitmix64(counter));
    return ((float)(int64_t)(h >> 40) + 1.0f) / (16777216.0f + 1.0f);
}

/* Seeded N(0,1) bf16 inputs: SplitMix64 counter stream -> Box-Muller ->
 * bf16 RNE.  Element i uses counters 2*(counter0+i) and 2*(counter0+i)+1. */
void ifo_fill_normal_bf16(uint16_t* dst, int64_t n, uint64_t seed,
                          uint64_t counter0) {
    for (int64_t i = 0; i < n; i++) {
        uint64_t c = 2ull * (counter0 + (uint64_t)i);
        double u1 = ifo_rng_uniform(seed, c);
        double u2 = ifo_rng_uniform(seed, c + 1);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = ifo_f32_to_bf16((float)z);
    }
}

/* SIMD[f32, 16].reduce_add as the halving tree of SIMD.reduce. */
float ifo_tree_sum16(const float* v) {
    float a[W];
    memcpy(a, v, sizeof(a));
    for (int w = W / 2; w >= 1; w >>= 1)
        for (int j = 0; j < w; j++) a[j] = a[j] + a[j + w];
    return a[0];
}

static float tree_max16(const float* v) {
    float a[W];
    memcpy(a, v, sizeof(a));
    for (int w = W / 2; w >= 1; w >>= 1)
        for (int j = 0; j < w; j++) a[j] = a[j] > a[j + w] ? a[j] : a[j + w];
    return a[0];
}

static inline float maxf_ref(float a, float b) { return a > b ? a : b; }

/* ------------------------------------------------------------------------ */
/* geometry and planning                                                     */
/* ------------------------------------------------------------------------ */

/* pow2_shift (kernels/attention_ops.mojo:32-37). */
int64_t ifo_pow2_shift(int64_t value) {
    int64_t shift = 0;
    while (((int64_t)1 << shift) < value) shift++;
    return shift;
}

/* flash_partial_stride (kernels/attention_ops.mojo:140-142). */
int64_t ifo_flash_partial_stride(int64_t num_q, int64_t head_dim) {
    return ((num_q * head_dim + 2 * num_q) * 4 + 63) / 64 * 16;
}

/* PagedKV.slot (kernels/attention_ops.mojo:47-51). */
int64_t ifo_paged_slot(const int32_t* base_rows, int64_t shift,
                       int64_t row_mask, int64_t page_mask,
                       int64_t start_pos, int64_t pos_t) {
    int64_t p = start_pos + pos_t;
    return (int64_t)base_rows[(p >> shift) & page_mask] + (p & row_mask);
}

/* worker_range (kernels/helpers.mojo:182-191). */
void ifo_worker_range(int64_t total, int64_t num_workers, int64_t worker_id,
                      int64_t base, int64_t* out2) {
    int64_t per = (total + num_workers - 1) / num_workers;
    int64_t start = base + worker_id * per;
    int64_t end = start + per;
    if (end > base + total) end = base + total;
    if (start >= base + total) {
        out2[0] = base + total;
        out2[1] = base + total;
        return;
    }
    out2[0] = start;
    out2[1] = end;
}

/* recommended_workers with DISPATCH_BW_PRODUCT and PARALLEL_AMORTIZED_BYTES
 * (kernels/helpers.mojo:206-219; kernels/dispatch_heuristics.mojo:10-11). */
int64_t ifo_recommended_workers(int64_t data_bytes, int64_t capacity) {
    if (capacity <= 1) return capacity;
    if (data_bytes >= 1024 * 1024) return capacity;
    int64_t target = data_bytes / 2280;
    int64_t n = 1;
    while ((n + 1) * (n + 1) <= target && n < capacity) n++;
    return n;
}

/* sliding_valid_len (kernels/attention_dispatch_kernels.mojo:29-33). */
int64_t ifo_sliding_valid_len(int64_t pos, int64_t window) {
    if (pos + 1 >= window) return window;
    return pos + 1;
}

/* full_local_kv_count (kernels/attention_ops.mojo:145-151). */
int64_t ifo_full_local_kv_count(int64_t rank, int64_t abs_pos,
                                int64_t degree) {
    if (abs_pos < 0) return 0;
    if (rank <= abs_pos % degree) return abs_pos / degree + 1;
    return abs_pos / degree;
}

/* plan_run_splits (kernels/attention_ops.mojo:99-137).
 * bands[i] = {buf_start, split_base, n_splits}. */
void ifo_plan_run_splits(const int64_t* kv_lens, const int64_t* buf_starts,
                         int64_t num_runs, int64_t cap, int64_t min_split,
                         int64_t* bands) {
    int64_t* max_splits = (int64_t*)malloc(sizeof(int64_t) * (size_t)(num_runs > 0 ? num_runs : 1));
    int64_t remaining = cap;
    for (int64_t i = 0; i < num_runs; i++) {
        int64_t kv = kv_lens[i];
        int64_t ceiling = kv > 0 ? (kv + min_split - 1) / min_split : 0;
        max_splits[i] = ceiling;
        int64_t seeded = (ceiling > 0 && remaining > 0) ? 1 : 0;
        remaining -= seeded;
        bands[3 * i + 0] = buf_starts[i];
        bands[3 * i + 1] = 0;
        bands[3 * i + 2] = seeded;
    }
    while (remaining > 0) {
        int64_t best = -1;
        for (int64_t i = 0; i < num_runs; i++) {
            int64_t n = bands[3 * i + 2];
            if (n == 0 || n >= max_splits[i]) continue;
            if (best < 0) {
                best = i;
                continue;
            }
            if (kv_lens[i] * bands[3 * best + 2] > kv_lens[best] * n) best = i;
        }
        if (best < 0) break;
        bands[3 * best + 2] += 1;
        remaining -= 1;
    }
    int64_t running = 0;
    for (int64_t i = 0; i < num_runs; i++) {
        bands[3 * i + 1] = running;
        running += bands[3 * i + 2];
    }
    free(max_splits);
}

/* ------------------------------------------------------------------------ */
/* bf16 score dot: bf16_panel_dot_to_scalars (kernels/dot_products.mojo:     */
/* 9-56,124-159) on an AVX-512 BF16 target: each VDPBF16PS lane adds the odd */
/* product then the even product, PU port-unrolled accumulators are summed   */
/* in order, then the 16 lanes are tree-reduced.                             */
/* ------------------------------------------------------------------------ */

static int64_t pick_port_unroll(int64_t width, int64_t cols) {
    if (cols % (8 * width) == 0) return 8;
    if (cols % (4 * width) == 0) return 4;
    if (cols % (2 * width) == 0) return 2;
    return 1;
}

/* reuse_panel_pu (kernels/attention_ops.mojo:183-190). */
static int64_t reuse_panel_pu(int64_t head_dim, int64_t gqa) {
    int64_t cap = pick_port_unroll(2 * W, head_dim);
    int64_t budget = 32 / gqa;
    int64_t pu = 1;
    while (pu * 2 <= cap && pu * 2 <= budget && pu * gqa < 8) pu *= 2;
    return pu;
}

#if defined(__AVX512BF16__) && defined(__AVX512F__)
/* The same lanes through the instruction itself, for a -march=native build on
 * a host with AVX-512 BF16 (the reference's own path on such hosts):
 * VDPBF16PS lane j adds x[2j+1]*k[2j+1] and then x[2j]*k[2j] to its f32
 * accumulator, each step rounded to nearest even; bf16 products are exact in
 * f32, so this equals the portable form below for all normal inputs (the
 * instruction treats denormal inputs and results as zero). */
static float bf16_dot_vdpbf16(const uint16_t* k_row, const uint16_t* x_row,
                              int64_t cols, int64_t pu) {
    __m512 acc[8];
    for (int64_t p = 0; p < pu; p++) acc[p] = _mm512_setzero_ps();
    int64_t stride = pu * 2 * W;
    for (int64_t i = 0; i < cols / stride; i++) {
        for (int64_t p = 0; p < pu; p++) {
            int64_t off = i * stride + p * 2 * W;
            __m512i xv = _mm512_loadu_si512((const void*)(x_row + off));
            __m512i kv = _mm512_loadu_si512((const void*)(k_row + off));
            acc[p] = _mm512_dpbf16_ps(acc[p], (__m512bh)xv, (__m512bh)kv);
        }
    }
    /* Port accumulators summed in order, then the halving tree of
     * SIMD.reduce_add (lanes j and j + w for w = 8, 4, 2, 1), lane for lane
     * as ifo_tree_sum16 adds them. */
    __m512 v = _mm512_setzero_ps();
    for (int64_t p = 0; p < pu; p++) v = _mm512_add_ps(v, acc[p]);
    __m256 h8 = _mm256_add_ps(_mm512_castps512_ps256(v), _mm512_extractf32x8_ps(v, 1));
    __m128 h4 = _mm_add_ps(_mm256_castps256_ps128(h8), _mm256_extractf128_ps(h8, 1));
    __m128 h2 = _mm_add_ps(h4, _mm_movehl_ps(h4, h4));
    __m128 h1 = _mm_add_ss(h2, _mm_shuffle_ps(h2, h2, 1));
    return _mm_cvtss_f32(h1);
}
#else
static float bf16_dot_vdpbf16(const uint16_t* k_row, const uint16_t* x_row,
                              int64_t cols, int64_t pu) {
    /* One 32-bit load holds a (even, odd) bf16 pair, as a VDPBF16PS lane
     * reads it: the odd element is the high half (bits & 0xFFFF0000 as f32),
     * the even one the low half (bits << 16).  The lanes are independent,
     * so the j loops vectorise without changing any lane's order. */
    float acc[8][W];
    for (int64_t p = 0; p < pu; p++)
        for (int j = 0; j < W; j++) acc[p][j] = 0.0f;
    int64_t stride = pu * 2 * W;
    const uint32_t* k32 = (const uint32_t*)k_row;
    const uint32_t* x32 = (const uint32_t*)x_row;
    for (int64_t i = 0; i < cols / stride; i++) {
        for (int64_t p = 0; p < pu; p++) {
            int64_t off = (i * stride + p * 2 * W) / 2;
            for (int j = 0; j < W; j++) {
                uint32_t xp = x32[off + j], kp = k32[off + j];
                float xo = bits_to_f32(xp & 0xFFFF0000u);
                float ko = bits_to_f32(kp & 0xFFFF0000u);
                float xe = bits_to_f32(xp << 16);
                float ke = bits_to_f32(kp << 16);
                float a = acc[p][j];
                a = a + xo * ko;
                a = a + xe * ke;
                acc[p][j] = a;
            }
        }
    }
    float s[W];
    for (int j = 0; j < W; j++) {
        float v = 0.0f;
        for (int64_t p = 0; p < pu; p++) v = v + acc[p][j];
        s[j] = v;
    }
    return ifo_tree_sum16(s);
}
#endif

/* Raw int8 score dot of bq_process_kv_tile: VPDPBUSD over (k ^ 0x80) read as
 * unsigned bytes times the signed q codes.  The sum is exact in int32, so any
 * order gives the same value. */
static int32_t i8_dot_vpdpbusd(const int8_t* k_row, const int8_t* q_row, int64_t D) {
#if defined(__AVX512VNNI__) && defined(__AVX512F__)
    if (D % 64 == 0) {
        __m512i acc = _mm512_setzero_si512();
        const __m512i flip = _mm512_set1_epi8((char)0x80);
        for (int64_t e = 0; e < D; e += 64) {
            __m512i kv = _mm512_xor_si512(_mm512_loadu_si512((const void*)(k_row + e)), flip);
            __m512i qv = _mm512_loadu_si512((const void*)(q_row + e));
            acc = _mm512_dpbusd_epi32(acc, kv, qv);
        }
        return _mm512_reduce_add_epi32(acc);
    }
#endif
    int32_t raw = 0;
    for (int64_t e = 0; e < D; e++)
        raw += (int32_t)((uint8_t)((uint8_t)k_row[e] ^ 0x80u)) * (int32_t)q_row[e];
    return raw;
}

/* ------------------------------------------------------------------------ */
/* attention work item: one (token or split) range through the paged cache   */
/* ------------------------------------------------------------------------ */

typedef struct {
    int is_bq;
    /* bf16 */
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    /* bq */
    const int8_t* qi;
    const float* qi_bias;
    const float* f_q;
    const int8_t* ki;
    const float* k_scale;
    const int8_t* vi;
    const float* v_scale;
    int64_t num_q, num_kv, head_dim, gqa, kv_stride;
    int64_t shift, row_mask, page_mask;
    int64_t partial_stride;
    float* partials;
} attn_ctx;

typedef struct {
    int64_t q_row;      /* token row of q (and of qi_bias / f_q) */
    const int32_t* rows;/* the run's base_rows */
    int64_t start_pos;
    int64_t start, end;
    int64_t stripe;     /* partial stripe written */
} attn_item;

/* online_softmax_tile (kernels/attention_ops.mojo:165-180) applied to one q
 * head; updates m, l, scales acc and returns the 16 weights. */
static void online_softmax_update(const float* scores16, float* m, float* l,
                                  float* acc, int64_t head_dim, float* w16) {
    float tile_max = tree_max16(scores16);
    float m_new = tile_max > *m ? tile_max : *m;
    float corr = ifo_fexp(maxf_ref(-87.0f, *m - m_new));
    for (int t = 0; t < W; t++)
        w16[t] = ifo_fexp(maxf_ref(-87.0f, scores16[t] - m_new));
    for (int64_t j = 0; j < head_dim; j++) acc[j] = acc[j] * corr;  /* scale_unrolled */
    float prod = *l * corr;
    *l = prod + ifo_tree_sum16(w16);
    *m = m_new;
}

/* process_kv_tile (kernels/attention_ops.mojo:193-253) and bq_process_kv_tile
 * (butterquant_kernels/attention.mojo:27-102). */
static void process_tile(const attn_ctx* c, const attn_item* it,
                         const int64_t* q_heads_off, int64_t pos,
                         int64_t tile_len, float* m, float* l, float* acc) {
    int64_t slots[TILE];
    int64_t D = c->head_dim;
    for (int64_t t = 0; t < tile_len; t++)
        slots[t] = ifo_paged_slot(it->rows, c->shift, c->row_mask,
                                  c->page_mask, it->start_pos, pos + t);
    int64_t groups = c->num_q / c->gqa;
    int64_t pu = reuse_panel_pu(D, c->gqa);
    const float inv127 = 1.0f / 127.0f;
    const float inv127sq = inv127 * inv127;
    float scores[TILE * 64];   /* gqa <= 64 */
    float weights[TILE * 64];
    for (int64_t g = 0; g < groups; g++) {
        int64_t base_q = g * c->gqa;
        int64_t head_off = g * D;
        for (int64_t t = 0; t < tile_len; t++) {
            if (!c->is_bq) {
                const uint16_t* k_head = c->k + slots[t] * c->kv_stride + head_off;
                for (int64_t r = 0; r < c->gqa; r++)
                    scores[t * c->gqa + r] = bf16_dot_vdpbf16(
                        k_head, c->q + q_heads_off[base_q + r], D, pu);
            } else {
                const int8_t* k_head = c->ki + slots[t] * c->kv_stride + head_off;
                float ks = c->k_scale[slots[t] * c->num_kv + g];
                for (int64_t r = 0; r < c->gqa; r++) {
                    int64_t qi = base_q + r;
                    const int8_t* qrow = c->qi + q_heads_off[qi];
                    int32_t raw = i8_dot_vpdpbusd(k_head, qrow, D);
                    float qb = c->qi_bias[it->q_row * c->num_q + qi];
                    float fq = c->f_q[it->q_row * c->num_q + qi];
                    float s = (float)raw - qb;
                    s = s * fq;
                    s = s * ks;
                    s = s * inv127sq;
                    scores[t * c->gqa + r] = s;
                }
            }
        }
        for (int64_t r = 0; r < c->gqa; r++) {
            int64_t qi = base_q + r;
            float sc[W], w16[W];
            for (int t = 0; t < W; t++) sc[t] = NEG_BIG;
            for (int64_t t = 0; t < tile_len; t++) sc[t] = scores[t * c->gqa + r];
            online_softmax_update(sc, &m[qi], &l[qi], acc + qi * D, D, w16);
            for (int64_t t = 0; t < tile_len; t++) weights[t * c->gqa + r] = w16[t];
        }
        for (int64_t t = 0; t < tile_len; t++) {
            if (!c->is_bq) {
                /* Each accumulator element takes one fma per key; the
                 * (r, j) loop order does not change any element's chain. */
                const uint16_t* v_head = c->v + slots[t] * c->kv_stride + head_off;
                for (int64_t r = 0; r < c->gqa; r++) {
                    float wr = weights[t * c->gqa + r];
                    float* a = acc + (base_q + r) * D;
                    for (int64_t j = 0; j < D; j++)
                        a[j] = fmaf(bits_to_f32((uint32_t)v_head[j] << 16), wr, a[j]);
                }
            } else {
                const int8_t* v_head = c->vi + slots[t] * c->kv_stride + head_off;
                float vs = c->v_scale[slots[t] * c->num_kv + g];
                float wts[64];
                for (int64_t r = 0; r < c->gqa; r++) {
                    float w = weights[t * c->gqa + r] * vs;
                    wts[r] = w * inv127;
                }
                for (int64_t r = 0; r < c->gqa; r++) {
                    float* a = acc + (base_q + r) * D;
                    for (int64_t j = 0; j < D; j++)
                        a[j] = fmaf((float)v_head[j], wts[r], a[j]);
                }
            }
        }
    }
}

/* FlashAttentionKernel.execute (kernels/flash_attention.mojo:28-58) and
 * BqFlashAttentionKernel.execute (butterquant_kernels/attention.mojo:128-161):
 * the item's range [start, end) is walked in TILE steps from `start`. */
static void run_item(const attn_ctx* c, const attn_item* it) {
    int64_t D = c->head_dim;
    float* part = c->partials + it->stripe * c->partial_stride;
    int64_t m_off = c->num_q * D;
    int64_t l_off = m_off + c->num_q;
    float m[64], l[64];
    int64_t q_heads_off[64];
    for (int64_t h = 0; h < c->num_q; h++) {
        m[h] = NEG_BIG;
        l[h] = 0.0f;
        q_heads_off[h] = it->q_row * c->num_q * D + h * D;
    }
    memset(part, 0, sizeof(float) * (size_t)(c->num_q * D));
    for (int64_t pos = it->start; pos < it->end; pos += TILE) {
        int64_t tile_len = it->end - pos < TILE ? it->end - pos : TILE;
        process_tile(c, it, q_heads_off, pos, tile_len, m, l, part);
    }
    for (int64_t h = 0; h < c->num_q; h++) {
        part[m_off + h] = m[h];
        part[l_off + h] = l[h];
    }
}

void ifo_flash_partial(const int32_t* base_rows, int64_t shift,
                       int64_t row_mask, int64_t page_mask,
                       const uint16_t* q, const uint16_t* k_base,
                       const uint16_t* v_base, float* partial,
                       int64_t num_q, int64_t head_dim, int64_t gqa_ratio,
                       int64_t kv_stride, int64_t start_pos, int64_t start,
                       int64_t end) {
    attn_ctx c;
    memset(&c, 0, sizeof(c));
    c.q = q;
    c.k = k_base;
    c.v = v_base;
    c.num_q = num_q;
    c.num_kv = num_q / gqa_ratio;
    c.head_dim = head_dim;
    c.gqa = gqa_ratio;
    c.kv_stride = kv_stride;
    c.shift = shift;
    c.row_mask = row_mask;
    c.page_mask = page_mask;
    c.partial_stride = 0;
    c.partials = partial;
    attn_item it = {0, base_rows, start_pos, start, end, 0};
    run_item(&c, &it);
}

/* merge_segments + write_finalized_head (kernels/logsum_merge.mojo:28-122)
 * for a single segment {seg_base, seg_stride, seg_n}. */
void ifo_finalize_head(uint16_t* dst, const float* seg_base,
                       int64_t seg_stride, int64_t seg_n, int64_t num_q,
                       int64_t head_dim, int64_t h) {
    int64_t m_off = num_q * head_dim;
    int64_t l_off = m_off + num_q;
    float global_m = NEG_BIG;
    for (int64_t s = 0; s < seg_n; s++) {
        float sm = seg_base[s * seg_stride + m_off + h];
        if (sm > global_m) global_m = sm;
    }
    float global_l = 0.0f;
    int first = 1;
    float* acc = (float*)calloc((size_t)head_dim, sizeof(float));
    for (int64_t bs = 0; bs < seg_n; bs += W) {
        int64_t be = bs + W < seg_n ? bs + W : seg_n;
        float deltas[W], ls[W], corrs[W], prod[W];
        for (int b = 0; b < W; b++) {
            deltas[b] = NEG_BIG;
            ls[b] = 0.0f;
        }
        for (int64_t b = 0; b < be - bs; b++) {
            const float* sp = seg_base + (bs + b) * seg_stride;
            deltas[b] = sp[m_off + h] - global_m;
            ls[b] = sp[l_off + h];
        }
        for (int b = 0; b < W; b++) {
            corrs[b] = ifo_fexp(maxf_ref(-87.0f, deltas[b]));
            corrs[b] = ls[b] > 0.0f ? corrs[b] : 0.0f;
            prod[b] = ls[b] * corrs[b];
        }
        global_l = global_l + ifo_tree_sum16(prod);
        for (int64_t b = 0; b < be - bs; b++) {
            float cv = corrs[b];
            if (cv <= 0.0f) continue;
            const float* src = seg_base + (bs + b) * seg_stride + h * head_dim;
            if (first) {
                for (int64_t j = 0; j < head_dim; j++) acc[j] = src[j] * cv;
                first = 0;
            } else {
                for (int64_t j = 0; j < head_dim; j++) acc[j] = fmaf(src[j], cv, acc[j]);
            }
        }
    }
    if (global_l <= 0.0f) {
        for (int64_t j = 0; j < head_dim; j++) dst[j] = 0;
    } else {
        float inv_l = 1.0f / global_l;
        for (int64_t j = 0; j < head_dim; j++) dst[j] = ifo_f32_to_bf16(acc[j] * inv_l);
    }
    free(acc);
}

/* Direct finalisation of the sliding prefill kernels
 * (kernels/flash_attention_prefill.mojo:95-106;
 * butterquant_kernels/attention.mojo:244-253). */
static void finalize_direct(uint16_t* dst, const float* part, int64_t num_q,
                            int64_t head_dim, int64_t h) {
    float l = part[num_q * head_dim + num_q + h];
    const float* acc = part + h * head_dim;
    if (l > 0.0f) {
        float inv_l = 1.0f / l;
        for (int64_t j = 0; j < head_dim; j++) dst[j] = ifo_f32_to_bf16(acc[j] * inv_l);
    } else {
        for (int64_t j = 0; j < head_dim; j++) dst[j] = 0;
    }
}

/* ------------------------------------------------------------------------ */
/* threaded item execution (one fan-out + join, as fanout_dispatch)          */
/* ------------------------------------------------------------------------ */

typedef struct {
    const attn_ctx* c;
    const attn_item* items;
    int64_t n;
    atomic_llong next;
} item_pool;

static void* item_worker(void* arg) {
    item_pool* p = (item_pool*)arg;
    for (;;) {
        long long i = atomic_fetch_add(&p->next, 1);
        if (i >= p->n) break;
        run_item(p->c, &p->items[i]);
    }
    return NULL;
}

static void run_items(const attn_ctx* c, const attn_item* items, int64_t n,
                      int64_t threads) {
    item_pool p;
    p.c = c;
    p.items = items;
    p.n = n;
    atomic_init(&p.next, 0);
    if (threads <= 1 || n <= 1) {
        item_worker(&p);
        return;
    }
    if (threads > n) threads = n;
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int64_t t = 1; t < threads; t++) pthread_create(&tids[t], NULL, item_worker, &p);
    item_worker(&p);
    for (int64_t t = 1; t < threads; t++) pthread_join(tids[t], NULL);
    free(tids);
}

/* ------------------------------------------------------------------------ */
/* dispatch: dispatch_flash_sliding / dispatch_flash_full at degree 1        */
/* (kernels/attention_dispatch_kernels.mojo:36-299, 302-426;                 */
/* butterquant_kernels/attention.mojo:354-491)                               */
/* ------------------------------------------------------------------------ */

static int run_dispatch(attn_ctx* c, int64_t kind, const int32_t* runs,
                        int64_t num_runs, const int32_t* base_rows,
                        uint16_t* out, int64_t window, int64_t seq_len,
                        int64_t cap, int64_t threads, int64_t elt_bytes) {
    int64_t D = c->head_dim;
    int64_t q_stride = c->num_q * D;
    if (seq_len <= 0) return 0;
    if (num_runs <= 0) return -1;
    if (cap < 1) cap = 1;
    c->partial_stride = ifo_flash_partial_stride(c->num_q, D);
    int is_sliding = kind == 0;

    if (seq_len == 1) {
        int64_t base_pos = runs[1];
        int64_t valid = is_sliding ? ifo_sliding_valid_len(base_pos, window)
                                   : ifo_full_local_kv_count(0, base_pos, 1);
        if (valid <= 0) {
            if (!is_sliding) memset(out, 0, sizeof(uint16_t) * (size_t)q_stride);
            return 0;
        }
        int64_t start_pos = is_sliding ? base_pos - valid + 1 : 0;
        int64_t nw = ifo_recommended_workers(valid * c->kv_stride * elt_bytes, cap);
        if (nw <= 0) nw = cap;
        if (nw > cap) nw = cap;
        if (nw > valid) nw = valid;
        c->partials = (float*)calloc((size_t)(nw * c->partial_stride), sizeof(float));
        attn_item* items = (attn_item*)malloc(sizeof(attn_item) * (size_t)nw);
        const int32_t* rows = base_rows + runs[2];
        for (int64_t w = 0; w < nw; w++) {
            int64_t wr[2];
            ifo_worker_range(valid, nw, w, 0, wr);
            attn_item it = {0, rows, start_pos, wr[0], wr[1], w};
            items[w] = it;
        }
        run_items(c, items, nw, threads);
        for (int64_t h = 0; h < c->num_q; h++)
            ifo_finalize_head(out + h * D, c->partials, c->partial_stride, nw,
                              c->num_q, D, h);
        free(items);
        free(c->partials);
        return 0;
    }

    if (num_runs == seq_len && num_runs > 1 && num_runs < cap) {
        int64_t* kv = (int64_t*)malloc(sizeof(int64_t) * (size_t)num_runs);
        int64_t* bs = (int64_t*)malloc(sizeof(int64_t) * (size_t)num_runs);
        int64_t* bands = (int64_t*)malloc(sizeof(int64_t) * 3 * (size_t)num_runs);
        for (int64_t i = 0; i < num_runs; i++) {
            int64_t p = runs[4 * i + 1];
            kv[i] = is_sliding ? ifo_sliding_valid_len(p, window)
                               : ifo_full_local_kv_count(0, p, 1);
            bs[i] = runs[4 * i + 0];
        }
        ifo_plan_run_splits(kv, bs, num_runs, cap, TILE, bands);
        int64_t total = 0;
        for (int64_t i = 0; i < num_runs; i++) total += bands[3 * i + 2];
        c->partials = (float*)calloc((size_t)((total > 0 ? total : 1) * c->partial_stride), sizeof(float));
        attn_item* items = (attn_item*)malloc(sizeof(attn_item) * (size_t)(total > 0 ? total : 1));
        int64_t n = 0;
        for (int64_t i = 0; i < num_runs; i++) {
            int64_t ns = bands[3 * i + 2];
            int64_t start_pos = is_sliding ? runs[4 * i + 1] - kv[i] + 1 : 0;
            for (int64_t s = 0; s < ns; s++) {
                int64_t wr[2];
                ifo_worker_range(kv[i], ns, s, 0, wr);
                attn_item it = {runs[4 * i + 0], base_rows + runs[4 * i + 2],
                                start_pos, wr[0], wr[1], bands[3 * i + 1] + s};
                items[n++] = it;
            }
        }
        run_items(c, items, n, threads);
        for (int64_t i = 0; i < num_runs; i++) {
            for (int64_t h = 0; h < c->num_q; h++)
                ifo_finalize_head(out + bands[3 * i + 0] * q_stride + h * D,
                                  c->partials + bands[3 * i + 1] * c->partial_stride,
                                  c->partial_stride, bands[3 * i + 2], c->num_q, D, h);
        }
        free(items);
        free(c->partials);
        free(kv);
        free(bs);
        free(bands);
        return 0;
    }

    /* token-partitioned prefill kernels: FlashPrefillSlidingKernel /
     * FlashPrefillFullKernel (kernels/flash_attention_prefill.mojo:41-193). */
    c->partials = (float*)calloc((size_t)(seq_len * c->partial_stride), sizeof(float));
    attn_item* items = (attn_item*)malloc(sizeof(attn_item) * (size_t)seq_len);
    int64_t r = 0;
    for (int64_t t = 0; t < seq_len; t++) {
        while (r + 1 < num_runs && t >= runs[4 * (r + 1)]) r++;
        int64_t abs_pos = runs[4 * r + 1] + (t - runs[4 * r]);
        int64_t lo, hi;
        if (is_sliding) {
            lo = abs_pos - window + 1;
            if (lo < 0) lo = 0;
            hi = abs_pos + 1;
        } else {
            lo = 0;
            hi = ifo_full_local_kv_count(0, abs_pos, 1);
        }
        attn_item it = {t, base_rows + runs[4 * r + 2], 0, lo, hi, t};
        items[t] = it;
    }
    run_items(c, items, seq_len, threads);
    for (int64_t t = 0; t < seq_len; t++) {
        for (int64_t h = 0; h < c->num_q; h++) {
            const float* part = c->partials + t * c->partial_stride;
            if (is_sliding)
                finalize_direct(out + t * q_stride + h * D, part, c->num_q, D, h);
            else   /* PrefillMergeKernel: one segment per rank (logsum_merge) */
                ifo_finalize_head(out + t * q_stride + h * D, part,
                                  c->partial_stride, 1, c->num_q, D, h);
        }
    }
    free(items);
    free(c->partials);
    return 0;
}

static int geometry(attn_ctx* c, int64_t kind, int64_t num_q, int64_t num_kv,
                    int64_t head_dim, int64_t kv_stride, int64_t cache_size,
                    int64_t page_len) {
    if (num_q <= 0 || num_kv <= 0 || num_q % num_kv != 0 || num_q > 64) return -1;
    if (head_dim % (2 * W) != 0 || num_q / num_kv > 8) return -1;
    if (page_len <= 0 || (page_len & (page_len - 1)) != 0) return -1;
    c->num_q = num_q;
    c->num_kv = num_kv;
    c->head_dim = head_dim;
    c->gqa = num_q / num_kv;
    c->kv_stride = kv_stride;
    c->shift = ifo_pow2_shift(page_len);
    c->row_mask = page_len - 1;
    if (kind == 0) {
        int64_t ring = cache_size / page_len;
        if (ring <= 0 || (ring & (ring - 1)) != 0) return -1;
        c->page_mask = ring - 1;
    } else {
        c->page_mask = -1;
    }
    return 0;
}

int ifo_attention(int64_t kind, const int32_t* runs, int64_t num_runs,
                  const int32_t* base_rows, const uint16_t* q,
                  const uint16_t* k_base, const uint16_t* v_base,
                  uint16_t* out, int64_t num_q, int64_t num_kv,
                  int64_t head_dim, int64_t kv_stride, int64_t window,
                  int64_t cache_size, int64_t page_len, int64_t seq_len,
                  int64_t cap, int64_t threads) {
    attn_ctx c;
    memset(&c, 0, sizeof(c));
    if (geometry(&c, kind, num_q, num_kv, head_dim, kv_stride, cache_size, page_len)) return -1;
    c.q = q;
    c.k = k_base;
    c.v = v_base;
    return run_dispatch(&c, kind, runs, num_runs, base_rows, out, window,
                        seq_len, cap, threads, 2);
}

int ifo_bq_attention(int64_t kind, const int32_t* runs, int64_t num_runs,
                     const int32_t* base_rows, const int8_t* q_i8,
                     const float* qi_bias, const float* f_q,
                     const int8_t* k_base, const float* k_scale,
                     const int8_t* v_base, const float* v_scale,
                     uint16_t* out, int64_t num_q, int64_t num_kv,
                     int64_t head_dim, int64_t kv_stride, int64_t window,
                     int64_t cache_size, int64_t page_len, int64_t seq_len,
                     int64_t cap, int64_t threads) {
    attn_ctx c;
    memset(&c, 0, sizeof(c));
    if (geometry(&c, kind, num_q, num_kv, head_dim, kv_stride, cache_size, page_len)) return -1;
    c.is_bq = 1;
    c.qi = q_i8;
    c.qi_bias = qi_bias;
    c.f_q = f_q;
    c.ki = k_base;
    c.k_scale = k_scale;
    c.vi = v_base;
    c.v_scale = v_scale;
    return run_dispatch(&c, kind, runs, num_runs, base_rows, out, window,
                        seq_len, cap, threads, 1);
}

/* ------------------------------------------------------------------------ */
/* MiniMax-M3 block-sparse attention (prototypes/, degree 1)                 */
/* ------------------------------------------------------------------------ */

/* The run a token belongs to, advancing `ri` as the reference's kernels do
 * (prototypes/lightning_indexer.mojo:161-169); returns the absolute position. */
static int64_t token_position(const int32_t* runs, int64_t num_runs, int64_t t,
                              int64_t* ri) {
    while (*ri + 1 < num_runs && t >= runs[4 * (*ri + 1)]) (*ri)++;
    return (int64_t)runs[4 * *ri + 1] + (t - runs[4 * *ri]);
}

/* IndexBlockScoreKernel.execute (prototypes/lightning_indexer.mojo:146-204):
 * per token, each causal position's index key is scored against every index
 * head's query (bf16_panel_dot_to_scalars, port unroll
 * pick_port_unroll(32, head_dim)), scaled, and max-folded (strict >) into its
 * block's cell, which starts at -1e30.  Rows are [token][head][block_stride]. */
void ifo_index_block_scores(const int32_t* runs, int64_t num_runs,
                            const int32_t* base_rows, const uint16_t* index_q,
                            const uint16_t* index_k, float* scores,
                            int64_t block_stride, int64_t num_heads,
                            int64_t head_dim, int64_t block_size, float scale,
                            int64_t page_len, int64_t seq_len) {
    int64_t shift = ifo_pow2_shift(page_len), row_mask = page_len - 1;
    int64_t pu = pick_port_unroll(2 * W, head_dim);
    int64_t ri = 0;
    for (int64_t t = 0; t < seq_len; t++) {
        int64_t abs_pos = token_position(runs, num_runs, t, &ri);
        if (abs_pos < 0) continue;
        int64_t nb = abs_pos / block_size + 1;
        float* tok = scores + t * num_heads * block_stride;
        for (int64_t h = 0; h < num_heads; h++)
            for (int64_t b = 0; b < nb; b++) tok[h * block_stride + b] = NEG_BIG;
        const int32_t* rows = base_rows + runs[4 * ri + 2];
        for (int64_t pos = 0; pos <= abs_pos; pos++) {
            int64_t slot = ifo_paged_slot(rows, shift, row_mask, -1, 0, pos);
            const uint16_t* kr = index_k + slot * head_dim;
            int64_t b = pos / block_size;
            for (int64_t h = 0; h < num_heads; h++) {
                float d = bf16_dot_vdpbf16(kr, index_q + (t * num_heads + h) * head_dim,
                                           head_dim, pu);
                float sh = d * scale;
                float* cell = tok + h * block_stride + b;
                if (sh > *cell) *cell = sh;
            }
        }
    }
}

/* reduce_argmax's winner (simd_math/matrixops.mojo:125-166) over a bank of
 * `cap` slots in cap/16 registers of 16 lanes: the across-register tree keeps
 * the lower register on ties, the in-lane butterfly the lower lane, so ties
 * go to the smaller lane (slot % 16), then the smaller register. */
static int64_t bank_argmax(const float* v, int64_t cap) {
    int64_t best = 0;
    for (int64_t s = 1; s < cap; s++) {
        if (v[s] > v[best]) {
            best = s;
        } else if (v[s] == v[best]) {
            int64_t ls = s % W, lb = best % W;
            if (ls < lb || (ls == lb && s / W < best / W)) best = s;
        }
    }
    return best;
}

/* reduce_top_k (matrixops.mojo:170-218): k argmax passes, each winner masked
 * to the sentinel in a copy of the bank. */
static void bank_top_k(const float* bank_v, const int32_t* bank_b, int64_t cap,
                       int64_t k, int32_t* keep_b, float* keep_v) {
    float work[256];
    for (int64_t s = 0; s < cap; s++) work[s] = bank_v[s];
    for (int64_t sel = 0; sel < k; sel++) {
        int64_t w = bank_argmax(work, cap);
        keep_v[sel] = work[w];
        keep_b[sel] = bank_b[w];
        work[w] = NEG_BIG;
    }
}

/* stream_select_blocks (prototypes/lightning_indexer.mojo:48-126) over one
 * row of block scores: blocks enter a bank of bank_cap(topk, 16) slots in
 * order (the last local_blocks and first init_blocks forced to 1e30); a full
 * bank keeps its top topk, in selection order, and refills from slot topk;
 * the final top topk with a score above -1e30 are written sorted ascending,
 * -1 padded. */
void ifo_select_blocks(const float* row_scores, int64_t num_blocks, int64_t topk,
                       int64_t local_blocks, int64_t init_blocks, int32_t* out_row) {
    int64_t cap = 1;
    while (cap < 2 * topk) cap <<= 1;
    if (cap < W) cap = W;
    float bank_v[256];
    int32_t bank_b[256], keep_b[128], ids[128];
    float keep_v[128];
    for (int64_t s = 0; s < cap; s++) {
        bank_v[s] = NEG_BIG;
        bank_b[s] = -1;
    }
    int64_t local_start = num_blocks - local_blocks;
    if (local_start < 0) local_start = 0;
    int64_t fill = 0;
    for (int64_t b = 0; b < num_blocks; b++) {
        float score = (b >= local_start || b < init_blocks) ? 1.0e30f : row_scores[b];
        bank_v[fill] = score;
        bank_b[fill] = (int32_t)b;
        fill++;
        if (fill == cap) {
            bank_top_k(bank_v, bank_b, cap, topk, keep_b, keep_v);
            for (int64_t s = 0; s < cap; s++) {
                bank_v[s] = NEG_BIG;
                bank_b[s] = -1;
            }
            for (int64_t s = 0; s < topk; s++) {
                bank_v[s] = keep_v[s];
                bank_b[s] = keep_b[s];
            }
            fill = topk;
        }
    }
    bank_top_k(bank_v, bank_b, cap, topk, keep_b, keep_v);
    int64_t n = 0;
    for (int64_t s = 0; s < topk; s++) ids[s] = -1;
    for (int64_t s = 0; s < topk; s++)
        if (keep_v[s] > NEG_BIG) ids[n++] = keep_b[s];
    for (int64_t i = 1; i < n; i++) {
        int32_t v = ids[i];
        int64_t j = i - 1;
        while (j >= 0 && ids[j] > v) {
            ids[j + 1] = ids[j];
            j--;
        }
        ids[j + 1] = v;
    }
    for (int64_t s = 0; s < topk; s++) out_row[s] = ids[s];
}

/* dispatch_lightning_indexer (prototypes/lightning_indexer.mojo:399-443) at
 * degree 1: block scores, then IndexTopkMergeKernel (:253-303) per (token,
 * head) row.  The reference's merge takes every token's position from the
 * first run (base_pos + t, :420 and :278, a one-sequence prototype); here each token's
 * own run gives it, which is the same for one run. */
void ifo_lightning_indexer(const int32_t* runs, int64_t num_runs,
                           const int32_t* base_rows, const uint16_t* index_q,
                           const uint16_t* index_k, int32_t* block_idx,
                           float* scores, int64_t block_stride, int64_t num_heads,
                           int64_t head_dim, int64_t block_size, int64_t topk,
                           int64_t local_blocks, int64_t init_blocks, float scale,
                           int64_t page_len, int64_t seq_len) {
    ifo_index_block_scores(runs, num_runs, base_rows, index_q, index_k, scores,
                           block_stride, num_heads, head_dim, block_size, scale,
                           page_len, seq_len);
    int64_t ri = 0;
    for (int64_t t = 0; t < seq_len; t++) {
        int64_t abs_pos = token_position(runs, num_runs, t, &ri);
        if (abs_pos < 0) continue;
        int64_t nb = abs_pos / block_size + 1;
        for (int64_t h = 0; h < num_heads; h++)
            ifo_select_blocks(scores + (t * num_heads + h) * block_stride, nb, topk,
                              local_blocks, init_blocks,
                              block_idx + (t * num_heads + h) * topk);
    }
}

/* BlockSparseFlashKernel.execute (prototypes/sparse_attention.mojo:59-131) at
 * degree 1: per token and kv head, the selected blocks in order (stopping at
 * the first -1), each clipped to the causal count and walked in 16-position
 * process_kv_tile steps from its first position over the head's gqa q heads;
 * then PrefillMergeKernel (kernels/flash_attention_prefill.mojo:221-240):
 * write_finalized_head over the token's one stripe. */
int ifo_block_sparse_attention(const int32_t* runs, int64_t num_runs,
                               const int32_t* base_rows, const uint16_t* q,
                               const uint16_t* k_base, const uint16_t* v_base,
                               const int32_t* block_idx, uint16_t* out,
                               int64_t num_q, int64_t num_kv, int64_t head_dim,
                               int64_t kv_stride, int64_t block_size, int64_t topk,
                               int64_t page_len, int64_t seq_len) {
    if (num_q <= 0 || num_kv <= 0 || num_q % num_kv != 0 || num_q > 64) return -1;
    if (head_dim % (2 * W) != 0 || head_dim > 512) return -1;
    if (page_len <= 0 || (page_len & (page_len - 1)) != 0) return -1;
    int64_t D = head_dim, gqa = num_q / num_kv;
    int64_t stride = ifo_flash_partial_stride(num_q, D);
    float* part = (float*)calloc((size_t)stride, sizeof(float));
    float* acc = (float*)malloc(sizeof(float) * (size_t)(gqa * D));
    attn_ctx c;
    memset(&c, 0, sizeof(c));
    c.num_q = gqa;
    c.num_kv = 1;
    c.gqa = gqa;
    c.head_dim = D;
    c.kv_stride = kv_stride;
    c.shift = ifo_pow2_shift(page_len);
    c.row_mask = page_len - 1;
    c.page_mask = -1;
    c.q = q;
    int64_t ri = 0;
    for (int64_t t = 0; t < seq_len; t++) {
        int64_t abs_pos = token_position(runs, num_runs, t, &ri);
        if (abs_pos < 0) continue;
        int64_t cap = abs_pos + 1;   /* full_local_kv_count(0, abs_pos, 1) */
        attn_item it = {t, base_rows + runs[4 * ri + 2], 0, 0, 0, 0};
        for (int64_t h = 0; h < num_kv; h++) {
            float m[64], l[64];
            int64_t q_off[64];
            for (int64_t r = 0; r < gqa; r++) {
                m[r] = NEG_BIG;
                l[r] = 0.0f;
                q_off[r] = (t * num_q + h * gqa + r) * D;
            }
            memset(acc, 0, sizeof(float) * (size_t)(gqa * D));
            c.k = k_base + h * D;
            c.v = v_base + h * D;
            const int32_t* row = block_idx + (t * num_kv + h) * topk;
            for (int64_t s = 0; s < topk; s++) {
                int64_t b = row[s];
                if (b < 0) break;
                int64_t plo = b * block_size;
                int64_t phi = (b + 1) * block_size;
                if (phi > cap) phi = cap;
                for (int64_t pos = plo; pos < phi; pos += TILE) {
                    int64_t tl = phi - pos < TILE ? phi - pos : TILE;
                    process_tile(&c, &it, q_off, pos, tl, m, l, acc);
                }
            }
            for (int64_t r = 0; r < gqa; r++) {
                int64_t qh = h * gqa + r;
                memcpy(part + qh * D, acc + r * D, sizeof(float) * (size_t)D);
                part[num_q * D + qh] = m[r];
                part[num_q * D + num_q + qh] = l[r];
            }
        }
        for (int64_t qh = 0; qh < num_q; qh++)
            ifo_finalize_head(out + (t * num_q + qh) * D, part, stride, 1, num_q, D, qh);
    }
    free(part);
    free(acc);
    return 0;
}

/* One (kv head h, slots [s0, s1)) pass of the bq block-sparse kernels over
 * the head's gqa q heads, into acc (gqa x D) and m, l (gqa): tiles of each
 * block in slot order through bq_process_kv_tile_head
 * (prototypes/bq_sparse_attention.mojo:29-91, the bq branch of process_tile).
 * A slot holding -1 ends the list (stop_at_neg) or is skipped. */
static void bq_sparse_pass(attn_ctx* c, const int32_t* rows, const int8_t* q_i8,
                           const float* qi_bias, const float* f_q, const int8_t* k_base,
                           const float* k_scale, const int8_t* v_base,
                           const float* v_scale, const int32_t* brow, int64_t t,
                           int64_t h, int64_t num_q, int64_t s0, int64_t s1,
                           int stop_at_neg, int64_t block_size, int64_t cap,
                           float* m, float* l, float* acc) {
    int64_t D = c->head_dim, gqa = c->gqa;
    int64_t q_off[64];
    for (int64_t r = 0; r < gqa; r++) {
        m[r] = NEG_BIG;
        l[r] = 0.0f;
        q_off[r] = (t * num_q + h * gqa + r) * D;
    }
    memset(acc, 0, sizeof(float) * (size_t)(gqa * D));
    c->qi = q_i8;
    c->qi_bias = qi_bias + t * num_q + h * gqa;   /* indexed [0 * gqa + r] */
    c->f_q = f_q + t * num_q + h * gqa;
    c->ki = k_base + h * D;
    c->vi = v_base + h * D;
    c->k_scale = k_scale + h;                    /* indexed [slot * num_kv + 0] */
    c->v_scale = v_scale + h;
    attn_item it = {0, rows, 0, 0, 0, 0};
    for (int64_t s = s0; s < s1; s++) {
        int64_t b = brow[s];
        if (b < 0) {
            if (stop_at_neg) break;
            continue;
        }
        int64_t plo = b * block_size;
        int64_t phi = (b + 1) * block_size;
        if (phi > cap) phi = cap;
        for (int64_t pos = plo; pos < phi; pos += TILE) {
            int64_t tl = phi - pos < TILE ? phi - pos : TILE;
            process_tile(c, &it, q_off, pos, tl, m, l, acc);
        }
    }
}

/* dispatch_bq_block_sparse_attention (prototypes/bq_sparse_attention.mojo:
 * 366-451) at degree 1.  seq_len > 1: BqBlockSparseFlashKernel (:94-200), one
 * stripe per token over its blocks in order, finalized by
 * PrefillMergeKernel.  seq_len == 1: BqBlockSparseFlashDecodeKernel
 * (:254-364): the num_kv * min(topk, causal blocks) (kv head, slot) units are
 * banded over min(cap, units) workers by worker_range (tile_dispatch,
 * kernels/helpers.mojo:264-282, saturate_workers), each worker writing one
 * stripe (untouched heads keep m = -1e30, l = 0), and the stripes merged per
 * head by write_finalized_head (dispatch_merge_context_flash_partials,
 * kernels/logsum_merge.mojo:251-292). */
int ifo_bq_block_sparse_attention(const int32_t* runs, int64_t num_runs,
                                  const int32_t* base_rows, const int8_t* q_i8,
                                  const float* qi_bias, const float* f_q,
                                  const int8_t* k_base, const float* k_scale,
                                  const int8_t* v_base, const float* v_scale,
                                  const int32_t* block_idx, uint16_t* out,
                                  int64_t num_q, int64_t num_kv, int64_t head_dim,
                                  int64_t kv_stride, int64_t block_size, int64_t topk,
                                  int64_t page_len, int64_t seq_len, int64_t cap) {
    if (num_q <= 0 || num_kv <= 0 || num_q % num_kv != 0 || num_q > 64) return -1;
    if (head_dim % (2 * W) != 0 || head_dim > 512) return -1;
    if (page_len <= 0 || (page_len & (page_len - 1)) != 0) return -1;
    if (seq_len <= 0 || cap < 1) return seq_len <= 0 ? 0 : -1;
    int64_t D = head_dim, gqa = num_q / num_kv;
    int64_t stride = ifo_flash_partial_stride(num_q, D);
    attn_ctx c;
    memset(&c, 0, sizeof(c));
    c.is_bq = 1;
    c.num_q = gqa;
    c.num_kv = num_kv;
    c.gqa = gqa;
    c.head_dim = D;
    c.kv_stride = kv_stride;
    c.shift = ifo_pow2_shift(page_len);
    c.row_mask = page_len - 1;
    c.page_mask = -1;
    float* acc = (float*)malloc(sizeof(float) * (size_t)(gqa * D));
    float m[64], l[64];
    if (seq_len == 1) {
        int64_t abs_pos = runs[1];
        if (abs_pos < 0) {
            free(acc);
            return 0;
        }
        int64_t causal = abs_pos / block_size + 1;
        int64_t pqb = topk < causal ? topk : causal;
        int64_t total = num_kv * pqb;
        int64_t workers = cap < total ? cap : total;
        float* part = (float*)calloc((size_t)(workers * stride), sizeof(float));
        const int32_t* rows = base_rows + runs[2];
        for (int64_t w = 0; w < workers; w++) {
            float* pw = part + w * stride;
            for (int64_t gh = 0; gh < num_q; gh++) {
                pw[num_q * D + gh] = NEG_BIG;
                pw[num_q * D + num_q + gh] = 0.0f;
            }
            int64_t wr[2];
            ifo_worker_range(total, workers, w, 0, wr);
            if (wr[0] >= wr[1]) continue;
            int64_t h0 = wr[0] / pqb, h1 = (wr[1] - 1) / pqb;
            for (int64_t h = h0; h <= h1; h++) {
                int64_t lo = (wr[0] > h * pqb ? wr[0] : h * pqb) - h * pqb;
                int64_t hi = (wr[1] < (h + 1) * pqb ? wr[1] : (h + 1) * pqb) - h * pqb;
                bq_sparse_pass(&c, rows, q_i8, qi_bias, f_q, k_base, k_scale, v_base,
                               v_scale, block_idx + h * topk, 0, h, num_q, lo, hi, 0,
                               block_size, abs_pos + 1, m, l, acc);
                for (int64_t r = 0; r < gqa; r++) {
                    int64_t gh = h * gqa + r;
                    memcpy(pw + gh * D, acc + r * D, sizeof(float) * (size_t)D);
                    pw[num_q * D + gh] = m[r];
                    pw[num_q * D + num_q + gh] = l[r];
                }
            }
        }
        for (int64_t gh = 0; gh < num_q; gh++)
            ifo_finalize_head(out + gh * D, part, stride, workers, num_q, D, gh);
        free(part);
        free(acc);
        return 0;
    }
    float* part = (float*)calloc((size_t)stride, sizeof(float));
    int64_t ri = 0;
    for (int64_t t = 0; t < seq_len; t++) {
        int64_t abs_pos = token_position(runs, num_runs, t, &ri);
        if (abs_pos < 0) continue;
        const int32_t* rows = base_rows + runs[4 * ri + 2];
        for (int64_t h = 0; h < num_kv; h++) {
            bq_sparse_pass(&c, rows, q_i8, qi_bias, f_q, k_base, k_scale, v_base, v_scale,
                           block_idx + (t * num_kv + h) * topk, t, h, num_q, 0, topk, 1,
                           block_size, abs_pos + 1, m, l, acc);
            for (int64_t r = 0; r < gqa; r++) {
                int64_t gh = h * gqa + r;
                memcpy(part + gh * D, acc + r * D, sizeof(float) * (size_t)D);
                part[num_q * D + gh] = m[r];
                part[num_q * D + num_q + gh] = l[r];
            }
        }
        for (int64_t gh = 0; gh < num_q; gh++)
            ifo_finalize_head(out + (t * num_q + gh) * D, part, stride, 1, num_q, D, gh);
    }
    free(part);
    free(acc);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* KV append: RopeCacheWriteKernel (kernels/rope.mojo:16-125)                */
/* ------------------------------------------------------------------------ */

static void rotate_pair_to(const uint16_t* src, uint16_t* dst,
                           const float* cos_row, const float* sin_row,
                           int64_t half, int64_t pair_stride) {
    for (int64_t j = 0; j < half; j++) {
        float x_lo = ifo_bf16_to_f32(src[j]);
        float x_hi = ifo_bf16_to_f32(src[pair_stride + j]);
        float cv = cos_row[j], sv = sin_row[j];
        float a = x_lo * cv, b = x_hi * sv;
        float c = x_hi * cv, d = x_lo * sv;
        dst[j] = ifo_f32_to_bf16(a - b);
        dst[pair_stride + j] = ifo_f32_to_bf16(c + d);
    }
}

/* rms_norm_row over one head (kernels/rmsnorm.mojo:15-48) as
 * ScaledNormKernel applies it per head row (:130-153):
 *   sum_sq = dot_to_scalar[head_dim](x, x) (kernels/dot_products.mojo:
 *     181-191): VDPBF16PS into pick_port_unroll(32, head_dim) accumulators
 *     of 16 lanes, the accumulators added in order per lane
 *     (panel_accs_to_scalars), then the halving-tree reduce_add;
 *   inv = sqrt_n / sqrt(sum_sq + n_eps);
 *   y = bf16((x * inv) * w)  (scaled: q and k heads), bf16(x * inv) (v). */
static void rms_norm_head(uint16_t* row, const uint16_t* w, int64_t head_dim,
                          float sqrt_n, float n_eps) {
    int64_t pu = pick_port_unroll(2 * W, head_dim);
    float ssq = bf16_dot_vdpbf16(row, row, head_dim, pu);
    float inv = sqrt_n / sqrtf(ssq + n_eps);
    for (int64_t e = 0; e < head_dim; e++) {
        float x = ifo_bf16_to_f32(row[e]);
        float y = x * inv;
        if (w) y = y * ifo_bf16_to_f32(w[e]);
        row[e] = ifo_f32_to_bf16(y);
    }
}

/* dispatch_rms_norm_qkv_heads (kernels/rmsnorm.mojo:168-215), in place:
 * q heads and k heads with their gains, v heads unscaled. */
void ifo_rms_norm_qkv_heads(uint16_t* q, uint16_t* k, uint16_t* v,
                            const uint16_t* q_weight, const uint16_t* k_weight,
                            int64_t num_q, int64_t num_kv, int64_t seq_len,
                            int64_t head_dim, float sqrt_n, float n_eps) {
    for (int64_t t = 0; t < seq_len; t++) {
        for (int64_t h = 0; h < num_q; h++)
            rms_norm_head(q + (t * num_q + h) * head_dim, q_weight, head_dim, sqrt_n, n_eps);
        for (int64_t h = 0; h < num_kv; h++) {
            rms_norm_head(k + (t * num_kv + h) * head_dim, k_weight, head_dim, sqrt_n, n_eps);
            rms_norm_head(v + (t * num_kv + h) * head_dim, NULL, head_dim, sqrt_n, n_eps);
        }
    }
}

void ifo_rope_cache_write(const int32_t* runs, int64_t num_runs,
                          const int32_t* base_rows, uint16_t* q,
                          const uint16_t* k_src, const uint16_t* v_src,
                          uint16_t* k_cache, uint16_t* v_cache,
                          const float* cos_table, const float* sin_table,
                          int64_t num_q, int64_t num_kv, int64_t cache_degree,
                          int64_t rank, int64_t page_shift, int64_t row_mask,
                          int64_t page_mask, int64_t seq_len, int64_t half,
                          int64_t pair_stride, int64_t head_dim) {
    if (seq_len <= 0 || num_runs <= 0) return;
    int64_t q_stride = num_q * head_dim;
    int64_t kv_stride = num_kv * head_dim;
    int64_t r = 0;
    for (int64_t tok = 0; tok < seq_len; tok++) {
        while (r + 1 < num_runs && tok >= runs[4 * (r + 1)]) r++;
        int64_t pos = runs[4 * r + 1] + (tok - runs[4 * r]);
        const float* cos_row = cos_table + pos * half;
        const float* sin_row = sin_table + pos * half;
        uint16_t* q_tok = q + tok * q_stride;
        for (int64_t h = 0; h < num_q; h++)
            rotate_pair_to(q_tok + h * head_dim, q_tok + h * head_dim, cos_row,
                           sin_row, half, pair_stride);
        if (pos % cache_degree == rank) {
            const int32_t* rows = base_rows + runs[4 * r + 2];
            int64_t slot = ifo_paged_slot(rows, page_shift, row_mask, page_mask,
                                          0, pos / cache_degree);
            const uint16_t* k_tok = k_src + tok * kv_stride;
            uint16_t* k_dst = k_cache + slot * kv_stride;
            for (int64_t h = 0; h < num_kv; h++) {
                const uint16_t* s = k_tok + h * head_dim;
                uint16_t* d = k_dst + h * head_dim;
                rotate_pair_to(s, d, cos_row, sin_row, half, pair_stride);
                if (half < pair_stride)
                    memcpy(d + half, s + half, sizeof(uint16_t) * (size_t)(pair_stride - half));
                if (pair_stride + half < head_dim)
                    memcpy(d + pair_stride + half, s + pair_stride + half,
                           sizeof(uint16_t) * (size_t)(head_dim - pair_stride - half));
            }
            memcpy(v_cache + slot * kv_stride, v_src + tok * kv_stride,
                   sizeof(uint16_t) * (size_t)kv_stride);
        }
    }
}

/* PageCopyKernel / dispatch_copy_jobs (kernels/page_copy.mojo:25-94): the
 * byte ranges of all jobs are copied; the worker split does not change the
 * result for non-overlapping jobs. */
void ifo_copy_jobs(uint8_t* arena, const int64_t* jobs, int64_t num_jobs) {
    for (int64_t i = 0; i < num_jobs; i++)
        memcpy(arena + jobs[3 * i + 1], arena + jobs[3 * i + 0], (size_t)jobs[3 * i + 2]);
}

/* GatherRowsKernel (kernels/gather.mojo:8-27). */
void ifo_gather_rows(const uint16_t* src, uint16_t* dst, const int32_t* rows,
                     int64_t num_rows, int64_t cols) {
    for (int64_t j = 0; j < num_rows; j++)
        memcpy(dst + j * cols, src + (int64_t)rows[j] * cols, sizeof(uint16_t) * (size_t)cols);
}

/* The reference's fanned-out forms: dispatch_copy_jobs
 * (kernels/page_copy.mojo:63-94) cuts the concatenated jobs' byte range
 * [0, total) into `workers` worker_range shares whose ends are rounded up to
 * 64 bytes (align_split, :18-22), and each PageCopyKernel (:25-60) copies its
 * share job segment by job segment; dispatch_gather_rows (gather.mojo:30-55)
 * gives each worker a worker_range share of the rows.  The shares run on
 * `threads` threads; the bytes written are those of the one-thread forms. */
typedef struct {
    uint8_t* arena;
    const int64_t* jobs;
    const int64_t* bounds;
    int64_t num_jobs, workers;
    const uint16_t* src;
    uint16_t* dst;
    const int32_t* rows;
    int64_t num_rows, cols;
    atomic_llong next;
} share_pool;

static int64_t align_split64(int64_t offset, int64_t total) {
    int64_t a = (offset + 63) / 64 * 64;
    return a < total ? a : total;
}

static void copy_share(share_pool* p, int64_t w) {
    int64_t total = p->bounds[p->num_jobs];
    int64_t wr[2];
    ifo_worker_range(total, p->workers, w, 0, wr);
    int64_t lo = align_split64(wr[0], total), hi = align_split64(wr[1], total);
    if (lo >= hi) return;
    int64_t j = 0;
    while (p->bounds[j + 1] <= lo) j++;
    for (int64_t cursor = lo; cursor < hi; j++) {
        int64_t seg_end = p->bounds[j + 1] < hi ? p->bounds[j + 1] : hi;
        int64_t off = cursor - p->bounds[j];
        memcpy(p->arena + p->jobs[3 * j + 1] + off, p->arena + p->jobs[3 * j + 0] + off,
               (size_t)(seg_end - cursor));
        cursor = seg_end;
    }
}

static void gather_share(share_pool* p, int64_t w) {
    int64_t wr[2];
    ifo_worker_range(p->num_rows, p->workers, w, 0, wr);
    for (int64_t j = wr[0]; j < wr[1]; j++)
        memcpy(p->dst + j * p->cols, p->src + (int64_t)p->rows[j] * p->cols,
               sizeof(uint16_t) * (size_t)p->cols);
}

static void* copy_share_worker(void* arg) {
    share_pool* p = (share_pool*)arg;
    for (long long w; (w = atomic_fetch_add(&p->next, 1)) < p->workers;) copy_share(p, w);
    return NULL;
}

static void* gather_share_worker(void* arg) {
    share_pool* p = (share_pool*)arg;
    for (long long w; (w = atomic_fetch_add(&p->next, 1)) < p->workers;) gather_share(p, w);
    return NULL;
}

static void run_shares(share_pool* p, void* (*fn)(void*), int64_t threads) {
    atomic_init(&p->next, 0);
    if (threads > p->workers) threads = p->workers;
    if (threads <= 1) {
        fn(p);
        return;
    }
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int64_t t = 1; t < threads; t++) pthread_create(&tids[t], NULL, fn, p);
    fn(p);
    for (int64_t t = 1; t < threads; t++) pthread_join(tids[t], NULL);
    free(tids);
}

void ifo_copy_jobs_workers(uint8_t* arena, const int64_t* jobs, int64_t num_jobs,
                           int64_t workers, int64_t threads) {
    if (num_jobs <= 0 || workers <= 0) return;
    int64_t* bounds = (int64_t*)malloc(sizeof(int64_t) * (size_t)(num_jobs + 1));
    bounds[0] = 0;
    for (int64_t i = 0; i < num_jobs; i++) bounds[i + 1] = bounds[i] + jobs[3 * i + 2];
    if (bounds[num_jobs] > 0) {
        share_pool p;
        memset(&p, 0, sizeof(p));
        p.arena = arena;
        p.jobs = jobs;
        p.bounds = bounds;
        p.num_jobs = num_jobs;
        p.workers = workers;
        run_shares(&p, copy_share_worker, threads);
    }
    free(bounds);
}

void ifo_gather_rows_workers(const uint16_t* src, uint16_t* dst, const int32_t* rows,
                             int64_t num_rows, int64_t cols, int64_t workers,
                             int64_t threads) {
    if (num_rows <= 0 || workers <= 0) return;
    share_pool p;
    memset(&p, 0, sizeof(p));
    p.src = src;
    p.dst = dst;
    p.rows = rows;
    p.num_rows = num_rows;
    p.cols = cols;
    p.workers = workers;
    run_shares(&p, gather_share_worker, threads);
}

/* ------------------------------------------------------------------------ */
/* butterquant head prep (butterquant/fwht.mojo, head_prep.mojo,             */
/* simd_math/ops.mojo:25-31, butterquant_kernels/attention.mojo:494-632)     */
/* ------------------------------------------------------------------------ */

/* fwht_apply (butterquant/fwht.mojo:20-57): strides 1, 2, ..., n/2; the
 * lower index of each pair becomes a+b and the upper a-b; then x 1/sqrt(n). */
void ifo_fwht(float* v, int64_t n) {
    for (int64_t stride = 1; stride < n; stride <<= 1) {
        for (int64_t i = 0; i < n; i++) {
            if (i & stride) continue;
            float a = v[i], b = v[i + stride];
            v[i] = a + b;
            v[i + stride] = a - b;
        }
    }
    float sq = sqrtf((float)n);
    float sc = (float)(1.0 / (double)sq);
    for (int64_t i = 0; i < n; i++) v[i] = v[i] * sc;
}

/* head_inv_rms (butterquant/head_prep.mojo:9-16): lane-wise FMA chain over
 * n/16 registers of 16 lanes, then the 16-lane tree sum. */
float ifo_head_inv_rms(const float* x, int64_t n, float sqrt_n, float n_eps) {
    int64_t width = n < W ? n : W;
    int64_t regs = n / width;
    float ssq[W];
    for (int64_t j = 0; j < W; j++) ssq[j] = 0.0f;
    for (int64_t j = 0; j < width; j++) ssq[j] = x[j] * x[j];
    for (int64_t ri = 1; ri < regs; ri++)
        for (int64_t j = 0; j < width; j++)
            ssq[j] = fmaf(x[ri * width + j], x[ri * width + j], ssq[j]);
    float total = ifo_tree_sum16(ssq);
    return sqrt_n / sqrtf(total + n_eps);
}

/* absmax_quantize_head (butterquant/head_prep.mojo:19-36) with quantize_i8
 * (simd_math/ops.mojo:25-31): roundeven, clamp [-128, 127]. */
float ifo_absmax_quantize(const float* x, int64_t n, int8_t* out,
                          int32_t* qsum) {
    float amax = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    if (amax < 1e-10f) amax = 1e-10f;
    float inv = 127.0f / amax;
    int32_t s = 0;
    for (int64_t i = 0; i < n; i++) {
        float v = nearbyintf(x[i] * inv);
        if (v < -128.0f) v = -128.0f;
        if (v > 127.0f) v = 127.0f;
        out[i] = (int8_t)v;
        s += (int32_t)out[i];
    }
    if (qsum) *qsum = s;
    return amax;
}

/* dispatch_gemm_cols[rows] (kernels/gemm.mojo:198-225): GemmColKernel over
 * bf16_microtile_runtime (kernels/panel.mojo:85-133).  Each (token, column)
 * has one W-lane f32 accumulator fed by VDPBF16PS over 32-element chunks of
 * the contraction (bf16_pair_dot, kernels/dot_products.mojo:10-35), lanes
 * reduced by the halving tree, then a scalar tail over cols % 32 added, and
 * the f32 sum cast to bf16 (emit_gemm_col_panel, gemm.mojo:122-150). */
void ifo_gemm_cols(const uint16_t* x, const uint16_t* w, uint16_t* out,
                   int64_t rows, int64_t cols, int64_t seq_len) {
    int64_t body = cols - cols % (2 * W);
    for (int64_t m = 0; m < seq_len; m++) {
        const uint16_t* xr = x + m * cols;
        for (int64_t n = 0; n < rows; n++) {
            const uint16_t* wr = w + n * cols;
            float v = bf16_dot_vdpbf16(wr, xr, body, 1);
            if (body < cols) {
                float tail = 0.0f;
                for (int64_t k = body; k < cols; k++)
                    tail = tail + ifo_bf16_to_f32(xr[k]) * ifo_bf16_to_f32(wr[k]);
                v = v + tail;
            }
            out[m * rows + n] = ifo_f32_to_bf16(v);
        }
    }
}

/* dispatch_bq_block_quant[apply_fwht=False] (butterquant_kernels/linear.mojo:
 * 151-206): per token, prepare_block_activation (butterquant/runtime.mojo:
 * 63-80) widens the bf16 row to f32 and quantize_activation_per_block
 * (butterquant/quantize.mojo:13-23) runs quant_segment[store_divided=False]
 * (butterquant/kernels.mojo:83-92) on each block: sa = amax (row_absmax
 * :63-70), inv = 127/amax or 0, code = quantize_i8 (simd_math/ops.mojo:26-31)
 * = clamp(roundeven(x * inv), -128, 127). */
void ifo_bq_block_quant(const uint16_t* src, int8_t* x_i8, float* x_sa,
                        int64_t cols, int64_t block, int64_t seq_len) {
    int64_t nb = cols / block;
    for (int64_t t = 0; t < seq_len; t++) {
        for (int64_t b = 0; b < nb; b++) {
            const uint16_t* s = src + t * cols + b * block;
            int8_t* d = x_i8 + t * cols + b * block;
            float amax = 0.0f;
            for (int64_t i = 0; i < block; i++) {
                float a = fabsf(ifo_bf16_to_f32(s[i]));
                amax = a > amax ? a : amax;
            }
            x_sa[t * nb + b] = amax;
            float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            for (int64_t i = 0; i < block; i++) {
                float r = rintf(ifo_bf16_to_f32(s[i]) * inv);
                r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
                d[i] = (int8_t)(int32_t)r;
            }
        }
    }
}

/* prep_head_qk_i8 (butterquant/head_prep.mojo:39-70). */
static float prep_head_qk(const uint16_t* src, const uint16_t* gamma,
                          const float* cos_row, const float* sin_row,
                          int8_t* out, int32_t* qsum, int64_t D,
                          int64_t rope_half, int64_t pair_stride,
                          float sqrt_n, float n_eps) {
    float r[512] = {0};
    for (int64_t i = 0; i < D; i++) r[i] = ifo_bf16_to_f32(src[i]);
    float inv_rms = ifo_head_inv_rms(r, D, sqrt_n, n_eps);
    for (int64_t i = 0; i < D; i++) {
        float g = ifo_bf16_to_f32(gamma[i]);
        float t = r[i] * inv_rms;
        r[i] = t * g;
    }
    for (int64_t j = 0; j < rope_half; j++) {
        float x_lo = r[j], x_hi = r[pair_stride + j];
        float cv = cos_row[j], sv = sin_row[j];
        float a = x_lo * cv, b = x_hi * sv;
        float c = x_hi * cv, d = x_lo * sv;
        r[j] = a - b;
        r[pair_stride + j] = c + d;
    }
    ifo_fwht(r, D);
    return ifo_absmax_quantize(r, D, out, qsum);
}

/* prep_head_v_i8 (butterquant/head_prep.mojo:73-87). */
static float prep_head_v(const uint16_t* src, int8_t* out, int64_t D) {
    float r[512];
    for (int64_t i = 0; i < D; i++) r[i] = ifo_bf16_to_f32(src[i]);
    ifo_fwht(r, D);
    return ifo_absmax_quantize(r, D, out, NULL);
}

/* BqAttnPrepKernel.execute (butterquant_kernels/attention.mojo:524-577). */
void ifo_bq_attn_prep(const int32_t* runs, int64_t num_runs,
                      const int32_t* base_rows, const uint16_t* q_src,
                      const uint16_t* k_src, const uint16_t* v_src,
                      const uint16_t* q_norm, const uint16_t* k_norm,
                      int8_t* q_i8, float* qi_bias, float* f_q,
                      int8_t* k_cache, float* k_scale, int8_t* v_cache,
                      float* v_scale, const float* cos_table,
                      const float* sin_table, int64_t num_q, int64_t num_kv,
                      int64_t cache_degree, int64_t rank, int64_t page_shift,
                      int64_t row_mask, int64_t page_mask, int64_t seq_len,
                      int64_t head_dim, int64_t rope_half,
                      int64_t pair_stride, float sqrt_n, float n_eps) {
    if (seq_len <= 0 || num_runs <= 0 || head_dim > 512) return;
    int64_t q_stride = num_q * head_dim;
    int64_t kv_stride = num_kv * head_dim;
    int64_t r = 0;
    float inv_sqrt_n = 1.0f / sqrt_n;
    for (int64_t tok = 0; tok < seq_len; tok++) {
        while (r + 1 < num_runs && tok >= runs[4 * (r + 1)]) r++;
        int64_t pos = runs[4 * r + 1] + (tok - runs[4 * r]);
        const float* cos_row = cos_table + pos * rope_half;
        const float* sin_row = sin_table + pos * rope_half;
        for (int64_t h = 0; h < num_q; h++) {
            int32_t qs = 0;
            float amax = prep_head_qk(q_src + tok * q_stride + h * head_dim, q_norm,
                                      cos_row, sin_row,
                                      q_i8 + tok * q_stride + h * head_dim, &qs,
                                      head_dim, rope_half, pair_stride, sqrt_n, n_eps);
            qi_bias[tok * num_q + h] = (float)qs * 128.0f;
            f_q[tok * num_q + h] = amax * inv_sqrt_n;
        }
        if (pos % cache_degree == rank) {
            const int32_t* rows = base_rows + runs[4 * r + 2];
            int64_t slot = ifo_paged_slot(rows, page_shift, row_mask, page_mask,
                                          0, pos / cache_degree);
            for (int64_t h = 0; h < num_kv; h++) {
                int32_t ks_unused = 0;
                k_scale[slot * num_kv + h] = prep_head_qk(
                    k_src + tok * kv_stride + h * head_dim, k_norm, cos_row, sin_row,
                    k_cache + slot * kv_stride + h * head_dim, &ks_unused,
                    head_dim, rope_half, pair_stride, sqrt_n, n_eps);
                v_scale[slot * num_kv + h] = prep_head_v(
                    v_src + tok * kv_stride + h * head_dim,
                    v_cache + slot * kv_stride + h * head_dim, head_dim);
            }
        }
    }
}
