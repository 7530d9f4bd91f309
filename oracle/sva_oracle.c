/*
 * sva_oracle.c -- CPU restatement of the SVA summon -> verify decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP path is
 * compared against; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Nothing in the shipped package links it.
 *
 * Every fp32 operation below is written with an explicit evaluation order so
 * that a GPU kernel following the same order reproduces it bit for bit:
 *
 *   projection / LUT dot products   sequential fmaf chain over the inner dim,
 *                                   starting from +0 (what MKL's sgemm does for
 *                                   the many-row products in sva/llama.py:615
 *                                   and sva/ops.py:19; verified bit-exact)
 *   torch.sum(dim=-1)               8-lane vectors, 4 interleaved accumulators,
 *                                   cascade levels, scalar tail, then lanes in
 *                                   order (torch's CPU cascade sum; verified
 *                                   bit-exact against torch 2.10 on fp32)
 *   PQ scan score                   ((0 + T_0[c_0]) + T_1[c_1]) + ... then / sqrt(R)
 *                                   (sva/ops.py:64-71)
 *   selection                       top-k by (score desc, key index asc)
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* order-preserving float key: a > b  <=>  key(a) > key(b); -0 folds onto +0 */
static inline uint32_t f2key(float x) {
    x = x + 0.0f;
    uint32_t u;
    memcpy(&u, &x, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

ORACLE_API uint32_t sva_oracle_float_key(float x) { return f2key(x); }

/* ------------------------------------------------------------------------ */
/* torch.sum(dim=-1) over a contiguous fp32 row (used by sva/ops.py:17-19 and
 * sva/llama.py:292, :495 for the rank scores).  Mirrors torch's CPU cascade
 * sum: the row is read as 8-float vectors grouped in rows of 4 (ILP 4); the
 * row sums are accumulated with a 4-level cascade whose level width is
 * 2^max(4, ceil(log2(rows))/4); leftover vectors go to accumulator 0; the 4
 * accumulators are folded in order; the scalar tail is summed first, then the
 * 8 lanes in order. */
static int64_t ceil_log2(int64_t x) {
    if (x <= 2) return x == 2 ? 1 : 0;
    int64_t r = 0;
    int64_t v = x - 1;
    while (v) { r++; v >>= 1; }
    return r;
}

static float torch_sum_f32(const float *x, int64_t k) {
    enum { W = 8, ILP = 4, LEVELS = 4 };
    const int64_t nvec = k / W;
    const int64_t rows = nvec / ILP;
    float acc[LEVELS][ILP][W];
    memset(acc, 0, sizeof(acc));
    const int64_t level_power = (ceil_log2(rows) / LEVELS) > 4 ? (ceil_log2(rows) / LEVELS) : 4;
    const int64_t level_step = (int64_t)1 << level_power;
    const int64_t level_mask = level_step - 1;
    int64_t i = 0;
    for (; i + level_step <= rows;) {
        for (int64_t j = 0; j < level_step; ++j, ++i) {
            for (int a = 0; a < ILP; ++a)
                for (int l = 0; l < W; ++l) acc[0][a][l] = acc[0][a][l] + x[(i * ILP + a) * W + l];
        }
        for (int j = 1; j < LEVELS; ++j) {
            for (int a = 0; a < ILP; ++a)
                for (int l = 0; l < W; ++l) {
                    acc[j][a][l] = acc[j][a][l] + acc[j - 1][a][l];
                    acc[j - 1][a][l] = 0.0f;
                }
            const int64_t mask = level_mask << (j * level_power);
            if ((i & mask) != 0) break;
        }
    }
    for (; i < rows; ++i)
        for (int a = 0; a < ILP; ++a)
            for (int l = 0; l < W; ++l) acc[0][a][l] = acc[0][a][l] + x[(i * ILP + a) * W + l];
    for (int j = 1; j < LEVELS; ++j)
        for (int a = 0; a < ILP; ++a)
            for (int l = 0; l < W; ++l) acc[0][a][l] = acc[0][a][l] + acc[j][a][l];
    float part[ILP][W];
    memcpy(part, acc[0], sizeof(part));
    for (int64_t v = rows * ILP; v < nvec; ++v)
        for (int l = 0; l < W; ++l) part[0][l] = part[0][l] + x[v * W + l];
    for (int a = 1; a < ILP; ++a)
        for (int l = 0; l < W; ++l) part[0][l] = part[0][l] + part[a][l];
    float total = 0.0f;
    for (int64_t t = nvec * W; t < k; ++t) total = total + x[t];
    for (int l = 0; l < W; ++l) total = total + part[0][l];
    return total;
}

ORACLE_API float sva_oracle_torch_sum(const float *x, int64_t k) { return torch_sum_f32(x, k); }

/* torch_sum of the elementwise products a*b (each product rounded to fp32). */
static float torch_dot_f32(const float *a, const float *b, int64_t k) {
    if (k <= 0) return 0.0f;
    float buf[1024] = {0};
    float *p = k <= 1024 ? buf : (float *)malloc(sizeof(float) * (size_t)k);
    for (int64_t i = 0; i < k; ++i) p[i] = a[i] * b[i];
    float s = torch_sum_f32(p, k);
    if (p != buf) free(p);
    return s;
}

ORACLE_API float sva_oracle_torch_dot(const float *a, const float *b, int64_t k) { return torch_dot_f32(a, b, k); }

/* ------------------------------------------------------------------------ */
/* Learned projection (sva/llama.py:211 q_low, :598/:615 k_low):
 * out[n][r] = sum_d x[n][d] * w[d][r] as a sequential fmaf chain over d. */
ORACLE_API void sva_oracle_project(const float *x, int64_t n, int64_t x_stride, const float *w, int64_t d,
                                   int64_t r, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float *xi = x + i * x_stride;
        for (int64_t j = 0; j < r; ++j) {
            float acc = 0.0f;
            for (int64_t t = 0; t < d; ++t) acc = fmaf(xi[t], w[t * r + j], acc);
            out[i * r + j] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* assign_to_centroids (sva/ops.py:10-21):
 *   dist = (x*x).sum(-1) - 2 * (x @ C^T) + (C*C).sum(-1);  label = first argmin.
 * x rows have `sub` floats at stride x_stride; cb is [C][sub]. */
ORACLE_API void sva_oracle_assign(const float *x, int64_t n, int64_t x_stride, int64_t sub, const float *cb,
                                  int64_t C, int64_t *labels, float *best_gap) {
    float *cn = (float *)malloc(sizeof(float) * (size_t)C);
    for (int64_t c = 0; c < C; ++c) cn[c] = torch_dot_f32(cb + c * sub, cb + c * sub, sub);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float *xi = x + i * x_stride;
        const float xx = torch_dot_f32(xi, xi, sub);
        float best = INFINITY, second = INFINITY;
        int64_t arg = 0;
        for (int64_t c = 0; c < C; ++c) {
            float xc = 0.0f;
            for (int64_t t = 0; t < sub; ++t) xc = fmaf(xi[t], cb[c * sub + t], xc);
            const float dist = (xx - 2.0f * xc) + cn[c];
            if (dist < best) {
                second = best;
                best = dist;
                arg = c;
            } else if (dist < second) {
                second = dist;
            }
        }
        labels[i] = arg;
        if (best_gap) best_gap[i] = second - best;
    }
    free(cn);
}

/* ------------------------------------------------------------------------ */
/* Per-query lookup table (sva/ops.py:68): lut[s][c] = q_low[s*sub:(s+1)*sub] . cb[s][c][:]
 * as a sequential fmaf chain. */
ORACLE_API void sva_oracle_lut(const float *q_low, int64_t S, int64_t C, int64_t sub, const float *cb, float *lut) {
    for (int64_t s = 0; s < S; ++s)
        for (int64_t c = 0; c < C; ++c) {
            float acc = 0.0f;
            const float *w = cb + (s * C + c) * sub;
            for (int64_t t = 0; t < sub; ++t) acc = fmaf(q_low[s * sub + t], w[t], acc);
            lut[s * C + c] = acc;
        }
}

static inline int64_t load_code(const void *codes, int code_bytes, int64_t off) {
    switch (code_bytes) {
    case 1: return ((const uint8_t *)codes)[off];
    case 2: return ((const int16_t *)codes)[off];
    case 4: return ((const int32_t *)codes)[off];
    default: return ((const int64_t *)codes)[off];
    }
}

/* PQ scan scores (sva/ops.py:64-71): score[n] = (((0 + T0[c0]) + T1[c1]) + ...) / sqrt_r.
 * codes row n starts at n*code_stride (elements), subspace s at +s. */
ORACLE_API void sva_oracle_pq_scores(const float *lut, int64_t S, int64_t C, const void *codes, int code_bytes,
                                     int64_t n, int64_t code_stride, float sqrt_r, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float acc = 0.0f;
        for (int64_t s = 0; s < S; ++s) acc = acc + lut[s * C + load_code(codes, code_bytes, i * code_stride + s)];
        out[i] = acc / sqrt_r;
    }
}

/* Low-rank rescore (sva/llama.py:292, :495):
 * out[i] = torch.sum(k_low[idx[i]] * q_low) / sqrt_r. */
ORACLE_API void sva_oracle_rank_scores(const float *k_low, int64_t R, const int64_t *idx, int64_t m,
                                       const float *q_low, float sqrt_r, float *out) {
    for (int64_t i = 0; i < m; ++i) out[i] = torch_dot_f32(k_low + idx[i] * R, q_low, R) / sqrt_r;
}

/* ------------------------------------------------------------------------ */
/* Top-k by (score desc, index asc) among allowed entries.  idx_map (optional)
 * maps position -> key index used for the tie rule and the output; when NULL
 * the position is the key index.  Returns the number selected = min(k, allowed). */
typedef struct {
    uint64_t key;
    int64_t pos;
} ranked_t;

static int cmp_ranked_desc(const void *a, const void *b) {
    const uint64_t ka = ((const ranked_t *)a)->key, kb = ((const ranked_t *)b)->key;
    return ka < kb ? 1 : (ka > kb ? -1 : 0);
}

static void select_top(ranked_t *v, int64_t m, int64_t k) {
    /* quickselect so that v[0..k) hold the k largest keys, then sort them */
    int64_t lo = 0, hi = m - 1;
    while (lo < hi && k < m) {
        const uint64_t pivot = v[lo + (hi - lo) / 2].key;
        int64_t i = lo, j = hi;
        while (i <= j) {
            while (v[i].key > pivot) i++;
            while (v[j].key < pivot) j--;
            if (i <= j) {
                ranked_t t = v[i];
                v[i] = v[j];
                v[j] = t;
                i++;
                j--;
            }
        }
        if (k - 1 <= j) hi = j;
        else if (k - 1 >= i) lo = i;
        else break;
    }
    qsort(v, (size_t)(k < m ? k : m), sizeof(ranked_t), cmp_ranked_desc);
}

ORACLE_API int64_t sva_oracle_topk(const float *scores, const uint8_t *allowed, const int64_t *idx_map, int64_t n,
                                   int64_t k, int64_t *out_pos) {
    ranked_t *v = (ranked_t *)malloc(sizeof(ranked_t) * (size_t)(n > 0 ? n : 1));
    int64_t m = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (allowed && !allowed[i]) continue;
        const int64_t key_index = idx_map ? idx_map[i] : i;
        v[m].key = ((uint64_t)f2key(scores[i]) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)key_index);
        v[m].pos = i;
        m++;
    }
    const int64_t take = k < m ? k : m;
    if (take > 0) select_top(v, m, take);
    for (int64_t i = 0; i < take; ++i) out_pos[i] = v[i].pos;
    free(v);
    return take;
}

/* ------------------------------------------------------------------------ */
/* Exact verifier reference in double precision (sva/llama.py:304-317,
 * :545-553): softmax(scaling * K[idx] . q) weighted sum of V[idx].  K and V
 * are [N][D] rows (already converted to float), idx the m selected keys. */
ORACLE_API void sva_oracle_verify(const float *q, const float *K, const float *V, int64_t D, const int64_t *idx,
                                  int64_t m, double scaling, double *out) {
    double *w = (double *)malloc(sizeof(double) * (size_t)(m > 0 ? m : 1));
    double mx = -INFINITY;
    for (int64_t i = 0; i < m; ++i) {
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += (double)K[idx[i] * D + d] * (double)q[d];
        w[i] = s * scaling;
        if (w[i] > mx) mx = w[i];
    }
    double z = 0.0;
    for (int64_t i = 0; i < m; ++i) {
        w[i] = exp(w[i] - mx);
        z += w[i];
    }
    for (int64_t d = 0; d < D; ++d) out[d] = 0.0;
    for (int64_t i = 0; i < m; ++i)
        for (int64_t d = 0; d < D; ++d) out[d] += (w[i] / z) * (double)V[idx[i] * D + d];
    free(w);
}

/* ------------------------------------------------------------------------ */
/* Whole scan-mode decode lookup for one query over H heads sharing G KV heads
 * (the synthetic cached-decode workload of
 * experiments/sva_million_cached_decode_benchmark.py:224-249, GQA-indexed):
 *   lut -> PQ scores -> top-L -> rank scores -> top-B -> verifier.
 * Inputs: q [H][D], q_low [H][R], K/V [G][cap][D] float, k_low [H][cap][R],
 * codebooks [H][S][C][sub], codes [H][cap][S] (code_bytes wide); the first N
 * of the cap rows of every head are the cache.
 * Outputs: shortlist [H][L], final [H][B] (key indices in selection order),
 * out [H][D].  Heads run in parallel (OpenMP).  Returns the thread count. */
ORACLE_API int sva_oracle_decode(int64_t H, int64_t G, int64_t N, int64_t cap, int64_t D, int64_t R, int64_t S,
                                 int64_t C,
                                 const float *q, const float *q_low, const float *K, const float *V,
                                 const float *k_low, const float *codebooks, const void *codes, int code_bytes,
                                 int64_t L, int64_t B, double scaling, int64_t *shortlist, int64_t *final_idx,
                                 double *out) {
    const int64_t sub = R / S;
    const float sqrt_r = (float)sqrt((double)R);
    const int64_t Lh = L < N ? L : N;
    const int64_t Bh = B < Lh ? B : Lh;
    int threads = 1;
    /* one thread per head at most: a larger team only spins at the barrier */
    int team = 1;
#ifdef _OPENMP
    team = omp_get_max_threads() < H ? omp_get_max_threads() : (int)H;
#endif
#pragma omp parallel num_threads(team)
    {
#ifdef _OPENMP
#pragma omp single
        threads = omp_get_num_threads();
#endif
#pragma omp for schedule(dynamic, 1)
        for (int64_t h = 0; h < H; ++h) {
            const int64_t g = h / (H / G);
            float *lut = (float *)malloc(sizeof(float) * (size_t)(S * C));
            float *sc = (float *)malloc(sizeof(float) * (size_t)N);
            sva_oracle_lut(q_low + h * R, S, C, sub, codebooks + h * S * C * sub, lut);
            const char *hc = (const char *)codes + (size_t)h * (size_t)cap * (size_t)S * (size_t)code_bytes;
            for (int64_t i = 0; i < N; ++i) {
                float acc = 0.0f;
                for (int64_t s = 0; s < S; ++s) acc = acc + lut[s * C + load_code(hc, code_bytes, i * S + s)];
                sc[i] = acc / sqrt_r;
            }
            int64_t *sl = shortlist + h * L;
            const int64_t got = sva_oracle_topk(sc, NULL, NULL, N, Lh, sl);
            float *rank = (float *)malloc(sizeof(float) * (size_t)(got > 0 ? got : 1));
            sva_oracle_rank_scores(k_low + (size_t)h * (size_t)cap * (size_t)R, R, sl, got, q_low + h * R, sqrt_r, rank);
            int64_t *pos = (int64_t *)malloc(sizeof(int64_t) * (size_t)(Bh > 0 ? Bh : 1));
            const int64_t kept = sva_oracle_topk(rank, NULL, sl, got, Bh, pos);
            for (int64_t b = 0; b < kept; ++b) final_idx[h * B + b] = sl[pos[b]];
            sva_oracle_verify(q + h * D, K + (size_t)g * (size_t)cap * (size_t)D, V + (size_t)g * (size_t)cap * (size_t)D, D,
                              final_idx + h * B, kept, scaling, out + h * D);
            free(pos);
            free(rank);
            free(sc);
            free(lut);
        }
    }
    return threads;
}
