/*
 * CPU oracle for the FreeML NanoLLM token loop — TEST INFRASTRUCTURE ONLY (see header).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: the reference's x86-64 build has no FMA,
 * so every a*b and +/- is rounded separately, and so must this file's).
 */
#define _GNU_SOURCE
#include "nanollm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------
 * Thread pool: restates ToolsLibrary/ThreadPool.h:15-106 (fixed workers, FIFO queue, a
 * latch per parallel call) so the CPU baseline splits work the way the reference does.
 * ------------------------------------------------------------------------------------- */
typedef void (*orc_range_fn)(void* arg, uint32_t begin, uint32_t end);

typedef struct {
    orc_range_fn fn;
    void* arg;
    uint32_t begin, end;
    int* latch;
} orc_task;

typedef struct {
    pthread_t* threads;
    int nthreads;
    pthread_mutex_t mu;
    pthread_cond_t cv;      /* work available / stopping */
    pthread_cond_t done_cv; /* a latch reached zero */
    orc_task* queue;
    int qcap, qhead, qcount;
    int stopping;
} orc_pool;

static void* orc_worker(void* p) {
    orc_pool* pool = (orc_pool*)p;
    for (;;) {
        pthread_mutex_lock(&pool->mu);
        while (!pool->stopping && pool->qcount == 0) pthread_cond_wait(&pool->cv, &pool->mu);
        if (pool->stopping && pool->qcount == 0) {
            pthread_mutex_unlock(&pool->mu);
            return NULL;
        }
        orc_task t = pool->queue[pool->qhead];
        pool->qhead = (pool->qhead + 1) % pool->qcap;
        pool->qcount--;
        pthread_mutex_unlock(&pool->mu);
        t.fn(t.arg, t.begin, t.end);
        pthread_mutex_lock(&pool->mu);
        if (--(*t.latch) == 0) pthread_cond_broadcast(&pool->done_cv);
        pthread_mutex_unlock(&pool->mu);
    }
}

static orc_pool* orc_pool_create(int n) {
    if (n < 1) n = 1;
    orc_pool* pool = (orc_pool*)calloc(1, sizeof(orc_pool));
    pool->nthreads = n;
    pool->qcap = 4 * n + 16;
    pool->queue = (orc_task*)calloc((size_t)pool->qcap, sizeof(orc_task));
    pthread_mutex_init(&pool->mu, NULL);
    pthread_cond_init(&pool->cv, NULL);
    pthread_cond_init(&pool->done_cv, NULL);
    pool->threads = (pthread_t*)calloc((size_t)n, sizeof(pthread_t));
    for (int i = 0; i < n; ++i) pthread_create(&pool->threads[i], NULL, orc_worker, pool);
    return pool;
}

static void orc_pool_destroy(orc_pool* pool) {
    if (!pool) return;
    pthread_mutex_lock(&pool->mu);
    pool->stopping = 1;
    pthread_cond_broadcast(&pool->cv);
    pthread_mutex_unlock(&pool->mu);
    for (int i = 0; i < pool->nthreads; ++i) pthread_join(pool->threads[i], NULL);
    pthread_mutex_destroy(&pool->mu);
    pthread_cond_destroy(&pool->cv);
    pthread_cond_destroy(&pool->done_cv);
    free(pool->threads);
    free(pool->queue);
    free(pool);
}

/* Splits [0, count) into nthreads chunks of ceil(count / nthreads) (MatrixBase_Mul.h:547-556)
 * and waits for all of them (the std::latch at :576-587). */
static void orc_parallel_for(orc_pool* pool, uint32_t count, orc_range_fn fn, void* arg) {
    if (count == 0) return;
    if (!pool || pool->nthreads <= 1) {
        fn(arg, 0, count);
        return;
    }
    uint32_t n = (uint32_t)pool->nthreads;
    uint32_t per = (count + n - 1) / n;
    int latch = 0;
    pthread_mutex_lock(&pool->mu);
    for (uint32_t t = 0; t < n; ++t) {
        uint32_t b = t * per;
        if (b >= count) break;
        uint32_t e = b + per < count ? b + per : count;
        int slot = (pool->qhead + pool->qcount) % pool->qcap;
        pool->queue[slot] = (orc_task){fn, arg, b, e, &latch};
        pool->qcount++;
        latch++;
    }
    pthread_cond_broadcast(&pool->cv);
    while (latch > 0) pthread_cond_wait(&pool->done_cv, &pool->mu);
    pthread_mutex_unlock(&pool->mu);
}

/* ---------------------------------------------------------------------------------------
 * GEMM: sequential-k fp32 dot products, blocked like MulBlock (MatrixBase_Mul.h:521-545).
 * The partial sum is reloaded from C at each 32-wide k block; that reload is exact, so every
 * output equals ((0 + a0*b0) + a1*b1) + ... in k order.
 * ------------------------------------------------------------------------------------- */
typedef struct {
    const float* A;
    const float* B;
    float* C;
    uint32_t M, N, K;
    uint32_t a_rs, a_cs, b_rs, b_cs, c_rs, c_cs;
    int tl, tr;
    int split_cols; /* 1: [begin,end) are column indices, 0: row indices */
} orc_gemm_args;

#define ORC_BLOCK 32u

static inline float orc_geta(const orc_gemm_args* g, uint32_t i, uint32_t k) {
    return g->tl ? g->A[(size_t)k * g->a_rs + (size_t)i * g->a_cs]
                 : g->A[(size_t)i * g->a_rs + (size_t)k * g->a_cs];
}
static inline float orc_getb(const orc_gemm_args* g, uint32_t k, uint32_t j) {
    return g->tr ? g->B[(size_t)j * g->b_rs + (size_t)k * g->b_cs]
                 : g->B[(size_t)k * g->b_rs + (size_t)j * g->b_cs];
}

/* The same blocks with the j loop innermost, for C rows with unit column stride: B's k-th row
 * slice (read along j, or copied out of a transposed B into bt) is added into C's row, so
 * C[i][j] still receives a(i,k0) b(k0,j), a(i,k0+1) b(k0+1,j), ... one rounded product and one
 * rounded sum at a time in k order -- the identical operation sequence per output as the
 * dot-product form above, which the compiler can now run on several j at once. */
static void orc_gemm_range_rows(const orc_gemm_args* g, uint32_t i_lo, uint32_t i_hi, uint32_t j_lo,
                                uint32_t j_hi) {
    float bt[ORC_BLOCK * ORC_BLOCK];
    for (uint32_t i = i_lo; i < i_hi; ++i)
        for (uint32_t j = j_lo; j < j_hi; ++j) g->C[(size_t)i * g->c_rs + j] = 0.0f;
    for (uint32_t i0 = i_lo; i0 < i_hi; i0 += ORC_BLOCK) {
        uint32_t ie = i0 + ORC_BLOCK < i_hi ? i0 + ORC_BLOCK : i_hi;
        for (uint32_t j0 = j_lo; j0 < j_hi; j0 += ORC_BLOCK) {
            uint32_t je = j0 + ORC_BLOCK < j_hi ? j0 + ORC_BLOCK : j_hi;
            const uint32_t nj = je - j0;
            for (uint32_t k0 = 0; k0 < g->K; k0 += ORC_BLOCK) {
                uint32_t ke = k0 + ORC_BLOCK < g->K ? k0 + ORC_BLOCK : g->K;
                const int direct = !g->tr && g->b_cs == 1;
                if (!direct)
                    for (uint32_t k = k0; k < ke; ++k)
                        for (uint32_t j = j0; j < je; ++j) bt[(k - k0) * ORC_BLOCK + (j - j0)] = orc_getb(g, k, j);
                for (uint32_t i = i0; i < ie; ++i) {
                    float* c = &g->C[(size_t)i * g->c_rs + j0];
                    for (uint32_t k = k0; k < ke; ++k) {
                        const float a = orc_geta(g, i, k);
                        const float* b = direct ? &g->B[(size_t)k * g->b_rs + j0] : &bt[(k - k0) * ORC_BLOCK];
                        for (uint32_t j = 0; j < nj; ++j) c[j] += a * b[j];
                    }
                }
            }
        }
    }
}

static void orc_gemm_range(void* p, uint32_t begin, uint32_t end) {
    const orc_gemm_args* g = (const orc_gemm_args*)p;
    uint32_t i_lo = 0, i_hi = g->M, j_lo = 0, j_hi = g->N;
    if (g->split_cols) { j_lo = begin; j_hi = end; } else { i_lo = begin; i_hi = end; }
    if (g->c_cs == 1) {
        orc_gemm_range_rows(g, i_lo, i_hi, j_lo, j_hi);
        return;
    }
    for (uint32_t i = i_lo; i < i_hi; ++i)
        for (uint32_t j = j_lo; j < j_hi; ++j) g->C[(size_t)i * g->c_rs + (size_t)j * g->c_cs] = 0.0f;
    for (uint32_t i0 = i_lo; i0 < i_hi; i0 += ORC_BLOCK) {
        uint32_t ie = i0 + ORC_BLOCK < i_hi ? i0 + ORC_BLOCK : i_hi;
        for (uint32_t j0 = j_lo; j0 < j_hi; j0 += ORC_BLOCK) {
            uint32_t je = j0 + ORC_BLOCK < j_hi ? j0 + ORC_BLOCK : j_hi;
            for (uint32_t k0 = 0; k0 < g->K; k0 += ORC_BLOCK) {
                uint32_t ke = k0 + ORC_BLOCK < g->K ? k0 + ORC_BLOCK : g->K;
                for (uint32_t i = i0; i < ie; ++i) {
                    for (uint32_t j = j0; j < je; ++j) {
                        float* c = &g->C[(size_t)i * g->c_rs + (size_t)j * g->c_cs];
                        float sum = *c;
                        for (uint32_t k = k0; k < ke; ++k) sum += orc_geta(g, i, k) * orc_getb(g, k, j);
                        *c = sum;
                    }
                }
            }
        }
    }
}

static void orc_gemm(orc_pool* pool, orc_gemm_args* g) {
    if (g->M == 0 || g->N == 0) return;
    /* MulBlock splits rows; with fewer rows than workers the split goes over columns
     * instead (one query row in the cached loop).  Neither changes a single output. */
    uint32_t n = pool ? (uint32_t)pool->nthreads : 1u;
    g->split_cols = (g->M < n && g->N >= 2u * n) ? 1 : 0;
    orc_parallel_for(pool, g->split_cols ? g->N : g->M, orc_gemm_range, g);
}

static void orc_mul_pool(orc_pool* pool, int mode, float* out, const float* L, const float* R,
                         uint32_t M, uint32_t N, uint32_t K) {
    int tl = (mode == ORC_LEFT || mode == ORC_BOTH);
    int tr = (mode == ORC_RIGHT || mode == ORC_BOTH);
    /* Row-major L (rows x cols): element (i,k) at i*cols + k; Left reads it transposed. */
    orc_gemm_args g = {L, R, out, M, N, K,
                       tl ? M : K, 1u, tr ? K : N, 1u, N, 1u, tl, tr, 0};
    orc_gemm(pool, &g);
}

void orc_mul(int mode, float* out, const float* L, const float* R,
             uint32_t M, uint32_t N, uint32_t K, int nthreads) {
    orc_pool* pool = nthreads > 1 ? orc_pool_create(nthreads) : NULL;
    orc_mul_pool(pool, mode, out, L, R, M, N, K);
    orc_pool_destroy(pool);
}

void orc_mul_strided(int mode, float* C, const float* A, const float* B,
                     uint32_t M, uint32_t N, uint32_t K,
                     uint32_t a_rs, uint32_t a_cs, uint32_t b_rs, uint32_t b_cs,
                     uint32_t c_rs, uint32_t c_cs) {
    int tl = (mode == ORC_LEFT || mode == ORC_BOTH);
    int tr = (mode == ORC_RIGHT || mode == ORC_BOTH);
    orc_gemm_args g = {A, B, C, M, N, K, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, tl, tr, 0};
    orc_gemm(NULL, &g);
}

/* ---------------------------------------------------------------------------------------
 * Element / row ops.
 * ------------------------------------------------------------------------------------- */
void orc_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                   float* xhat, uint32_t rows, uint32_t cols, float eps) {
    const float inv_cols = 1.0f / (float)cols;
    for (uint32_t r = 0; r < rows; ++r) {
        const float* x = in + (size_t)r * cols;
        float mean = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) mean += x[c];
        mean *= inv_cols;
        float var = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) {
            const float d = x[c] - mean;
            var += d * d;
        }
        var *= inv_cols;
        const float inv_std = 1.0f / sqrtf(var + eps);
        for (uint32_t c = 0; c < cols; ++c) {
            const float nrm = (x[c] - mean) * inv_std;
            if (xhat) xhat[(size_t)r * cols + c] = nrm;
            const float b = beta ? beta[c] : 0.0f;
            out[(size_t)r * cols + c] = nrm * gamma[c] + b;
        }
    }
}

void orc_softmax(float* out, const float* in, uint32_t rows, uint32_t cols) {
    for (uint32_t r = 0; r < rows; ++r) {
        const float* x = in + (size_t)r * cols;
        float* y = out + (size_t)r * cols;
        float mx = x[0];
        for (uint32_t c = 1; c < cols; ++c) mx = (mx < x[c]) ? x[c] : mx; /* std::max */
        float sum = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) {
            const float v = expf(x[c] - mx);
            y[c] = v;
            sum += v;
        }
        for (uint32_t c = 0; c < cols; ++c) y[c] /= sum;
    }
}

void orc_scale_add(float* out, const float* in, float scale, const float* add, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) out[i] = in[i] * scale + add[i];
}

void orc_gelu(float* out, const float* in, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) {
        const float x = in[i];
        out[i] = 0.5f * x * (1.0f + erff(x / sqrtf(2.0f)));
    }
}

void orc_add(float* out, const float* a, const float* b, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void orc_gather_rows(float* out, const float* src, const float* ids, uint32_t width,
                     uint32_t rows) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint32_t s = (uint32_t)ids[r];
        memcpy(out + (size_t)r * width, src + (size_t)s * width, sizeof(float) * width);
    }
}

void orc_split_qkv(float* q, float* k, float* v, const float* packed, uint32_t rows,
                   uint32_t dC) {
    for (uint32_t r = 0; r < rows; ++r) {
        const float* p = packed + (size_t)r * 3u * dC;
        memcpy(q + (size_t)r * dC, p, sizeof(float) * dC);
        memcpy(k + (size_t)r * dC, p + dC, sizeof(float) * dC);
        memcpy(v + (size_t)r * dC, p + 2u * dC, sizeof(float) * dC);
    }
}

void orc_triangle_lower(float* out, uint32_t rows, uint32_t cols, float true_val,
                        float false_val) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint32_t keep = r + 1 < cols ? r + 1 : cols;
        for (uint32_t c = 0; c < cols; ++c) out[(size_t)r * cols + c] = c < keep ? true_val : false_val;
    }
}

uint32_t orc_argmax(const float* row, uint32_t n) {
    uint32_t best = 0;
    float bv = row[0];
    for (uint32_t v = 1; v < n; ++v)
        if (row[v] > bv) { bv = row[v]; best = v; }
    return best;
}

/* ---------------------------------------------------------------------------------------
 * Model.
 * ------------------------------------------------------------------------------------- */
typedef struct {
    const float *w_qkv, *w_proj, *w_fc, *w_proj2, *ln0_g, *ln0_b, *ln1_g, *ln1_b;
} orc_layer;

struct orc_model {
    uint32_t V, T, C, H, L, hd;
    const float *tok, *pos, *lnf_g, *lnf_b, *lm;
    orc_layer* layers;
    orc_pool* pool;
    float scale;
    float* mask; /* T x T, 0 / -inf (CausalSelfAttentionLayer.h:66-67) */
};

orc_model* orc_model_create(uint32_t vocab, uint32_t block_size, uint32_t n_embed,
                            uint32_t n_head, uint32_t n_layer,
                            const float* tok_emb, const float* pos_emb,
                            const float* const* layer_ptrs,
                            const float* lnf_gamma, const float* lnf_beta,
                            const float* lm_head, int nthreads) {
    if (!vocab || !block_size || !n_embed || !n_head || !n_layer || n_embed % n_head) return NULL;
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->V = vocab; m->T = block_size; m->C = n_embed; m->H = n_head; m->L = n_layer;
    m->hd = n_embed / n_head;
    m->tok = tok_emb; m->pos = pos_emb; m->lnf_g = lnf_gamma; m->lnf_b = lnf_beta; m->lm = lm_head;
    m->layers = (orc_layer*)calloc(n_layer, sizeof(orc_layer));
    for (uint32_t l = 0; l < n_layer; ++l) {
        const float* const* p = layer_ptrs + 8u * l;
        m->layers[l] = (orc_layer){p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]};
    }
    /* scale = 1 / sqrt(head_dim) in float (CausalSelfAttentionLayer.h:73-74). */
    m->scale = 1.0f / sqrtf((float)m->hd);
    m->mask = (float*)malloc(sizeof(float) * (size_t)block_size * block_size);
    orc_triangle_lower(m->mask, block_size, block_size, 0.0f, -INFINITY);
    m->pool = nthreads > 1 ? orc_pool_create(nthreads) : NULL;
    return m;
}

void orc_model_destroy(orc_model* m) {
    if (!m) return;
    orc_pool_destroy(m->pool);
    free(m->mask);
    free(m->layers);
    free(m);
}

/* Embedding x2 + AddLayer (Embedding.h:161-170, AddLayer.h:149): x[r] = tok[id] + pos[r0+r].
 * The embedding dropout at p = 0 multiplies by a mask of ones and a scale of 1
 * (DropoutLayer.h:125-147), which leaves every value unchanged. */
static void orc_embed(const orc_model* m, const int32_t* ids, uint32_t r0, uint32_t n, float* x) {
    for (uint32_t r = 0; r < n; ++r)
        for (uint32_t c = 0; c < m->C; ++c)
            x[(size_t)r * m->C + c] = m->tok[(size_t)ids[r] * m->C + c] + m->pos[(size_t)(r0 + r) * m->C + c];
}

/* Full-window forward: Model::Run over embedding -> blocks -> ln_f -> flatten -> lm_head. */
int orc_forward_window(orc_model* m, const int32_t* ids, float* logits) {
    const uint32_t T = m->T, C = m->C, H = m->H, hd = m->hd, V = m->V;
    for (uint32_t r = 0; r < T; ++r)
        if (ids[r] < 0 || (uint32_t)ids[r] >= V) return -1;
    const size_t TC = (size_t)T * C;
    float* x = (float*)malloc(sizeof(float) * TC);
    float* ln = (float*)malloc(sizeof(float) * TC);
    float* qkv = (float*)malloc(sizeof(float) * TC * 3);
    float* q = (float*)malloc(sizeof(float) * TC);
    float* k = (float*)malloc(sizeof(float) * TC);
    float* v = (float*)malloc(sizeof(float) * TC);
    float* y = (float*)malloc(sizeof(float) * TC);
    float* att = (float*)malloc(sizeof(float) * TC);
    float* buf = (float*)malloc(sizeof(float) * TC);
    float* h = (float*)malloc(sizeof(float) * TC * 4);
    float* mlp = (float*)malloc(sizeof(float) * TC);
    float* scores = (float*)malloc(sizeof(float) * (size_t)T * T);
    float* probs = (float*)malloc(sizeof(float) * (size_t)T * T);

    orc_embed(m, ids, 0, T, x);
    for (uint32_t l = 0; l < m->L; ++l) {
        const orc_layer* w = &m->layers[l];
        /* TransformerBlockLayer::Forward (TransformerBlock.h:355-401). */
        orc_layernorm(ln, x, w->ln0_g, w->ln0_b, NULL, T, C, 1e-5f);
        /* CausalSelfAttentionLayer::Forward (CausalSelfAttentionLayer.h:371-514). */
        orc_mul_pool(m->pool, ORC_NONE, qkv, ln, w->w_qkv, T, 3 * C, C);
        orc_split_qkv(q, k, v, qkv, T, C);
        for (uint32_t hh = 0; hh < H; ++hh) {
            /* scores = Q_h K_h^T (MatMul_Strided<Right>, :445-450), row stride C. */
            orc_gemm_args gs = {q + hh * hd, k + hh * hd, scores, T, T, hd,
                                C, 1u, C, 1u, T, 1u, 0, 1, 0};
            orc_gemm(m->pool, &gs);
            orc_scale_add(scores, scores, m->scale, m->mask, T * T); /* :453 */
            orc_softmax(probs, scores, T, T);                          /* :458 */
            /* Y_h = P V_h (MatMul_Strided<None>, :492-497) into the head's column slice. */
            orc_gemm_args gv = {probs, v + hh * hd, y + hh * hd, T, hd, T,
                                T, 1u, C, 1u, C, 1u, 0, 0, 0};
            orc_gemm(m->pool, &gv);
        }
        orc_mul_pool(m->pool, ORC_RIGHT, att, y, w->w_proj, T, C, C); /* :502-503 */
        orc_add(buf, x, att, (uint32_t)TC);                            /* TransformerBlock.h:382 */
        orc_layernorm(ln, buf, w->ln1_g, w->ln1_b, NULL, T, C, 1e-5f);
        orc_mul_pool(m->pool, ORC_NONE, h, ln, w->w_fc, T, 4 * C, C);  /* :390-391 */
        orc_gelu(h, h, (uint32_t)(TC * 4));
        orc_mul_pool(m->pool, ORC_NONE, mlp, h, w->w_proj2, T, C, 4 * C); /* :394-395 */
        orc_add(x, buf, mlp, (uint32_t)TC);                            /* :400 */
    }
    orc_layernorm(ln, x, m->lnf_g, m->lnf_b, NULL, T, C, 1e-5f);      /* ln_f */
    orc_mul_pool(m->pool, ORC_RIGHT, logits, ln, m->lm, T, V, C);      /* lm_head */

    free(x); free(ln); free(qkv); free(q); free(k); free(v); free(y); free(att);
    free(buf); free(h); free(mlp); free(scores); free(probs);
    return 0;
}

int orc_greedy_window(orc_model* m, const int32_t* prompt, uint32_t prompt_len,
                      uint32_t n_gen, int32_t* tokens_out, float* logits_out) {
    const uint32_t T = m->T, V = m->V;
    if (prompt_len == 0 || prompt_len + n_gen - 1 > T) return -2;
    int32_t* hist = (int32_t*)calloc(T + 1, sizeof(int32_t));
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * V);
    memcpy(hist, prompt, sizeof(int32_t) * prompt_len);
    uint32_t len = prompt_len;
    int rc = 0;
    for (uint32_t s = 0; s < n_gen; ++s) {
        int32_t* window = (int32_t*)calloc(T, sizeof(int32_t)); /* padding id 0 */
        memcpy(window, hist, sizeof(int32_t) * len);
        rc = orc_forward_window(m, window, logits);
        free(window);
        if (rc) break;
        const float* row = logits + (size_t)(len - 1) * V;
        if (logits_out) memcpy(logits_out + (size_t)s * V, row, sizeof(float) * V);
        const int32_t next = (int32_t)orc_argmax(row, V);
        tokens_out[s] = next;
        if (len < T) hist[len++] = next;
    }
    free(hist);
    free(logits);
    return rc;
}

/* Causal attention of query rows [begin, end) (absolute positions r0 + r, each attending to
 * keys 0 .. r0 + r), every head, as the full-window path computes a row of scores, softmax and
 * P V_h: rows are independent, so the pool splits them.  The P V_h sums run over j in order for
 * every d (the j loop outside, a row of V at a time): the same sequence per output as a d-outer
 * loop, with V read along its rows. */
typedef struct {
    const float *q, *K, *V;
    float* y;
    uint32_t r0, C, H, hd;
    float scale;
} orc_attn_rows_args;

static void orc_attn_rows(void* p, uint32_t begin, uint32_t end) {
    const orc_attn_rows_args* a = (const orc_attn_rows_args*)p;
    const uint32_t C = a->C, hd = a->hd;
    float* sc = (float*)malloc(sizeof(float) * (a->r0 + end));
    float* acc = (float*)malloc(sizeof(float) * hd);
    for (uint32_t r = begin; r < end; ++r) {
        const uint32_t i = a->r0 + r; /* absolute position; attends to 0..i */
        for (uint32_t hh = 0; hh < a->H; ++hh) {
            const float* qi = a->q + (size_t)r * C + hh * hd;
            float mx = -INFINITY;
            for (uint32_t j = 0; j <= i; ++j) {
                const float* kj = a->K + (size_t)j * C + hh * hd;
                float s = 0.0f;
                for (uint32_t d = 0; d < hd; ++d) s += qi[d] * kj[d];
                s = s * a->scale + 0.0f; /* ScaleAdd with mask 0 on j <= i */
                sc[j] = s;
                if (j == 0) mx = s; else mx = (mx < s) ? s : mx;
            }
            /* Masked entries are -inf: they cannot raise the max, exp() gives exactly 0
             * and adding 0 (or 0 * v) leaves the sequential sums unchanged. */
            float sum = 0.0f;
            for (uint32_t j = 0; j <= i; ++j) {
                sc[j] = expf(sc[j] - mx);
                sum += sc[j];
            }
            for (uint32_t j = 0; j <= i; ++j) sc[j] /= sum;
            for (uint32_t d = 0; d < hd; ++d) acc[d] = 0.0f;
            for (uint32_t j = 0; j <= i; ++j) {
                const float pj = sc[j];
                const float* vj = a->V + (size_t)j * C + hh * hd;
                for (uint32_t d = 0; d < hd; ++d) acc[d] += pj * vj[d];
            }
            float* yi = a->y + (size_t)r * C + hh * hd;
            for (uint32_t d = 0; d < hd; ++d) yi[d] = acc[d];
        }
    }
    free(acc);
    free(sc);
}

/* Forward of rows [r0, r0+n) given K/V of rows < r0 in kc/vc (T x C each, per layer). */
static void orc_forward_rows(orc_model* m, const int32_t* ids, uint32_t r0, uint32_t n,
                             float* kc, float* vc, float* logits_last) {
    const uint32_t C = m->C, H = m->H, hd = m->hd, V = m->V, T = m->T;
    const size_t nC = (size_t)n * C;
    float* x = (float*)malloc(sizeof(float) * nC);
    float* ln = (float*)malloc(sizeof(float) * nC);
    float* qkv = (float*)malloc(sizeof(float) * nC * 3);
    float* q = (float*)malloc(sizeof(float) * nC);
    float* y = (float*)malloc(sizeof(float) * nC);
    float* att = (float*)malloc(sizeof(float) * nC);
    float* buf = (float*)malloc(sizeof(float) * nC);
    float* h = (float*)malloc(sizeof(float) * nC * 4);
    float* mlp = (float*)malloc(sizeof(float) * nC);

    orc_embed(m, ids + r0, r0, n, x);
    for (uint32_t l = 0; l < m->L; ++l) {
        const orc_layer* w = &m->layers[l];
        float* K = kc + (size_t)l * T * C;
        float* Vv = vc + (size_t)l * T * C;
        orc_layernorm(ln, x, w->ln0_g, w->ln0_b, NULL, n, C, 1e-5f);
        orc_mul_pool(m->pool, ORC_NONE, qkv, ln, w->w_qkv, n, 3 * C, C);
        orc_split_qkv(q, K + (size_t)r0 * C, Vv + (size_t)r0 * C, qkv, n, C);
        orc_attn_rows_args aa = {q, K, Vv, y, r0, C, H, hd, m->scale};
        orc_parallel_for(m->pool, n, orc_attn_rows, &aa);
        orc_mul_pool(m->pool, ORC_RIGHT, att, y, w->w_proj, n, C, C);
        orc_add(buf, x, att, (uint32_t)nC);
        orc_layernorm(ln, buf, w->ln1_g, w->ln1_b, NULL, n, C, 1e-5f);
        orc_mul_pool(m->pool, ORC_NONE, h, ln, w->w_fc, n, 4 * C, C);
        orc_gelu(h, h, (uint32_t)(nC * 4));
        orc_mul_pool(m->pool, ORC_NONE, mlp, h, w->w_proj2, n, C, 4 * C);
        orc_add(x, buf, mlp, (uint32_t)nC);
    }
    /* Only the last row's logits are needed by the loop. */
    orc_layernorm(ln, x + (size_t)(n - 1) * C, m->lnf_g, m->lnf_b, NULL, 1, C, 1e-5f);
    orc_mul_pool(m->pool, ORC_RIGHT, logits_last, ln, m->lm, 1, V, C);
    free(x); free(ln); free(qkv); free(q); free(y); free(att); free(buf); free(h); free(mlp);
}

int orc_greedy_cached(orc_model* m, const int32_t* prompt, uint32_t prompt_len,
                      uint32_t n_gen, int32_t* tokens_out, float* logits_out) {
    const uint32_t T = m->T, V = m->V, C = m->C;
    if (prompt_len == 0 || prompt_len + n_gen - 1 > T) return -2;
    for (uint32_t r = 0; r < prompt_len; ++r)
        if (prompt[r] < 0 || (uint32_t)prompt[r] >= V) return -1;
    float* kc = (float*)calloc((size_t)m->L * T * C, sizeof(float));
    float* vc = (float*)calloc((size_t)m->L * T * C, sizeof(float));
    int32_t* hist = (int32_t*)calloc(T + 1, sizeof(int32_t));
    float* row = (float*)malloc(sizeof(float) * V);
    memcpy(hist, prompt, sizeof(int32_t) * prompt_len);
    uint32_t len = prompt_len, done = 0;
    for (uint32_t s = 0; s < n_gen; ++s) {
        orc_forward_rows(m, hist, done, len - done, kc, vc, row);
        done = len;
        if (logits_out) memcpy(logits_out + (size_t)s * V, row, sizeof(float) * V);
        const int32_t next = (int32_t)orc_argmax(row, V);
        tokens_out[s] = next;
        if (len < T) hist[len++] = next;
    }
    free(kc); free(vc); free(hist); free(row);
    return 0;
}

/* ---- training-step restatements ---------------------------------------------------------- */

void orc_softmax_backward(float* out, const float* p, const float* dp, uint32_t rows, uint32_t cols) {
    for (uint32_t r = 0; r < rows; ++r) {
        const size_t o = (size_t)r * cols;
        float dot = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) dot += dp[o + c] * p[o + c];
        for (uint32_t c = 0; c < cols; ++c) out[o + c] = p[o + c] * (dp[o + c] - dot);
    }
}

/* Mean, two-pass variance and 1/sqrt(var + eps) of one row, as :626-642 / :660-675 compute
 * them. */
static void ln_row_stats(const float* x, uint32_t cols, float inv_cols, float eps, float* mean,
                         float* inv_std) {
    float m = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) m += x[c];
    m *= inv_cols;
    float var = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) {
        const float d = x[c] - m;
        var += d * d;
    }
    var *= inv_cols;
    *mean = m;
    *inv_std = 1.0f / sqrtf(var + eps);
}

void orc_layernorm_backward(float* dx, const float* dy, const float* in, const float* gamma,
                            float* dgamma, float* dbeta, const float* xhat, uint32_t rows,
                            uint32_t cols, float eps) {
    const float inv_cols = 1.0f / (float)cols;
    for (uint32_t c = 0; c < cols; ++c) {
        dgamma[c] = 0.0f;
        if (dbeta) dbeta[c] = 0.0f;
    }
    for (uint32_t r = 0; r < rows; ++r) {
        const size_t o = (size_t)r * cols;
        float mean = 0.0f, inv_std = 0.0f;
        if (!xhat) ln_row_stats(in + o, cols, inv_cols, eps, &mean, &inv_std);
        for (uint32_t c = 0; c < cols; ++c) {
            const float d = dy[o + c];
            const float xh = xhat ? xhat[o + c] : (in[o + c] - mean) * inv_std;
            if (dbeta) dbeta[c] += d;
            dgamma[c] += d * xh;
        }
    }
    for (uint32_t r = 0; r < rows; ++r) {
        const size_t o = (size_t)r * cols;
        float mean, inv_std;
        ln_row_stats(in + o, cols, inv_cols, eps, &mean, &inv_std);
        const float inv_std3 = inv_std * inv_std * inv_std;
        float dvar = 0.0f, dmean = 0.0f, sdiff = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) {
            const float diff = in[o + c] - mean;
            const float dxh = dy[o + c] * gamma[c];
            dvar += dxh * diff * -0.5f * inv_std3;
            dmean += dxh * -inv_std;
            sdiff += diff;
        }
        dmean += dvar * -2.0f * sdiff * inv_cols;
        for (uint32_t c = 0; c < cols; ++c) {
            const float diff = in[o + c] - mean;
            const float dxh = dy[o + c] * gamma[c];
            dx[o + c] = dxh * inv_std + dvar * 2.0f * diff * inv_cols + dmean * inv_cols;
        }
    }
}

void orc_gelu_derivative(float* out, const float* in, uint32_t n) {
    const float sqrt2 = sqrtf(2.0f);
    const float sqrt2pi = sqrtf(2.0f * 3.14159265358979323846f);
    for (uint32_t i = 0; i < n; ++i) {
        const float x = in[i];
        const float erf_term = erff(x / sqrt2);
        const float exp_term = expf(-0.5f * x * x);
        out[i] = 0.5f * (1.0f + erf_term) + (x * exp_term) / sqrt2pi;
    }
}

void orc_scatter_add_rows(float* out, const float* src, const float* idx, uint32_t width,
                          uint32_t src_rows, uint32_t src_batch, uint32_t out_rows,
                          uint32_t out_batch) {
    for (uint32_t z = 0; z < src_batch; ++z) {
        const uint32_t oz = out_batch == 1 ? 0u : z;
        for (uint32_t r = 0; r < src_rows; ++r) {
            const uint32_t d = (uint32_t)idx[(size_t)z * src_rows + r];
            const float* s = src + ((size_t)z * src_rows + r) * width;
            float* o = out + ((size_t)oz * out_rows + d) * width;
            for (uint32_t x = 0; x < width; ++x) o[x] += s[x];
        }
    }
}

void orc_merge_qkv(float* packed, const float* q, const float* k, const float* v,
                   uint32_t head_dim, uint32_t tokens, uint32_t n_head) {
    const uint32_t dC = head_dim * n_head;
    for (uint32_t r = 0; r < tokens; ++r)
        for (uint32_t h = 0; h < n_head; ++h) {
            const size_t so = ((size_t)h * tokens + r) * head_dim;
            float* p = packed + (size_t)r * 3u * dC + (size_t)h * head_dim;
            memcpy(p, q + so, sizeof(float) * head_dim);
            memcpy(p + dC, k + so, sizeof(float) * head_dim);
            memcpy(p + 2u * dC, v + so, sizeof(float) * head_dim);
        }
}

/* Row maximum (first element, then strict '>') and the sequential sum of exp(z - max). */
static void cce_row(const float* z, uint32_t vocab, float* mx, float* sum) {
    float m = z[0];
    for (uint32_t i = 1; i < vocab; ++i)
        if (z[i] > m) m = z[i];
    float s = 0.0f;
    for (uint32_t i = 0; i < vocab; ++i) s += expf(z[i] - m);
    *mx = m;
    *sum = s;
}

float orc_cce_logits(float* grad, const float* target, const float* logits, uint32_t vocab,
                     uint32_t steps, uint32_t batch, uint32_t target_cols, uint32_t target_batch) {
    float total = 0.0f;
    if (target_cols == 1) {
        uint32_t valid = 0;
        for (uint32_t z = 0; z < batch; ++z)
            for (uint32_t t = 0; t < steps; ++t)
                if ((int32_t)target[(size_t)(target_batch == 1 ? 0 : z) * steps + t] != -1) ++valid;
        const float inv_valid = valid > 0 ? 1.0f / (float)valid : 0.0f;
        for (uint32_t z = 0; z < batch; ++z)
            for (uint32_t t = 0; t < steps; ++t) {
                const int32_t id = (int32_t)target[(size_t)(target_batch == 1 ? 0 : z) * steps + t];
                const float* lz = logits + ((size_t)z * steps + t) * vocab;
                float* g = grad ? grad + ((size_t)z * steps + t) * vocab : NULL;
                if (id == -1) {
                    if (g)
                        for (uint32_t i = 0; i < vocab; ++i) g[i] = 0.0f;
                    continue;
                }
                float m, s;
                cce_row(lz, vocab, &m, &s);
                if (g)
                    for (uint32_t i = 0; i < vocab; ++i) {
                        const float p = expf(lz[i] - m) / s;
                        const float ti = (uint32_t)id == i ? 1.0f : 0.0f;
                        g[i] = (ti - p) * inv_valid;
                    }
                total += ((m + logf(s)) - lz[id]);
            }
        return valid ? total / (float)valid : 0.0f;
    }
    for (uint32_t z = 0; z < batch; ++z)
        for (uint32_t t = 0; t < steps; ++t) {
            const float* tg = target + ((size_t)(target_batch == 1 ? 0 : z) * steps + t) * vocab;
            const float* lz = logits + ((size_t)z * steps + t) * vocab;
            float m, s;
            cce_row(lz, vocab, &m, &s);
            if (grad) {
                float* g = grad + ((size_t)z * steps + t) * vocab;
                for (uint32_t i = 0; i < vocab; ++i) g[i] = tg[i] - expf(lz[i] - m) / s;
            }
            for (uint32_t i = 0; i < vocab; ++i)
                if (tg[i] > 0.5f) {
                    total += ((m + logf(s)) - lz[i]);
                    break;
                }
        }
    return total;
}

void orc_adamw_update(float* param, const float* grad, float* mt, float* vt, uint32_t n, float lr,
                      float beta1, float beta2, float beta1_pow_t, float beta2_pow_t, float eps,
                      float weight_decay) {
    const float inv_b1 = 1.0f - beta1, inv_b2 = 1.0f - beta2;
    const float inv_b1p = 1.0f - beta1_pow_t, inv_b2p = 1.0f - beta2_pow_t;
    for (uint32_t i = 0; i < n; ++i) {
        const float g = grad[i];
        const float m = beta1 * mt[i] + inv_b1 * g;
        const float v = beta2 * vt[i] + inv_b2 * g * g;
        mt[i] = m;
        vt[i] = v;
        const float m_hat = m / inv_b1p;
        const float v_hat = v / inv_b2p;
        const float p = param[i];
        const float update = lr * m_hat / (sqrtf(v_hat) + eps);
        const float decay = lr * weight_decay * p;
        param[i] = p + update - decay;
    }
}

/* SumColumns: the reference's column loop, rows added in order (MatrixBase_Functions.h:1109-1117). */
void orc_sum_columns(float* out, const float* in, uint32_t rows, uint32_t cols) {
    for (uint32_t c = 0; c < cols; ++c) {
        float sum = 0.0f;
        for (uint32_t r = 0; r < rows; ++r) sum += in[(size_t)r * cols + c];
        out[c] = sum;
    }
}

/* UpdateMask's three branches (DropoutLayer.h:105-122): Fill(one), Fill(zero), or one buffered
 * uniform per element in element order. */
uint64_t orc_dropout_mask(float* mask, uint64_t n, const float* uniforms, uint64_t count, uint64_t start,
                          float prob) {
    if (n == 0) return 0;
    if (prob <= 0.0f || prob >= 1.0f) {
        for (uint64_t i = 0; i < n; ++i) mask[i] = prob <= 0.0f ? 1.0f : 0.0f;
        return 0;
    }
    for (uint64_t i = 0; i < n; ++i) mask[i] = uniforms[(start + i) % count] < prob ? 0.0f : 1.0f;
    return n;
}
