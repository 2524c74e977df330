/*
 * ssa_oracle.c -- CPU restatement of the SSA forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (package ssa_amd) never
 * links, loads or calls it.
 *
 * What it restates (reference = chenxingqiang/SSA):
 *   oracle_normalize      F.normalize(x, dim=-1)            ssa/router.py:116-118
 *   oracle_route_vectors  W_qr/W_kr projection, GQA mean,   ssa/router.py:102-117
 *                         then normalize
 *   oracle_code_topk      codebook scoring / temperature,   ssa/router.py:121-130,141
 *                         top-b (keys) and top-a (queries)  (get_code_assignment :261-275)
 *   oracle_build_index    inverted index code -> keys       (no reference counterpart; its
 *                                                           set is ssa/router.py:224-235)
 *   oracle_select         candidate set, full rescoring,    ssa/router.py:151-259
 *                         top-k with filler and zero pad
 *   oracle_sparse_attention  gathered exact softmax . V     ssa/attention.py:12-115
 *   oracle_dense_attention   dense SDPA with GQA expand     ssa/attention.py:118-158
 *   oracle_sparse_attention_backward  d/dq, d/dk, d/dv of   ssa/attention.py:64-113
 *                         oracle_sparse_attention (the reference's autograd of
 *                         gather -> einsum -> / scale -> softmax -> einsum)
 *
 * Canonical arithmetic contract (the HIP kernels reproduce it bit for bit):
 *   - every score is fp32; inputs (bf16 or fp32) are widened exactly to fp32;
 *   - a dot product over a dimension is ONE fmaf chain in ascending index
 *     order starting from +0.0f: acc = fmaf(x[t], y[t], acc);
 *   - the GQA mean over g heads is  s = p_0; s = s + p_1; ... ; s / (float)g;
 *   - normalize: r = sqrtf(chain(x*x)); x / fmaxf(r, 1e-12f)  (IEEE div/sqrt);
 *   - rescoring divides each per-head dot by score_div = (float)sqrt(d) before
 *     the GQA mean (ssa/router.py:180-182,191);
 *   - selections order by (score desc, index asc): the composite key
 *     (ordered_bits(score) << 32) | (0xFFFFFFFF - index), -0.0 folded into +0.0;
 *   - fewer than k candidates: the remaining slots take the lowest indices
 *     that are not candidates, ascending (the reference leaves these -inf
 *     slots unspecified, ssa/router.py:200-204); k > n pads with index 0
 *     (ssa/router.py:206-211).
 *
 * Attention outputs are computed in double precision (tolerance checks only).
 * Build: see oracle/Makefile.  Compile WITHOUT -ffast-math and with
 * -ffp-contract=off so that only the explicit fmaf calls fuse.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_VERSION 1

#if defined(__x86_64__)
#define HOT __attribute__((target_clones("fma", "default")))
#else
#define HOT
#endif

int oracle_version(void) { return ORACLE_VERSION; }

void oracle_set_threads(int t) {
#ifdef _OPENMP
  if (t > 0) omp_set_num_threads(t);
#else
  (void)t;
#endif
}

int oracle_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* Monotone float -> uint32 map: a > b (as reals) <=> key(a) > key(b); -0 == +0. */
uint32_t oracle_score_key(float s) {
  uint32_t u = f2u(s);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static inline uint64_t composite(float s, int64_t idx) {
  return ((uint64_t)oracle_score_key(s) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

static int cmp_desc_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return (x < y) - (x > y);
}

/* ---------------------------------------------------------------- stage (a) */

/* x[d_s] -> x / max(||x||, 1e-12), ||x|| = sqrtf(fmaf chain of x*x).
 * Restates F.normalize(x, dim=-1) (ssa/router.py:116-118). */
HOT static void normalize_vec(const float* x, int d_s, float* out) {
  float acc = 0.0f;
  for (int s = 0; s < d_s; ++s) acc = fmaf(x[s], x[s], acc);
  float den = fmaxf(sqrtf(acc), 1e-12f);
  for (int s = 0; s < d_s; ++s) out[s] = x[s] / den;
}

void oracle_normalize(const float* x, int64_t rows, int d_s, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) normalize_vec(x + r * d_s, d_s, out + r * d_s);
}

/* Routing vectors for one batch element.
 *   x   [n][h_in][d]  (fp32, contiguous)
 *   w   [d_s][d]      (nn.Linear weight, ssa/router.py:61-62)
 *   out [h_in/group][n][d_s]
 * out[h][i] = normalize( (sum_{gg<group} x[i][h*group+gg] . w^T) / group ).
 * Projection before the group mean, as ssa/router.py:102,111-112. */
HOT void oracle_route_vectors(const float* x, int64_t n, int h_in, int group, int d,
                              const float* w, int d_s, float* out) {
  int h_out = h_in / group;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < (int64_t)h_out * n; ++r) {
    int h = (int)(r / n);
    int64_t i = r % n;
    float tmp[1024];
    for (int s = 0; s < d_s; ++s) {
      const float* wr = w + (int64_t)s * d;
      float sum = 0.0f;
      for (int gg = 0; gg < group; ++gg) {
        const float* xr = x + (i * h_in + (int64_t)h * group + gg) * d;
        float acc = 0.0f;
        for (int t = 0; t < d; ++t) acc = fmaf(xr[t], wr[t], acc);
        sum = (gg == 0) ? acc : sum + acc;
      }
      tmp[s] = sum / (float)group;
    }
    normalize_vec(tmp, d_s, out + r * d_s);
  }
}

/* Codebook scoring and top-`top` selection.
 *   xhat  [h][rows][d_s]   normalized routing vectors
 *   chat  [h][n_c][d_s]    normalized codebook
 *   codes [h][rows][top]   (score desc, code asc)
 *   scores (nullable) [h][rows][top]
 * score(c) = chain_s fmaf(xhat[s], chat[c][s]); divided by temperature unless it is 1.
 * Restates ssa/router.py:121-130 (keys, top-b) and :121-122,141 (queries, top-a). */
HOT void oracle_code_topk(const float* xhat, int h, int64_t rows, const float* chat, int n_c,
                          int d_s, float temperature, int top, int32_t* codes, float* scores) {
#pragma omp parallel
  {
    uint64_t* best = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(top + 1));
    float* sc = (float*)malloc(sizeof(float) * (size_t)n_c);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < (int64_t)h * rows; ++r) {
      int hh = (int)(r / rows);
      const float* q = xhat + r * d_s;
      const float* cb = chat + (int64_t)hh * n_c * d_s;
      int cnt = 0;
      for (int c = 0; c < n_c; ++c) {
        const float* cr = cb + (int64_t)c * d_s;
        float acc = 0.0f;
        for (int s = 0; s < d_s; ++s) acc = fmaf(q[s], cr[s], acc);
        if (temperature != 1.0f) acc = acc / temperature;
        sc[c] = acc;
        uint64_t key = composite(acc, c);
        if (cnt == top && key <= best[top - 1]) continue;
        int p = (cnt < top) ? cnt++ : top - 1;
        while (p > 0 && best[p - 1] < key) {
          best[p] = best[p - 1];
          --p;
        }
        best[p] = key;
      }
      for (int m = 0; m < top; ++m) {
        int32_t c = (int32_t)(0xFFFFFFFFu - (uint32_t)(best[m] & 0xFFFFFFFFu));
        codes[r * top + m] = c;
        if (scores) scores[r * top + m] = sc[c];
      }
    }
    free(best);
    free(sc);
  }
}

/* ---------------------------------------------------------------- stage (b) */

/* Inverted index for one batch element.
 *   k_codes  [h][n][b]
 *   offsets  [h][n_c+1]   exclusive prefix of bucket sizes
 *   postings [h][n*b]     key indices, ascending inside each bucket
 * A key j is in bucket c of head h iff c is one of k_codes[h][j][:], i.e. the
 * key side of the candidate-set definition in ssa/router.py:224-235,255-256. */
void oracle_build_index(const int32_t* k_codes, int h, int64_t n, int b, int n_c,
                        int32_t* offsets, int32_t* postings) {
  for (int hh = 0; hh < h; ++hh) {
    const int32_t* kc = k_codes + (int64_t)hh * n * b;
    int32_t* off = offsets + (int64_t)hh * (n_c + 1);
    int32_t* post = postings + (int64_t)hh * n * b;
    memset(off, 0, sizeof(int32_t) * (size_t)(n_c + 1));
    for (int64_t e = 0; e < n * b; ++e) off[kc[e] + 1]++;
    for (int c = 0; c < n_c; ++c) off[c + 1] += off[c];
    int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)n_c);
    memcpy(cur, off, sizeof(int32_t) * (size_t)n_c);
    for (int64_t e = 0; e < n * b; ++e) post[cur[kc[e]]++] = (int32_t)(e / b);
    free(cur);
  }
}

/* ---------------------------------------------------------------- stage (c) */

/* Canonical rescoring of key j for query row (i, h):
 *   mean over gg of ( chain_t fmaf(q[i][h*g+gg][t], k[j][h][t]) / score_div ).
 * Restates ssa/router.py:177-191. */
HOT static float rescore(const float* qrow /*[g][d]*/, const float* krow /*[d]*/, int g, int d,
                         float score_div) {
  float sum = 0.0f;
  for (int gg = 0; gg < g; ++gg) {
    const float* qr = qrow + (int64_t)gg * d;
    float acc = 0.0f;
    for (int t = 0; t < d; ++t) acc = fmaf(qr[t], krow[t], acc);
    float s = acc / score_div;
    sum = (gg == 0) ? s : sum + s;
  }
  return sum / (float)g;
}

/* Candidate selection for one batch element.
 *   q [n][h_q][d], k [n][h_kv][d]        fp32 (bf16 values widened)
 *   q_codes [h_kv][n][a], offsets/postings as oracle_build_index (b codes per key)
 *   mask_mode 0: no mask; 1: causal (j <= i); 2: dense bool mask[i*n + j]
 *   rows (nullable): query positions to evaluate (else 0..n-1), n_rows of them
 *   out [n_rows][h_kv][top_k] int64
 *   n_cand (nullable) [n_rows][h_kv]: |candidate set|; n_raw (nullable): postings read
 *     (for causal: postings with j <= i)
 *   sorted != 0 lists the selected keys by (score desc, index asc); 0 lists the
 *     same set ascending (torch.topk(sorted=False)-style), before the filler
 * Candidate set (ssa/router.py:224-235): keys sharing >= 1 code with the query and
 * allowed by the mask.  Ranking by canonical rescoring; filler and pad as the
 * file header states. */
static int cmp_asc_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return (x > y) - (x < y);
}

HOT void oracle_select(const float* q, const float* k, int64_t n, int h_q, int h_kv, int d,
                       const int32_t* q_codes, int a, const int32_t* offsets,
                       const int32_t* postings, int n_c, int b, int top_k, int mask_mode,
                       const uint8_t* mask, float score_div, int sorted, const int64_t* rows,
                       int64_t n_rows, int64_t* out, int32_t* n_cand, int32_t* n_raw) {
  int g = h_q / h_kv;
  int64_t k_eff = top_k < n ? top_k : n;
  int64_t nrow = rows ? n_rows : n;
#pragma omp parallel
  {
    uint32_t* bitmap = (uint32_t*)calloc((size_t)(n + 31) / 32, sizeof(uint32_t));
    uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(n > 0 ? n : 1));
    int64_t* list = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n > 0 ? n : 1));
    float* qrow = (float*)malloc(sizeof(float) * (size_t)g * d);
#pragma omp for schedule(dynamic, 16)
    for (int64_t rr = 0; rr < nrow * h_kv; ++rr) {
      int64_t ri = rr / h_kv;
      int h = (int)(rr % h_kv);
      int64_t i = rows ? rows[ri] : ri;
      const int32_t* qc = q_codes + ((int64_t)h * n + i) * a;
      const int32_t* off = offsets + (int64_t)h * (n_c + 1);
      const int32_t* hp = postings + (int64_t)h * n * b;
      int64_t C = 0, R = 0;
      for (int m = 0; m < a; ++m) {
        int c = qc[m];
        for (int32_t p = off[c]; p < off[c + 1]; ++p) {
          int64_t j = hp[p];
          if (mask_mode == 1 && j > i) break; /* postings ascend inside a bucket */
          ++R;
          if (mask_mode == 2 && !mask[i * n + j]) continue;
          uint32_t bit = 1u << (j & 31);
          if (bitmap[j >> 5] & bit) continue;
          bitmap[j >> 5] |= bit;
          list[C++] = j;
        }
      }
      for (int gg = 0; gg < g; ++gg)
        memcpy(qrow + (int64_t)gg * d, q + (i * h_q + (int64_t)h * g + gg) * d,
               sizeof(float) * (size_t)d);
      for (int64_t m = 0; m < C; ++m) {
        int64_t j = list[m];
        float s = rescore(qrow, k + (j * h_kv + h) * d, g, d, score_div);
        keys[m] = composite(s, j);
      }
      qsort(keys, (size_t)C, sizeof(uint64_t), cmp_desc_u64);
      int64_t* o = out + rr * top_k;
      int64_t w = 0;
      for (; w < C && w < k_eff; ++w) o[w] = (int64_t)(0xFFFFFFFFu - (uint32_t)(keys[w] & 0xFFFFFFFFu));
      if (!sorted) qsort(o, (size_t)w, sizeof(int64_t), cmp_asc_i64);
      for (int64_t j = 0; w < k_eff && j < n; ++j)
        if (!(bitmap[j >> 5] & (1u << (j & 31)))) o[w++] = j;
      for (; w < top_k; ++w) o[w] = 0;
      if (n_cand) n_cand[rr] = (int32_t)C;
      if (n_raw) n_raw[rr] = (int32_t)R;
      for (int64_t m = 0; m < C; ++m) bitmap[list[m] >> 5] = 0u;
    }
    free(bitmap);
    free(keys);
    free(list);
    free(qrow);
  }
}

/* ---------------------------------------------------------------- stage (d) */

/* Gathered exact attention for one batch element, in double precision.
 *   idx [n][h_kv][kk] int64, or [n_rows][h_kv][kk] aligned with `rows` when rows
 *   is given; out [n_rows][h_q][d] double.
 * logits = q . K[idx] / scale_div (scale is a divisor, ssa/attention.py:37-38,107),
 * softmax over the kk slots (duplicates count twice, no mask: ssa/attention.py:109),
 * out = p . V[idx] (ssa/attention.py:112).  causal != 0 additionally drops slots with
 * idx > i (an extension); a row with every slot dropped outputs zeros. */
void oracle_sparse_attention(const float* q, const float* k, const float* v, int64_t n, int h_q,
                             int h_kv, int d, const int64_t* idx, int kk, double scale_div,
                             int causal, const int64_t* rows, int64_t n_rows, double* out) {
  int g = h_q / h_kv;
  int64_t nrow = rows ? n_rows : n;
#pragma omp parallel
  {
    double* lg = (double*)malloc(sizeof(double) * (size_t)(kk > 0 ? kk : 1));
#pragma omp for schedule(static)
    for (int64_t rr = 0; rr < nrow * h_q; ++rr) {
      int64_t ri = rr / h_q;
      int hq = (int)(rr % h_q);
      int h = hq / g;
      int64_t i = rows ? rows[ri] : ri;
      const float* qr = q + (i * h_q + hq) * d;
      const int64_t* ix = idx + ((rows ? ri : i) * h_kv + h) * kk;
      double mx = -INFINITY;
      for (int m = 0; m < kk; ++m) {
        int64_t j = ix[m];
        if (causal && j > i) {
          lg[m] = -INFINITY;
          continue;
        }
        const float* kr = k + (j * h_kv + h) * d;
        double acc = 0.0;
        for (int t = 0; t < d; ++t) acc += (double)qr[t] * (double)kr[t];
        lg[m] = acc / scale_div;
        if (lg[m] > mx) mx = lg[m];
      }
      double* o = out + rr * d;
      for (int t = 0; t < d; ++t) o[t] = 0.0;
      if (mx == -INFINITY) continue;
      double den = 0.0;
      for (int m = 0; m < kk; ++m) {
        if (lg[m] == -INFINITY) continue;
        double p = exp(lg[m] - mx);
        den += p;
        const float* vr = v + (ix[m] * h_kv + h) * d;
        for (int t = 0; t < d; ++t) o[t] += p * (double)vr[t];
      }
      for (int t = 0; t < d; ++t) o[t] /= den;
    }
    free(lg);
  }
}

/* Gradients of oracle_sparse_attention for one batch element (double precision),
 * given dout [n][h_q][d]: the chain rule through ssa/attention.py:64-113 (gather
 * :70-100, logits / scale :107, softmax :109, p . V :112).  With p the softmax
 * of a (query, head) row over its slots, o = sum p v and D = dout . o:
 *   dv[idx_m] += p_m dout;  ds_m = p_m (dout . v[idx_m] - D);
 *   dq += ds_m k[idx_m] / scale;  dk[idx_m] += ds_m q / scale.
 * A slot repeated in idx contributes once per slot; causal != 0 drops slots
 * with idx > i.  Indices must lie in [0, n).  dq [n][h_q][d], dk, dv
 * [n][h_kv][d] are overwritten.  One thread per kv head (dk, dv of a head are
 * written by its thread only). */
void oracle_sparse_attention_backward(const float* q, const float* k, const float* v, int64_t n,
                                      int h_q, int h_kv, int d, const int64_t* idx, int kk,
                                      double scale_div, int causal, const double* dout,
                                      double* dq, double* dk, double* dv) {
  int g = h_q / h_kv;
  memset(dq, 0, sizeof(double) * (size_t)(n * h_q * d));
  memset(dk, 0, sizeof(double) * (size_t)(n * h_kv * d));
  memset(dv, 0, sizeof(double) * (size_t)(n * h_kv * d));
#pragma omp parallel
  {
    double* pr = (double*)malloc(sizeof(double) * (size_t)(kk > 0 ? kk : 1));
    double* o = (double*)malloc(sizeof(double) * (size_t)d);
#pragma omp for schedule(static)
    for (int h = 0; h < h_kv; ++h) {
      for (int64_t i = 0; i < n; ++i) {
        const int64_t* ix = idx + (i * h_kv + h) * kk;
        for (int hq = h * g; hq < (h + 1) * g; ++hq) {
          const float* qr = q + (i * h_q + hq) * d;
          const double* dor = dout + (i * h_q + hq) * d;
          double mx = -INFINITY;
          for (int m = 0; m < kk; ++m) {
            int64_t j = ix[m];
            if (causal && j > i) {
              pr[m] = -INFINITY;
              continue;
            }
            const float* kr = k + (j * h_kv + h) * d;
            double acc = 0.0;
            for (int t = 0; t < d; ++t) acc += (double)qr[t] * (double)kr[t];
            pr[m] = acc / scale_div;
            if (pr[m] > mx) mx = pr[m];
          }
          if (mx == -INFINITY) continue;  /* no slot: zero output, zero gradients */
          double den = 0.0;
          for (int m = 0; m < kk; ++m) {
            if (pr[m] == -INFINITY) {
              pr[m] = 0.0;
              continue;
            }
            pr[m] = exp(pr[m] - mx);
            den += pr[m];
          }
          for (int t = 0; t < d; ++t) o[t] = 0.0;
          for (int m = 0; m < kk; ++m) {
            pr[m] /= den;
            if (pr[m] == 0.0) continue;
            const float* vr = v + (ix[m] * h_kv + h) * d;
            for (int t = 0; t < d; ++t) o[t] += pr[m] * (double)vr[t];
          }
          double dd = 0.0;
          for (int t = 0; t < d; ++t) dd += dor[t] * o[t];
          double* dqr = dq + (i * h_q + hq) * d;
          for (int m = 0; m < kk; ++m) {
            int64_t j = ix[m];
            if (causal && j > i) continue;
            const float* kr = k + (j * h_kv + h) * d;
            const float* vr = v + (j * h_kv + h) * d;
            double dp = 0.0;
            for (int t = 0; t < d; ++t) dp += dor[t] * (double)vr[t];
            double ds = pr[m] * (dp - dd);
            double* dkr = dk + (j * h_kv + h) * d;
            double* dvr = dv + (j * h_kv + h) * d;
            for (int t = 0; t < d; ++t) {
              dqr[t] += ds * (double)kr[t] / scale_div;
              dkr[t] += ds * (double)qr[t] / scale_div;
              dvr[t] += pr[m] * dor[t];
            }
          }
        }
      }
    }
    free(pr);
    free(o);
  }
}

/* Dense attention for one batch element (double precision), ssa/attention.py:118-158.
 * causal != 0 applies the lower-triangular mask (build_causal_mask, ssa/utils.py:75-86). */
void oracle_dense_attention(const float* q, const float* k, const float* v, int64_t n, int h_q,
                            int h_kv, int d, double scale_div, int causal, double* out) {
  int g = h_q / h_kv;
#pragma omp parallel
  {
    double* lg = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
#pragma omp for schedule(static)
    for (int64_t rr = 0; rr < n * h_q; ++rr) {
      int64_t i = rr / h_q;
      int hq = (int)(rr % h_q);
      int h = hq / g;
      const float* qr = q + (i * h_q + hq) * d;
      int64_t jend = causal ? i + 1 : n;
      double mx = -INFINITY;
      for (int64_t j = 0; j < jend; ++j) {
        const float* kr = k + (j * h_kv + h) * d;
        double acc = 0.0;
        for (int t = 0; t < d; ++t) acc += (double)qr[t] * (double)kr[t];
        lg[j] = acc / scale_div;
        if (lg[j] > mx) mx = lg[j];
      }
      double* o = out + rr * d;
      for (int t = 0; t < d; ++t) o[t] = 0.0;
      double den = 0.0;
      for (int64_t j = 0; j < jend; ++j) {
        double p = exp(lg[j] - mx);
        den += p;
        const float* vr = v + (j * h_kv + h) * d;
        for (int t = 0; t < d; ++t) o[t] += p * (double)vr[t];
      }
      for (int t = 0; t < d; ++t) o[t] /= den;
    }
    free(lg);
  }
}
