/*
 * moe_oracle.c -- plain-C restatement of the contest reference
 * full-agent-pipeline/references/moe.py (function `run`, moe.py:28-202).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): this is the checker the HIP path is
 * compared with, and the CPU baseline the benchmark reports.  It is never part
 * of the product path.
 *
 * Arithmetic follows moe.py op by op, in fp32:
 *   dequantisation   A = fp32(a) * scale            (moe.py:95-104)
 *                    W = fp32(w) * scale            (moe.py:107-118)
 *   sigmoid          s = 1 / (1 + exp(-x))          (moe.py:127)
 *   biased score     sb = s + bias                  (moe.py:128)
 *   group score      top-2 sum per group of 32      (moe.py:135-136)
 *   group choice     top-4 of 8 groups              (moe.py:139-146)
 *   expert choice    top-8 of sb, other groups -> finfo.min (moe.py:149-151)
 *   weights          (s / (sum_8 s + 1e-20)) * rsf  (moe.py:154-158)
 *   per local expert G1 = A_e W13_e^T; C = X2/(1+exp(-X2)) * X1 with
 *                    X1 = G1[:, :I], X2 = G1[:, I:]; O = C W2_e^T;
 *                    out += O * w   (ascending local expert)  (moe.py:168-200)
 *   cast             out.to(bfloat16)               (moe.py:202)
 * Where moe.py leaves an order open this file fixes one and says so:
 *   - topk: torch's CPU selection algorithm is restated (q_nth_element), so
 *     exact ties resolve as the reference resolves them;
 *   - the 8 weights are summed in ascending expert-id order (torch's
 *     vectorised sum order depends on the host's SIMD width);
 *   - dot products accumulate in 16 interleaved fp32 partial sums (FMA).
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------------------------------------------------------------- */
/* routing (moe.py:123-158)                                                */
/* ---------------------------------------------------------------------- */
/* torch.topk(..., sorted=False) on CPU (torch 2.10.0, the reference's pin in
 * full-agent-pipeline/uv.lock) fills a queue of (value, index) pairs in index
 * order and calls std::nth_element(q, q + k - 1, q_end, greater) (GCC 11
 * libstdc++: introselect = median-of-3 unguarded partitions, insertion sort
 * below 4 elements, heap-select fallback at depth 2*floor(log2 n)); the first k
 * queue entries are the result.  The selected set, including how exact ties are
 * resolved, therefore follows that algorithm, restated here. */
typedef struct {
  double v;
  int i;
} qe_t;

static inline int q_greater(const qe_t* x, const qe_t* y) {
  return (isnan(x->v) && !isnan(y->v)) || (x->v > y->v);
}
static inline void q_swap(qe_t* a, qe_t* b) {
  qe_t t = *a;
  *a = *b;
  *b = t;
}

static void q_push_heap(qe_t* first, long hole, long top, qe_t value) {
  long parent = (hole - 1) / 2;
  while (hole > top && q_greater(first + parent, &value)) {
    first[hole] = first[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  first[hole] = value;
}

static void q_adjust_heap(qe_t* first, long hole, long len, qe_t value) {
  const long top = hole;
  long child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (q_greater(first + child, first + (child - 1))) child--;
    first[hole] = first[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    first[hole] = first[child - 1];
    hole = child - 1;
  }
  q_push_heap(first, hole, top, value);
}

static void q_make_heap(qe_t* first, qe_t* last) {
  const long len = last - first;
  if (len < 2) return;
  long parent = (len - 2) / 2;
  for (;;) {
    q_adjust_heap(first, parent, len, first[parent]);
    if (parent == 0) return;
    parent--;
  }
}

static void q_heap_select(qe_t* first, qe_t* middle, qe_t* last) {
  q_make_heap(first, middle);
  for (qe_t* i = middle; i < last; ++i)
    if (q_greater(i, first)) {
      /* pop_heap(first, middle, i) */
      qe_t value = *i;
      *i = *first;
      q_adjust_heap(first, 0, middle - first, value);
    }
}

static void q_move_median_to_first(qe_t* result, qe_t* a, qe_t* b, qe_t* c) {
  if (q_greater(a, b)) {
    if (q_greater(b, c))
      q_swap(result, b);
    else if (q_greater(a, c))
      q_swap(result, c);
    else
      q_swap(result, a);
  } else if (q_greater(a, c))
    q_swap(result, a);
  else if (q_greater(b, c))
    q_swap(result, c);
  else
    q_swap(result, b);
}

static qe_t* q_unguarded_partition(qe_t* first, qe_t* last, qe_t* pivot) {
  for (;;) {
    while (q_greater(first, pivot)) ++first;
    --last;
    while (q_greater(pivot, last)) --last;
    if (!(first < last)) return first;
    q_swap(first, last);
    ++first;
  }
}

static void q_insertion_sort(qe_t* first, qe_t* last) {
  if (first == last) return;
  for (qe_t* i = first + 1; i != last; ++i) {
    if (q_greater(i, first)) {
      qe_t val = *i;
      memmove(first + 1, first, (size_t)(i - first) * sizeof(qe_t));
      *first = val;
    } else {
      qe_t val = *i;
      qe_t* hole = i;
      qe_t* next = i - 1;
      while (q_greater(&val, next)) {
        *hole = *next;
        hole = next;
        --next;
      }
      *hole = val;
    }
  }
}

static int q_lg(long n) {
  int r = 0;
  while (n >>= 1) r++;
  return r;
}

static void q_nth_element(qe_t* first, qe_t* nth, qe_t* last) {
  if (first == last || nth == last) return;
  int depth = 2 * q_lg(last - first);
  while (last - first > 3) {
    if (depth == 0) {
      q_heap_select(first, nth + 1, last);
      q_swap(first, nth);
      return;
    }
    --depth;
    qe_t* mid = first + (last - first) / 2;
    q_move_median_to_first(first, first + 1, mid, last - 1);
    qe_t* cut = q_unguarded_partition(first + 1, last, first);
    if (cut <= nth)
      first = cut;
    else
      last = cut;
  }
  q_insertion_sort(first, last);
}

static int int_cmp(const void* a, const void* b) {
  return (*(const int32_t*)a > *(const int32_t*)b) - (*(const int32_t*)a < *(const int32_t*)b);
}

static void route_one(const float* x, const float* bias_f, float rsf, int32_t* ids, float* w,
                      float* s_out, float* sb_out) {
  float s[ORC_E_GLOBAL], sb[ORC_E_GLOBAL];
  for (int e = 0; e < ORC_E_GLOBAL; ++e) {
    /* moe.py:127  s = 1.0 / (1.0 + torch.exp(-logits)) */
    const float ex = orc_exp_f32(-x[e]);
    s[e] = 1.0f / (1.0f + ex);
    /* moe.py:128  s_with_bias = s + bias */
    sb[e] = s[e] + bias_f[e];
  }
  if (s_out) memcpy(s_out, s, sizeof s);
  if (sb_out) memcpy(sb_out, sb, sizeof sb);

  /* moe.py:135-136  per-group top-2 sum (the two values; their order does not
   * change the fp32 sum) */
  qe_t gq[ORC_N_GROUP];
  for (int g = 0; g < ORC_N_GROUP; ++g) {
    float m1 = -INFINITY, m2 = -INFINITY;
    for (int j = 0; j < ORC_GROUP_SIZE; ++j) {
      const float v = sb[g * ORC_GROUP_SIZE + j];
      if (v > m1) {
        m2 = m1;
        m1 = v;
      } else if (v > m2) {
        m2 = v;
      }
    }
    gq[g].v = (double)(m1 + m2);
    gq[g].i = g;
  }
  /* moe.py:139-146  top-4 groups */
  q_nth_element(gq, gq + ORC_TOPK_GROUP - 1, gq + ORC_N_GROUP);
  int keep[ORC_N_GROUP] = {0};
  for (int j = 0; j < ORC_TOPK_GROUP; ++j) keep[gq[j].i] = 1;

  /* moe.py:149-151  top-8 over the kept groups (others masked to finfo.min) */
  qe_t cand[ORC_E_GLOBAL];
  for (int e = 0; e < ORC_E_GLOBAL; ++e) {
    cand[e].v = keep[e / ORC_GROUP_SIZE] ? (double)sb[e] : (double)-FLT_MAX;
    cand[e].i = e;
  }
  q_nth_element(cand, cand + ORC_TOP_K - 1, cand + ORC_E_GLOBAL);
  for (int k = 0; k < ORC_TOP_K; ++k) ids[k] = cand[k].i;
  qsort(ids, ORC_TOP_K, sizeof(int32_t), int_cmp);

  /* moe.py:154-158  weights from the un-biased s, normalised then scaled */
  float sum = 0.0f;
  for (int k = 0; k < ORC_TOP_K; ++k) sum = sum + s[ids[k]];
  const float denom = sum + 1e-20f;
  for (int k = 0; k < ORC_TOP_K; ++k) w[k] = (s[ids[k]] / denom) * rsf;
}

void orc_route(const float* logits, const uint16_t* bias, int64_t T, float rsf, int32_t* ids,
               float* w, float* s_out, float* sb_out) {
  float bias_f[ORC_E_GLOBAL];
  for (int e = 0; e < ORC_E_GLOBAL; ++e) bias_f[e] = orc_bf16_to_f32(bias[e]);
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t)
    route_one(logits + t * ORC_E_GLOBAL, bias_f, rsf, ids + t * ORC_TOP_K, w + t * ORC_TOP_K,
              s_out ? s_out + t * ORC_E_GLOBAL : NULL, sb_out ? sb_out + t * ORC_E_GLOBAL : NULL);
}

/* ---------------------------------------------------------------------- */
/* dense helpers                                                           */
/* ---------------------------------------------------------------------- */
static float dot_f32(const float* a, const float* b, int n) {
  float acc[16] = {0};
  int k = 0;
  for (; k + 16 <= n; k += 16)
    for (int j = 0; j < 16; ++j) acc[j] = fmaf(a[k + j], b[k + j], acc[j]);
  for (; k < n; ++k) acc[0] = fmaf(a[k], b[k], acc[0]);
  float s = 0.0f;
  for (int j = 0; j < 16; ++j) s = s + acc[j];
  return s;
}

static float e4m3_lut[256];
static int e4m3_lut_ready = 0;
static void ensure_lut(void) {
  if (e4m3_lut_ready) return;
  for (int i = 0; i < 256; ++i) e4m3_lut[i] = orc_e4m3_to_f32((uint8_t)i);
  e4m3_lut_ready = 1;
}

/* A row: fp32(a) * hidden_states_scale[k/128, t]   (moe.py:95-104) */
static void dequant_hidden_row(const uint8_t* hs, const float* hs_scale, int64_t T, int64_t t,
                               float* dst) {
  for (int k = 0; k < ORC_H; ++k)
    dst[k] = e4m3_lut[hs[t * ORC_H + k]] * hs_scale[(int64_t)(k / ORC_BLOCK) * T + t];
}

/* weight row r of expert le of a [E, R, C] tensor: fp32(w) * S[le, r/128, c/128] */
static void dequant_weight_row(const uint8_t* w, const float* s, int R, int C, int le, int r,
                               float* dst) {
  const uint8_t* src = w + ((int64_t)le * R + r) * C;
  const float* srow = s + ((int64_t)le * (R / ORC_BLOCK) + r / ORC_BLOCK) * (C / ORC_BLOCK);
  for (int c = 0; c < C; ++c) dst[c] = e4m3_lut[src[c]] * srow[c / ORC_BLOCK];
}

/* silu(x2) * x1 exactly as moe.py:190-193 */
static inline float swiglu(float x1, float x2) {
  const float silu = x2 / (1.0f + orc_exp_f32(-x2));
  return silu * x1;
}

/* G1 -> C -> O for n rows of one expert.  A: [n, H] fp32 rows.  Weights come
 * either from fp32 copies (w13f/w2f, dequant_all mode) or are dequantised per
 * row on the fly. */
static int expert_forward(const float* A, int64_t n, int le, const uint8_t* w13,
                          const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                          const float* w13f, const float* w2f, float* C /*[n, I]*/,
                          float* O /*[n, H] or NULL*/) {
  float* G1 = (float*)malloc(sizeof(float) * (size_t)n * ORC_2I);
  if (!G1) return -1;
  /* moe.py:187  G1 = A_e.matmul(W13_e.t()) */
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * ORC_H);
#pragma omp for schedule(static)
    for (int r = 0; r < ORC_2I; ++r) {
      const float* wr;
      if (w13f) {
        wr = w13f + ((int64_t)le * ORC_2I + r) * ORC_H;
      } else {
        dequant_weight_row(w13, w13_scale, ORC_2I, ORC_H, le, r, row);
        wr = row;
      }
      for (int64_t i = 0; i < n; ++i) G1[i * ORC_2I + r] = dot_f32(A + i * ORC_H, wr, ORC_H);
    }
    free(row);
  }
  /* moe.py:190-193 */
  for (int64_t i = 0; i < n; ++i)
    for (int d = 0; d < ORC_I; ++d)
      C[i * ORC_I + d] = swiglu(G1[i * ORC_2I + d], G1[i * ORC_2I + ORC_I + d]);
  free(G1);
  if (!O) return 0;
  /* moe.py:196  O = C.matmul(W2_e.t()) */
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * ORC_I);
#pragma omp for schedule(static)
    for (int h = 0; h < ORC_H; ++h) {
      const float* wr;
      if (w2f) {
        wr = w2f + ((int64_t)le * ORC_H + h) * ORC_I;
      } else {
        dequant_weight_row(w2, w2_scale, ORC_H, ORC_I, le, h, row);
        wr = row;
      }
      for (int64_t i = 0; i < n; ++i) O[i * ORC_H + h] = dot_f32(C + i * ORC_I, wr, ORC_I);
    }
    free(row);
  }
  return 0;
}

int orc_moe(const float* logits, const uint16_t* bias, const uint8_t* hs, const float* hs_scale,
            const uint8_t* w13, const float* w13_scale, const uint8_t* w2, const float* w2_scale,
            int64_t local_expert_offset, float rsf, int64_t T, const int32_t* tokens,
            int64_t n_tok, uint16_t* out, int dequant_all) {
  ensure_lut();
  if (!tokens) n_tok = T;
  int rc = -1;
  int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_tok > 0 ? n_tok : 1));
  float* acc = (float*)calloc((size_t)(n_tok > 0 ? n_tok : 1) * ORC_H, sizeof(float));
  int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_tok > 0 ? n_tok : 1) * ORC_TOP_K);
  float* wts = (float*)malloc(sizeof(float) * (size_t)(n_tok > 0 ? n_tok : 1) * ORC_TOP_K);
  float* lg = (float*)malloc(sizeof(float) * (size_t)(n_tok > 0 ? n_tok : 1) * ORC_E_GLOBAL);
  float *w13f = NULL, *w2f = NULL;
  if (!tok || !acc || !ids || !wts || !lg) goto done;
  for (int64_t i = 0; i < n_tok; ++i) tok[i] = tokens ? tokens[i] : (int32_t)i;

  if (dequant_all) {
    /* moe.py:107-118: fp32 copies of every local expert's weights */
    w13f = (float*)malloc(sizeof(float) * (size_t)ORC_E_LOCAL * ORC_2I * ORC_H);
    w2f = (float*)malloc(sizeof(float) * (size_t)ORC_E_LOCAL * ORC_H * ORC_I);
    if (!w13f || !w2f) goto done;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)ORC_E_LOCAL * ORC_2I; ++r)
      dequant_weight_row(w13, w13_scale, ORC_2I, ORC_H, (int)(r / ORC_2I), (int)(r % ORC_2I),
                         w13f + r * ORC_H);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)ORC_E_LOCAL * ORC_H; ++r)
      dequant_weight_row(w2, w2_scale, ORC_H, ORC_I, (int)(r / ORC_H), (int)(r % ORC_H),
                         w2f + r * ORC_I);
  }

  /* routing of the requested tokens (rows are independent) */
  for (int64_t i = 0; i < n_tok; ++i)
    memcpy(lg + i * ORC_E_GLOBAL, logits + (int64_t)tok[i] * ORC_E_GLOBAL,
           sizeof(float) * ORC_E_GLOBAL);
  orc_route(lg, bias, n_tok, rsf, ids, wts, NULL, NULL);

  /* moe.py:168-200: per local expert, ascending */
  for (int le = 0; le < ORC_E_LOCAL; ++le) {
    const int64_t ge = local_expert_offset + le;
    if (ge < 0 || ge >= ORC_E_GLOBAL) continue;
    int64_t n = 0;
    for (int64_t i = 0; i < n_tok; ++i)
      for (int k = 0; k < ORC_TOP_K; ++k)
        if (ids[i * ORC_TOP_K + k] == ge) n++;
    if (n == 0) continue;
    int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
    float* wsel = (float*)malloc(sizeof(float) * (size_t)n);
    float* A = (float*)malloc(sizeof(float) * (size_t)n * ORC_H);
    float* C = (float*)malloc(sizeof(float) * (size_t)n * ORC_I);
    float* O = (float*)malloc(sizeof(float) * (size_t)n * ORC_H);
    if (!rows || !wsel || !A || !C || !O) {
      free(rows), free(wsel), free(A), free(C), free(O);
      goto done;
    }
    int64_t j = 0;
    for (int64_t i = 0; i < n_tok; ++i)
      for (int k = 0; k < ORC_TOP_K; ++k)
        if (ids[i * ORC_TOP_K + k] == ge) {
          rows[j] = i;
          wsel[j] = wts[i * ORC_TOP_K + k];
          j++;
        }
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) dequant_hidden_row(hs, hs_scale, T, tok[rows[r]], A + r * ORC_H);
    if (expert_forward(A, n, le, w13, w13_scale, w2, w2_scale, w13f, w2f, C, O) != 0) {
      free(rows), free(wsel), free(A), free(C), free(O);
      goto done;
    }
    /* moe.py:199-200  output.index_add_(0, token_idx, O * w_tok) */
    for (int64_t r = 0; r < n; ++r) {
      float* dst = acc + rows[r] * ORC_H;
      const float wr = wsel[r];
      for (int h = 0; h < ORC_H; ++h) {
        const float p = O[r * ORC_H + h] * wr;
        dst[h] = dst[h] + p;
      }
    }
    free(rows), free(wsel), free(A), free(C), free(O);
  }
  /* moe.py:202 */
  for (int64_t i = 0; i < n_tok * ORC_H; ++i) out[i] = orc_f32_to_bf16(acc[i]);
  rc = 0;
done:
  free(tok), free(acc), free(ids), free(wts), free(lg), free(w13f), free(w2f);
  return rc;
}

int orc_expert_rows(const uint8_t* hs, const float* hs_scale, int64_t T, const uint8_t* w13,
                    const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                    const int32_t* pair_token, const int32_t* pair_local_expert, int64_t n_pairs,
                    float* c_out, float* o_out) {
  ensure_lut();
  int rc = 0;
  int64_t* idx = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n_pairs > 0 ? n_pairs : 1));
  if (!idx) return -1;
  for (int le = 0; le < ORC_E_LOCAL && rc == 0; ++le) {
    int64_t n = 0;
    for (int64_t p = 0; p < n_pairs; ++p)
      if (pair_local_expert[p] == le) idx[n++] = p;
    if (n == 0) continue;
    float* A = (float*)malloc(sizeof(float) * (size_t)n * ORC_H);
    float* C = (float*)malloc(sizeof(float) * (size_t)n * ORC_I);
    float* O = o_out ? (float*)malloc(sizeof(float) * (size_t)n * ORC_H) : NULL;
    if (!A || !C || (o_out && !O)) {
      rc = -1;
    } else {
      for (int64_t r = 0; r < n; ++r)
        dequant_hidden_row(hs, hs_scale, T, pair_token[idx[r]], A + r * ORC_H);
      rc = expert_forward(A, n, le, w13, w13_scale, w2, w2_scale, NULL, NULL, C, O);
      for (int64_t r = 0; r < n && rc == 0; ++r) {
        if (c_out) memcpy(c_out + idx[r] * ORC_I, C + r * ORC_I, sizeof(float) * ORC_I);
        if (o_out) memcpy(o_out + idx[r] * ORC_H, O + r * ORC_H, sizeof(float) * ORC_H);
      }
    }
    free(A), free(C), free(O);
  }
  free(idx);
  return rc;
}
