/*
 * CPU oracle for the PrunePath routing arithmetic -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker. The product path never calls it.
 *
 * What it restates (reference files under /root/reference, read not run):
 *   softmax_thresholding      src/MoEBlock_origin.py:50-97 (twin src/MoEBlock.py:49-95)
 *     y_soft  = torch.softmax(logits, -1)                      :70
 *     sorted  = torch.sort(y_soft, -1, descending=True)        :71
 *     cum     = torch.cumsum(sorted, -1); mask = cum < tau     :74-75
 *     scatter back, top-1 fallback                             :77-88
 *     gates   = sigmoid(where(mask, logits, finfo.min))        :91-93
 *   canonical bucket layout   src/tl_kernel_optimized_Ultimate_PanGU.py:133-266
 *     experts ascending, tokens ascending inside an expert.
 *
 * Bit-level recipe of torch 2.10 CPU (AVX512) for fp32 rows:
 *   exp      = SLEEF expf_u10 (Shibata & Petrogalli, IEEE TPDS 2020; SLEEF is
 *              Boost-licensed). torch maps Vectorized<float>::exp() to
 *              Sleef_expf16_u10 (torch/include/ATen/cpu/vec/vec512/vec512_float.h:307-309).
 *   row sum  = vec::reduce_all (torch/include/ATen/cpu/vec/functional_base.h:185-203):
 *              rows shorter than 16 are summed left to right; longer rows are
 *              summed lane-wise over 16-wide chunks (the partial tail chunk only
 *              touches its low lanes) and then folded lane i + lane i^8, i^4,
 *              i^2, i^1 (functional_base.h:79-101).
 *   probs    = e * (1.0f / sum).
 *   cumsum   = fp32 output of a float64 running sum (torch CPU accumulates
 *              float cumsum in double).
 *   sort     = std::sort (introsort) of (value, index) pairs, descending; stable
 *              for E <= 16, implementation-ordered ties above (see oracle_sort_desc).
 *   sigmoid  = 1 / (1 + exp(-x)) with the same exp.
 * Build: see oracle/Makefile (-O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define ORACLE_VL 16  /* AVX512 float lanes */

static inline float pow2i_f(int q) {
  /* 2^q for q in the normal exponent range, built from the exponent bits. */
  uint32_t bits = (uint32_t)(q + 0x7f) << 23;
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

/* SLEEF expf_u10, FMA variant. */
float oracle_expf_u10(float d) {
  const float R_LN2f = 1.442695040888963407359924681001892137426645954152985934135449406931f;
  const float L2Uf = 0.693145751953125f;
  const float L2Lf = 1.428606765330187045e-06f;
  float t = d * R_LN2f;
  int q = (int)rintf(t); /* round half to even (default rounding mode) */
  float s = fmaf((float)q, -L2Uf, d);
  s = fmaf((float)q, -L2Lf, s);
  float u = 0.000198527617612853646278381f;
  u = fmaf(u, s, 0.00139304355252534151077271f);
  u = fmaf(u, s, 0.00833336077630519866943359f);
  u = fmaf(u, s, 0.0416664853692054748535156f);
  u = fmaf(u, s, 0.166666671633720397949219f);
  u = fmaf(u, s, 0.5f);
  float ss = s * s;
  u = 1.0f + fmaf(ss, u, s);
  int qh = q >> 1;
  u = (u * pow2i_f(qh)) * pow2i_f(q - qh);
  if (d < -104.0f) u = 0.0f;
  if (d > 104.0f) u = INFINITY;
  if (isnan(d)) u = NAN;
  return u;
}

float oracle_sigmoid(float x) {
  float e = oracle_expf_u10(0.0f - x);
  return 1.0f / (e + 1.0f);
}

/* torch vec::reduce_all(+) over e[0..n) with 16 float lanes. */
static float reduce_sum_vl16(const float* e, int n) {
  if (n < ORACLE_VL) {
    float acc = e[0];
    for (int i = 1; i < n; ++i) acc = acc + e[i];
    return acc;
  }
  float acc[ORACLE_VL];
  for (int i = 0; i < ORACLE_VL; ++i) acc[i] = e[i];
  int d = ORACLE_VL;
  for (; d < n - (n % ORACLE_VL); d += ORACLE_VL)
    for (int i = 0; i < ORACLE_VL; ++i) acc[i] = acc[i] + e[d + i];
  if (n - d > 0)
    for (int i = 0; i < n - d; ++i) acc[i] = acc[i] + e[d + i];
  for (int stride = 8; stride >= 1; stride >>= 1) {
    float nxt[ORACLE_VL];
    for (int i = 0; i < ORACLE_VL; ++i) nxt[i] = acc[i] + acc[i ^ stride];
    memcpy(acc, nxt, sizeof acc);
  }
  return acc[0];
}

/* Softmax over rows of length E, bit-compatible with torch CPU fp32. */
void oracle_softmax_rows(const float* logits, int64_t n, int32_t E, float* probs) {
  float* e = (float*)malloc(sizeof(float) * (size_t)E);
  for (int64_t t = 0; t < n; ++t) {
    const float* x = logits + t * E;
    float m = x[0];
    for (int j = 1; j < E; ++j) m = (x[j] > m || isnan(x[j])) ? x[j] : m;
    for (int j = 0; j < E; ++j) e[j] = oracle_expf_u10(x[j] - m);
    float s = reduce_sum_vl16(e, E);
    float r = 1.0f / s;
    for (int j = 0; j < E; ++j) probs[t * E + j] = e[j] * r;
  }
  free(e);
}

/*
 * Sort order of torch.sort(p, descending=True) on CPU: torch's CPU sort kernel
 * calls std::sort on (value, index) pairs with a descending comparator (NaN
 * first). libstdc++'s std::sort is introsort: quicksort with a median-of-three
 * pivot moved to the front and an unguarded partition while a range holds more
 * than 16 elements (depth limit 2*floor(log2 n), then heapsort), followed by a
 * final insertion sort. Ranges of at most 16 elements are therefore sorted
 * stably; longer ranges order equal values in the way the partition leaves them.
 * Restated from the published libstdc++ algorithm (bits/stl_algo.h, stl_heap.h).
 */
typedef struct { float key; int32_t idx; } kv_t;

static inline int kv_before(kv_t a, kv_t b) { /* comparator: a sorts before b */
  return (isnan(a.key) && !isnan(b.key)) || a.key > b.key;
}
static inline void kv_swap(kv_t* A, int i, int j) { kv_t t = A[i]; A[i] = A[j]; A[j] = t; }

static void kv_adjust_heap(kv_t* A, int hole, int len, kv_t val) {
  int top = hole, sc = hole;
  while (sc < (len - 1) / 2) {
    sc = 2 * (sc + 1);
    if (kv_before(A[sc], A[sc - 1])) sc--;
    A[hole] = A[sc];
    hole = sc;
  }
  if ((len & 1) == 0 && sc == (len - 2) / 2) {
    sc = 2 * (sc + 1);
    A[hole] = A[sc - 1];
    hole = sc - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && kv_before(A[parent], val)) {
    A[hole] = A[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  A[hole] = val;
}

static void kv_heapsort(kv_t* A, int len) {
  if (len >= 2) {
    for (int parent = (len - 2) / 2;; --parent) {
      kv_adjust_heap(A, parent, len, A[parent]);
      if (parent == 0) break;
    }
  }
  for (int last = len; last > 1;) {
    --last;
    kv_t val = A[last];
    A[last] = A[0];
    kv_adjust_heap(A, 0, last, val);
  }
}

static void kv_unguarded_linear_insert(kv_t* A, int last) {
  kv_t val = A[last];
  int nxt = last - 1;
  while (kv_before(val, A[nxt])) { A[last] = A[nxt]; last = nxt; --nxt; }
  A[last] = val;
}

static void kv_insertion_sort(kv_t* A, int f, int l) {
  for (int i = f + 1; i < l; ++i) {
    if (kv_before(A[i], A[f])) {
      kv_t v = A[i];
      for (int j = i; j > f; --j) A[j] = A[j - 1];
      A[f] = v;
    } else {
      kv_unguarded_linear_insert(A, i);
    }
  }
}

static void kv_introsort(kv_t* A, int n) {
  if (n <= 0) return;
  int lg = 0;
  while ((2 << lg) <= n) ++lg;
  int stf[64], stl[64], std_[64], sp = 0;
  stf[sp] = 0; stl[sp] = n; std_[sp] = 2 * lg; ++sp;
  while (sp > 0) {
    --sp;
    int f = stf[sp], l = stl[sp], depth = std_[sp];
    while (l - f > 16) {
      if (depth == 0) { kv_heapsort(A + f, l - f); break; }
      --depth;
      int mid = f + (l - f) / 2, a = f + 1, b = mid, c = l - 1, s;
      if (kv_before(A[a], A[b])) {
        if (kv_before(A[b], A[c])) s = b;
        else if (kv_before(A[a], A[c])) s = c;
        else s = a;
      } else if (kv_before(A[a], A[c])) s = a;
      else if (kv_before(A[b], A[c])) s = c;
      else s = b;
      kv_swap(A, f, s);
      int lo = f + 1, hi = l;
      for (;;) {
        while (kv_before(A[lo], A[f])) ++lo;
        --hi;
        while (kv_before(A[f], A[hi])) --hi;
        if (!(lo < hi)) break;
        kv_swap(A, lo, hi);
        ++lo;
      }
      stf[sp] = lo; stl[sp] = l; std_[sp] = depth; ++sp; /* right part */
      l = lo;
    }
  }
  if (n > 16) {
    kv_insertion_sort(A, 0, 16);
    for (int i = 16; i < n; ++i) kv_unguarded_linear_insert(A, i);
  } else {
    kv_insertion_sort(A, 0, n);
  }
}

/* Descending sort order of p[0..E) as torch CPU returns it. */
void oracle_sort_desc(const float* p, int32_t E, int32_t* order) {
  kv_t* A = (kv_t*)malloc(sizeof(kv_t) * (size_t)(E > 0 ? E : 1));
  for (int j = 0; j < E; ++j) { A[j].key = p[j]; A[j].idx = j; }
  kv_introsort(A, E);
  for (int j = 0; j < E; ++j) order[j] = A[j].idx;
  free(A);
}

/*
 * Tau selection for n rows of E logits.
 * Outputs (any may be NULL):
 *   probs  [n,E]  softmax probabilities (y_soft)
 *   gates  [n,E]  sigmoid(logit) where selected, 0 elsewhere (y_gated)
 *   mask   [n,E]  1 where selected
 *   ranked [n,E]  expert ids in descending-probability order (full sort)
 *   count  [n]    number of selected experts (selected = the first count ranks)
 */
void oracle_select_rows(const float* logits, int64_t n, int32_t E, float tau,
                        float* probs, float* gates, uint8_t* mask,
                        int32_t* ranked, int32_t* count) {
  float* p = (float*)malloc(sizeof(float) * (size_t)E);
  int32_t* order = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  const float tau32 = tau;
  for (int64_t t = 0; t < n; ++t) {
    const float* x = logits + t * E;
    oracle_softmax_rows(x, 1, E, p);
    oracle_sort_desc(p, E, order);
    double acc = 0.0;
    int kept = 0;
    for (int r = 0; r < E; ++r) {
      acc += (double)p[order[r]];
      float cum = (float)acc;
      if (cum < tau32) kept = r + 1;
      else break; /* cum is non-decreasing: no later rank can pass */
    }
    if (kept == 0) kept = 1; /* top-1 fallback */
    if (probs) memcpy(probs + t * E, p, sizeof(float) * (size_t)E);
    if (ranked) memcpy(ranked + t * E, order, sizeof(int32_t) * (size_t)E);
    if (count) count[t] = kept;
    for (int j = 0; j < E; ++j) {
      if (gates) gates[t * E + j] = 0.0f;
      if (mask) mask[t * E + j] = 0;
    }
    for (int r = 0; r < kept; ++r) {
      int j = order[r];
      if (gates) gates[t * E + j] = oracle_sigmoid(x[j]);
      if (mask) mask[t * E + j] = 1;
    }
  }
  free(p);
  free(order);
}

/*
 * Canonical bucket layout from a selection mask.
 *   offsets     [E+1]  CSR offsets, experts in ascending id order
 *   token_ids   [P]    tokens ascending inside each expert segment
 *   pair_gates  [P]    gates[token, expert] of each pair
 *   token_pairs [n,E]  for token t, the pair positions of its selected experts
 *                      in ascending expert-id order, -1 padded
 */
void oracle_bucket(const uint8_t* mask, const float* gates, int64_t n, int32_t E,
                   int32_t* offsets, int32_t* token_ids, float* pair_gates,
                   int32_t* token_pairs) {
  int64_t* cnt = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  for (int64_t t = 0; t < n; ++t)
    for (int j = 0; j < E; ++j) cnt[j] += mask[t * E + j] ? 1 : 0;
  offsets[0] = 0;
  for (int j = 0; j < E; ++j) offsets[j + 1] = offsets[j] + (int32_t)cnt[j];
  int64_t* cur = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  for (int j = 0; j < E; ++j) cur[j] = offsets[j];
  for (int64_t t = 0; t < n; ++t) {
    int slot = 0;
    for (int j = 0; j < E; ++j) {
      if (token_pairs) token_pairs[t * E + j] = -1;
    }
    for (int j = 0; j < E; ++j) {
      if (!mask[t * E + j]) continue;
      int64_t pos = cur[j]++;
      if (token_ids) token_ids[pos] = (int32_t)t;
      if (pair_gates) pair_gates[pos] = gates ? gates[t * E + j] : 0.0f;
      if (token_pairs) token_pairs[t * E + slot] = (int32_t)pos;
      ++slot;
    }
  }
  free(cnt);
  free(cur);
}
