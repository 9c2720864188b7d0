/*
 * shortlist_oracle.c -- TEST INFRASTRUCTURE ONLY (CPU oracle).
 *
 * C restatement of the reference shortlist builder
 * (src/proteus_attention/kernels/sparse_attn.py:376-596 of
 * Proteus-Flux-Attention), used by tests/ to check the HIP builder at full
 * sizes and by bench.py's cpu_baseline leg.  Never linked into the product.
 *
 * Per row: concatenate local window, strided anchors and the prototype
 * prefix top-K (ties -> lowest index), clamp to [0, T-1], min with the row,
 * append the row, sort, drop duplicates, keep the smallest L, pad with the
 * row; length = max(count, 1)  -- the reference's own procedure, not the
 * merge-path formulation of the device kernel.
 *
 * The prototype prefix sets are maintained by one walk over the tokens of
 * each batch row: a binary min-heap on (value asc, index desc) holds the
 * current K best, and a position-sorted array mirrors it (new tokens append
 * at the end, evictions delete in place).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct { float v; int32_t i; } item_t;

/* a is "worse" than b: smaller value, or equal value and larger index */
static int worse(item_t a, item_t b) {
  if (a.v != a.v) return !(b.v != b.v) || a.i > b.i; /* NaN is worst */
  if (b.v != b.v) return 0;
  return (a.v < b.v) || (a.v == b.v && a.i > b.i);
}

static void heap_push(item_t* h, int* n, item_t x) {
  int c = (*n)++;
  h[c] = x;
  while (c > 0) {
    int p = (c - 1) / 2;
    if (worse(h[c], h[p])) { item_t t = h[c]; h[c] = h[p]; h[p] = t; c = p; } else break;
  }
}

static void heap_replace_top(item_t* h, int n, item_t x) {
  h[0] = x;
  int c = 0;
  for (;;) {
    int l = 2 * c + 1, r = l + 1, m = c;
    if (l < n && worse(h[l], h[m])) m = l;
    if (r < n && worse(h[r], h[m])) m = r;
    if (m == c) break;
    item_t t = h[c]; h[c] = h[m]; h[m] = t; c = m;
  }
}

static int cmp_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return (x > y) - (x < y);
}

typedef struct { int64_t tok; int64_t row; } order_t;
static int cmp_order(const void* a, const void* b) {
  const order_t* x = (const order_t*)a; const order_t* y = (const order_t*)b;
  if (x->tok != y->tok) return (x->tok > y->tok) - (x->tok < y->tok);
  return (x->row > y->row) - (x->row < y->row);
}

static void build_row(int64_t t, int64_t T, int L, int local_w, int stride, int slots,
                      const int32_t* pset, int pcount, int64_t* buf, int32_t* out, int32_t* len_out) {
  int64_t n = 0;
  if (local_w > 0) {
    int64_t ln = t + 1 < local_w ? t + 1 : local_w;
    int64_t start = t - ln + 1;
    for (int j = 0; j < local_w; ++j) buf[n++] = (j < ln) ? start + j : t;
  }
  if (slots > 0 && stride > 0) {
    for (int j = 1; j <= slots; ++j) { int64_t a = t - (int64_t)j * stride; buf[n++] = a < 0 ? 0 : a; }
  }
  for (int j = 0; j < pcount; ++j) buf[n++] = pset[j];
  for (int64_t j = 0; j < n; ++j) {
    int64_t c = buf[j];
    if (c < 0) c = 0;
    if (c > T - 1) c = T - 1;
    if (c > t) c = t;
    buf[j] = c;
  }
  buf[n++] = t;
  qsort(buf, (size_t)n, sizeof(int64_t), cmp_i64);
  int64_t u = 0;
  for (int64_t j = 0; j < n; ++j) {
    if (j > 0 && buf[j] == buf[j - 1]) continue;
    if (u < L) out[u] = (int32_t)buf[j];
    ++u;
  }
  int64_t keep = u < L ? u : L;
  for (int64_t j = keep; j < L; ++j) out[j] = (int32_t)t;
  *len_out = (int32_t)(keep < 1 ? 1 : keep);
}

/*
 * rows/row_batch: (N) tokens and batch ids (row_batch may be NULL).
 * scores: (B, Ts) row-major or NULL; K = proto set size (0 = no proto).
 * cand_out (N, L) int32, len_out (N) int32.  Returns 0 on success.
 */
int oracle_shortlist_build(const int32_t* rows, const int32_t* row_batch, int64_t N, int64_t T, int L,
                           int local_w, int stride, int slots, const float* scores, int B, int64_t Ts, int K,
                           int32_t* cand_out, int32_t* len_out) {
  int64_t cap = (int64_t)local_w + slots + K + 2;
  int64_t* buf = (int64_t*)malloc(sizeof(int64_t) * cap);
  if (!buf) return 1;
  if (scores == NULL || K <= 0) {
    for (int64_t r = 0; r < N; ++r)
      build_row(rows[r], T, L, local_w, stride, slots, NULL, 0, buf, cand_out + r * L, len_out + r);
    free(buf);
    return 0;
  }
  item_t* heap = (item_t*)malloc(sizeof(item_t) * (size_t)K);
  int32_t* sorted = (int32_t*)malloc(sizeof(int32_t) * (size_t)K);
  order_t* ord = (order_t*)malloc(sizeof(order_t) * (size_t)(N > 0 ? N : 1));
  if (!heap || !sorted || !ord) { free(buf); free(heap); free(sorted); free(ord); return 1; }
  for (int b = 0; b < B; ++b) {
    int64_t m = 0;
    for (int64_t r = 0; r < N; ++r)
      if ((row_batch ? row_batch[r] : 0) == b) { ord[m].tok = rows[r]; ord[m].row = r; ++m; }
    if (m == 0) continue;
    qsort(ord, (size_t)m, sizeof(order_t), cmp_order);
    const float* s = scores + (int64_t)b * Ts;
    int hn = 0, sn = 0;
    int64_t next = 0; /* next token to insert */
    for (int64_t q = 0; q < m; ++q) {
      int64_t t = ord[q].tok;
      int64_t upto = t < Ts - 1 ? t : Ts - 1;
      while (next <= upto) {
        item_t it = {s[next], (int32_t)next};
        if (hn < K) {
          heap_push(heap, &hn, it);
          sorted[sn++] = (int32_t)next;
        } else if (worse(heap[0], it)) {
          int32_t ev = heap[0].i;
          heap_replace_top(heap, hn, it);
          /* delete ev from the position-sorted array, append next */
          int lo = 0, hi = sn - 1;
          while (lo < hi) { int mid = (lo + hi) / 2; if (sorted[mid] < ev) lo = mid + 1; else hi = mid; }
          memmove(sorted + lo, sorted + lo + 1, sizeof(int32_t) * (size_t)(sn - lo - 1));
          sorted[sn - 1] = (int32_t)next;
        }
        ++next;
      }
      build_row(t, T, L, local_w, stride, slots, sorted, sn, buf, cand_out + ord[q].row * L,
                len_out + ord[q].row);
    }
  }
  free(buf); free(heap); free(sorted); free(ord);
  return 0;
}
