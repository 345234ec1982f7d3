/*
 * geo_oracle.c — CPU restatement of the reference semantics for the geometry kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (gdl_amd/, geoembodied/) may load or call
 * this file; it is the checker used by tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline.
 *
 * Build: see oracle/build.py (gcc -O2 -ffp-contract=off -fopenmp -fPIC -shared).  The KNN
 * and radius loops run their queries / targets on OpenMP threads (each writes only its own
 * outputs, so results do not depend on the thread count).  Every float
 * operation below is a single IEEE fp32 operation (x86-64 SSE, no contraction), so distances
 * round exactly like the reference's (fl(dx*dx) + fl(dy*dy)) + fl(dz*dz).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float sqd(const float* a, const float* b) {
  const float dx = a[0] - b[0];
  const float dy = a[1] - b[1];
  const float dz = a[2] - b[2];
  const float xx = dx * dx, yy = dy * dy, zz = dz * dz;
  const float s = xx + yy;
  return s + zz;
}

/*
 * FPS.  Follows _fps_iterative_fallback (geoembodied/csrc/__init__.py:600-654):
 *   k = min(k_b, n) (:627), k <= 0 -> skip (:629-630), k >= n -> arange (:634-636),
 *   selected[0] = 0 (:640), min_dists = +inf (:641),
 *   dist = (local_pos - current).pow(2).sum(-1) (:645), torch.minimum (:646),
 *   selected[i+1] = argmax (first maximum) (:648).
 * out_ptr[b] gives each cloud's output offset (the caller clamps k and scans).
 */
void oracle_fps(const float* pos, const int64_t* ptr, const int64_t* k_per_batch, int64_t B,
                const int64_t* out_ptr, int64_t* out) {
  for (int64_t b = 0; b < B; ++b) {
    const int64_t start = ptr[b], n = ptr[b + 1] - ptr[b];
    int64_t k = k_per_batch[b];
    if (k > n) k = n;
    if (k <= 0) continue;
    int64_t* o = out + out_ptr[b];
    if (k >= n) {
      for (int64_t i = 0; i < n; ++i) o[i] = start + i;
      continue;
    }
    const float* P = pos + 3 * start;
    float* md = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = 0; i < n; ++i) md[i] = INFINITY;
    int64_t cur = 0;
    o[0] = start;
    for (int64_t it = 0; it < k; ++it) {
      const float* c = P + 3 * cur;
      float best = -INFINITY;
      int64_t arg = 0;
      for (int64_t i = 0; i < n; ++i) {
        const float d = sqd(P + 3 * i, c);
        const float m = d < md[i] ? d : md[i];
        md[i] = m;
        if (m > best) { best = m; arg = i; }
      }
      if (it + 1 < k) {
        cur = arg;
        o[it + 1] = start + arg;
      }
    }
    free(md);
  }
}

/* (d, j) ordered max-heap for the k smallest keys. */
typedef struct { float d; int64_t j; } Key;
static inline int key_less(Key a, Key b) { return a.d < b.d || (a.d == b.d && a.j < b.j); }

static void heap_sift_down(Key* h, int64_t n, int64_t i) {
  for (;;) {
    int64_t l = 2 * i + 1, r = l + 1, m = i;
    if (l < n && key_less(h[m], h[l])) m = l;
    if (r < n && key_less(h[m], h[r])) m = r;
    if (m == i) return;
    Key t = h[i]; h[i] = h[m]; h[m] = t;
    i = m;
  }
}
static void heap_sift_up(Key* h, int64_t i) {
  while (i > 0) {
    int64_t p = (i - 1) / 2;
    if (!key_less(h[p], h[i])) return;
    Key t = h[i]; h[i] = h[p]; h[p] = t;
    i = p;
  }
}
static int key_cmp(const void* a, const void* b) {
  const Key* x = (const Key*)a;
  const Key* y = (const Key*)b;
  return key_less(*x, *y) ? -1 : (key_less(*y, *x) ? 1 : 0);
}

/* Keeps the `cap` smallest finite keys; returns the count (sorted ascending into h). */
typedef struct { Key* h; int64_t n, cap; } TopK;
static inline void topk_push(TopK* t, Key k) {
  if (!(k.d <= INFINITY) || isinf(k.d)) return; /* non-finite distances never selected */
  if (t->n < t->cap) {
    t->h[t->n] = k;
    heap_sift_up(t->h, t->n);
    t->n++;
  } else if (t->cap > 0 && key_less(k, t->h[0])) {
    t->h[0] = k;
    heap_sift_down(t->h, t->n, 0);
  }
}

/*
 * KNN.  Follows _knn_bruteforce (geoembodied/csrc/__init__.py:435-492): per cloud,
 * diff = q - s, d = (diff*diff).sum(-1) (:480-483), k smallest (:485-486), global source
 * index = local + s_start (:489), padding -1 / 1e30 (:461-462), empty clouds skipped
 * (:468-469).  Ties: ascending source index (the reference's topk leaves them unspecified).
 */
void oracle_knn(const float* query, const float* source, const int64_t* ptr_q,
                const int64_t* ptr_s, int64_t B, int64_t k, int64_t Nq, int64_t* out_idx,
                float* out_dist) {
  for (int64_t i = 0; i < Nq * k; ++i) { out_idx[i] = -1; out_dist[i] = 1e30f; }
  for (int64_t b = 0; b < B; ++b) {
    const int64_t qa = ptr_q[b], qc = ptr_q[b + 1], sa = ptr_s[b], sc = ptr_s[b + 1];
    /* queries are independent: each thread owns its heap and writes only its query's row */
#pragma omp parallel
    {
      Key* heap = (Key*)malloc(sizeof(Key) * (size_t)(k > 0 ? k : 1));
#pragma omp for schedule(dynamic, 16)
      for (int64_t q = qa; q < qc; ++q) {
        TopK t = {heap, 0, k};
        for (int64_t j = sa; j < sc; ++j) {
          Key key = {sqd(query + 3 * q, source + 3 * j), j};
          topk_push(&t, key);
        }
        qsort(heap, (size_t)t.n, sizeof(Key), key_cmp);
        for (int64_t m = 0; m < t.n; ++m) {
          out_idx[q * k + m] = heap[m].j;
          out_dist[q * k + m] = heap[m].d;
        }
      }
      free(heap);
    }
  }
}

/*
 * Radius graph.  Follows _radius_graph_batched / _single
 * (geoembodied/functional/radius_graph.py:204-335) with the exact squared distance:
 *   masked points take part in no edge (:240-245, :308-312), d >= r2 -> no edge (:248, :315)
 *   with r2 = fl32(r*r) (:232, :302 and the fp32 comparison), no self edges unless loop
 *   (:250-252, :317-319), at most K = max_num_neighbors sources per target kept by smallest
 *   (d, j) (:233, :255-257, :321-326).  cloud[i] < 0 marks an excluded point.
 * Two-pass interface: with row/col == NULL it only writes deg[i]; otherwise it writes the
 * edges at row_ptr[i] sorted by source index.
 */
void oracle_radius(const float* x, int64_t N, const int64_t* cloud, float r2, int64_t K, int loop,
                   int64_t* deg, const int64_t* row_ptr, int64_t* row, int64_t* col) {
  /* group points by cloud (stable) so each target scans only its own cloud */
  int64_t maxc = -1;
  for (int64_t i = 0; i < N; ++i) if (cloud[i] > maxc) maxc = cloud[i];
  const int64_t nc = maxc + 1;
  int64_t* start = (int64_t*)calloc((size_t)(nc + 1), sizeof(int64_t));
  int64_t* members = (int64_t*)malloc(sizeof(int64_t) * (size_t)(N > 0 ? N : 1));
  for (int64_t i = 0; i < N; ++i) if (cloud[i] >= 0) start[cloud[i] + 1]++;
  for (int64_t c = 0; c < nc; ++c) start[c + 1] += start[c];
  int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nc > 0 ? nc : 1));
  for (int64_t c = 0; c < nc; ++c) fill[c] = start[c];
  for (int64_t i = 0; i < N; ++i) if (cloud[i] >= 0) members[fill[cloud[i]]++] = i;
  /* targets are independent: each thread owns its heap and writes only its target's outputs */
#pragma omp parallel
  {
  Key* heap = (Key*)malloc(sizeof(Key) * (size_t)(K > 0 ? K : 1));
  int64_t* js = (int64_t*)malloc(sizeof(int64_t) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(dynamic, 64)
  for (int64_t i = 0; i < N; ++i) {
    if (deg && !row) deg[i] = 0;
    if (cloud[i] < 0) continue;
    const int64_t c = cloud[i];
    TopK t = {heap, 0, K};
    for (int64_t m = start[c]; m < start[c + 1]; ++m) {
      const int64_t j = members[m];
      if (!loop && j == i) continue;
      const float d = sqd(x + 3 * i, x + 3 * j);
      if (d < r2) {
        Key key = {d, j};
        topk_push(&t, key);
      }
    }
    if (!row) {
      if (deg) deg[i] = t.n;
      continue;
    }
    for (int64_t m = 0; m < t.n; ++m) js[m] = t.h[m].j;
    /* sort the kept sources by index */
    for (int64_t a = 1; a < t.n; ++a) {
      int64_t v = js[a], b2 = a;
      while (b2 > 0 && js[b2 - 1] > v) { js[b2] = js[b2 - 1]; --b2; }
      js[b2] = v;
    }
    for (int64_t m = 0; m < t.n; ++m) {
      row[row_ptr[i] + m] = js[m];
      col[row_ptr[i] + m] = i;
    }
  }
  free(js); free(heap);
  }
  free(fill); free(members); free(start);
}

/*
 * CSR build.  Stable counting sort by target, the ordering the reference's CUDA path gets from
 * CUB's stable radix sort (geoembodied/csrc/segment_reduce_kernel.cu:118-152); offsets as in
 * the CPU path's bincount + cumsum (geoembodied/functional/segment_reduce.py:96-102).  Targets
 * outside [0, N) sort last (reported as N) and belong to no segment.
 */
void oracle_csr(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted, int32_t* perm,
                int32_t* node_start, int32_t* node_end) {
  int64_t* cnt = (int64_t*)calloc((size_t)(N + 2), sizeof(int64_t));
  for (int64_t e = 0; e < E; ++e) {
    const int64_t c = (col[e] >= 0 && col[e] < N) ? col[e] : N;
    cnt[c + 1]++;
  }
  for (int64_t c = 0; c <= N; ++c) cnt[c + 1] += cnt[c];
  for (int64_t n = 0; n < N; ++n) {
    node_start[n] = (int32_t)cnt[n];
    node_end[n] = (int32_t)cnt[n + 1];
  }
  for (int64_t e = 0; e < E; ++e) {
    const int64_t c = (col[e] >= 0 && col[e] < N) ? col[e] : N;
    const int64_t p = cnt[c]++;
    col_sorted[p] = (int32_t)c;
    perm[p] = (int32_t)e;
  }
  free(cnt);
}
