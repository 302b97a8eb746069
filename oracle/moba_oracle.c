/*
 * CPU oracle for MoBA sparse block attention.  TEST INFRASTRUCTURE ONLY:
 * this file is linked by the test-suite, by __graft_entry__.smoke() (as the
 * checker) and by bench.py's cpu_baseline leg.  The product path never calls it.
 *
 * Two kinds of functions live here:
 *
 *  1. Canonical-order FP32 routing (chunk means, gate scores, stable top-k,
 *     decode block means and decode route scores).  The summation order is
 *     DEFINED here and implemented identically by the HIP kernels, so block
 *     selection can be compared bit-for-bit:
 *        mean[d]   = tree64(part) / C  (fp32), part[j] = sequential sum of the
 *                    tokens t = j, j+64, j+128, ... of the chunk (0.0f start),
 *                    tree64: for off = 32,16,8,4,2,1: part[j] += part[j+off]
 *                    (j < off); the result is part[0]
 *        gate      = fma(mean[D-1], q[D-1], ... fma(mean[1], q[1], fma(mean[0], q[0], 0)))
 *        top-k     = descending score, exact ties -> lowest chunk index,
 *                    -inf (illegal) never selected.
 *     References: chunk means / gate / mask / top-k of the prefill path
 *     (src/moba_opt/grouped_attention.py:48-71, src/moba_opt/diagnostic.py:386-426),
 *     the tie rule of src/moba_opt/ops/prepared_decode.py:77-88 and
 *     grouped_attention.py:61-69, decode means src/moba_opt/ops/paged_decode.py:26-44
 *     and decode scores paged_decode.py:47-64.
 *
 *  2. FP64 fixed-route attention: forward O/LSE, the backward dQ/dK/dV, the
 *     merge closed form and decode attention.  These restate
 *     reference/fixed_route_attention.py:66-119, reference/grouped_reference.py:6-36,
 *     reference/merge_reference.py:10-69 and reference/decode_reference.py:9-38
 *     as a per-(query, head) gather of the routed tokens.
 *
 * Element inputs of the routing functions are raw 16-bit patterns
 * (dtype 0 = bf16, 1 = fp16) so the oracle sees exactly the bits the GPU sees.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ dtypes */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) {
    /* zero / subnormal: m * 2^-24, exact in fp32 */
    float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (e == 31) return bits_to_f32(sign | 0x7f800000u | (m << 13));
  return bits_to_f32(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t oracle_float_to_half(float f) {
  uint32_t x = f32_to_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  uint32_t e = a >> 23, mant = (a & 0x7fffffu) | 0x800000u;
  if (e < 113) { /* half subnormal: value = mant * 2^(e-150) = n * 2^-24 */
    uint32_t shift = 126 - e;
    if (shift > 24) return (uint16_t)sign;
    uint32_t n = mant >> shift, rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (n & 1))) n++;
    return (uint16_t)(sign | n);
  }
  uint32_t h = ((e - 112) << 10) | ((a & 0x7fffffu) >> 13), rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

float oracle_bf16_to_float(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

uint16_t oracle_float_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float to_f32(uint16_t v, int dtype) {
  return dtype == 0 ? oracle_bf16_to_float(v) : oracle_half_to_float(v);
}
static inline uint16_t from_f32(float v, int dtype) {
  return dtype == 0 ? oracle_float_to_bf16(v) : oracle_float_to_half(v);
}
float oracle_round_to_dtype(float v, int dtype) { return to_f32(from_f32(v, dtype), dtype); }

void oracle_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n < 1 ? 1 : n);
#else
  (void)n;
#endif
}

/* ----------------------------------------------------- canonical routing */

/* Canonical fp32 sum of n values x(t), t = 0..n-1: 64 strided partial sums
 * (lane j of a wave owns t = j, j+64, ...), then a fixed pairwise tree. */
#define CANON_SUM(n, x_of_t, result)                                          \
  do {                                                                        \
    float part_[64];                                                          \
    for (int j_ = 0; j_ < 64; ++j_) {                                         \
      float a_ = 0.0f;                                                        \
      for (int t = j_; t < (n); t += 64) a_ = a_ + (x_of_t);                  \
      part_[j_] = a_;                                                         \
    }                                                                         \
    for (int off_ = 32; off_ > 0; off_ >>= 1)                                 \
      for (int j_ = 0; j_ < off_; ++j_) part_[j_] = part_[j_] + part_[j_ + off_]; \
    (result) = part_[0];                                                      \
  } while (0)

/* Chunk means of the F routing candidates, canonical sum, then / C.
 * precision 0 ("upstream"): the mean is rounded to the input dtype and widened
 * back (torch's keys.mean(1).float(), grouped_attention.py:52);
 * precision 1 ("fp32"): kept in fp32 (keys.float().mean(1)). */
void oracle_chunk_means(const uint16_t* k, int dtype, int T, int Hkv, int D,
                        const int* chunk_start, int F, int C, int precision,
                        float* means) {
  (void)T;
  for (int f = 0; f < F; ++f)
    for (int h = 0; h < Hkv; ++h)
      for (int d = 0; d < D; ++d) {
        float acc;
        CANON_SUM(C, to_f32(k[((size_t)(chunk_start[f] + t) * Hkv + h) * D + d], dtype), acc);
        float m = acc / (float)C;
        if (precision == 0) m = oracle_round_to_dtype(m, dtype);
        means[((size_t)f * Hkv + h) * D + d] = m;
      }
}

static inline float gate_dot(const float* mean, const uint16_t* q, int dtype, int D) {
  float acc = 0.0f;
  for (int d = 0; d < D; ++d) acc = fmaf(mean[d], to_f32(q[d], dtype), acc);
  return acc;
}

/* Stable top-k over n scores: descending, exact ties -> lowest index,
 * -inf never chosen (slot gets -1).  Returns the number chosen. */
int oracle_stable_topk(const float* scores, int n, int k, int* idx, float* val) {
  int cnt = 0;
  for (int i = 0; k > 0 && i < n; ++i) {
    float s = scores[i];
    if (!(s > -INFINITY)) continue;
    if (cnt == k && !(s > val[k - 1])) continue;   /* ties keep the earlier index */
    int pos = cnt < k ? cnt : k - 1;
    while (pos > 0 && s > val[pos - 1]) { val[pos] = val[pos - 1]; idx[pos] = idx[pos - 1]; pos--; }
    val[pos] = s; idx[pos] = i;
    if (cnt < k) cnt++;
  }
  for (int j = cnt; j < k; ++j) { idx[j] = -1; val[j] = -INFINITY; }
  return cnt;
}

/* Prefill routing.  cu_chunk[nchunk+1] / chunk_batch[nchunk] follow
 * calc_chunks (src/moba_opt/diagnostic.py:30-80).  Query s of batch b may
 * select any chunk c of b that ends at or before s (grouped_attention.py:56-60);
 * those are exactly the chunks before s's own chunk, all of them "filtered"
 * candidates with filtered index f = c - b.  sel[T,Hq,R] lists the chosen
 * GLOBAL chunk ids ascending, -1 padded.  gate[F,Hq,T] (optional) receives the
 * masked gate scores (-inf where illegal). */
void oracle_route_prefill(const uint16_t* q, int dtype, int T, int Hq, int Hkv, int D,
                          const float* means, const int* cu_chunk, int nchunk,
                          const int* chunk_batch, int R, float* gate, int* sel) {
  int G = Hq / Hkv;
  int F = nchunk - (chunk_batch[nchunk - 1] + 1);
  int* first = (int*)malloc(sizeof(int) * (size_t)nchunk);
  for (int c = 0; c < nchunk; ++c)
    first[c] = (c > 0 && chunk_batch[c - 1] == chunk_batch[c]) ? first[c - 1] : c;
  if (gate)
    for (size_t i = 0; i < (size_t)F * Hq * T; ++i) gate[i] = -INFINITY;
  float* sc = (float*)malloc(sizeof(float) * (size_t)(nchunk + 1));
  int* idx = (int*)malloc(sizeof(int) * (size_t)(R + 1));
  float* val = (float*)malloc(sizeof(float) * (size_t)(R + 1));
  int c_s = 0;
  for (int s = 0; s < T; ++s) {
    while (cu_chunk[c_s + 1] <= s) c_s++;
    int b = chunk_batch[c_s], c0 = first[c_s], n = c_s - c0;
    for (int h = 0; h < Hq; ++h) {
      const uint16_t* qrow = q + ((size_t)s * Hq + h) * D;
      for (int c = c0; c < c_s; ++c) {
        int f = c - b;
        sc[c - c0] = gate_dot(means + ((size_t)f * Hkv + h / G) * D, qrow, dtype, D);
        if (gate) gate[((size_t)f * Hq + h) * T + s] = sc[c - c0];
      }
      int cnt = oracle_stable_topk(sc, n, R, idx, val);
      /* ascending chunk order */
      for (int i = 1; i < cnt; ++i) {
        int x = idx[i], j = i - 1;
        while (j >= 0 && idx[j] > x) { idx[j + 1] = idx[j]; j--; }
        idx[j + 1] = x;
      }
      int* out = sel + ((size_t)s * Hq + h) * R;
      for (int j = 0; j < R; ++j) out[j] = j < cnt ? idx[j] + c0 : -1;
    }
  }
  free(first); free(sc); free(idx); free(val);
}

/* ------------------------------------------------- FP64 attention (prefill) */

/* Keys of (s,h): its own chunk's tokens [cu_chunk[c_s], s] (causal) plus every
 * token of each selected chunk.  Natural-log LSE. */
static int chunk_of(const int* cu_chunk, int nchunk, int s) {
  int lo = 0, hi = nchunk - 1;
  while (lo < hi) { int mid = (lo + hi + 1) / 2; if (cu_chunk[mid] <= s) lo = mid; else hi = mid - 1; }
  return lo;
}

static int gather_keys(const int* cu_chunk, int nchunk, const int* selrow, int R, int s, int* keys) {
  int c = chunk_of(cu_chunk, nchunk, s), n = 0;
  for (int j = 0; j < R; ++j) {
    int cc = selrow ? selrow[j] : -1;
    if (cc < 0) continue;
    for (int t = cu_chunk[cc]; t < cu_chunk[cc + 1]; ++t) keys[n++] = t;
  }
  for (int t = cu_chunk[c]; t <= s; ++t) keys[n++] = t;
  return n;
}

void oracle_attention_fwd(const double* q, const double* k, const double* v,
                          int T, int Hq, int Hkv, int D, const int* cu_chunk, int nchunk,
                          const int* sel, int R, double scale, double* out, double* lse) {
  int G = Hq / Hkv;
#pragma omp parallel
  {
    int* keys = (int*)malloc(sizeof(int) * (size_t)T);
    double* lg = (double*)malloc(sizeof(double) * (size_t)T);
#pragma omp for schedule(dynamic, 16)
    for (long r = 0; r < (long)T * Hq; ++r) {
      int s = (int)(r / Hq), h = (int)(r % Hq), kh = h / G;
      int n = gather_keys(cu_chunk, nchunk, R ? sel + (size_t)r * R : NULL, R, s, keys);
      const double* qr = q + (size_t)r * D;
      double m = -INFINITY;
      for (int i = 0; i < n; ++i) {
        const double* kr = k + ((size_t)keys[i] * Hkv + kh) * D;
        double a = 0;
        for (int d = 0; d < D; ++d) a += qr[d] * kr[d];
        lg[i] = a * scale;
        if (lg[i] > m) m = lg[i];
      }
      double z = 0;
      for (int i = 0; i < n; ++i) { lg[i] = exp(lg[i] - m); z += lg[i]; }
      double* o = out + (size_t)r * D;
      for (int d = 0; d < D; ++d) o[d] = 0;
      for (int i = 0; i < n; ++i) {
        const double* vr = v + ((size_t)keys[i] * Hkv + kh) * D;
        double p = lg[i] / z;
        for (int d = 0; d < D; ++d) o[d] += p * vr[d];
      }
      lse[r] = m + log(z);
    }
    free(keys); free(lg);
  }
}

/* FP64 backward of the same fixed-route attention (standard softmax VJP):
 *   P = exp(scale*q.k - lse), dP_t = dO.v_t, Delta = sum_t P_t dP_t,
 *   dS_t = P_t (dP_t - Delta), dq = scale sum dS_t k_t,
 *   dk_t += scale dS_t q, dv_t += P_t dO.
 * Parallel over KV heads so dk/dv accumulation is race-free. */
void oracle_attention_bwd(const double* q, const double* k, const double* v, const double* dout,
                          int T, int Hq, int Hkv, int D, const int* cu_chunk, int nchunk,
                          const int* sel, int R, double scale, const double* lse,
                          double* dq, double* dk, double* dv) {
  int G = Hq / Hkv;
  memset(dk, 0, sizeof(double) * (size_t)T * Hkv * D);
  memset(dv, 0, sizeof(double) * (size_t)T * Hkv * D);
#pragma omp parallel
  {
    int* keys = (int*)malloc(sizeof(int) * (size_t)T);
    double* p = (double*)malloc(sizeof(double) * (size_t)T);
    double* dp = (double*)malloc(sizeof(double) * (size_t)T);
#pragma omp for schedule(dynamic, 1)
    for (int kh = 0; kh < Hkv; ++kh)
      for (int g = 0; g < G; ++g)
        for (int s = 0; s < T; ++s) {
          int h = kh * G + g;
          size_t r = (size_t)s * Hq + h;
          int n = gather_keys(cu_chunk, nchunk, R ? sel + r * R : NULL, R, s, keys);
          const double* qr = q + r * D;
          const double* gr = dout + r * D;
          double delta = 0;
          for (int i = 0; i < n; ++i) {
            const double* kr = k + ((size_t)keys[i] * Hkv + kh) * D;
            const double* vr = v + ((size_t)keys[i] * Hkv + kh) * D;
            double a = 0, b = 0;
            for (int d = 0; d < D; ++d) { a += qr[d] * kr[d]; b += gr[d] * vr[d]; }
            p[i] = exp(a * scale - lse[r]);
            dp[i] = b;
            delta += p[i] * b;
          }
          double* dqr = dq + r * D;
          for (int d = 0; d < D; ++d) dqr[d] = 0;
          for (int i = 0; i < n; ++i) {
            double ds = p[i] * (dp[i] - delta);
            const double* kr = k + ((size_t)keys[i] * Hkv + kh) * D;
            double* dkr = dk + ((size_t)keys[i] * Hkv + kh) * D;
            double* dvr = dv + ((size_t)keys[i] * Hkv + kh) * D;
            for (int d = 0; d < D; ++d) {
              dqr[d] += scale * ds * kr[d];
              dkr[d] += scale * ds * qr[d];
              dvr[d] += p[i] * gr[d];
            }
          }
        }
    free(keys); free(p); free(dp);
  }
}

/* ------------------------------------------------------------------ merge */

/* Closed-form global-softmax merge (reference/merge_reference.py:10-26,
 * docs/semantics.md section 6): per row p, m = max l, w = exp(l - m),
 * O = sum w o / sum w, L = m + log sum w.  mapping[m] = destination row. */
void oracle_merge(const double* self_out, const double* self_lse, int P, int D,
                  const double* remote_out, const double* remote_lse, const int64_t* mapping,
                  int M, double* out, double* lse) {
  double* mx = (double*)malloc(sizeof(double) * (size_t)P);
  double* z = (double*)malloc(sizeof(double) * (size_t)P);
  for (int p = 0; p < P; ++p) mx[p] = self_lse[p];
  for (int i = 0; i < M; ++i) if (remote_lse[i] > mx[mapping[i]]) mx[mapping[i]] = remote_lse[i];
  for (int p = 0; p < P; ++p) {
    double w = exp(self_lse[p] - mx[p]);
    z[p] = w;
    for (int d = 0; d < D; ++d) out[(size_t)p * D + d] = w * self_out[(size_t)p * D + d];
  }
  for (int i = 0; i < M; ++i) {
    int64_t p = mapping[i];
    double w = exp(remote_lse[i] - mx[p]);
    z[p] += w;
    for (int d = 0; d < D; ++d) out[(size_t)p * D + d] += w * remote_out[(size_t)i * D + d];
  }
  for (int p = 0; p < P; ++p) {
    for (int d = 0; d < D; ++d) out[(size_t)p * D + d] /= z[p];
    lse[p] = mx[p] + log(z[p]);
  }
  free(mx); free(z);
}

/* ----------------------------------------------------------------- decode */

/* Closed-chunk means of one sequence's logical keys k[L,Hkv,D] (bits), stored
 * in the cache dtype (paged_decode.py:26-44 stores tl.sum/C into a cache-dtype
 * tensor).  Canonical sum as above.  out[nclosed,Hkv,D] bits. */
void oracle_decode_means(const uint16_t* k, int dtype, int L, int Hkv, int D, int C,
                         uint16_t* out) {
  int nclosed = L / C;
  for (int c = 0; c < nclosed; ++c)
    for (int h = 0; h < Hkv; ++h)
      for (int d = 0; d < D; ++d) {
        float acc;
        CANON_SUM(C, to_f32(k[((size_t)(c * C + t) * Hkv + h) * D + d], dtype), acc);
        out[((size_t)c * Hkv + h) * D + d] = from_f32(acc / (float)C, dtype);
      }
}

/* Decode route of one query row: scores over the legal closed chunks
 * (c+1)*C <= pos (paged_decode.py:47-64) using the cache-dtype means, then the
 * stable top-R.  sel[Hq, 1+R]: slot 0 = pos / C, then chosen chunks in
 * descending-score order, -1 padded.  scores[Hq, width] (optional): -inf for
 * illegal chunks. */
void oracle_decode_route(const uint16_t* q, const uint16_t* means, int dtype, int Hq, int Hkv,
                         int D, int C, int pos, int width, int R, float* scores, int* sel) {
  int G = Hq / Hkv;
  int legal = pos / C;  /* chunks 0..legal-1 satisfy (c+1)*C <= pos */
  float* sc = (float*)malloc(sizeof(float) * (size_t)(width > legal ? width : legal) + 4);
  float* mf = (float*)malloc(sizeof(float) * (size_t)D);
  int* idx = (int*)malloc(sizeof(int) * (size_t)(R + 1));
  float* val = (float*)malloc(sizeof(float) * (size_t)(R + 1));
  for (int h = 0; h < Hq; ++h) {
    int nl = legal < width ? legal : width;
    for (int c = 0; c < nl; ++c) {
      for (int d = 0; d < D; ++d) mf[d] = to_f32(means[((size_t)c * Hkv + h / G) * D + d], dtype);
      sc[c] = gate_dot(mf, q + (size_t)h * D, dtype, D);
    }
    if (scores)
      for (int c = 0; c < width; ++c) scores[(size_t)h * width + c] = c < nl ? sc[c] : -INFINITY;
    oracle_stable_topk(sc, nl, R, idx, val);
    int* out = sel + (size_t)h * (R + 1);
    out[0] = pos / C;
    for (int j = 0; j < R; ++j) out[1 + j] = idx[j];
  }
  free(sc); free(mf); free(idx); free(val);
}

/* FP64 decode attention for one query row over one sequence's logical K/V
 * (reference/decode_reference.py:9-38).  chunks[Hq, nslot] (slot 0 current,
 * -1 pad) or NULL for dense (tokens 0..pos). */
void oracle_decode_attention(const double* q, const double* k, const double* v, int Hq, int Hkv,
                             int D, int C, int pos, const int* chunks, int nslot,
                             double* out, double* lse) {
  int G = Hq / Hkv;
  double* lg = (double*)malloc(sizeof(double) * (size_t)(pos + 1));
  int* tok = (int*)malloc(sizeof(int) * (size_t)(pos + 1));
  double scale = 1.0 / sqrt((double)D);
  for (int h = 0; h < Hq; ++h) {
    int n = 0;
    if (!chunks) {
      for (int t = 0; t <= pos; ++t) tok[n++] = t;
    } else {
      for (int j = 0; j < nslot; ++j) {
        int c = chunks[(size_t)h * nslot + j];
        if (c < 0) continue;
        for (int t = c * C; t < (c + 1) * C && t <= pos; ++t) tok[n++] = t;
      }
    }
    int kh = h / G;
    double m = -INFINITY;
    for (int i = 0; i < n; ++i) {
      double a = 0;
      for (int d = 0; d < D; ++d) a += q[(size_t)h * D + d] * k[((size_t)tok[i] * Hkv + kh) * D + d];
      lg[i] = a * scale;
      if (lg[i] > m) m = lg[i];
    }
    double z = 0;
    for (int i = 0; i < n; ++i) { lg[i] = exp(lg[i] - m); z += lg[i]; }
    for (int d = 0; d < D; ++d) {
      double o = 0;
      for (int i = 0; i < n; ++i) o += lg[i] * v[((size_t)tok[i] * Hkv + kh) * D + d];
      out[(size_t)h * D + d] = o / z;
    }
    lse[h] = m + log(z);
  }
  free(lg); free(tok);
}
