// Paged-KV MoBA decode on gfx950.
//
// Replaces the Triton kernels of src/moba_opt/ops/paged_decode.py:10-144 and
// src/moba_opt/ops/prepared_decode.py:6-94:
//   paged_append      : scatter new K/V tokens into the page pool through the
//                       page table (_append_kernel)
//   block_means       : closed-chunk key means, fp32 sum in canonical order,
//                       stored in the cache dtype (_closed_means_kernel /
//                       _step_means)
//   decode_route      : fp32 route scores over the closed chunks + stable top-k
//                       + the selected-slot list (_route_kernel, topk,
//                       _stable_topk, _selected)
//   paged_attention   : GQA-grouped split-K attention straight through the page
//                       table (_attention_kernel), then a deterministic combine
//   decode_metadata   : page-table delta, positions, length advance (_metadata)
//
// paged_attention: one wave per (query, kv head, 16-head block, chunk of the
// union of the group's selections, sub-block of <= kSub tokens).  Each
// selected page is read once for all the q heads of the group.  Scores are
// S^T = K Q^T on v_mfma_f32_16x16x32 (16 tokens x 16 heads, K read straight
// from the pool), O^T += V^T P^T with V^T taken from a row-major LDS tile by
// the transposed LDS read.  Partials (o, max, sum) per (query, head, slot,
// sub-block) are merged in a fixed order by combine_kernel.
#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int DT>
MOBA_DEV f32x4v mfma16(const u16x8_t& a, const u16x8_t& b, const f32x4v& c) {
  if constexpr (DT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

constexpr int kSub = 128;  // tokens per attention work item
constexpr int kMaxRemote = 8;

// ------------------------------------------------------------------ append
__global__ void append_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                              int N, int Hkv, int D, uint16_t* __restrict__ kc,
                              uint16_t* __restrict__ vc, int P, const int* __restrict__ table,
                              int W, const int* __restrict__ seq, const int* __restrict__ pos) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)N * Hkv * D;
  if (idx >= total) return;
  const int d = (int)(idx % D);
  const int hk = (int)((idx / D) % Hkv);
  const int n = (int)(idx / ((int64_t)D * Hkv));
  const int sid = seq[n], p = pos[n];
  const int page = table[(int64_t)sid * W + p / P];
  if (page < 0) return;  // unmapped logical page: never write outside the pool
  const int64_t dst = (((int64_t)page * P + p % P) * Hkv + hk) * D + d;
  kc[dst] = k[idx];
  vc[dst] = v[idx];
}

__global__ void append_vec_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                  int N, int Hkv, int D, uint16_t* __restrict__ kc,
                                  uint16_t* __restrict__ vc, int P, const int* __restrict__ table,
                                  int W, const int* __restrict__ seq, const int* __restrict__ pos) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one 16-byte chunk
  const int nd = D / 8;
  const int64_t total = (int64_t)N * Hkv * nd;
  if (idx >= total) return;
  const int dc = (int)(idx % nd) * 8;
  const int hk = (int)((idx / nd) % Hkv);
  const int n = (int)(idx / ((int64_t)nd * Hkv));
  const int sid = seq[n], p = pos[n];
  const int page = table[(int64_t)sid * W + p / P];
  if (page < 0) return;  // unmapped logical page: never write outside the pool
  const int64_t dst = (((int64_t)page * P + p % P) * Hkv + hk) * D + dc;
  const int64_t src = ((int64_t)n * Hkv + hk) * D + dc;
  st8(kc + dst, ld8(k + src));
  st8(vc + dst, ld8(v + src));
}

// ------------------------------------------------------------------- means
// One wave per (item, kv head, 8 consecutive d); lane j sums tokens j, j+64,
// ... of the chunk through the page table, then the canonical tree.
// mode 0: item i closes chunk chunk_or_pos[i] of sequence seq[i].
// mode 1: item i is a query row at position chunk_or_pos[i]; it closes chunk
//         pos / C only when (pos + 1) % C == 0 (prepared decode step).
template <int DT, bool VEC>
__global__ __launch_bounds__(64) void means_kernel(const uint16_t* __restrict__ kc, int Hkv,
                                                   int D, int P, const int* __restrict__ table,
                                                   int W, const int* __restrict__ seq,
                                                   const int* __restrict__ chunk_or_pos, int mode,
                                                   int C, uint16_t* __restrict__ means,
                                                   int max_chunks) {
  const int nd8 = (D + 7) / 8;
  const int db = blockIdx.x % nd8;
  const int kh = (blockIdx.x / nd8) % Hkv;
  const int i = blockIdx.x / (nd8 * Hkv);
  const int lane = threadIdx.x;
  const int sid = seq[i];
  int chunk = chunk_or_pos[i];
  if (mode == 1) {
    if ((chunk + 1) % C != 0) return;
    chunk = chunk / C;
  }
  const int* trow = table + (int64_t)sid * W;
  const int d0 = db * 8;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  for (int t = chunk * C + lane; t < (chunk + 1) * C; t += 64) {
    const int page = trow[t / P];
    if (page < 0) continue;  // unmapped page (caller bug): read nothing
    const int64_t off = (((int64_t)page * P + t % P) * Hkv + kh) * D + d0;
    if constexpr (VEC) {
      const u16x8_t x = ld8(kc + off);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] + to_f32<DT>(x[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (d0 + e < D) acc[e] = acc[e] + to_f32<DT>(kc[off + e]);
    }
  }
  uint16_t res[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) res[e] = from_f32<DT>(canon_tree(acc[e]) / (float)C);
  if (lane == 0) {
    uint16_t* dst = means + (((int64_t)sid * max_chunks + chunk) * Hkv + kh) * D + d0;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (d0 + e < D) dst[e] = res[e];
  }
}

// ------------------------------------------------------------------- route
// One wave per (query row, q head).  Lane j scores chunks j, j+64, ... (fp32
// fma chain over d, the canonical gate order) against the cache-dtype means;
// the stable top-R is R rounds of a wave argmax: each round takes the best
// candidate strictly after the previous pick in (score desc, chunk asc) order.
template <int DT>
__global__ __launch_bounds__(64) void route_kernel(const uint16_t* __restrict__ q, int Hq, int Hkv,
                                                   int D, const uint16_t* __restrict__ means,
                                                   int max_chunks, const int* __restrict__ seq,
                                                   const int* __restrict__ pos, int C, int width,
                                                   int R, float* __restrict__ scores,
                                                   int* __restrict__ selected) {
  __shared__ float qs[256];
  const int idx = blockIdx.x;  // row * Hq + h
  const int row = idx / Hq, h = idx % Hq;
  const int kh = h / (Hq / Hkv);
  const int lane = threadIdx.x;
  const int sid = seq[row], p = pos[row];
  for (int d = lane; d < D; d += 64) qs[d] = to_f32<DT>(q[(int64_t)idx * D + d]);
  __syncthreads();
  const int legal = min(p / C, width);  // chunks c with (c+1)*C <= p
  float* srow = scores + (int64_t)idx * width;
  for (int c = lane; c < width; c += 64) {
    float acc = -INFINITY;
    if (c < legal) {
      const uint16_t* mr = means + (((int64_t)sid * max_chunks + c) * Hkv + kh) * D;
      acc = 0.0f;
      for (int d = 0; d < D; ++d) acc = fmaf(to_f32<DT>(mr[d]), qs[d], acc);
    }
    srow[c] = acc;
  }
  __syncthreads();  // scores of this row are re-read by other lanes below
  int* out = selected + (int64_t)idx * (R + 1);
  if (lane == 0) out[0] = p / C;
  float last_v = INFINITY;
  int last_c = -1;
  for (int r = 0; r < R; ++r) {
    float bv = -INFINITY;
    int bc = 0x7fffffff;
    for (int c = lane; c < legal; c += 64) {
      const float v = srow[c];
      const bool after = v < last_v || (v == last_v && c > last_c);
      if (after && (v > bv || (v == bv && c < bc))) { bv = v; bc = c; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oc = __shfl_xor(bc, off, 64);
      if (ov > bv || (ov == bv && oc < bc)) { bv = ov; bc = oc; }
    }
    const bool found = bv > -INFINITY;
    if (lane == 0) out[1 + r] = found ? bc : -1;
    if (found) { last_v = bv; last_c = bc; } else { last_v = -INFINITY; last_c = 0x7fffffff; }
  }
}

// --------------------------------------------------------------- attention
struct AttnArgs {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  int Nq, Hq, Hkv, D, G, NHB;
  int P, W, C, nslot, nsub, dense;
  float scale_log2;
  const int* table;
  const int* lengths;
  const int* seq;
  const int* pos;
  const int* selected;
  float* part_o;
  float* part_ml;
  uint16_t* out;
  float* lse;
};

// Token range of (chunk c, sub-block b) for a query at p over a sequence of
// length len; empty when t0 >= t1.
MOBA_DEV void sub_range(int c, int b, int C, int p, int len, int& t0, int& t1) {
  t0 = c * C + b * kSub;
  t1 = min(min(t0 + kSub, (c + 1) * C), min(p + 1, len));
}

template <int DT, int DP, bool VEC>
__global__ __launch_bounds__(64) void attn_kernel(AttnArgs a) {
  constexpr int NKS = DP / 32;  // 32-d k-steps of S^T
  constexpr int NDB = DP / 16;  // 16-d blocks of O^T
  constexpr int VS = DP + 8;
  __shared__ __attribute__((aligned(16))) uint16_t Vs[32 * VS];

  const int lane = threadIdx.x, g4 = lane >> 4, c16 = lane & 15;
  const int bx = blockIdx.x;
  const int qrow = bx / (a.Hkv * a.NHB), kh = (bx / a.NHB) % a.Hkv, hb = bx % a.NHB;
  const int G = a.G, D = a.D;
  const int sid = a.seq[qrow], p = a.pos[qrow], len = a.lengths[sid];
  const int u = blockIdx.y, b = blockIdx.z;
  const int hg = hb * 16 + c16;  // this lane's head within the group
  const int h = kh * G + hg;
  const bool head_ok = hg < G;

  int c, jh = -1;
  if (a.dense) {
    c = u;
    if (c > p / a.C) return;
    jh = head_ok ? c : -1;
  } else {
    const int* sel = a.selected + ((int64_t)qrow * a.Hq + kh * G) * a.nslot;
    const int gu = u / a.nslot, ju = u % a.nslot;
    c = sel[gu * a.nslot + ju];
    if (c < 0) return;
    for (int x = 0; x < gu * a.nslot + ju; ++x)  // first occurrence in the union only
      if (sel[x] == c) return;
    if (head_ok)
      for (int j = 0; j < a.nslot; ++j)
        if (sel[hg * a.nslot + j] == c) { jh = j; break; }
  }
  if (__ballot(jh >= 0) == 0) return;
  int t0, t1;
  sub_range(c, b, a.C, p, len, t0, t1);
  if (t0 >= t1) return;

  const int* trow = a.table + (int64_t)sid * a.W;
  u16x8_t qf[NKS];
  {
    const uint16_t* qp = a.q + ((int64_t)qrow * a.Hq + h) * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 32 + g4 * 8;
      if constexpr (VEC) {
        qf[ks] = (head_ok && d < D) ? ld8(qp + d) : zero8();
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[ks][e] = (head_ok && d + e < D) ? qp[d + e] : (uint16_t)0;
      }
    }
  }
  f32x4v oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, lsum = 0.0f;

  for (int tt = t0; tt < t1; tt += 32) {
    // K rows of the two 16-token tiles (A operand, straight from the pool)
    f32x4v sc[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int tok = tt + half * 16 + c16;
      const int page = tok < t1 ? trow[tok / a.P] : -1;
      const bool tok_ok = page >= 0;  // unmapped pages read as zero, never out of the pool
      const int64_t base = tok_ok ? (((int64_t)page * a.P + tok % a.P) * a.Hkv + kh) * D : 0;
      sc[half] = (f32x4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d = ks * 32 + g4 * 8;
        u16x8_t kv;
        if constexpr (VEC) {
          kv = (tok_ok && d < D) ? ld8(a.kc + base + d) : zero8();
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) kv[e] = (tok_ok && d + e < D) ? a.kc[base + d + e] : (uint16_t)0;
        }
        sc[half] = mfma16<DT>(kv, qf[ks], sc[half]);
      }
    }
    // stage the V rows of these 32 tokens (row-major) for the transposed read
    for (int id = lane; id < 32 * (DP / 8); id += 64) {
      const int r = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      const int tok = tt + r;
      u16x8_t vv = zero8();
      const int page = tok < t1 ? trow[tok / a.P] : -1;
      if (page >= 0) {
        const int64_t base = (((int64_t)page * a.P + tok % a.P) * a.Hkv + kh) * D;
        if constexpr (VEC) {
          if (dc < D) vv = ld8(a.vc + base + dc);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) vv[e] = dc + e < D ? a.vc[base + dc + e] : (uint16_t)0;
        }
      }
      st8(&Vs[r * VS + dc], vv);
    }
    // online softmax for this lane's head over tokens {4g4+i, 16+4g4+i}
    float mx = -INFINITY;
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = tt + half * 16 + 4 * g4 + i;
        const float x = tok < t1 ? sc[half][i] * a.scale_log2 : -INFINITY;
        sc[half][i] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - mn);
    m_run = mn;
    float pr[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = fast_exp2(sc[0][i] - mn);
      pr[4 + i] = fast_exp2(sc[1][i] - mn);
    }
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ps += pr[e];
    lsum = lsum * alpha + ps;
    const u16x8_t pv = pack8<DT>(pr);
    __syncthreads();
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      // A = V^T (16 d x 32 tokens): column db*16 + c16, rows 4g4.. and 16+4g4..
      const uint16_t* p0 = Vs + (4 * g4 + (c16 >> 2)) * VS + db * 16 + 4 * (c16 & 3);
      const u16x4_t lo = ld_tr4(p0), hi = ld_tr4(p0 + 16 * VS);
      u16x8_t av;
      av[0] = lo[0]; av[1] = lo[1]; av[2] = lo[2]; av[3] = lo[3];
      av[4] = hi[0]; av[5] = hi[1]; av[6] = hi[2]; av[7] = hi[3];
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[db][i] *= alpha;
      oacc[db] = mfma16<DT>(av, pv, oacc[db]);
    }
    __syncthreads();
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (jh < 0) return;
  const int64_t entry = (((int64_t)qrow * a.Hq + h) * a.nslot + jh) * a.nsub + b;
  const float inv = 1.0f / lsum;
  float* po = a.part_o + entry * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = db * 16 + 4 * g4 + i;
      if (d < D) po[d] = oacc[db][i] * inv;
    }
  if (g4 == 0) {  // (max, sum) in the log2 domain: exact to merge at any magnitude
    a.part_ml[2 * entry] = m_run;
    a.part_ml[2 * entry + 1] = lsum;
  }
}

// One wave per (query, head): merge the partials of every slot / sub-block
// in ascending order.
template <int DT>
__global__ __launch_bounds__(64) void combine_kernel(AttnArgs a) {
  const int row = blockIdx.x;  // qrow * Hq + h
  const int qrow = row / a.Hq;
  const int lane = threadIdx.x, D = a.D;
  const int sid = a.seq[qrow], p = a.pos[qrow], len = a.lengths[sid];
  const int* sel = a.selected + (int64_t)row * a.nslot;
  const int nj = a.dense ? p / a.C + 1 : a.nslot;
  float M = -INFINITY;
  for (int j = 0; j < nj; ++j) {
    const int c = a.dense ? j : sel[j];
    if (c < 0) continue;
    for (int b = 0; b < a.nsub; ++b) {
      int t0, t1;
      sub_range(c, b, a.C, p, len, t0, t1);
      if (t0 < t1) M = fmaxf(M, a.part_ml[2 * (((int64_t)row * a.nslot + j) * a.nsub + b)]);
    }
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float z = 0.0f;
  for (int j = 0; j < nj; ++j) {
    const int c = a.dense ? j : sel[j];
    if (c < 0) continue;
    for (int b = 0; b < a.nsub; ++b) {
      int t0, t1;
      sub_range(c, b, a.C, p, len, t0, t1);
      if (t0 >= t1) continue;
      const int64_t entry = ((int64_t)row * a.nslot + j) * a.nsub + b;
      const float w = a.part_ml[2 * entry + 1] * fast_exp2(a.part_ml[2 * entry] - M);
      z += w;
      const float* po = a.part_o + entry * D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) acc[i] += w * po[d];
      }
    }
  }
  const float invz = 1.0f / z;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) a.out[(int64_t)row * D + d] = from_f32<DT>(acc[i] * invz);
  }
  if (lane == 0) a.lse[row] = (M + log2f(z)) * kLn2;
}

// ---------------------------------------------------------------- metadata
__global__ void metadata_kernel(int* __restrict__ table, int W, int* __restrict__ lengths,
                                const int* __restrict__ ids, int* __restrict__ positions,
                                const int* __restrict__ delta, int B, int append) {
  for (int row = threadIdx.x; row < B; row += blockDim.x) {
    const int sid = ids[row];
    const int logical = delta[row], physical = delta[B + row];
    if (logical >= 0) table[(int64_t)sid * W + logical] = physical;
    const int length = lengths[sid];
    if (append) {
      positions[row] = length;
      lengths[sid] = length + 1;
    } else {
      positions[row] = length - 1;
    }
  }
}

template <int DT, int DP>
int launch_attn(const AttnArgs& a, int n_items, hipStream_t st) {
  dim3 grid((unsigned)(a.Nq * a.Hkv * a.NHB), (unsigned)n_items, (unsigned)a.nsub);
  if (a.D % 8 == 0)
    hipLaunchKernelGGL((attn_kernel<DT, DP, true>), grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((attn_kernel<DT, DP, false>), grid, dim3(64), 0, st, a);
  hipLaunchKernelGGL(combine_kernel<DT>, dim3((unsigned)(a.Nq * a.Hq)), dim3(64), 0, st, a);
  return moba_launch_status("paged_attention");
}

template <int DT>
int dispatch_attn(const AttnArgs& a, int n_items, hipStream_t st) {
  if (a.D <= 32) return launch_attn<DT, 32>(a, n_items, st);
  if (a.D <= 64) return launch_attn<DT, 64>(a, n_items, st);
  if (a.D <= 128) return launch_attn<DT, 128>(a, n_items, st);
  return launch_attn<DT, 256>(a, n_items, st);
}

}  // namespace

extern "C" int moba_hip_decode_sub_tokens(void) { return kSub; }

extern "C" int moba_hip_paged_append(const void* k, const void* v, int dtype, int N, int Hkv, int D,
                                     void* k_cache, void* v_cache, int page_size,
                                     const int* table, int table_width, const int* token_seq,
                                     const int* token_pos, void* stream) {
  (void)dtype;
  if (N <= 0) return MOBA_OK;
  hipStream_t st = (hipStream_t)stream;
  if (D % 8 == 0) {
    const int64_t n = (int64_t)N * Hkv * (D / 8);
    hipLaunchKernelGGL(append_vec_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const uint16_t*)k, (const uint16_t*)v, N, Hkv, D, (uint16_t*)k_cache,
                       (uint16_t*)v_cache, page_size, table, table_width, token_seq, token_pos);
  } else {
    const int64_t n = (int64_t)N * Hkv * D;
    hipLaunchKernelGGL(append_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const uint16_t*)k, (const uint16_t*)v, N, Hkv, D, (uint16_t*)k_cache,
                       (uint16_t*)v_cache, page_size, table, table_width, token_seq, token_pos);
  }
  return moba_launch_status("paged_append");
}

extern "C" int moba_hip_block_means(const void* k_cache, int dtype, int Hkv, int D, int page_size,
                                    const int* table, int table_width, const int* item_seq,
                                    const int* item_chunk_or_pos, int n_items, int mode, int chunk,
                                    void* means, int max_chunks, void* stream) {
  if (n_items <= 0) return MOBA_OK;
  if (dtype != 0 && dtype != 1) { moba_set_error("block_means: dtype must be 0 or 1"); return MOBA_ERR_ARG; }
  dim3 grid((unsigned)((int64_t)n_items * Hkv * ((D + 7) / 8))), block(64);
  hipStream_t st = (hipStream_t)stream;
#define MOBA_MEANS(DT_, VEC_)                                                                   \
  hipLaunchKernelGGL((means_kernel<DT_, VEC_>), grid, block, 0, st, (const uint16_t*)k_cache,   \
                     Hkv, D, page_size, table, table_width, item_seq, item_chunk_or_pos, mode,  \
                     chunk, (uint16_t*)means, max_chunks)
  if (D % 8 == 0) { if (dtype == 0) MOBA_MEANS(0, true); else MOBA_MEANS(1, true); }
  else { if (dtype == 0) MOBA_MEANS(0, false); else MOBA_MEANS(1, false); }
#undef MOBA_MEANS
  return moba_launch_status("block_means");
}

extern "C" int moba_hip_decode_route(const void* q, int dtype, int Nq, int Hq, int Hkv, int D,
                                     const void* means, int max_chunks, const int* q_seq,
                                     const int* q_pos, int chunk, int width, int R, float* scores,
                                     int* selected, void* stream) {
  if (R < 0 || R > kMaxRemote) { moba_set_error("decode_route: remote count must be in [0,8]"); return MOBA_ERR_ARG; }
  if (Hq % Hkv) { moba_set_error("decode_route: Hq must be a multiple of Hkv"); return MOBA_ERR_ARG; }
  if (D < 1 || D > 256) { moba_set_error("decode_route: head_dim must be in [1,256]"); return MOBA_ERR_ARG; }
  if (R > 0 && (scores == nullptr || width < 1)) { moba_set_error("decode_route: scores workspace [Nq,Hq,width] required"); return MOBA_ERR_ARG; }
  const int64_t n = (int64_t)Nq * Hq;
  if (n == 0) return MOBA_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == 0)
    hipLaunchKernelGGL(route_kernel<0>, dim3((unsigned)n), dim3(64), 0, st, (const uint16_t*)q, Hq,
                       Hkv, D, (const uint16_t*)means, max_chunks, q_seq, q_pos, chunk, width, R,
                       scores, selected);
  else
    hipLaunchKernelGGL(route_kernel<1>, dim3((unsigned)n), dim3(64), 0, st, (const uint16_t*)q, Hq,
                       Hkv, D, (const uint16_t*)means, max_chunks, q_seq, q_pos, chunk, width, R,
                       scores, selected);
  return moba_launch_status("decode_route");
}

extern "C" int moba_hip_paged_attention(const void* q, int dtype, int Nq, int Hq, int Hkv, int D,
                                        const void* k_cache, const void* v_cache, int page_size,
                                        const int* table, int table_width, const int* lengths,
                                        const int* q_seq, const int* q_pos, const int* selected,
                                        int nslot, int dense, int chunk, int max_chunks_bound,
                                        float* part_o, float* part_ml, void* out, float* lse,
                                        void* stream) {
  if (dtype != 0 && dtype != 1) { moba_set_error("paged_attention: dtype must be 0 or 1"); return MOBA_ERR_ARG; }
  if (D < 1 || D > 256) { moba_set_error("paged_attention: head_dim must be in [1,256]"); return MOBA_ERR_ARG; }
  if (Hq % Hkv) { moba_set_error("paged_attention: Hq must be a multiple of Hkv"); return MOBA_ERR_ARG; }
  if (Nq <= 0) return MOBA_OK;
  AttnArgs a;
  a.q = (const uint16_t*)q; a.kc = (const uint16_t*)k_cache; a.vc = (const uint16_t*)v_cache;
  a.Nq = Nq; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv; a.NHB = (a.G + 15) / 16;
  a.P = page_size; a.W = table_width; a.C = chunk;
  a.dense = dense ? 1 : 0;
  a.nslot = dense ? max_chunks_bound : nslot;
  a.nsub = (chunk + kSub - 1) / kSub;
  a.scale_log2 = (1.0f / sqrtf((float)D)) * kLog2e;
  a.table = table; a.lengths = lengths; a.seq = q_seq; a.pos = q_pos; a.selected = selected;
  a.part_o = part_o; a.part_ml = part_ml; a.out = (uint16_t*)out; a.lse = lse;
  const int n_items = dense ? max_chunks_bound : a.G * nslot;
  if (n_items <= 0 || n_items > 65535 || a.nsub > 65535) { moba_set_error("paged_attention: work grid out of range"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  return dtype == 0 ? dispatch_attn<0>(a, n_items, st) : dispatch_attn<1>(a, n_items, st);
}

extern "C" int moba_hip_decode_metadata(int* table, int table_width, int* lengths, const int* ids,
                                        int* positions, const int* delta, int B, int append,
                                        void* stream) {
  if (B <= 0) return MOBA_OK;
  hipLaunchKernelGGL(metadata_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, table,
                     table_width, lengths, ids, positions, delta, B, append);
  return moba_launch_status("decode_metadata");
}
