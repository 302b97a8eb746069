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
//   decode_step       : prepared-decode step prologue in one launch: page-table
//                       delta + positions + length advance, the scatter of the
//                       new token, and the mean of a chunk the token closes
//
// decode_route builds, per (query, kv head, block of 16 q heads), a work list:
// the union of the chunks the heads selected (first-occurrence order), each
// with the mask of heads that chose it and their slot indices.
// paged_attention runs one 8-wave workgroup per work item (one whole chunk):
// every selected page is read once for all the q heads of the group.  Scores
// are S^T = K Q^T on v_mfma_f32_16x16x32 (16 tokens x 16 heads, K straight from
// the pool), O^T += V^T P^T with V^T taken from a row-major LDS tile by the
// transposed LDS read.  The waves split the chunk's tokens and merge in LDS;
// partials (o, max, sum) per (query, head, slot) are merged in slot order by
// combine_kernel.
#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {

typedef f32x4_t f32x4v;

constexpr int kWaves = 8;  // waves per attention workgroup
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
// Lane j's partial sums (8 dims from d0) of a chunk's keys: tokens t0 + j,
// t0 + j + 64, ... (at most kMeansPer of them, C <= 1024), added in that order
// (the canonical order; canon_tree then combines the 64 lanes).  All page
// lookups, then all row loads, are issued unconditionally (addresses clamped
// to token t0 / page offset 0) and masked after: guarded loads compiled to
// one full wait each.  A masked token adds +0, an exact no-op on a sum that
// starts at +0.
constexpr int kMeansPer = 16;

template <int DT, bool VEC>
MOBA_DEV void chunk_partials(const uint16_t* __restrict__ kc, const int* __restrict__ trow, int P,
                             int Hkv, int D, int kh, int d0, int t0, int C, int lane,
                             float (&acc)[8]) {
  int pg[kMeansPer];
#pragma unroll
  for (int k = 0; k < kMeansPer; ++k) {
    const int j = lane + 64 * k;
    pg[k] = trow[(t0 + (j < C ? j : 0)) / P];
  }
  u16x8_t x[kMeansPer];
#pragma unroll
  for (int k = 0; k < kMeansPer; ++k) {
    const int j = lane + 64 * k, t = t0 + (j < C ? j : 0);
    const int64_t off = pg[k] >= 0 ? (((int64_t)pg[k] * P + t % P) * Hkv + kh) * D + d0 : 0;
    if constexpr (VEC) {
      x[k] = ld8(kc + off);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] = kc[off + (d0 + e < D ? e : 0)];
    }
  }
#pragma unroll
  for (int k = 0; k < kMeansPer; ++k) {
    const bool on = lane + 64 * k < C && pg[k] >= 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = acc[e] + (on ? to_f32<DT>(x[k][e]) : 0.0f);
  }
}

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
  chunk_partials<DT, VEC>(kc, trow, P, Hkv, D, kh, d0, chunk * C, C, lane, acc);
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
// One workgroup (up to 8 waves) per (query row, kv head, block of 16 q heads).
// Wave w scores the heads g = w, w+nw, ... of the block: lane j takes chunks
// j, j+64, ... (fp32 fma
// chain over d, the canonical gate order) against the cache-dtype means; the
// stable top-R is R rounds of a wave argmax, each round taking the best
// candidate strictly after the previous pick in (score desc, chunk asc) order.
// The workgroup then writes its block's work list.
struct WorkItem {
  int chunk, mask, slots_lo, slots_hi;  // slots: 4 bits per head of the block
};

// Waves per route workgroup: at most 8, or 4 above 128 dims, where the q
// row and a means row held in registers take 256 of them.
template <int DP> constexpr int route_max_waves() { return DP > 128 ? 4 : 8; }

template <int DT, int DP, bool VEC>
__global__ __launch_bounds__(64 * route_max_waves<DP>()) void route_kernel(const uint16_t* __restrict__ q, int Hq, int Hkv,
                                                     int D, const uint16_t* __restrict__ means,
                                                     int max_chunks, const int* __restrict__ seq,
                                                     const int* __restrict__ pos, int C, int width,
                                                     int R, float* __restrict__ scores,
                                                     int* __restrict__ selected,
                                                     WorkItem* __restrict__ items,
                                                     int* __restrict__ item_counts, int max_items) {
  extern __shared__ float sc_lds[];  // [waves][width]
  __shared__ int sel_s[64 * 9];
  __shared__ int first_s[16 * 9], rank_s[16 * 9];
  __shared__ WorkItem it_s[16 * 9];
  __shared__ int n_s;
  const int G = Hq / Hkv, NHB = (G + 15) / 16;
  const int nw = blockDim.x >> 6;
  const int hb = blockIdx.x % NHB, rk = blockIdx.x / NHB;  // rk = qrow * Hkv + kh
  const int qrow = rk / Hkv, kh = rk % Hkv;
  const int g_lo = hb * 16, g_hi = min(G, g_lo + 16);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sid = seq[qrow], p = pos[qrow];
  const int legal = min(p / C, width);  // chunks c with (c+1)*C <= p
  float* sc = sc_lds + w * width;
  for (int g0 = g_lo; g0 < g_hi; g0 += nw) {
    const int g = g0 + w;
    if (g < g_hi) {
      const int h = kh * G + g;
      const int64_t idx = (int64_t)qrow * Hq + h;
      const uint16_t* qr = q + idx * D;
      if constexpr (VEC) {
        // the whole q row in registers; every means row loaded in one burst
        u16x8_t qv[DP / 8];
#pragma unroll
        for (int x = 0; x < DP / 8; ++x) qv[x] = x * 8 < D ? ld8(qr + x * 8) : zero8();
        for (int c = lane; c < width; c += 64) {
          float acc = -INFINITY;
          if (c < legal) {
            const uint16_t* mr = means + (((int64_t)sid * max_chunks + c) * Hkv + kh) * D;
            u16x8_t mv[DP / 8];
#pragma unroll
            for (int x = 0; x < DP / 8; ++x) mv[x] = x * 8 < D ? ld8(mr + x * 8) : zero8();
            acc = 0.0f;
#pragma unroll
            for (int x = 0; x < DP / 8; ++x)
              if (x * 8 < D) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                  acc = fmaf(to_f32<DT>(mv[x][e]), to_f32<DT>(qv[x][e]), acc);
              }
          }
          sc[c] = acc;
          scores[idx * width + c] = acc;
        }
      } else {
        for (int c = lane; c < width; c += 64) {
          float acc = -INFINITY;
          if (c < legal) {
            const uint16_t* mr = means + (((int64_t)sid * max_chunks + c) * Hkv + kh) * D;
            acc = 0.0f;
            for (int d = 0; d < D; ++d) acc = fmaf(to_f32<DT>(mr[d]), to_f32<DT>(qr[d]), acc);
          }
          sc[c] = acc;
          scores[idx * width + c] = acc;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      int* out = selected + idx * (R + 1);
      if (lane == 0) { out[0] = p / C; sel_s[g * (R + 1)] = p / C; }
      float last_v = INFINITY;
      int last_c = -1;
      for (int r = 0; r < R; ++r) {
        float bv = -INFINITY;
        int bc = 0x7fffffff;
        for (int c = lane; c < legal; c += 64) {
          const float v = sc[c];
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
        if (lane == 0) {
          out[1 + r] = found ? bc : -1;
          sel_s[g * (R + 1) + 1 + r] = found ? bc : -1;
        }
        if (found) { last_v = bv; last_c = bc; } else { last_v = -INFINITY; last_c = 0x7fffffff; }
      }
    }
    __syncthreads();  // the wave's score buffer is reused by its next head
  }
  if (items == nullptr) return;
  // Work list of each 16-head block: distinct chunks in first-occurrence
  // order over the flattened (head, slot) entries, with the mask of heads that
  // chose each chunk and their slot indices.  Built in parallel: entry e finds
  // its first occurrence by comparison, ranks come from a ballot prefix count.
  const int S = R + 1;
  {
    const int ng = g_hi - g_lo, E = ng * S;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      const int c = sel_s[g_lo * S + e];
      int first = -1;
      if (c >= 0) {
        first = e;
        for (int e2 = 0; e2 < e; ++e2)
          if (sel_s[g_lo * S + e2] == c) { first = e2; break; }
      }
      first_s[e] = first;
      it_s[e].chunk = 0; it_s[e].mask = 0; it_s[e].slots_lo = 0; it_s[e].slots_hi = 0;
    }
    __syncthreads();
    if (w == 0) {
      int base = 0;
      for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const bool is_first = e < E && first_s[e] == e;
        const uint64_t m = __ballot(is_first);
        if (e < E) rank_s[e] = base + __popcll(m & ((1ull << lane) - 1ull));
        base += __popcll(m);
      }
      if (lane == 0) n_s = base;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      const int f = first_s[e];
      if (f < 0) continue;
      const int x = rank_s[f], b = e / S, j = e % S;
      if (f == e) it_s[x].chunk = sel_s[g_lo * S + e];
      atomicOr(&it_s[x].mask, 1 << b);
      if (b < 8) atomicOr(&it_s[x].slots_lo, j << (4 * b));
      else atomicOr(&it_s[x].slots_hi, j << (4 * (b - 8)));
    }
    __syncthreads();
    const int n = n_s;
    WorkItem* it = items + ((int64_t)rk * NHB + hb) * max_items;
    for (int x = threadIdx.x; x < n; x += blockDim.x) it[x] = it_s[x];
    if (threadIdx.x == 0) item_counts[rk * NHB + hb] = n;
    __syncthreads();
  }
}

// --------------------------------------------------------------- attention
struct AttnArgs {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  int Nq, Hq, Hkv, D, G, NHB;
  int P, W, C, nslot, dense, max_items;
  float scale_log2;
  const int* table;
  const int* lengths;
  const int* seq;
  const int* pos;
  const int* selected;
  const WorkItem* items;
  const int* item_counts;
  float* part_o;
  float* part_ml;
  uint16_t* out;
  float* lse;
};

// Waves per attention workgroup: 8, or 4 above 128 dims, where the K/V
// register blocks and O accumulators of a wave need more than the 256
// registers of two waves per SIMD (8 waves spilled 145-655 registers).
template <int DP> constexpr int attn_waves() { return DP > 128 ? 4 : kWaves; }

template <int DT, int DP, bool VEC>
__global__ __launch_bounds__(64 * attn_waves<DP>()) void attn_kernel(AttnArgs a) {
  constexpr int NW = attn_waves<DP>();
  constexpr int NKS = DP / 32;  // 32-d k-steps of S^T
  constexpr int NDB = DP / 16;  // 16-d blocks of O^T
  constexpr int VS = DP + 8;
  constexpr int STAGE = 32 * VS;  // per-wave V tile (elements)
  constexpr int STAGE_BYTES = NW * STAGE * 2;
  constexpr int MERGE_BYTES = NW * (16 * DP + 32) * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds[STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES];
  uint16_t* Vs = reinterpret_cast<uint16_t*>(lds) + (threadIdx.x >> 6) * STAGE;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g4 = lane >> 4, c16 = lane & 15;
  const int r = blockIdx.x;  // (qrow * Hkv + kh) * NHB + hb
  const int hb = r % a.NHB, kh = (r / a.NHB) % a.Hkv, qrow = r / (a.NHB * a.Hkv);
  const int G = a.G, D = a.D;
  const int p = a.pos[qrow];
  const int n_items = a.dense ? p / a.C + 1 : a.item_counts[r];
  if ((int)blockIdx.y >= n_items) return;
  const int sid = a.seq[qrow], len = a.lengths[sid];
  // the workgroup takes work items blockIdx.y, blockIdx.y + gridDim.y, ...
  for (int i = blockIdx.y; i < n_items; i += gridDim.y) {
  int c, mask, jh = -1;
  if (a.dense) {
    c = i;
    const int nh = min(16, G - hb * 16);
    mask = (int)((1u << nh) - 1u);
    jh = c;
  } else {
    const WorkItem it = a.items[(int64_t)r * a.max_items + i];
    c = it.chunk;
    mask = it.mask;
    jh = c16 < 8 ? (it.slots_lo >> (4 * c16)) & 15 : (it.slots_hi >> (4 * (c16 - 8))) & 15;
  }
  const bool head_on = (mask >> c16) & 1;
  const int hg = hb * 16 + c16;
  const int h = kh * G + hg;
  const int t_begin = c * a.C;
  const int t_end = min(min((c + 1) * a.C, p + 1), len);
  const int* trow = a.table + (int64_t)sid * a.W;

  u16x8_t qf[NKS];
  {
    const uint16_t* qp = a.q + ((int64_t)qrow * a.Hq + h) * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 32 + g4 * 8;
      if constexpr (VEC) {
        qf[ks] = (head_on && d < D) ? ld8(qp + d) : zero8();
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[ks][e] = (head_on && d + e < D) ? qp[d + e] : (uint16_t)0;
      }
    }
  }
  f32x4v oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, lsum = 0.0f;

  // wave w takes the 32-token steps w, w + NW, ... of the chunk; the K rows and
  // V rows of the next step are loaded into registers while this one computes
  constexpr int VLD = 32 * (DP / 8) / 64;  // 16-byte V chunks per lane per step
  // Page of token t0 + r (0 <= r < 32) from one division per step: pages of at
  // least 32 tokens hold the step in at most two pages.
  auto page_of = [&](int t0, int pg0, int off0, int r) -> int {
    const int tok = t0 + r;
    if (tok >= t_end) return -1;
    int off = off0 + r, pg = pg0;
    if (off >= a.P) {
      if (a.P >= 32) { pg += 1; } else { pg += off / a.P; }
    }
    return trow[pg];
  };
  auto tok_off = [&](int off0, int r) -> int {  // row of token t0 + r inside its page
    const int off = off0 + r;
    return off < a.P ? off : (a.P >= 32 ? off - a.P : off % a.P);
  };
  auto load = [&](int t0, u16x8_t (&kr)[2][NKS], u16x8_t (&vr)[VLD]) {
    const int pg0 = t0 / a.P, off0 = t0 - pg0 * a.P;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int tok = t0 + half * 16 + c16;
      const int page = page_of(t0, pg0, off0, half * 16 + c16);
      const bool tok_ok = page >= 0;  // unmapped pages read as zero, never out of the pool
      const int64_t base =
          tok_ok ? (((int64_t)page * a.P + tok_off(off0, half * 16 + c16)) * a.Hkv + kh) * D : 0;
      (void)tok;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d = ks * 32 + g4 * 8;
        if constexpr (VEC) {
          kr[half][ks] = (tok_ok && d < D) ? ld8(a.kc + base + d) : zero8();
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            kr[half][ks][e] = (tok_ok && d + e < D) ? a.kc[base + d + e] : (uint16_t)0;
        }
      }
    }
#pragma unroll
    for (int x = 0; x < VLD; ++x) {
      const int id = lane + 64 * x, rr = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      const int page = page_of(t0, pg0, off0, rr);
      u16x8_t vv = zero8();
      if (page >= 0) {
        const int64_t base = (((int64_t)page * a.P + tok_off(off0, rr)) * a.Hkv + kh) * D;
        if constexpr (VEC) {
          if (dc < D) vv = ld8(a.vc + base + dc);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) vv[e] = dc + e < D ? a.vc[base + dc + e] : (uint16_t)0;
        }
      }
      vr[x] = vv;
    }
  };
  auto compute = [&](int tt, const u16x8_t (&kr)[2][NKS], const u16x8_t (&vr)[VLD]) {
    f32x4v sc[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      sc[half] = (f32x4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) sc[half] = mfma16<DT>(kr[half][ks], qf[ks], sc[half]);
    }
#pragma unroll
    for (int x = 0; x < VLD; ++x) {
      const int id = lane + 64 * x, rr = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      st8(&Vs[rr * VS + dc], vr[x]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = tt + half * 16 + 4 * g4 + e;
        const float xv = tok < t_end ? sc[half][e] * a.scale_log2 : -INFINITY;
        sc[half][e] = xv;
        mx = fmaxf(mx, xv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - mn);
    m_run = mn;
    float pr[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pr[e] = fast_exp2(sc[0][e] - mn);
      pr[4 + e] = fast_exp2(sc[1][e] - mn);
    }
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ps += pr[e];
    lsum = lsum * alpha + ps;
    const u16x8_t pv = pack8<DT>(pr);
    // the V tile is private to this wave: order its LDS stores before the reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      // A = V^T (16 d x 32 tokens): column db*16 + c16, rows 4g4.. and 16+4g4..
      const uint16_t* p0 = Vs + (4 * g4 + (c16 >> 2)) * VS + db * 16 + 4 * (c16 & 3);
      const u16x4_t lo = ld_tr4(p0), hi = ld_tr4(p0 + 16 * VS);
      u16x8_t av;
      av[0] = lo[0]; av[1] = lo[1]; av[2] = lo[2]; av[3] = lo[3];
      av[4] = hi[0]; av[5] = hi[1]; av[6] = hi[2]; av[7] = hi[3];
#pragma unroll
      for (int e = 0; e < 4; ++e) oacc[db][e] *= alpha;
      oacc[db] = mfma16<DT>(av, pv, oacc[db]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  constexpr int kStride = 32 * NW;
  int tt = t_begin + 32 * w;
  if (tt < t_end) {
    u16x8_t kr[2][NKS], vr[VLD];
    load(tt, kr, vr);
    for (; tt + kStride < t_end; tt += kStride) {
      u16x8_t kn[2][NKS], vn[VLD];
      load(tt + kStride, kn, vn);
      compute(tt, kr, vr);
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) kr[half][ks] = kn[half][ks];
#pragma unroll
      for (int x = 0; x < VLD; ++x) vr[x] = vn[x];
    }
    compute(tt, kr, vr);
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // merge the waves in LDS: per wave [16 heads][DP] of O^T plus (m, l) per head
  __shared__ int slot_s[16];
  if (tid < 16) slot_s[tid] = jh;  // lanes 0..15 of wave 0 hold heads 0..15
  __syncthreads();
  float* mrg = reinterpret_cast<float*>(lds);
  float* wo = mrg + w * (16 * DP + 32);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 4; ++e) wo[c16 * DP + db * 16 + 4 * g4 + e] = oacc[db][e];
  if (g4 == 0) { wo[16 * DP + c16] = m_run; wo[16 * DP + 16 + c16] = lsum; }
  __syncthreads();
  for (int x = tid; x < 16 * DP; x += 64 * NW) {
    const int hh = x / DP, d = x % DP;
    if (!((mask >> hh) & 1) || d >= D) continue;
    float M = -INFINITY;
    for (int ww = 0; ww < NW; ++ww) {
      const float* o = mrg + ww * (16 * DP + 32);
      if (o[16 * DP + 16 + hh] > 0.0f) M = fmaxf(M, o[16 * DP + hh]);
    }
    float z = 0.0f, acc = 0.0f;
    for (int ww = 0; ww < NW; ++ww) {
      const float* o = mrg + ww * (16 * DP + 32);
      const float l = o[16 * DP + 16 + hh];
      if (l > 0.0f) {
        const float f = fast_exp2(o[16 * DP + hh] - M);
        z += l * f;
        acc += o[hh * DP + d] * f;
      }
    }
    const int hj = hb * 16 + hh;
    const int j = slot_s[hh];
    const int64_t entry = ((int64_t)qrow * a.Hq + kh * G + hj) * a.nslot + j;
    a.part_o[entry * D + d] = acc / z;
    if (d == 0) { a.part_ml[2 * entry] = M; a.part_ml[2 * entry + 1] = z; }
  }
  __syncthreads();  // the merge buffer aliases the V tiles of the next item
  }
}

// One wave per (query, head): merge the per-slot partials in slot order.
template <int DT>
__global__ __launch_bounds__(64) void combine_kernel(AttnArgs a) {
  const int row = blockIdx.x;  // qrow * Hq + h
  const int qrow = row / a.Hq;
  const int lane = threadIdx.x, D = a.D;
  const int p = a.pos[qrow];
  const int* sel = a.selected + (int64_t)row * a.nslot;
  const int nj = a.dense ? p / a.C + 1 : a.nslot;
  // Each slot's loads are issued together and masked after (slots below
  // nslot are in the row's allocation, columns clamped): guarded loads
  // compiled to one full wait each.
  float M = -INFINITY;
  for (int j = 0; j < nj; ++j) {
    const bool on = a.dense || sel[j] >= 0;
    const float mj = a.part_ml[2 * ((int64_t)row * a.nslot + j)];
    M = on ? fmaxf(M, mj) : M;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float z = 0.0f;
  for (int j = 0; j < nj; ++j) {
    const bool on = a.dense || sel[j] >= 0;
    const int64_t entry = (int64_t)row * a.nslot + j;
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + 2 * entry);
    const float* po = a.part_o + entry * D;
    float o[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int d = lane + 64 * x;
      o[x] = po[d < D ? d : 0];
    }
    const float wgt = on ? ml.y * fast_exp2(ml.x - M) : 0.0f;
    z += wgt;
#pragma unroll
    for (int x = 0; x < 4; ++x) acc[x] += (on && lane + 64 * x < D) ? wgt * o[x] : 0.0f;
  }
  const float invz = 1.0f / z;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int d = lane + 64 * x;
    if (d < D) a.out[(int64_t)row * D + d] = from_f32<DT>(acc[x] * invz);
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

// Prepared-decode step prologue, one workgroup per active row: page-table
// delta, position / length advance, scatter of the new token, and, when the
// token closes its chunk, that chunk's mean (canonical order, one wave per
// (kv head, 8 d)).
template <int DT>
__global__ __launch_bounds__(256) void step_kernel(int* __restrict__ table, int W,
                                                   int* __restrict__ lengths,
                                                   const int* __restrict__ ids,
                                                   int* __restrict__ positions,
                                                   const int* __restrict__ delta, int B,
                                                   const uint16_t* __restrict__ k,
                                                   const uint16_t* __restrict__ v,
                                                   uint16_t* __restrict__ kc,
                                                   uint16_t* __restrict__ vc, int P, int Hkv,
                                                   int D, int C, uint16_t* __restrict__ means,
                                                   int max_chunks) {
  __shared__ int s_pos, s_page;
  const int row = blockIdx.x, tid = threadIdx.x;
  const int sid = ids[row];
  if (tid == 0) {
    const int logical = delta[row], physical = delta[B + row];
    if (logical >= 0) table[(int64_t)sid * W + logical] = physical;
    const int length = lengths[sid];
    positions[row] = length;
    lengths[sid] = length + 1;
    s_pos = length;
    s_page = table[(int64_t)sid * W + length / P];
  }
  __syncthreads();
  const int p = s_pos, page = s_page;
  if (page >= 0) {
    const int64_t dst = (((int64_t)page * P + p % P) * Hkv) * D;
    const int64_t src = (int64_t)row * Hkv * D;
    for (int x = tid; x < Hkv * D; x += 256) {
      kc[dst + x] = k[src + x];
      vc[dst + x] = v[src + x];
    }
  }
  if ((p + 1) % C != 0) return;  // workgroup-uniform
  __syncthreads();  // the token written above is part of the chunk mean
  const int chunk = p / C, nd8 = (D + 7) / 8;
  const int lane = tid & 63, w = tid >> 6;
  const int* trow = table + (int64_t)sid * W;
  for (int item = w; item < Hkv * nd8; item += 4) {
    const int kh = item / nd8, d0 = (item % nd8) * 8;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    if (D % 8 == 0) chunk_partials<DT, true>(kc, trow, P, Hkv, D, kh, d0, chunk * C, C, lane, acc);
    else chunk_partials<DT, false>(kc, trow, P, Hkv, D, kh, d0, chunk * C, C, lane, acc);
    uint16_t res[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) res[e] = from_f32<DT>(canon_tree(acc[e]) / (float)C);
    if (lane == 0) {
      uint16_t* dstm = means + (((int64_t)sid * max_chunks + chunk) * Hkv + kh) * D + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (d0 + e < D) dstm[e] = res[e];
    }
  }
}

template <int DT, int DP>
int launch_attn(const AttnArgs& a, int n_items, hipStream_t st) {
  // enough workgroups to fill the chip twice; each loops over its items
  const int rows = a.Nq * a.Hkv * a.NHB;
  int ny = (512 + rows - 1) / rows;
  if (ny > n_items) ny = n_items;
  if (ny < 1) ny = 1;
  dim3 grid((unsigned)rows, (unsigned)ny);
  if (a.D % 8 == 0)
    hipLaunchKernelGGL((attn_kernel<DT, DP, true>), grid, dim3(64 * attn_waves<DP>()), 0, st, a);
  else
    hipLaunchKernelGGL((attn_kernel<DT, DP, false>), grid, dim3(64 * attn_waves<DP>()), 0, st, a);
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

extern "C" int moba_hip_decode_work_items(int Hq, int Hkv, int nslot) {
  return (Hq / Hkv) * nslot;
}

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
  if (chunk < 1 || chunk > 1024) { moba_set_error("block_means: chunk must be in [1,1024]"); return MOBA_ERR_ARG; }
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
                                     int* selected, void* work_items, int* work_counts,
                                     void* stream) {
  if (R < 0 || R > kMaxRemote) { moba_set_error("decode_route: remote count must be in [0,8]"); return MOBA_ERR_ARG; }
  if (Hq % Hkv) { moba_set_error("decode_route: Hq must be a multiple of Hkv"); return MOBA_ERR_ARG; }
  if (Hq / Hkv > 64) { moba_set_error("decode_route: at most 64 q heads per kv head"); return MOBA_ERR_ARG; }
  if (D < 1 || D > 256) { moba_set_error("decode_route: head_dim must be in [1,256]"); return MOBA_ERR_ARG; }
  if (width < 0 || width > 8192) { moba_set_error("decode_route: width must be in [0,8192]"); return MOBA_ERR_ARG; }
  if (R > 0 && (scores == nullptr || width < 1)) { moba_set_error("decode_route: scores workspace [Nq,Hq,width] required"); return MOBA_ERR_ARG; }
  if (Nq <= 0) return MOBA_OK;
  hipStream_t st = (hipStream_t)stream;
  const int G = Hq / Hkv;
  // one wave per q head of a 16-head block, at most route_max_waves (the
  // kernel's register budget), bounded by the score buffers' LDS
  const int wmax = D % 8 != 0 ? route_max_waves<8>() : D <= 128 ? route_max_waves<128>()
                                                                : route_max_waves<256>();
  int nw = G < wmax ? G : wmax;
  const int wb = (width > 0 ? width : 1) * (int)sizeof(float);
  while (nw > 1 && nw * wb > 96 * 1024) --nw;
  const size_t lds = (size_t)nw * wb;
  const int max_items = G * (R + 1);
  const int NHB = (G + 15) / 16;
  dim3 grid((unsigned)(Nq * Hkv * NHB)), block(64 * nw);
#define MOBA_ROUTE(DT_, DP_, VEC_)                                                              \
  hipLaunchKernelGGL((route_kernel<DT_, DP_, VEC_>), grid, block, lds, st, (const uint16_t*)q,   \
                     Hq, Hkv, D, (const uint16_t*)means, max_chunks, q_seq, q_pos, chunk, width, \
                     R, scores, selected, (WorkItem*)work_items, work_counts, max_items)
#define MOBA_ROUTE_D(DT_)                                                                       \
  if (D % 8 != 0) MOBA_ROUTE(DT_, 8, false);                                                    \
  else if (D <= 64) MOBA_ROUTE(DT_, 64, true);                                                  \
  else if (D <= 128) MOBA_ROUTE(DT_, 128, true);                                                \
  else MOBA_ROUTE(DT_, 256, true)
  if (dtype == 0) { MOBA_ROUTE_D(0); } else { MOBA_ROUTE_D(1); }
#undef MOBA_ROUTE_D
#undef MOBA_ROUTE
  return moba_launch_status("decode_route");
}

extern "C" int moba_hip_paged_attention(const void* q, int dtype, int Nq, int Hq, int Hkv, int D,
                                        const void* k_cache, const void* v_cache, int page_size,
                                        const int* table, int table_width, const int* lengths,
                                        const int* q_seq, const int* q_pos, const int* selected,
                                        int nslot, const void* work_items, const int* work_counts,
                                        int dense, int chunk, int max_chunks_bound, float* part_o,
                                        float* part_ml, void* out, float* lse, void* stream) {
  if (dtype != 0 && dtype != 1) { moba_set_error("paged_attention: dtype must be 0 or 1"); return MOBA_ERR_ARG; }
  if (D < 1 || D > 256) { moba_set_error("paged_attention: head_dim must be in [1,256]"); return MOBA_ERR_ARG; }
  if (Hq % Hkv) { moba_set_error("paged_attention: Hq must be a multiple of Hkv"); return MOBA_ERR_ARG; }
  if (!dense && (nslot < 1 || nslot > 9 || work_items == nullptr || work_counts == nullptr)) {
    moba_set_error("paged_attention: moba mode needs 1..9 slots and the route work list");
    return MOBA_ERR_ARG;
  }
  if (Nq <= 0) return MOBA_OK;
  AttnArgs a;
  a.q = (const uint16_t*)q; a.kc = (const uint16_t*)k_cache; a.vc = (const uint16_t*)v_cache;
  a.Nq = Nq; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv; a.NHB = (a.G + 15) / 16;
  a.P = page_size; a.W = table_width; a.C = chunk;
  a.dense = dense ? 1 : 0;
  a.nslot = dense ? max_chunks_bound : nslot;
  a.max_items = a.G * nslot;
  a.scale_log2 = (1.0f / sqrtf((float)D)) * kLog2e;
  a.table = table; a.lengths = lengths; a.seq = q_seq; a.pos = q_pos; a.selected = selected;
  a.items = (const WorkItem*)work_items; a.item_counts = work_counts;
  a.part_o = part_o; a.part_ml = part_ml; a.out = (uint16_t*)out; a.lse = lse;
  const int n_items = dense ? max_chunks_bound : a.G * nslot;
  if (n_items <= 0 || n_items > 65535) { moba_set_error("paged_attention: work grid out of range"); return MOBA_ERR_ARG; }
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

extern "C" int moba_hip_decode_step(int* table, int table_width, int* lengths, const int* ids,
                                    int* positions, const int* delta, int B, const void* k,
                                    const void* v, int dtype, void* k_cache, void* v_cache,
                                    int page_size, int Hkv, int D, int chunk, void* means,
                                    int max_chunks, void* stream) {
  if (B <= 0) return MOBA_OK;
  if (dtype != 0 && dtype != 1) { moba_set_error("decode_step: dtype must be 0 or 1"); return MOBA_ERR_ARG; }
  if (chunk < 1 || chunk > 1024) { moba_set_error("decode_step: chunk must be in [1,1024]"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  if (dtype == 0)
    hipLaunchKernelGGL(step_kernel<0>, dim3(B), dim3(256), 0, st, table, table_width, lengths, ids,
                       positions, delta, B, (const uint16_t*)k, (const uint16_t*)v,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, page_size, Hkv, D, chunk,
                       (uint16_t*)means, max_chunks);
  else
    hipLaunchKernelGGL(step_kernel<1>, dim3(B), dim3(256), 0, st, table, table_width, lengths, ids,
                       positions, delta, B, (const uint16_t*)k, (const uint16_t*)v,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, page_size, Hkv, D, chunk,
                       (uint16_t*)means, max_chunks);
  return moba_launch_status("decode_step");
}
