// One-launch paged MoBA decode on gfx950.
//
// Replaces, for one query per row, the whole launch sequence of a decode step
// of src/moba_opt/ops/prepared_decode.py:6-94 and src/moba_opt/ops/paged_decode.py:
// page-table delta + position / length advance (_metadata), the scatter of
// the new token (_append_kernel), the mean of the chunk the token closes
// (_step_means), route scores + stable top-k + selected slots (_route_kernel,
// _stable_topk, _selected) and the attention (_attention_kernel).
//
// Two launches.  fused_kernel, grid (splits S, query rows x kv heads): every
// workgroup of a (query, kv head) first recomputes the route of the group's
// G <= 16 q heads (the work is tiny: G x closed chunks dot products against
// the stored means), giving every workgroup the same union of selected
// chunks.  The union's tokens, cut into 32-token blocks, are split evenly over
// the S workgroups; each workgroup's 8 waves take its blocks round-robin:
// S^T = K Q^T on v_mfma_f32_16x16x32 (16 tokens x the 16 heads, K straight
// from the page pool, heads that did not select the block's chunk masked),
// O^T += V^T P^T with V^T from a wave-private LDS tile by the transposed read.
// The waves merge in LDS into one (o, max, sum) partial per (head, split).
// merge_kernel, one workgroup per (query, q head), then combines the S
// partials in a fixed order (deterministic for a fixed S).  The launch boundary orders the
// partial stores before the merge reads, with no device-scope fences or
// arrival counters inside either kernel.
//
// Step mode: the new token's K/V are read from the input rows (so no
// workgroup waits for the scatter); split 0 scatters them and applies the
// page-table delta, the last split computes the closing chunk mean, and the
// merge advances the row's position and length.
#include <mutex>

#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

// Phase timestamps for profiling builds (-DMOBA_DECODE_TRACE): thread 0 of
// each workgroup of fused_kernel records s_memrealtime (100 MHz) at the
// phase boundaries below into a device array that moba_decode_trace_read
// copies out.  Compiled out of the product library.
#ifdef MOBA_DECODE_TRACE
__device__ unsigned long long g_decode_trace[16 * 8192];
extern "C" int moba_decode_trace_read(void* dst) {
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_trace), sizeof(g_decode_trace), 0,
                                  hipMemcpyDeviceToHost);
}
#define DTRACE(i)                                                              \
  do {                                                                         \
    if (threadIdx.x == 0) {                                                    \
      const unsigned wg = blockIdx.y * gridDim.x + blockIdx.x;                 \
      if (wg < 8192) g_decode_trace[wg * 16 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    }                                                                          \
  } while (0)
#else
#define DTRACE(i) do { } while (0)
#endif

namespace {

// Waves per workgroup (one workgroup per CU, 256 workgroups over the
// chip).  Eight waves run the route's (head, chunk) items in one pass of 512
// threads where four waves needed two, and halve the split partials the
// merge reads against 4-wave workgroups two per CU (cfg5 68.0 -> 65.9 us).
// Each of them streams its blocks through two register buffers (251
// registers, 2 waves per SIMD).  A launch whose workgroups carry many blocks
// instead takes 12 waves of one buffer each (167 registers, 3 waves per
// SIMD): with one block's load latency exposed per block either way, 1.5
// times the waves keep 1.5 times the bytes in flight (cfg5 64.5 -> 62.6 us;
// cfg4, about 4 blocks per workgroup, 26.0 -> 26.8 us with 12 waves, so it
// keeps 8).  D > 128 keeps 8 waves: 12 V tiles of 256 dims exceed LDS.
constexpr int kFwNarrow = 8;
constexpr int kFwWide = 12;
constexpr int kWideBlocksPerWorkgroup = 16;  // expected blocks at which 12 waves pay
constexpr int kMaxSlots = 9;    // current chunk + up to 8 routed chunks
constexpr int kMaxSeg = 64;     // 64-chunk segments of the parallel union (more: one wave)
constexpr int kGroupMax = 16;   // q heads of one (virtual) kv-head group: the MFMA's 16 columns
constexpr size_t kDynMax = 64 * 1024;  // dynamic LDS of one launch (route scratch + table row)

struct FusedArgs {
  const uint16_t* q;   // [Nq, Hq, D]
  const uint16_t* k;   // [Nq, Hkv, D] new tokens (step mode)
  const uint16_t* v;
  uint16_t* kc;        // pool [pages, P, Hkv, D]
  uint16_t* vc;
  // G: q heads per workgroup group (<= 16).  A kv head with more q heads is
  // served as Vg virtual kv heads of G q heads each (Vg * G = Hq / Hkv):
  // they share the physical head's K/V, means and page table, and the first
  // of them does the kv head's side work (scatter, closing mean).
  int Nq, Hq, Hkv, Vg, D, G, P, W, C, width, R, max_chunks, dense, pos_mode;
  float scale_log2;
  int* table;          // [B, W]
  int* lengths;        // [B]
  const int* ids;      // [Nq]
  int* positions;      // [Nq] (read when pos_mode == 0, written otherwise)
  const int* delta;    // [2, Nq] (logical slot, physical page) or null
  uint16_t* means;     // [B, max_chunks, Hkv, D]
  int* selected;       // [Nq, Hq, R + 1] or null
  float* part_o;       // [Nq, Hq, smax, D]
  float* part_ml;      // [Nq, Hq, smax, 2]
  const int* sched;    // null: uniform splits; else per workgroup (row x kv head, split,
                       // splits of that row), then splits per (row x kv head)
  int n_sched, smax;
  uint16_t* out;       // [Nq, Hq, D]
  float* lse;          // [Nq, Hq]
};

// Route scratch in dynamic LDS (ints / floats):
//   sc[G * width] | umask[width + 1] | item_c[width + 1] | item_m[width + 1] |
//   bp[width + 2] | sel[16 * kMaxSlots] | table row [table width, rounded up to 4]
inline size_t fused_route_lds(int G, int width, int table_width) {
  return sizeof(int) * ((size_t)G * width + 3 * (size_t)(width + 1) + (width + 2) +
                        16 * kMaxSlots + (((size_t)table_width + 3) & ~(size_t)3));
}

// Static LDS of fused_kernel<., DP, FW>: the per-wave V tiles (rows of
// DP + 8 elements), aliased after the attention by the waves' partials
// (rows of DP + 4 floats: float4 stores of 16 lanes hit 16 distinct bank
// groups).
constexpr size_t fused_static_lds(int DP, int FW) {
  return (size_t)FW * 32 * (DP + 8) * 2 > (size_t)FW * (16 * (DP + 4) + 32) * 4
             ? (size_t)FW * 32 * (DP + 8) * 2
             : (size_t)FW * (16 * (DP + 4) + 32) * 4;
}
constexpr size_t kLdsBytes = 160 * 1024;

// WROUTE: the launch has rows with more than 64 closed chunks (the wide
// score and top-k forms below are compiled in only then).
template <int DT, int DP, int FW, bool WROUTE>
__global__ __launch_bounds__(64 * FW) void fused_kernel(FusedArgs a) {
  constexpr int kFW = FW;
  constexpr int NKS = DP / 32;  // 32-d k-steps of S^T
  constexpr int NDB = DP / 16;  // 16-d blocks of O^T
  constexpr int VS = DP + 8;
  constexpr int STAGE = 32 * VS;  // per-wave V tile (elements)
  constexpr int STAGE_BYTES = kFW * STAGE * 2;
  constexpr int WS = DP + 4;
  constexpr int MERGE_BYTES = kFW * (16 * WS + 32) * 4;
  static_assert(fused_static_lds(DP, FW) == (STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES),
                "static LDS size");
  constexpr int VLD = 32 * (DP / 8) / 64;  // 16-byte V chunks per lane per block
  static_assert(64 * (DP + 8) * 2 + 16 * DP * 4 <= (STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES),
                "route staging must fit the V-tile / merge buffer");
  __shared__ __attribute__((aligned(16))) unsigned char lds[STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES];
  extern __shared__ int dyn[];
  __shared__ int s_info[8];
  __shared__ int s_segn[kMaxSeg], s_segb[kMaxSeg];  // per 64-chunk segment: items, blocks

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g4 = lane >> 4, c16 = lane & 15;
  int split, S, rowk;
  if (a.sched != nullptr) {
    const int* e = a.sched + 3 * blockIdx.x;
    rowk = e[0]; split = e[1]; S = e[2];
  } else {
    split = blockIdx.x; S = gridDim.x; rowk = blockIdx.y;
  }
  const int Hv = a.Hkv * a.Vg;  // (virtual) kv heads per row
  const int qrow = rowk / Hv, vh = rowk % Hv, kh = vh / a.Vg;
  const int G = a.G, D = a.D, C = a.C, width = a.width;
  const int hb = vh * G;                // first q head of the group
  const bool lead = vh % a.Vg == 0;     // does the physical kv head's side work

  DTRACE(0);
  // Row state comes from uniform (scalar) loads; the loads that need only the
  // slot (q rows, the first 64 closed-chunk means, the page-table row) are
  // issued before the position is known, so they overlap the lengths load.
  const int sid = a.ids != nullptr ? a.ids[qrow] : qrow;  // null ids: row i is slot i
  const int* trow = a.table + (int64_t)sid * a.W;
  int* tbl = dyn + (G * width + 3 * (width + 1) + (width + 2) + 16 * kMaxSlots);
  constexpr int RC = DP / 8;                  // 16-byte pieces per row
  constexpr int NSTG = (64 * RC + 64 * kFW - 1) / (64 * kFW);
  constexpr int MS = DP + 8;                         // padded row: conflict-free 16-byte reads
  uint16_t* ms = reinterpret_cast<uint16_t*>(lds);  // [64][MS] means rows (cache dtype)
  float* qsf = reinterpret_cast<float*>(ms + 64 * MS);  // [16][DP] q rows in fp32
  auto load_means = [&](int c0, int nc, u16x8_t (&stg)[NSTG]) {
#pragma unroll
    for (int i = 0; i < NSTG; ++i) {
      const int x = tid + i * 64 * kFW, cl = x / RC, j = x % RC;
      // issued unconditionally at a clamped address, masked after (a guarded
      // load costs a branch and a full wait each)
      const int clc = min(cl, nc - 1), jc = min(j, D / 8 - 1);
      stg[i] = ld8(a.means + (((int64_t)sid * a.max_chunks + c0 + clc) * a.Hkv + kh) * D + jc * 8);
      if (!(cl < nc && j * 8 < D)) stg[i] = zero8();
    }
  };
  auto store_means = [&](const u16x8_t (&stg)[NSTG]) {
#pragma unroll
    for (int i = 0; i < NSTG; ++i) {
      const int x = tid + i * 64 * kFW, cl = x / RC, j = x % RC;
      if (cl < 64) st8(ms + cl * MS + j * 8, stg[i]);
    }
  };
  constexpr int NQ = (16 * RC + 64 * kFW - 1) / (64 * kFW);
  u16x8_t qv[NQ], stg[NSTG];
  int t[4];
  {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int x = tid + i * 64 * kFW, qg = x / RC, qj = x % RC;
      qv[i] = ld8(a.q + ((int64_t)qrow * a.Hq + hb + min(qg, G - 1)) * D +
                  min(qj, D / 8 - 1) * 8);
      if (!(qg < G && qj * 8 < D)) qv[i] = zero8();
    }
    // rows past the position's closed chunks are staged but never scored
    if (!a.dense) load_means(0, min(64, width), stg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int x = tid + i * 64 * kFW;
      t[i] = trow[min(x, a.W - 1)];
    }
  }
  int p;
  if (a.pos_mode == 0) {
    p = a.positions[qrow];
  } else {
    const int len = a.lengths[sid];
    p = a.pos_mode == 2 ? len : len - 1;
  }
  const int dl = a.delta ? a.delta[qrow] : -1, dp = a.delta ? a.delta[a.Nq + qrow] : -1;
  DTRACE(1);
  const bool step = a.pos_mode == 2;
  // the position is published for the merge launch before any early exit (no
  // workgroup of this launch reads it in prepared modes)
  if (a.pos_mode != 0 && split == 0 && vh == 0 && tid == 0) a.positions[qrow] = p;
  if (p < 0 || p / C > width) return;  // caller contract: width covers every position
  const int npg = min(p / a.P + 1, a.W);
  const int cur = p / C;  // the current chunk (always attended, by every head)
  const int legal = a.dense ? 0 : min(cur, width);  // chunks c with (c + 1) * C <= p
  {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int x = tid + i * 64 * kFW;
      if (x < npg) tbl[x] = t[i];
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int x = tid + i * 64 * kFW, qg = x / RC, qj = x % RC;
      if (!a.dense && qg < G) {
        f32x4_t lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) { lo[e] = to_f32<DT>(qv[i][e]); hi[e] = to_f32<DT>(qv[i][4 + e]); }
        *reinterpret_cast<f32x4_t*>(qsf + qg * DP + qj * 8) = lo;
        *reinterpret_cast<f32x4_t*>(qsf + qg * DP + qj * 8 + 4) = hi;
      }
    }
    if (!a.dense) store_means(stg);
    for (int x0 = 4 * 64 * kFW; x0 < npg; x0 += 64 * kFW) {  // long rows
      const int x = x0 + tid;
      if (x < npg) tbl[x] = trow[x];
    }
  }
  __syncthreads();
  DTRACE(2);
  // page of logical slot `slot`; the page-table delta of this launch wins
  auto page_at = [&](int slot) -> int { return slot == dl ? dp : tbl[slot]; };

  // ---- side work of a step: table delta + scatter (split 0), closing mean
  if (a.pos_mode != 0 && split == 0 && vh == 0 && tid == 0 && dl >= 0)
    a.table[(int64_t)sid * a.W + dl] = dp;
  if (step && split == 0 && lead) {
    const int page = page_at(p / a.P);
    if (page >= 0) {
      const int64_t dst = (((int64_t)page * a.P + p % a.P) * a.Hkv + kh) * D;
      const int64_t src = ((int64_t)qrow * a.Hkv + kh) * D;
      for (int x = tid * 8; x < D; x += 64 * kFW * 8) {
        st8(a.kc + dst + x, ld8(a.k + src + x));
        st8(a.vc + dst + x, ld8(a.v + src + x));
      }
    }
  }
  if (step && lead && (p + 1) % C == 0) {
    // The mean of the chunk this token closes, canonical order: lane j sums
    // tokens j, j+64, ... of the chunk in order, then the fixed tree.  Its
    // D/8 items of 8 dims are spread over the row's splits and waves (item i:
    // split i % S, wave (i / S) % 4), each item's loads issued together.
    const int cc = p / C, nd8 = D / 8;
    for (int item = split + S * w; item < nd8; item += S * kFW) {
      const int d0 = item * 8;
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
      for (int t0 = 0; t0 < C; t0 += 64 * 16) {
        u16x8_t x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int tl = t0 + lane + 64 * i, tok = tl < C ? cc * C + tl : p;
          const uint16_t* src =
              tok == p ? a.k + ((int64_t)qrow * a.Hkv + kh) * D + d0
                       : a.kc + (((int64_t)max(page_at(tok / a.P), 0) * a.P + tok % a.P) * a.Hkv + kh) * D + d0;
          x[i] = ld8(src);
          if (tl >= C) x[i] = zero8();
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] = acc[e] + to_f32<DT>(x[i][e]);
      }
      uint16_t res[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) res[e] = from_f32<DT>(canon_tree(acc[e]) / (float)C);
      if (lane == 0) {
        uint16_t* m = a.means + (((int64_t)sid * a.max_chunks + cc) * a.Hkv + kh) * D + d0;
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = res[e];
      }
    }
  }
  DTRACE(3);

  // ---- route: scores, stable top-R per head, union of the chosen chunks
  float* sc = reinterpret_cast<float*>(dyn);
  int* umask = dyn + G * width;
  int* item_c = umask + (width + 1);
  int* item_m = item_c + (width + 1);
  int* bp = item_m + (width + 1);
  int* sel_s = bp + (width + 2);
  const int all_heads = (int)((1u << G) - 1u);
  const int S1 = a.R + 1;
  for (int c = tid; c <= cur; c += 64 * kFW) umask[c] = (a.dense || c == cur) ? all_heads : 0;
  for (int x = tid; x < G * S1; x += 64 * kFW) sel_s[x] = x % S1 == 0 ? cur : -1;
  if (!a.dense) {
    if constexpr (WROUTE) {
      // Scores: each is the sequential fp32 fma chain over d of a staged means
      // row (64 rows per tile) and the head's q row (fp32 in LDS).  Wide routes
      // (more than 64 closed chunks) stream the means rows with lanes as chunks;
      // narrow ones take one (head, chunk) item per thread.  The next tile's
      // means rows are loaded into registers while a tile is scored.
      const bool wide = legal > 64;
      for (int c0 = 0; c0 < legal; c0 += 64) {
        const int nc = min(64, legal - c0);
        // the first 64 rows came with the first burst; the wide form reads all
        // of its rows itself in the first pass
        if (wide && c0 > 0) break;
        const bool more = !wide && c0 + 64 < legal;
        if (more) load_means(c0 + 64, min(64, legal - c0 - 64), stg);
        if (wide) {
          // unit u = (tile u / nq, heads hpu (u % nq) .. + hpu - 1), nq =
          // ceil(G / hpu), dealt to the waves, its head chains interleaved.
          // lane = chunk.  The lane's means
          // row comes from global memory (L2) into registers and feeds the
          // unit's head chains; head g's q row sits 16 dims per register, dim
          // 16 i + j in lane j of each 16-lane row, and reaches the chain by DPP
          // row broadcast.  Lanes past the closed chunks compute on a clamped
          // row and store nothing.  (All tiles are scored in the first pass.)
          if (c0 == 0) {
            const int ntile = (legal + 63) / 64;
            const int hpu = 4;  // four interleaved chains (two were slower at G = 4)
            const int nq = (G + hpu - 1) / hpu;
            for (int u = w; u < ntile * nq; u += kFW) {
              const int t0 = (u / nq) * 64, g0 = (u % nq) * hpu;
              const int c = min(t0 + lane, legal - 1);
              const uint16_t* mrow = a.means + (((int64_t)sid * a.max_chunks + c) * a.Hkv + kh) * D;
              u16x8_t mv[RC];
#pragma unroll
              for (int j = 0; j < RC; ++j) mv[j] = j * 8 < D ? ld8(mrow + j * 8) : zero8();
              float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int i = 0; i < DP / 16; ++i) {
                float qb[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) qb[k] = qsf[min(g0 + k, G - 1) * DP + 16 * i + c16];
#pragma unroll
                for (int hlf = 0; hlf < 2; ++hlf) {
                  float m[8];
#pragma unroll
                  for (int e = 0; e < 8; ++e) m[e] = to_f32<DT>(mv[2 * i + hlf][e]);
                  if (hlf == 0) fma8_bcast4<0>(acc, qb, m); else fma8_bcast4<8>(acc, qb, m);
                }
              }
              if (t0 + lane < legal) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                  if (k < hpu && g0 + k < G) sc[(g0 + k) * width + t0 + lane] = acc[k];
              }
            }
          }
        } else {
          for (int x = tid; x < G * nc; x += 64 * kFW) {
            const int g = x / nc, cl = x % nc;
            const float* qg = qsf + g * DP;
            const uint16_t* mr = ms + cl * MS;
            float acc = 0.0f;
            // operands of 8 pieces (64 d) are read in one batch, then the chain
            // runs on registers; pieces past D are zero in both rows, and
            // fma(0, 0, acc) == acc
            constexpr int JB = RC % 8 == 0 ? 8 : RC % 6 == 0 ? 6 : RC;  // divides RC
#pragma unroll
            for (int j0 = 0; j0 < RC; j0 += JB) {
              u16x8_t mv[JB];
              f32x4_t qa[JB], qb[JB];
#pragma unroll
              for (int j = 0; j < JB; ++j) {
                mv[j] = ld8(mr + (j0 + j) * 8);
                qa[j] = *reinterpret_cast<const f32x4_t*>(qg + (j0 + j) * 8);
                qb[j] = *reinterpret_cast<const f32x4_t*>(qg + (j0 + j) * 8 + 4);
              }
#pragma unroll
              for (int j = 0; j < JB; ++j) {
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = fmaf(to_f32<DT>(mv[j][e]), qa[j][e], acc);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = fmaf(to_f32<DT>(mv[j][4 + e]), qb[j][e], acc);
              }
            }
            sc[g * width + c0 + cl] = acc;
          }
        }
        if (more) {
          __syncthreads();  // this tile's scores are done
          store_means(stg);
          __syncthreads();
        }
      }
    } else {
      // Scores: thread x takes (head x / nc, chunk x % nc) of the tile; each
      // score is the sequential fp32 fma chain over d of the staged mean row
      // and the head's q row (fp32 in LDS).
      for (int c0 = 0; c0 < legal; c0 += 64) {
        const int nc = min(64, legal - c0);
        if (c0 > 0) {  // the first 64 means rows came with the first burst
          load_means(c0, nc, stg);
          __syncthreads();  // the previous tile's scores are done
          store_means(stg);
          __syncthreads();
        }
        for (int x = tid; x < G * nc; x += 64 * kFW) {
          const int g = x / nc, cl = x % nc;
          const float* qg = qsf + g * DP;
          const uint16_t* mr = ms + cl * MS;
          float acc = 0.0f;
          // operands of 8 pieces (64 d) are read in one batch, then the chain
          // runs on registers; pieces past D are zero in both rows, and
          // fma(0, 0, acc) == acc
          constexpr int JB = RC % 8 == 0 ? 8 : RC % 6 == 0 ? 6 : RC;  // divides RC
#pragma unroll
          for (int j0 = 0; j0 < RC; j0 += JB) {
            u16x8_t mv[JB];
            f32x4_t qa[JB], qb[JB];
#pragma unroll
            for (int j = 0; j < JB; ++j) {
              mv[j] = ld8(mr + (j0 + j) * 8);
              qa[j] = *reinterpret_cast<const f32x4_t*>(qg + (j0 + j) * 8);
              qb[j] = *reinterpret_cast<const f32x4_t*>(qg + (j0 + j) * 8 + 4);
            }
#pragma unroll
            for (int j = 0; j < JB; ++j) {
#pragma unroll
              for (int e = 0; e < 4; ++e) acc = fmaf(to_f32<DT>(mv[j][e]), qa[j][e], acc);
#pragma unroll
              for (int e = 0; e < 4; ++e) acc = fmaf(to_f32<DT>(mv[j][4 + e]), qb[j][e], acc);
            }
          }
          sc[g * width + c0 + cl] = acc;
        }
      }
    }
    __syncthreads();
    DTRACE(4);
    // stable top-R by rank: chunk c of head g takes slot 1 + rank, where rank
    // counts the chunks ahead of it in (score desc, chunk asc) order; -inf
    // and NaN scores are never selected.  Same picks as R rounds of "best
    // candidate strictly after the previous pick".
    //
    // Wide routes (more than 64 closed chunks; counting ranks costs G x
    // legal^2 comparisons): wave w takes heads w, w + kFW, ...; each lane
    // keeps the best R of its chunks (lane, lane + 64, ...) as order keys
    // (score desc, chunk asc), then R rounds of a wave-wide maximum pick the
    // head's chunks in rank order -- the same picks.
    if (WROUTE && legal > 64) {
      for (int g = w; g < G; g += kFW) {
        const float* sg = sc + g * width;
        uint64_t bk[kMaxSlots - 1];
#pragma unroll
        for (int r = 0; r < kMaxSlots - 1; ++r) bk[r] = 0;
        for (int c = lane; c < legal; c += 64) {
          uint64_t x = route_key(sg[c], c);
#pragma unroll
          for (int r = 0; r < kMaxSlots - 1; ++r) {  // insertion into the descending list
            const uint64_t hi = bk[r] > x ? bk[r] : x, lo = bk[r] > x ? x : bk[r];
            bk[r] = hi;
            x = lo;
          }
        }
        for (int r = 0; r < a.R; ++r) {
          uint64_t m = bk[0];
#pragma unroll
          for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t yl = __shfl_xor((uint32_t)m, o, 64);
            const uint32_t yh = __shfl_xor((uint32_t)(m >> 32), o, 64);
            const uint64_t y = ((uint64_t)yh << 32) | yl;
            m = m > y ? m : y;
          }
          if (m == 0) break;  // no selectable chunk left
          if (bk[0] == m) {   // the one lane holding it (keys are distinct)
#pragma unroll
            for (int q2 = 0; q2 < kMaxSlots - 2; ++q2) bk[q2] = bk[q2 + 1];
            bk[kMaxSlots - 2] = 0;
          }
          if (lane == 0) {
            const int c = 0x7fffffff - (int)(uint32_t)m;
            sel_s[g * S1 + 1 + r] = c;
            atomicOr(&umask[c], 1 << g);
          }
        }
      }
    } else
    for (int x = tid; x < G * legal; x += 64 * kFW) {
      const int g = x / legal, c = x % legal;
      const float* sg = sc + g * width;
      const float v = sg[c];
      if (!(v > -INFINITY)) continue;
      // 32 scores per batch, all read before the comparisons, entries past
      // `legal` as -inf (the reads stay inside the route scratch).  Count the
      // higher scores and the equal ones (v itself included); only exact ties
      // need the chunk order, in a per-lane pass over the lower chunks.
      int gt = 0, eq = 0;
      for (int c0 = 0; c0 < legal; c0 += 32) {
        float u[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) u[i] = sg[c0 + i];
        if (c0 + 32 > legal) {
#pragma unroll
          for (int i = 0; i < 32; ++i) u[i] = c0 + i < legal ? u[i] : -INFINITY;
        }
        // one comparison at a time: hoisted together, their lane masks
        // exhausted the scalar registers and spilled
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          gt += (int)(u[i] > v);
          eq += (int)(u[i] == v);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      int rank = gt;
      if (eq > 1)
        for (int j = 0; j < c; ++j) rank += (int)(sg[j] == v);
      if (rank < a.R) {
        sel_s[g * S1 + 1 + rank] = c;
        atomicOr(&umask[c], 1 << g);
      }
    }
  }
  __syncthreads();
  DTRACE(5);
  if (!a.dense && split == 0 && a.selected != nullptr) {
    for (int x = tid; x < G * S1; x += 64 * kFW) {
      const int g = x / S1, j = x % S1;
      a.selected[((int64_t)qrow * a.Hq + hb + g) * S1 + j] = sel_s[x];
    }
  }
  if constexpr (WROUTE) {
    // items: the union's chunks in ascending order with their head masks, and
    // the prefix count of 32-token blocks.  Chunks go in segments of 64, one
    // lane each: with one segment, wave 0 does it; with several, the waves
    // count their segments' items and blocks, then place them after the counts
    // of the segments before.
    const int nseg = cur / 64 + 1;
    auto seg_items = [&](int sg, int n0, int nb0, bool place, int& cnt, int& nblk) {
      const int c = sg * 64 + lane;
      const int m = c <= cur ? umask[c] : 0;
      const uint64_t bal = __ballot(m != 0);
      const int ntok = c < cur ? C : p + 1 - cur * C;
      const int blocks = m != 0 ? (ntok + 31) / 32 : 0;
      int incl = blocks;  // inclusive scan of the block counts over the wave
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
      if (place && m != 0) {
        const int rank = n0 + __popcll(bal & ((1ull << lane) - 1ull));
        item_c[rank] = c;
        item_m[rank] = m;
        bp[rank] = nb0 + incl - blocks;
      }
      cnt = __popcll(bal);
      nblk = __shfl(incl, 63, 64);
    };
    if (nseg == 1 || nseg > kMaxSeg) {
      if (w == 0) {
        int n = 0, nb = 0;
        for (int sg = 0; sg < nseg; ++sg) {
          int cnt, nblk;
          seg_items(sg, n, nb, true, cnt, nblk);
          n += cnt;
          nb += nblk;
        }
        if (lane == 0) {
          bp[n] = nb;
          s_info[4] = n;
          s_info[5] = nb;
        }
      }
    } else {
      for (int sg = w; sg < nseg; sg += kFW) {
        int cnt, nblk;
        seg_items(sg, 0, 0, false, cnt, nblk);
        if (lane == 0) { s_segn[sg] = cnt; s_segb[sg] = nblk; }
      }
      __syncthreads();
      for (int sg = w; sg < nseg; sg += kFW) {
        int n0 = 0, nb0 = 0;
        for (int k = 0; k < sg; ++k) { n0 += s_segn[k]; nb0 += s_segb[k]; }
        int cnt, nblk;
        seg_items(sg, n0, nb0, true, cnt, nblk);
        if (sg == nseg - 1 && lane == 0) {
          bp[n0 + cnt] = nb0 + nblk;
          s_info[4] = n0 + cnt;
          s_info[5] = nb0 + nblk;
        }
      }
    }
  } else {
    // items: the union's chunks in ascending order with their head masks, and
    // the prefix count of 32-token blocks
    if (w == 0) {
      int n = 0, nb = 0;
      for (int c0 = 0; c0 <= cur; c0 += 64) {
        const int c = c0 + lane;
        const int m = c <= cur ? umask[c] : 0;
        const uint64_t bal = __ballot(m != 0);
        const int rank = n + __popcll(bal & ((1ull << lane) - 1ull));
        const int ntok = c < cur ? C : p + 1 - cur * C;
        int blocks = m != 0 ? (ntok + 31) / 32 : 0;
        // inclusive scan of the block counts over the wave
        int incl = blocks;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int y = __shfl_up(incl, off, 64);
          if (lane >= off) incl += y;
        }
        if (m != 0) {
          item_c[rank] = c;
          item_m[rank] = m;
          bp[rank] = nb + incl - blocks;
        }
        n += __popcll(bal);
        nb += __shfl(incl, 63, 64);
      }
      if (lane == 0) {
        bp[n] = nb;
        s_info[4] = n;
        s_info[5] = nb;
      }
    }
  }
  __syncthreads();
  const int n_items = s_info[4], NB = s_info[5];
  DTRACE(6);
  const int b0 = (int)((int64_t)split * NB / S), b1 = (int)((int64_t)(split + 1) * NB / S);

  // ---- attention over blocks [b0, b1)
  uint16_t* Vs = reinterpret_cast<uint16_t*>(lds) + w * STAGE;
  const bool head_ok = c16 < G;
  const int h = hb + (head_ok ? c16 : 0);
  u16x8_t qf[NKS];
  {
    const uint16_t* qp = a.q + ((int64_t)qrow * a.Hq + h) * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 32 + g4 * 8;
      qf[ks] = (head_ok && d < D) ? ld8(qp + d) : zero8();
    }
  }
  f32x4_t oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, lsum = 0.0f;

  struct Blk { int t0, t_end, mask; };
  auto block_info = [&](int b) -> Blk {
    int lo = 0, hi = n_items - 1;  // last item with bp[i] <= b
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (bp[mid] <= b) lo = mid; else hi = mid - 1;
    }
    const int c = item_c[lo];
    Blk r;
    r.t0 = c * C + (b - bp[lo]) * 32;
    r.t_end = min((c + 1) * C, p + 1);
    r.mask = item_m[lo];
    return r;
  };
  // K rows of tokens t0 + half*16 + c16 and the V rows of the block.  A row
  // is (source, element offset): the new token of a step comes from the input
  // row; tokens past the block end or on unmapped pages read as zero.
  // The input rows are addressed as an element distance from the cache, so
  // the per-lane choice of source is an integer add: a per-lane choice
  // between the two argument pointers compiled to a load of the chosen
  // pointer, and waiting for it also waited for every K/V load in flight.
  const int64_t k_in_off = ((int64_t)(uintptr_t)a.k - (int64_t)(uintptr_t)a.kc) / 2;
  const int64_t v_in_off = ((int64_t)(uintptr_t)a.v - (int64_t)(uintptr_t)a.vc) / 2;
  auto row_of = [&](int tok, bool& from_input) -> int64_t {
    from_input = false;
    if (tok >= 0 && step && tok == p) {
      from_input = true;
      return ((int64_t)qrow * a.Hkv + kh) * D;
    }
    const int pg = page_at(tok / a.P);
    if (pg < 0) return -1;
    return (((int64_t)pg * a.P + tok % a.P) * a.Hkv + kh) * D;
  };
  auto load = [&](const Blk& bk, u16x8_t (&kr)[2][NKS], u16x8_t (&vr)[VLD]) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int tok = bk.t0 + half * 16 + c16;
      bool inp = false;
      const int64_t base = tok < bk.t_end ? row_of(tok, inp) : -1;
      const uint16_t* kp = a.kc + (inp ? k_in_off : 0);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d = ks * 32 + g4 * 8;
        const bool ok = base >= 0 && d < D;
        kr[half][ks] = ok ? ld8(kp + base + d) : zero8();
      }
    }
#pragma unroll
    for (int x = 0; x < VLD; ++x) {
      const int id = lane + 64 * x, rr = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      const int tok = bk.t0 + rr;
      bool inp = false;
      const int64_t base = tok < bk.t_end ? row_of(tok, inp) : -1;
      const uint16_t* vp = a.vc + (inp ? v_in_off : 0);
      const bool ok = base >= 0 && dc < D;
      vr[x] = ok ? ld8(vp + base + dc) : zero8();
    }
  };
  auto compute = [&](const Blk& bk, const u16x8_t (&kr)[2][NKS], const u16x8_t (&vr)[VLD]) {
    f32x4_t s4[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      s4[half] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) s4[half] = mfma16<DT>(kr[half][ks], qf[ks], s4[half]);
    }
#pragma unroll
    for (int x = 0; x < VLD; ++x) {
      const int id = lane + 64 * x, rr = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      st8(&Vs[rr * VS + dc], vr[x]);
    }
    const bool on = head_ok && ((bk.mask >> c16) & 1);
    float mx = -INFINITY;
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = bk.t0 + half * 16 + 4 * g4 + e;
        const float xv = (on && tok < bk.t_end) ? s4[half][e] * a.scale_log2 : -INFINITY;
        s4[half][e] = xv;
        mx = fmaxf(mx, xv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m_run, mx);
    const float ms = mn == -INFINITY ? 0.0f : mn;  // no finite score yet: all weights 0
    const float alpha = fast_exp2(m_run - ms);
    m_run = mn;
    float pr[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pr[e] = fast_exp2(s4[0][e] - ms);
      pr[4 + e] = fast_exp2(s4[1][e] - ms);
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
  {
    // wave w takes blocks b0 + w, b0 + w + kFW, ...: 12-wave form and head
    // dims above 128 one register buffer, 8-wave form two (ping-pong: block
    // b + kFW loads while block b computes).  Two 256-wide buffers need more
    // than the 256 registers of a 2-wave-per-SIMD launch (about 700 spilled).
    int b = b0 + w;
    if constexpr (FW > kFwNarrow || DP > 128) {
      // one register buffer: load, then compute, block after block
      for (; b < b1; b += kFW) {
        u16x8_t kA[2][NKS], vA[VLD];
        const Blk bA = block_info(b);
        load(bA, kA, vA);
        compute(bA, kA, vA);
      }
    } else if (b < b1) {
      u16x8_t kA[2][NKS], vA[VLD], kB[2][NKS], vB[VLD];
      Blk bA = block_info(b), bB;
      load(bA, kA, vA);
      __builtin_amdgcn_sched_barrier(0);
      for (;;) {
        const int bn = b + kFW;
        if (bn < b1) {
          bB = block_info(bn);
          load(bB, kB, vB);
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(bA, kA, vA);
        if (bn >= b1) break;
        const int bn2 = bn + kFW;
        if (bn2 < b1) {
          bA = block_info(bn2);
          load(bA, kA, vA);
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(bB, kB, vB);
        if (bn2 >= b1) break;
        b = bn2;
      }
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // ---- merge the waves in LDS into this split's partial per head
  __syncthreads();  // all V tiles consumed: the merge buffer aliases them
  DTRACE(7);
  float* mrg = reinterpret_cast<float*>(lds);
  {
    float* wo = mrg + w * (16 * WS + 32);
    // head c16's row, dims db*16 + 4*g4 .. +3: one 16-byte store per block
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      *reinterpret_cast<f32x4_t*>(wo + c16 * WS + db * 16 + 4 * g4) = oacc[db];
    if (g4 == 0) { wo[16 * WS + c16] = m_run; wo[16 * WS + 16 + c16] = lsum; }
  }
  __syncthreads();
  // thread x: head x / (D/4), dims 4 (x % (D/4)) .. +3 (16-byte LDS reads
  // and global stores; D is a multiple of 8)
  const int nd4 = D / 4;
  for (int x = tid; x < G * nd4; x += 64 * kFW) {
    const int g = x / nd4, d = (x % nd4) * 4;
    float mw[kFW], lw[kFW];
#pragma unroll
    for (int ww = 0; ww < kFW; ++ww) {
      const float* o = mrg + ww * (16 * WS + 32);
      mw[ww] = o[16 * WS + g];
      lw[ww] = o[16 * WS + 16 + g];
    }
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kFW; ++ww) M = lw[ww] > 0.0f ? fmaxf(M, mw[ww]) : M;
    float z = 0.0f;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < kFW; ++ww) {
      const f32x4_t ov = *reinterpret_cast<const f32x4_t*>(mrg + ww * (16 * WS + 32) + g * WS + d);
      const float f = lw[ww] > 0.0f ? fast_exp2(mw[ww] - M) : 0.0f;
      z += lw[ww] * f;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += lw[ww] > 0.0f ? ov[e] * f : 0.0f;
    }
    const float iz = z > 0.0f ? 1.0f / z : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= iz;
    const int64_t entry = ((int64_t)qrow * a.Hq + hb + g) * a.smax + split;
    *reinterpret_cast<f32x4_t*>(a.part_o + entry * D + d) = acc;
    if (d == 0) { a.part_ml[2 * entry] = M; a.part_ml[2 * entry + 1] = z; }
  }
  DTRACE(8);
}

// Combines the S split partials of one (query, q head): weights
// w_s = z_s 2^(m_s - M), O = sum w_s o_s / sum w_s, LSE = M + log2(sum w_s)
// (natural log on output).  Wave w takes splits w, w + 4, ...: every partial
// load is issued before any arithmetic.
// Each wave sums its splits in order, then the 4 wave sums are added in wave
// order (deterministic for a fixed S).  The row's position is read from
// `positions` (given in mode 0, published by the attention launch
// otherwise); in step mode head 0 advances the row's length: every attention
// workgroup has read it by now.
constexpr int kMergeWaves = 4;
constexpr int kMergePer = 64 / kMergeWaves;  // splits per wave (S <= 64)

template <int DT>
__global__ __launch_bounds__(64 * kMergeWaves) void merge_kernel(FusedArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rh = blockIdx.x, qrow = rh / a.Hq, h = rh % a.Hq;
  const int S = a.sched != nullptr ? a.sched[3 * a.n_sched + qrow * a.Hkv * a.Vg + h / a.G] : a.smax;
  // the row's position decides only whether anything is written: its loads
  // (ids -> lengths) run beside the partial loads below, which stay inside
  // the row's own slots either way
  // the row's position: given (mode 0) or published by the attention launch
  // (one load; the slot id is needed only for the length store at the end)
  const int p = a.positions[qrow];
  const int64_t e0 = (int64_t)rh * a.smax;
  const int d = lane * 4;
  const bool dok = d < a.D;
  float m[kMergePer], z[kMergePer];
  f32x4_t o[kMergePer];
  // All loads are issued unconditionally, back to back, at slots clamped to
  // the row's S (the repeats hit the cache, so only S slots' bytes move);
  // slots past S are dropped by a select afterwards.  Guarded loads compiled
  // to one branch and one full wait per slot.
  const int dl = dok ? d : 0;
#pragma unroll
  for (int i = 0; i < kMergePer; ++i) {
    const int s = min(w + kMergeWaves * i, S - 1);
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + 2 * (e0 + s));
    m[i] = ml.x;
    z[i] = ml.y;
    o[i] = *reinterpret_cast<const f32x4_t*>(a.part_o + (e0 + s) * a.D + dl);
  }
#pragma unroll
  for (int i = 0; i < kMergePer; ++i) {
    const bool ok = w + kMergeWaves * i < S;
    m[i] = ok ? m[i] : -INFINITY;
    z[i] = ok ? z[i] : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[i][e] = (ok && dok) ? o[i][e] : 0.0f;
  }
  if (p < 0 || p / a.C > a.width) return;  // the attention launch skipped this row
  __shared__ float wm[kMergeWaves], wz[kMergeWaves];
  __shared__ f32x4_t wo[kMergeWaves][64];
  float mw = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMergePer; ++i) mw = fmaxf(mw, z[i] > 0.0f ? m[i] : -INFINITY);
  if (lane == 0) wm[w] = mw;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMergeWaves; ++i) M = fmaxf(M, wm[i]);
  float Zw = 0.0f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kMergePer; ++i) {
    const float wt = z[i] > 0.0f ? z[i] * fast_exp2(m[i] - M) : 0.0f;
    Zw += wt;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += wt * o[i][e];
  }
  wo[w][lane] = acc;
  if (lane == 0) wz[w] = Zw;
  __syncthreads();
  if (w != 0) return;
  float Z = 0.0f;
  f32x4_t tot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kMergeWaves; ++i) {
    Z += wz[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) tot[e] += wo[i][lane][e];
  }
  if (dok) {
    const float iz = Z > 0.0f ? 1.0f / Z : 0.0f;
    u16x4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = from_f32<DT>(tot[e] * iz);
    *reinterpret_cast<u16x4_t*>(a.out + (int64_t)rh * a.D + d) = r;
  }
  if (lane == 0) {
    a.lse[rh] = (M + log2f(Z)) * kLn2;
    if (a.pos_mode == 2 && h == 0) a.lengths[a.ids != nullptr ? a.ids[qrow] : qrow] = p + 1;
  }
}

// Whether the launch's workgroups carry enough 32-token blocks for the
// 12-wave form: at most min(width, R + 1) chunks of C / 32 blocks per
// (row, kv head) (every chunk when dense), over that row's workgroups.
bool wide_launch(const FusedArgs& a, int splits, int DP, size_t dyn) {
  if (dyn + fused_static_lds(DP, kFwWide) > kLdsBytes) return false;
  const int64_t chunks = a.dense ? a.width : std::min(a.width, a.R + 1);
  const int64_t blocks = chunks * ((a.C + 31) / 32);
  const int64_t per_row = a.sched != nullptr ? std::max(1, a.n_sched / (a.Nq * a.Hkv * a.Vg)) : splits;
  return blocks >= (int64_t)kWideBlocksPerWorkgroup * per_row;
}

template <int DT, int DP, bool WROUTE>
int launch_fused(const FusedArgs& a, int splits, size_t dyn, hipStream_t st) {
  const dim3 grid = a.sched != nullptr ? dim3((unsigned)a.n_sched)
                                        : dim3((unsigned)splits, (unsigned)(a.Nq * a.Hkv * a.Vg));
  bool wide = false;
  if constexpr (DP <= 128) {
    wide = wide_launch(a, splits, DP, dyn);
    if (wide) hipLaunchKernelGGL((fused_kernel<DT, DP, kFwWide, WROUTE>), grid, dim3(64 * kFwWide), dyn, st, a);
  }
  if (!wide) hipLaunchKernelGGL((fused_kernel<DT, DP, kFwNarrow, WROUTE>), grid, dim3(64 * kFwNarrow), dyn, st, a);
  hipLaunchKernelGGL((merge_kernel<DT>), dim3((unsigned)(a.Nq * a.Hq)), dim3(64 * kMergeWaves), 0, st, a);
  return moba_launch_status("decode_fused");
}

template <int DT, int DP>
int launch_fused(const FusedArgs& a, int splits, size_t dyn, hipStream_t st) {
  // closed chunks of a row are at most `width`
  return a.width > 64 && !a.dense ? launch_fused<DT, DP, true>(a, splits, dyn, st)
                                  : launch_fused<DT, DP, false>(a, splits, dyn, st);
}

template <int DT>
int dispatch_fused(const FusedArgs& a, int splits, size_t dyn, hipStream_t st) {
  if (a.D <= 32) return launch_fused<DT, 32>(a, splits, dyn, st);
  if (a.D <= 64) return launch_fused<DT, 64>(a, splits, dyn, st);
  // 96 wide: 3 k-steps / 6 d blocks instead of a masked quarter of 128
  if (a.D <= 96) return launch_fused<DT, 96>(a, splits, dyn, st);
  if (a.D <= 128) return launch_fused<DT, 128>(a, splits, dyn, st);
  return launch_fused<DT, 256>(a, splits, dyn, st);
}

}  // namespace

namespace {
// Uniform split count of an unscheduled launch: about two workgroups per CU
// over the grid (the host wrapper's default, fused_splits in ops/decode.py).
// Workgroups of a decode launch: one per CU.
constexpr int kGridWorkgroups = 256;

int uniform_splits(int Nq, int Hkv) {
  const int64_t rows = (int64_t)Nq * Hkv;
  if (rows < 1) return 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>(64, (kGridWorkgroups + rows - 1) / rows));
}
}  // namespace

extern "C" int moba_hip_decode_fused_groups(int Hq, int Hkv) {
  if (Hkv < 1 || Hq < 1 || Hq % Hkv) return 0;
  const int G = Hq / Hkv;
  for (int vg = (G + kGroupMax - 1) / kGroupMax; vg <= G; ++vg)
    if (G % vg == 0) return vg;  // the fewest groups of equal size <= 16
  return 0;
}

extern "C" int moba_hip_decode_fused_supported(int Hq, int Hkv, int D, int width, int table_width) {
  const int vg = moba_hip_decode_fused_groups(Hq, Hkv);
  if (vg < 1 || D % 8 || D < 8 || D > 256 || table_width < 1 || width < 0) return 0;
  const int DP = D <= 32 ? 32 : D <= 64 ? 64 : D <= 96 ? 96 : D <= 128 ? 128 : 256;
  const size_t dyn = fused_route_lds(Hq / Hkv / vg, width, table_width);
  return dyn <= kDynMax && dyn + fused_static_lds(DP, kFwNarrow) <= kLdsBytes ? 1 : 0;
}

extern "C" int moba_hip_decode_fused(const void* q, const void* k, const void* v, int dtype, int Nq,
                                     int Hq, int Hkv, int D, void* k_cache, void* v_cache,
                                     int page_size, int* table, int table_width, int* lengths,
                                     const int* ids, int* positions, const int* delta, void* means,
                                     int max_chunks, int chunk, int width, int R, int dense,
                                     int pos_mode, int splits, const int* sched, int n_sched,
                                     int* selected, float* part_o,
                                     float* part_ml, void* out, float* lse,
                                     void* stream) {
  if (dtype != 0 && dtype != 1) { moba_set_error("decode_fused: dtype must be 0 (bf16) or 1 (fp16)"); return MOBA_ERR_ARG; }
  if (!moba_hip_decode_fused_supported(Hq, Hkv, D, width, table_width)) {
    moba_set_error("decode_fused: needs Hq a multiple of Hkv, head_dim a multiple of 8 in [8,256], "
                   "and a route width and page-table width that fit LDS");
    return MOBA_ERR_CAPACITY;
  }
  if (R < 0 || R + 1 > kMaxSlots) { moba_set_error("decode_fused: routed chunk count must be in [0,8]"); return MOBA_ERR_ARG; }
  if (pos_mode < 0 || pos_mode > 2) { moba_set_error("decode_fused: pos_mode must be 0 (given), 1 (attend) or 2 (step)"); return MOBA_ERR_ARG; }
  if (splits < 1 || splits > 64) { moba_set_error("decode_fused: splits must be in [1,64]"); return MOBA_ERR_ARG; }
  const int vg = moba_hip_decode_fused_groups(Hq, Hkv);
  if (sched != nullptr && n_sched < Nq * Hkv * vg) { moba_set_error("decode_fused: a schedule needs at least one workgroup per (row, kv head)"); return MOBA_ERR_ARG; }
  if (page_size < 1 || chunk < 1 || width < 0 || Nq < 1) { moba_set_error("decode_fused: bad sizes"); return MOBA_ERR_ARG; }
  if (pos_mode == 2 && (k == nullptr || v == nullptr)) { moba_set_error("decode_fused: step mode needs the new K/V rows"); return MOBA_ERR_ARG; }
  FusedArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.kc = (uint16_t*)k_cache; a.vc = (uint16_t*)v_cache;
  a.Nq = Nq; a.Hq = Hq; a.Hkv = Hkv; a.Vg = vg; a.D = D; a.G = Hq / Hkv / vg; a.P = page_size;
  a.W = table_width;
  a.C = chunk; a.width = width; a.R = dense ? 0 : R; a.max_chunks = max_chunks; a.dense = dense;
  a.pos_mode = pos_mode;
  a.scale_log2 = kLog2e / sqrtf((float)D);
  a.table = table; a.lengths = lengths; a.ids = ids; a.positions = positions; a.delta = delta;
  a.means = (uint16_t*)means; a.selected = selected; a.part_o = part_o; a.part_ml = part_ml;
  a.out = (uint16_t*)out; a.lse = lse;
  a.sched = sched; a.n_sched = n_sched; a.smax = splits;
  const size_t dyn = fused_route_lds(a.G, width, table_width);
  hipStream_t st = (hipStream_t)stream;
  return dtype == 0 ? dispatch_fused<0>(a, splits, dyn, st) : dispatch_fused<1>(a, splits, dyn, st);
}

// ---------------------------------------------------------------- no-alloc
// Split partials of moba_hip_decode_attend_noalloc live in this file-scope
// device array instead of caller workspaces.  Host code never passes the
// array's name to a kernel: each device's copy is located once with
// hipGetSymbolAddress (with that device current) and that address is used.
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of the current device's scratch array (resolved once per device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { moba_set_error("decode_attend_noalloc: hipGetDevice: %s", hipGetErrorString(e)); return MOBA_ERR_LAUNCH; }
  if (dev < 0 || dev >= kMaxDevices) { moba_set_error("decode_attend_noalloc: device %d out of range", dev); return MOBA_ERR_ARG; }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      moba_set_error("decode_attend_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return MOBA_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOBA_OK;
}
}  // namespace

extern "C" int moba_hip_decode_attend_noalloc(const void* q, int dtype, int Nq, int Hq, int Hkv,
                                              int D, const void* k_cache, const void* v_cache,
                                              int page_size, const int* table, int table_width,
                                              const int* lengths, const int* ids,
                                              const int* positions, const void* means,
                                              int max_chunks, int chunk, int width, int R,
                                              int dense, int* selected, void* out, float* lse,
                                              void* stream) {
  if (Nq < 1 || Hkv < 1 || Hq < 1 || D < 1) { moba_set_error("decode_attend_noalloc: bad sizes"); return MOBA_ERR_ARG; }
  const int splits = uniform_splits(Nq, Hkv * std::max(1, moba_hip_decode_fused_groups(Hq, Hkv)));
  const int64_t rows = (int64_t)Nq * Hq * splits;
  const int64_t part_o_bytes = (rows * D * 4 + 255) / 256 * 256;
  const int64_t need = part_o_bytes + rows * 2 * 4;
  if (need > (int64_t)kNoAllocScratchBytes) {
    moba_set_error("decode_attend_noalloc: %lld bytes of split partials (Nq*Hq*splits*(D+2)*4, "
                   "splits %d) exceed the %lld-byte static scratch; use moba_hip_decode_fused "
                   "with caller workspaces", (long long)need, splits,
                   (long long)kNoAllocScratchBytes);
    return MOBA_ERR_CAPACITY;
  }
  void* base = nullptr;
  if (int rc = scratch_address(&base)) return rc;
  float* part_o = (float*)base;
  float* part_ml = (float*)((char*)base + part_o_bytes);
  return moba_hip_decode_fused(q, nullptr, nullptr, dtype, Nq, Hq, Hkv, D, (void*)k_cache,
                               (void*)v_cache, page_size, (int*)table, table_width, (int*)lengths,
                               ids, (int*)positions, nullptr, (void*)means, max_chunks, chunk,
                               width, R, dense, 0, splits, nullptr, 0, selected, part_o, part_ml,
                               out, lse, stream);
}
