// MoBA prefill backward on gfx950 (deterministic, no atomics).
//
// Replaces OptMixedAttention.backward (src/moba_opt/mixed_attention.py:141-225):
// the self-branch and remote-branch flash-attention backwards, both evaluated
// with the GLOBAL output O and GLOBAL LSE of the merged forward
// (docs/semantics.md section 7), plus the autograd scatter of the packed
// remote dq/dkv back into q/k/v (grouped_attention.py:81-89), which is where
// GQA gradients of the heads sharing a KV head are summed.
//
//   delta_kernel : Delta = rowsum(dO * O)                                  [T*Hq]
//   dq_kernel<REMOTE> : query-major.  S^T = K Q^T, dP^T = V dO^T,
//        P = exp(S*scale - LSE), dS = P (dP - Delta), dQ^T += K^T dS^T.
//        REMOTE tiles (expert rows) write dq partials into the row's slot;
//        SELF tiles (causal within the chunk) add the slots in ascending order.
//   dkdv_kernel : key-major.  One workgroup owns a tile of one chunk's keys for
//        one KV head and walks every query row that attends them: the causal
//        rows of the chunk for all G heads of the group, then the expert rows
//        that selected the chunk.  dK, dV accumulate in registers and are
//        written once.
#include <type_traits>

#include "common.h"
#include "bwd_args.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {


constexpr int kBN = 64;   // dq: keys per LDS tile

// ------------------------------------------------------------------ delta
template <int DT>
__global__ __launch_bounds__(256) void delta_kernel(const uint16_t* __restrict__ o,
                                                    const uint16_t* __restrict__ g,
                                                    const float* __restrict__ lse, int64_t rows,
                                                    int D, float* __restrict__ delta,
                                                    float scale, float* __restrict__ lse_k) {
  const int sub = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  float acc = 0.0f;
  if (row < rows) {
    for (int d = sub * 8; d < D; d += 128) {
      const u16x8_t x = ld8(o + row * D + d), y = ld8(g + row * D + d);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += to_f32<DT>(x[e]) * to_f32<DT>(y[e]);
    }
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (row < rows && sub == 0) {
    delta[row] = acc;
    lse_k[row] = lse[row] / scale;
  }
}

// --------------------------------------------------------------------- dq
// Per wave two blocks of 32 query rows; K/V tiles of 64 keys double-buffered
// in LDS (row-major).  S^T = K Q^T and dP^T = V dO^T take K / V rows as the A
// operand; dQ^T = K^T dS^T reads K^T with the transposed LDS read.
template <int DT, int DP, bool REMOTE, int QB>
__global__ __launch_bounds__(256, attn_occupancy<DP>()) void dq_kernel(BwdArgs a) {
  constexpr int NKS = DP / 16, NDB = DP / 32;
  constexpr int TILE = kBN * DP, NB = DP / 8, NDMA = kBN * NB / 256;
  // Two stages of K and V tiles (swz<DP> layout) filled by buffer loads
  // straight into LDS, as in the forward kernel.
  __shared__ __attribute__((aligned(16))) uint16_t K0[TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V0[TILE];
  __shared__ __attribute__((aligned(16))) uint16_t K1[TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V1[TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int D = a.D;

  int s[QB], h[QB], slot[QB];
  int pidx[QB];  // packed index of an expert row (row_off order)
  bool valid[QB];
  int kh, k_lo, k_hi, s_wave0 = 0;
  if constexpr (REMOTE) {
    const int t = xcd_contiguous(blockIdx.x, a.tile_off[a.E]);
    if (t < 0) return;
    int lo = 0, hi = a.E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.tile_off[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    kh = e % a.Hkv;
    const int c = a.filtered[e / a.Hkv];
    k_lo = a.cu_chunk[c];
    k_hi = a.cu_chunk[c + 1];
    const int cnt = a.counts[e], base = a.row_off[e];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int local = (t - a.tile_off[e]) * (128 * QB) + wave * (32 * QB) + qb * 32 + qi;
      valid[qb] = local < cnt;
      pidx[qb] = base + local;
      const int packed = valid[qb] ? a.rows[base + local] : 0;  // (row << 3) | j
      const int sh = packed >> 3;
      slot[qb] = sh * a.R + (packed & 7);
      s[qb] = sh / a.Hq;
      h[qb] = sh % a.Hq;
    }
  } else {
    // 1-D grid over (tile, q head within the kv group), tiles in the
    // host's order of 8 XCD runs: workgroup L runs on XCD L % 8 and takes
    // entry xcd_contiguous(L) / G, so each run's tiles share that XCD's L2.
    // Entries are (chunk, first row, kv head); chunk -1 pads a run.
    const int t = xcd_contiguous(blockIdx.x, a.n_self_wg);
    if (t < 0) return;
    const int e = t / a.G, g = t - e * a.G;
    const int c = a.self_tiles[3 * e];
    if (c < 0) return;
    const int row0 = a.self_tiles[3 * e + 1];
    kh = a.self_tiles[3 * e + 2];
    k_lo = a.cu_chunk[c];
    const int c_end = a.cu_chunk[c + 1];
    k_hi = min(c_end, k_lo + row0 + 128 * QB);
    s_wave0 = k_lo + row0 + wave * (32 * QB);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      h[qb] = kh * a.G + g;
      s[qb] = s_wave0 + qb * 32 + qi;
      valid[qb] = s[qb] < c_end;
      if (!valid[qb]) s[qb] = k_hi - 1;
    }
  }
  u16x8_t qf[QB][NKS], gf[QB][NKS];
  float lse2[QB], lk[QB], dl[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t row = (int64_t)s[qb] * a.Hq + h[qb];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 16 + hh * 8;
      const bool ok = valid[qb] && d < D;
      qf[qb][ks] = ok ? ld8(a.q + row * D + d) : zero8();
      gf[qb][ks] = ok ? ld8(a.dout + row * D + d) : zero8();
    }
    const float lr = valid[qb] ? a.lse[row] : INFINITY;
    lse2[qb] = lr * kLog2e;
    lk[qb] = lr / a.scale;
    dl[qb] = valid[qb] ? a.delta[row] : 0.0f;
  }
  if constexpr (REMOTE && DP <= 128) {
    // The key-major dK/dV kernel reads the expert rows packed contiguously in
    // row_off order; this kernel holds exactly those rows, so it writes the
    // packed q / dO / lse_k / delta (the values delta_kernel and the loads above
    // produce) instead of a separate gather pass.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (!valid[qb]) continue;
      const int64_t m = pidx[qb];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d = ks * 16 + hh * 8;
        if (d < D) {
          st8(a.pack_q + m * D + d, qf[qb][ks]);
          st8(a.pack_g + m * D + d, gf[qb][ks]);
        }
      }
      if (hh == 0) {
        a.pack_lse_k[m] = lk[qb];
        a.pack_delta[m] = dl[qb];
      }
    }
  }

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  // Lane l of wave w loads blocks j = (n * 4 + w) * 64 + l: row j / NB,
  // physical block j % NB.  The row advances by 256 / NB per n, a multiple of
  // 16 when DP <= 128, and the swizzle depends on the row mod 16 only, so
  // every n has the same column and its offset is the n = 0 offset plus a
  // uniform step (added per load, not held in NDMA registers).
  constexpr bool UNI = (256 / NB) % 16 == 0;
  uint32_t voff[UNI ? 1 : NDMA];
  bool vok[UNI ? 1 : NDMA];
#pragma unroll
  for (int n = 0; n < (UNI ? 1 : NDMA); ++n) {
    const int j = (n * 4 + wave_s) * 64 + lane, row = j / NB;
    const int col = swz<DP>(row, (j % NB) * 8) - row * DP;  // swizzle is an involution
    voff[n] = (uint32_t)(((row * a.Hkv + kh) * D + col) * 2);
    vok[n] = col < D;
  }
  const uint32_t vstep = (uint32_t)((256 / NB) * a.Hkv * D * 2);
  const int n_keys = k_hi - k_lo;
  const uint32_t nrec = (uint32_t)((((int64_t)(n_keys - 1) * a.Hkv + kh + 1) * D) * 2);
  const uint16_t* kbase = a.k + (int64_t)k_lo * a.Hkv * D;
  const uint16_t* vbase = a.v + (int64_t)k_lo * a.Hkv * D;
  const uint32_t tile_bytes = (uint32_t)(kBN * a.Hkv * D * 2);
  auto dma = [&](uint16_t* Kd, uint16_t* Vd, int it) {
    const uint32_t soff = (uint32_t)it * tile_bytes;
    const uint32_t v0 = opaque(voff[0]);
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      if (vok[UNI ? 0 : n]) {
        const uint32_t vo = UNI ? v0 + n * vstep : voff[n];
        load_lds16(make_rsrc(kbase, nrec), Kd + (n * 4 + wave_s) * 64 * 8, vo, soff);
        load_lds16(make_rsrc(vbase, nrec), Vd + (n * 4 + wave_s) * 64 * 8, vo, soff);
      }
    }
  };
  if (D < DP) {  // column blocks past D stay zero
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int j = (n * 4 + wave) * 64 + lane;
      st8(K0 + j * 8, zero8()); st8(V0 + j * 8, zero8());
      st8(K1 + j * 8, zero8()); st8(V1 + j * 8, zero8());
    }
    __syncthreads();
  }
  const uint32_t kbase0 = swz_b128_base<DP>(lane);
  const uint32_t trb0 = swz_tr_base<DP>(lane, 0), trb1 = swz_tr_base<DP>(lane, 1);

  f32x16_t acc[QB][NDB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[qb][db] = zero16();
  const float c2 = a.scale_log2;

  const int ntiles = (n_keys + kBN - 1) / kBN;
  auto tile = [&](const uint16_t* Kb, const uint16_t* Vb, const int it, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int kt0 = k_lo + it * kBN;
    const uint32_t kq = opaque(kbase0), t0 = opaque(trb0), t1 = opaque(trb1);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16_t sa[QB], pa[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) { sa[qb] = zero16(); pa[qb] = zero16(); }
      wave_prio<1>();
      if constexpr (REMOTE && DP > 64) {
        // the expert variant holds more per-row state: above D = 64 no room
        // for a ring (it spills); at D <= 64 it takes the ring path below
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const uint32_t o = kb * 32 * DP * 2 + swz_b128<DP>(kq, ks);
          const u16x8_t ka = lds8(Kb, o), va = lds8(Vb, o);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            sa[qb] = mfma32<DT>(ka, qf[qb][ks], sa[qb]);
            pa[qb] = mfma32<DT>(va, gf[qb][ks], pa[qb]);
          }
        }
      } else {
        // K / V operand reads run PF k-steps ahead of the MFMAs, in this
        // order (the scheduling fences keep the compiler from sinking them)
        constexpr int PF = 3;
        u16x8_t rk[PF], rv[PF];
#pragma unroll
        for (int i = 0; i < PF && i < NKS; ++i) {
          const uint32_t o = kb * 32 * DP * 2 + swz_b128<DP>(kq, i);
          rk[i] = lds8(Kb, o);
          rv[i] = lds8(Vb, o);
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const u16x8_t ka = rk[ks % PF], va = rv[ks % PF];
          if (ks + PF < NKS) {
            const uint32_t o = kb * 32 * DP * 2 + swz_b128<DP>(kq, ks + PF);
            rk[ks % PF] = lds8(Kb, o);
            rv[ks % PF] = lds8(Vb, o);
          }
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            sa[qb] = mfma32<DT>(ka, qf[qb][ks], sa[qb]);
            pa[qb] = mfma32<DT>(va, gf[qb][ks], pa[qb]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      wave_prio<0>();
      u16x8_t dsv[QB][2];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float tmp[16];
        const float nl = -lse2[qb];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(fmaf(sa[qb][r], c2, nl));
          if constexpr (MASK) {
            const int key = kt0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
            p = (key < k_hi && (REMOTE || key <= s[qb])) ? p : 0.0f;
          }
          tmp[r] = p * (pa[qb][r] - dl[qb]);
        }
        dsv[qb][0] = pack8<DT>(tmp);
        dsv[qb][1] = pack8<DT>(tmp + 8);
      }
      wave_prio<1>();
      if constexpr (REMOTE && DP > 64) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const uint32_t ro = (kb * 32 + t * 16) * DP * 2;
            const u16x8_t kt = lds_tr8(Kb, ro + swz_tr<DP>(t0, db), ro + swz_tr<DP>(t1, db));
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) acc[qb][db] = mfma32<DT>(kt, dsv[qb][t], acc[qb][db]);
          }
        // issue order for this 32-key block: LDS operand reads run at most
        // two MFMAs ahead, which bounds the registers they hold
        if constexpr (QB == 1) {
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
          for (int i = 0; i < NKS - 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 200, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
          for (int i = 0; i < 2 * NDB - 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
      } else {
        // K^T operand reads pipelined the same way; step i is d block i / 2
        // of 16-key half i % 2
        constexpr int N2 = 2 * NDB, PF = 4;
        u16x8_t ring[PF];
        auto rd = [&](int i) __attribute__((always_inline)) {
          const uint32_t ro = (kb * 32 + (i % 2) * 16) * DP * 2;
          return lds_tr8(Kb, ro + swz_tr<DP>(t0, i / 2), ro + swz_tr<DP>(t1, i / 2));
        };
#pragma unroll
        for (int i = 0; i < PF && i < N2; ++i) ring[i] = rd(i);
#pragma unroll
        for (int i = 0; i < N2; ++i) {
          const u16x8_t kt = ring[i % PF];
          if (i + PF < N2) ring[i % PF] = rd(i + PF);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) acc[qb][i / 2] = mfma32<DT>(kt, dsv[qb][i % 2], acc[qb][i / 2]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto stage_sync = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's tile loads landed
    __builtin_amdgcn_s_barrier();
  };
  auto run = [&](const uint16_t* Kb, const uint16_t* Vb, int it) {
    const int kt0 = k_lo + it * kBN;
    // a causal tile wholly above this wave's rows adds exact zeros: skip it
    // (the wave still joins the stage barriers)
    if (!REMOTE && kt0 > s_wave0 + 32 * QB - 1) return;
    const bool need_mask = (kt0 + kBN > k_hi) || (!REMOTE && kt0 + kBN - 1 > s_wave0);
    if (need_mask) tile(Kb, Vb, it, std::true_type{}); else tile(Kb, Vb, it, std::false_type{});
  };
  dma(K0, V0, 0);
  stage_sync();
  for (int it = 0; it < ntiles; it += 2) {
    if (it + 1 < ntiles) dma(K1, V1, it + 1);
    run(K0, V0, it);
    stage_sync();
    if (it + 1 >= ntiles) break;
    if (it + 2 < ntiles) dma(K0, V0, it + 2);
    run(K1, V1, it + 1);
    stage_sync();
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if (!valid[qb]) continue;
    const int64_t row = (int64_t)s[qb] * a.Hq + h[qb];
    if constexpr (REMOTE) {
      uint16_t* po = a.part_dq + (int64_t)slot[qb] * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d0 = db * 32 + 8 * j + 4 * hh;
          if (d0 < D) {
            f32x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = acc[qb][db][4 * j + i] * a.scale;
            u16x4_t ob;
#pragma unroll
            for (int i = 0; i < 4; ++i) ob[i] = from_f32<DT>(o[i]);
            *reinterpret_cast<u16x4_t*>(po + d0) = ob;
          }
        }
    } else {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[qb][db][r] *= a.scale;
      // one slot per iteration, all of its loads issued together: slots
      // below R are in the row's allocation, columns past D are clamped and
      // masked, unselected slots (sel < 0) add zero
      for (int jj = 0; jj < a.R; ++jj) {
        const int64_t sl = row * a.R + jj;
        const bool on = a.sel[sl] >= 0;
        const uint16_t* po = a.part_dq + sl * D;
        u16x4_t o[NDB][4];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int d0 = db * 32 + 8 * j + 4 * hh;
            o[db][j] = *reinterpret_cast<const u16x4_t*>(po + (d0 < D ? d0 : 0));
          }
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool ok = on && db * 32 + 8 * j + 4 * hh < D;
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[qb][db][4 * j + i] += ok ? to_f32<DT>(o[db][j][i]) : 0.0f;
          }
      }
      uint16_t* orow = a.dq + row * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d0 = db * 32 + 8 * j + 4 * hh;
          if (d0 < D) {
            u16x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = from_f32<DT>(acc[qb][db][4 * j + i]);
            *reinterpret_cast<u16x4_t*>(orow + d0) = o;
          }
        }
    }
  }
}

// ------------------------------------------------------------------- dkdv
// Key-major dK/dV.  A workgroup of 8 waves owns 128 keys of one chunk and one
// KV head, as 4 pairs of waves; each pair owns 32 keys.  Within a pair the
// work is split by role so that each wave holds only half the operands:
//   role P (waves 0-3): K in registers; S = Q K^T, P = exp2(S*c - lse), P to
//                       LDS (fp32), then dV += P^T dO
//   role D (waves 4-7): V in registers; dP = dO V^T, reads P, dS = P (dP - delta),
//                       then dK += dS^T Q
// Query tiles of 32*QB rows (Q and dO, row-major) are double-buffered in LDS,
// the next tile prefetched through registers and its row indices one tile
// further ahead (a gathered expert row costs two dependent global loads: its
// index, then its data).  The MFMA D-layout of S / dP (one key per lane) is
// exactly the A layout of P^T / dS^T; dO and Q enter as B through the
// transposed LDS read.  Waves w and w+4 share a SIMD, so one wave's
// exponentials overlap its partner's MFMAs.
constexpr int kDkdvPairKeys = 32;

template <int DP> constexpr int dkdv_qb() { return DP <= 128 ? 2 : 1; }

template <int DT, int DP>
__global__ __launch_bounds__(512, 1) void dkdv_kernel(BwdArgs a) {
  constexpr int QB = dkdv_qb<DP>();
  constexpr int NKS = DP / 16, NDB = DP / 32;
  constexpr int BQ = 32 * QB;                 // query rows per tile
  constexpr int NB = DP / 8;                  // 16-byte blocks per row
  constexpr int NDMA = (BQ * NB + 511) / 512; // blocks per thread per operand
  constexpr int WKEYS = kDkdvPairKeys;        // keys per wave pair
  // Q / dO tiles in two named stages (swz<DP> layout), filled by buffer loads
  // straight into LDS while the other stage is being used.
  __shared__ __attribute__((aligned(16))) uint16_t Q0[BQ * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G0[BQ * DP];
  __shared__ __attribute__((aligned(16))) uint16_t Q1[BQ * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G1[BQ * DP];
  __shared__ __attribute__((aligned(16))) float lse2s[2][BQ];
  __shared__ __attribute__((aligned(16))) float dels[2][BQ];
  // P handed from role P to role D as a pair of input-dtype values: Px holds
  // P rounded to the input dtype (the operand dV uses), Pr the rounding
  // residual, so dS = (Px + Pr)(dP - delta) sees P to about 16 mantissa bits
  // (dS from the rounded P alone doubled the dK error at D = 256).
  // [pair][qb][half][lane], 8 values per lane
  __shared__ __attribute__((aligned(16))) u16x8_t Px[4][QB][2][64];
  __shared__ __attribute__((aligned(16))) u16x8_t Pr[4][QB][2][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int pair = wave & 3;
  const bool role_p = wave < 4;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int D = a.D, G = a.G;
  int ti, s_lo, s_hi, slot;
  if (!kv_work(a, ti, s_lo, s_hi, slot)) return;
  const int* tile = a.kv_tiles + 4 * ti;
  const int c = tile[0], kt0 = tile[1], f = tile[2], kh = tile[3];
  if (c < 0) return;                        // padding entry of the XCD-ordered list
  const int c_lo = a.cu_chunk[c], c_hi = a.cu_chunk[c + 1];
  const int key0 = c_lo + kt0;              // first key of the workgroup
  const int wkey0 = key0 + pair * WKEYS;    // first key of this pair
  const int mykey = wkey0 + qi;             // this lane's key (B operand column)

  // Uninitialised LDS could hold NaN patterns that a zero probability would
  // not cancel; column blocks past D are never loaded and must read zero.
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int j = n * 512 + tid;
    if (j < BQ * NB) {
      st8(Q0 + j * 8, zero8()); st8(G0 + j * 8, zero8());
      st8(Q1 + j * 8, zero8()); st8(G1 + j * 8, zero8());
    }
  }
  __syncthreads();

  // The two roles run as separate instantiations of the body, so each wave's
  // code holds only its own role's registers.
  auto body = [&](auto role_tag) {
    constexpr bool ROLE_P = decltype(role_tag)::value;
    // role P holds K, role D holds V (B operands: column = key, k = d)
    u16x8_t kv[NKS];
    const uint16_t* kvsrc = ROLE_P ? a.k : a.v;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 16 + hh * 8;
      const bool ok = mykey < c_hi && d < D;
      kv[ks] = ok ? ld8(kvsrc + ((int64_t)mykey * a.Hkv + kh) * D + d) : zero8();
    }
    f32x16_t acc[NDB];                        // dV (role P) or dK (role D)
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc[i] = zero16();

    // query tiles: G * n_self causal tiles (rows from key0 to the chunk end, for
    // every head of the group), then the expert's gathered rows
    const int self_begin = key0;
    const int n_self = (max(0, c_hi - self_begin) + BQ - 1) / BQ;
    const int e = (f >= 0 && a.R > 0) ? f * a.Hkv + kh : -1;
    const int n_rem = e >= 0 ? a.counts[e] : 0;
    const int rbase = e >= 0 ? a.row_off[e] : 0;
    const int n_tiles = G * n_self + (n_rem + BQ - 1) / BQ;
    const int it_lo = s_lo, it_hi = min(s_hi, n_tiles);  // this workgroup's share

    auto row_of = [&](int it, int qr) -> int {  // row index s*Hq+h, or -1
      if (it < G * n_self) {
        const int g = it / n_self, s = self_begin + (it % n_self) * BQ + qr;
        return s < c_hi ? s * a.Hq + kh * G + g : -1;
      }
      const int local = (it - G * n_self) * BQ + qr;
      return local < n_rem ? a.rows[rbase + local] >> 3 : -1;
    };

    // Thread t loads blocks j = n * 512 + t of a tile: row j / NB, physical
    // block j % NB, logical column block (j % NB) ^ f(row).
    int nrow[NDMA], nlrow = -1;
    auto fetch_rows = [&](int it) {
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        const int q = (n * 512 + tid) / NB;
        nrow[n] = q < BQ ? row_of(it, q) : -1;
      }
      nlrow = tid < BQ ? row_of(it, tid) : -1;
    };
    const uint32_t qbytes = (uint32_t)((int64_t)a.T * a.Hq * D * 2);
    auto dma = [&](uint16_t* Qd, uint16_t* Gd) {
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        const int j = n * 512 + tid, q = j / NB;
        const int col = swz<DP>(q, (j % NB) * 8) - q * DP;
        if (j < BQ * NB && col < D) {
          // rows of -1 read past the end of the tensor: zeros
          const uint32_t off = nrow[n] >= 0 ? (uint32_t)(((int64_t)nrow[n] * D + col) * 2) : qbytes;
          const int jb = n * 512 + wave_s * 64;  // first block of this wave's 64
          load_lds16(make_rsrc(a.q, qbytes), Qd + jb * 8, off, 0);
          load_lds16(make_rsrc(a.dout, qbytes), Gd + jb * 8, off, 0);
        }
      }
    };
    float lse_r = INFINITY, del_r = 0.0f;
    auto load_ld = [&]() {
      lse_r = nlrow >= 0 ? a.lse[nlrow] * kLog2e : INFINITY;
      del_r = nlrow >= 0 ? a.delta[nlrow] : 0.0f;
    };
    auto store_ld = [&](int buf) {
      if (tid < BQ) { lse2s[buf][tid] = lse_r; dels[buf][tid] = del_r; }
    };

    const uint32_t kq0 = swz_b128_base<DP>(lane);
    const uint32_t trb0 = swz_tr_base<DP>(lane, 0), trb1 = swz_tr_base<DP>(lane, 1);
    const float c2 = a.scale_log2;

    auto compute = [&](const uint16_t* Qb, const uint16_t* Gb, const int buf, const int it) {
      const uint32_t kq = opaque(kq0), t0 = opaque(trb0), t1 = opaque(trb1);
      const bool is_self = it < G * n_self;
      const int sq0 = is_self ? self_begin + (it % n_self) * BQ : 0;
      // causal rows that end before the pair's first key contribute nothing
      const bool skip = is_self && sq0 + BQ - 1 < wkey0;
      const bool need_mask = (wkey0 + WKEYS > c_hi) || (is_self && sq0 < wkey0 + WKEYS - 1);
      // ---- first half: S -> P (role P) or dP (role D)
      const uint16_t* A1 = ROLE_P ? Qb : Gb;
      f32x16_t sp[QB];
      u16x8_t pk[QB][2];  // role P: P as the A operand of dV += P^T dO
      u16x8_t pr[QB][2];  // role P: rounding residual of pk
      if (!skip) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sp[qb] = zero16();
        // operand reads run PF steps ahead of the MFMAs, in this order (the
        // scheduling fences keep the compiler from sinking them)
        {
          constexpr int N1 = NKS * QB, PF = 6;
          u16x8_t ring[PF];
          auto rd = [&](int i) __attribute__((always_inline)) {
            return lds8(A1, (i % QB) * 32 * DP * 2 + swz_b128<DP>(kq, i / QB));
          };
#pragma unroll
          for (int i = 0; i < PF && i < N1; ++i) ring[i] = rd(i);
#pragma unroll
          for (int i = 0; i < N1; ++i) {
            const u16x8_t x = ring[i % PF];
            if (i + PF < N1) ring[i % PF] = rd(i + PF);
            sp[i % QB] = mfma32<DT>(x, kv[i / QB], sp[i % QB]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        if constexpr (ROLE_P) {
          auto to_p = [&](auto mask_tag) {
            constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int r0 = qb * 32 + 8 * j + 4 * hh;
                const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(&lse2s[buf][r0]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  float p = fast_exp2(fmaf(sp[qb][4 * j + i], c2, -l4[i]));
                  if constexpr (MASK)
                    p = (mykey < c_hi && (!is_self || mykey <= sq0 + r0 + i)) ? p : 0.0f;
                  const uint16_t hi = from_f32<DT>(p);
                  pk[qb][j >> 1][(j & 1) * 4 + i] = hi;
                  pr[qb][j >> 1][(j & 1) * 4 + i] = from_f32<DT>(p - to_f32<DT>(hi));
                }
              }
          };
          if (need_mask) to_p(std::true_type{}); else to_p(std::false_type{});
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            Px[pair][qb][0][lane] = pk[qb][0];
            Px[pair][qb][1][lane] = pk[qb][1];
            Pr[pair][qb][0][lane] = pr[qb][0];
            Pr[pair][qb][1][lane] = pr[qb][1];
          }
        }
      }
      lds_barrier();
      // ---- second half: dV += P^T dO (role P) or dK += dS^T Q (role D)
      if (!skip) {
        u16x8_t op[QB][2];
        if constexpr (ROLE_P) {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) { op[qb][0] = pk[qb][0]; op[qb][1] = pk[qb][1]; }
        } else {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            const u16x8_t px[2] = {Px[pair][qb][0][lane], Px[pair][qb][1][lane]};
            const u16x8_t rx[2] = {Pr[pair][qb][0][lane], Pr[pair][qb][1][lane]};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const f32x4_t d4 =
                  *reinterpret_cast<const f32x4_t*>(&dels[buf][qb * 32 + 8 * j + 4 * hh]);
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int r = 4 * j + i, h2 = j >> 1, x = (j & 1) * 4 + i;
                const float pv = to_f32<DT>(px[h2][x]) + to_f32<DT>(rx[h2][x]);
                op[qb][h2][x] = from_f32<DT>(pv * (sp[qb][r] - d4[i]));
              }
            }
          }
        }
        const uint16_t* B2 = ROLE_P ? Gb : Qb;
        {
          constexpr int N2 = NDB * QB * 2, PF = 6;
          u16x8_t ring[PF];
          // step i: d block i / (2 QB), row block (i / 2) % QB, half i % 2
          auto rd = [&](int i) __attribute__((always_inline)) {
            const uint32_t ro = (((i / 2) % QB) * 32 + (i % 2) * 16) * DP * 2;
            const int db = i / (2 * QB);
            return lds_tr8(B2, ro + swz_tr<DP>(t0, db), ro + swz_tr<DP>(t1, db));
          };
#pragma unroll
          for (int i = 0; i < PF && i < N2; ++i) ring[i] = rd(i);
#pragma unroll
          for (int i = 0; i < N2; ++i) {
            const u16x8_t b = ring[i % PF];
            if (i + PF < N2) ring[i % PF] = rd(i + PF);
            acc[i / (2 * QB)] = mfma32<DT>(op[(i / 2) % QB][i % 2], b, acc[i / (2 * QB)]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    };

    if (it_lo < it_hi) {
      fetch_rows(it_lo);
      load_ld();
      dma(Q0, G0);
      store_ld(0);
      fetch_rows(it_lo + 1);
    }
    stage_barrier();
    for (int it = it_lo; it < it_hi; it += 2) {
      if (it + 1 < it_hi) {
        load_ld();
        dma(Q1, G1);
        fetch_rows(it + 2);
      }
      compute(Q0, G0, 0, it);
      if (it + 1 < it_hi) store_ld(1);
      stage_barrier();
      if (it + 1 >= it_hi) break;
      if (it + 2 < it_hi) {
        load_ld();
        dma(Q0, G0);
        fetch_rows(it + 3);
      }
      compute(Q1, G1, 1, it + 1);
      if (it + 2 < it_hi) store_ld(0);
      stage_barrier();
    }

    // D-layout: lane holds column d = i*32 + qi, keys 8j + 4hh + r.  A row
    // split writes fp32 partials to its slot for the fixed-order reduction.
    if (slot >= 0) {
      float* pdst = a.part_dkv + (int64_t)slot * kv_slot_floats(D) + (ROLE_P ? kKvTileKeys * D : 0);
#pragma unroll
      for (int i = 0; i < NDB; ++i) {
        const int d = i * 32 + qi;
        if (d >= D) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = wkey0 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key < c_hi) pdst[(key - key0) * D + d] = acc[i][r];
        }
      }
      return;
    }
    uint16_t* dst = ROLE_P ? a.dv : a.dk;
    const float osc = ROLE_P ? 1.0f : a.scale;
#pragma unroll
    for (int i = 0; i < NDB; ++i) {
      const int d = i * 32 + qi;
      if (d >= D) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = wkey0 + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (key < c_hi) dst[((int64_t)key * a.Hkv + kh) * D + d] = from_f32<DT>(acc[i][r] * osc);
      }
    }
  };
  if (role_p) body(std::true_type{}); else body(std::false_type{});
}

// Row-split schedule of the key-major kernels, built on the device because
// the expert row counts live there.  Tile t costs n_t row tiles (its causal
// tiles for the G heads plus its expert's packed tiles, the count every
// key-major kernel derives).  The kernel picks the smallest segment length L
// with sum ceil(n_t / L) <= nwg, cuts each tile into that many equal
// segments, and deals the segments, in the XCD-grouped order of the host's
// list (its entries L % 8 == x, i.e. whole (chunk, kv head) groups per XCD),
// to the XCDs in contiguous runs: workgroup g runs on XCD g % 8, so a run of
// segments that share query rows stays in one L2.  One workgroup; a fixed
// function of the counts, so the sums below keep a fixed order.
constexpr int kSchedMaxTiles = 4096;

__device__ int block_sum_1024(int v, int* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) t += red[i];
  return t;
}

template <int ROWS>
__global__ __launch_bounds__(1024) void dkdv_sched_kernel(BwdArgs a, int n_kv, int nwg, int* sched,
                                                          int* seg) {
  __shared__ int work[kSchedMaxTiles];
  __shared__ int first[kSchedMaxTiles + 1];
  __shared__ int red[16];
  const int tid = threadIdx.x;
  const bool grouped = n_kv % 8 == 0;
  const int ni = n_kv / 8;
  auto tile_of = [&](int o) { return grouped ? (o % ni) * 8 + o / ni : o; };
  int wmax = 0, wsum = 0, nvalid = 0;
  for (int o = tid; o < n_kv; o += 1024) {
    const int* t = a.kv_tiles + 4 * tile_of(o);
    int n = 0;
    if (t[0] >= 0) {
      const int c = t[0], kt0 = t[1], f = t[2], kh = t[3];
      const int c_hi = a.cu_chunk[c + 1], key0 = a.cu_chunk[c] + kt0;
      const int n_self = (max(0, c_hi - key0) + ROWS - 1) / ROWS;
      const int n_rem = (f >= 0 && a.R > 0) ? a.counts[f * a.Hkv + kh] : 0;
      n = max(1, a.G * n_self + (n_rem + ROWS - 1) / ROWS);  // >= 1: its keys get written
    }
    work[o] = n;
    wmax = max(wmax, n);
    wsum += n;
    nvalid += n > 0;
  }
  // sum ceil(n_t / L) lies in [W / L, W / L + valid tiles]: the answer lies in
  // [ceil(W / nwg), ceil(W / (nwg - valid))], and max n_t always fits
  const int W = block_sum_1024(wsum, red), nv = block_sum_1024(nvalid, red);
  // block max through the sum helper's scratch (values are >= 0)
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wmax = max(wmax, __shfl_xor(wmax, o, 64));
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = wmax;
  __syncthreads();
  int hi = 1;
#pragma unroll
  for (int i = 0; i < 16; ++i) hi = max(hi, red[i]);
  if (nwg > nv) hi = min(hi, max(1, (W + (nwg - nv) - 1) / (nwg - nv)));
  int lo = min(hi, max(1, (W + nwg - 1) / nwg));
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    int cnt = 0;
    for (int o = tid; o < n_kv; o += 1024) cnt += (work[o] + mid - 1) / mid;
    if (block_sum_1024(cnt, red) <= nwg) hi = mid; else lo = mid + 1;
  }
  const int L = lo;
  // exclusive scan of the segment counts: thread tid owns a contiguous run
  const int per = (n_kv + 1023) / 1024;
  const int o0 = min(n_kv, tid * per), o1 = min(n_kv, o0 + per);
  int mine = 0;
  for (int o = o0; o < o1; ++o) mine += (work[o] + L - 1) / L;
  int inc = mine;  // inclusive scan over the wave, then over the waves
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if ((tid & 63) >= o) inc += y;
  }
  __syncthreads();
  if ((tid & 63) == 63) red[tid >> 6] = inc;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < (tid >> 6); ++i) base += red[i];
  int run = base + inc - mine;
  for (int o = o0; o < o1; ++o) {
    first[o] = run;
    run += (work[o] + L - 1) / L;
  }
  int S = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) S += red[i];
  if (tid == 0) first[n_kv] = S;
  __syncthreads();
  for (int o = tid; o < n_kv; o += 1024) {
    seg[2 * tile_of(o)] = first[o];
    seg[2 * tile_of(o) + 1] = first[o + 1] - first[o];
  }
  for (int g = tid; g < nwg; g += 1024) {
    int j = g;
    bool ok = g < S;
    if (grouped) {  // XCD x = g % 8 takes segments [ceil(x S / 8), ceil((x+1) S / 8))
      const int x = g % 8, s0 = (x * S + 7) / 8, s1 = ((x + 1) * S + 7) / 8;
      j = s0 + g / 8;
      ok = j < s1;
    }
    int4 w = {-1, 0, 0, -1};
    if (ok) {
      int l = 0, h = n_kv - 1;  // last o with first[o] <= j
      while (l < h) {
        const int m = (l + h + 1) >> 1;
        if (first[m] <= j) l = m; else h = m - 1;
      }
      const int ns = first[l + 1] - first[l], sidx = j - first[l], n = work[l];
      w = {tile_of(l), (int)((int64_t)n * sidx / ns), (int)((int64_t)n * (sidx + 1) / ns),
           ns > 1 ? j : -1};
    }
    reinterpret_cast<int4*>(sched)[g] = w;
  }
}

// dK / dV of the split tiles: workgroups (kv tile, y) share a tile's 16-byte
// elements, each summed over the tile's slots in slot order (tiles with one
// slot were written by the key-major kernel itself).
constexpr int kReduceSplit = 8;
template <int DT>
__global__ __launch_bounds__(256) void dkdv_reduce_kernel(BwdArgs a) {
  const int* t = a.kv_tiles + 4 * blockIdx.x;
  if (t[0] < 0) return;
  const int j0 = a.kv_seg[2 * blockIdx.x], ns = a.kv_seg[2 * blockIdx.x + 1];
  if (ns <= 1) return;
  const int c = t[0], kh = t[3], D = a.D;
  const int key0 = a.cu_chunk[c] + t[1];
  const int nk = min(kKvTileKeys, a.cu_chunk[c + 1] - key0);
  const int n4 = nk * D / 4;
  const int64_t slot4 = kv_slot_floats(D) / 4;
  const f32x4_t* part = reinterpret_cast<const f32x4_t*>(a.part_dkv) + j0 * slot4;
  for (int i = blockIdx.y * 256 + threadIdx.x; i < 2 * n4; i += 256 * kReduceSplit) {
    const int which = i >= n4;  // 0 = dK, 1 = dV
    const int jj = which ? i - n4 : i;
    const f32x4_t* src = part + which * (kKvTileKeys * D / 4) + jj;
    f32x4_t acc = src[0];
    int s = 1;
    for (; s + 4 <= ns; s += 4) {  // four loads in flight, added in slot order
      f32x4_t x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] = src[(s + u) * slot4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += x[u][e];
    }
    for (; s < ns; ++s) {
      const f32x4_t x = src[s * slot4];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += x[e];
    }
    const float sc = which ? 1.0f : a.scale;
    u16x4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = from_f32<DT>(acc[e] * sc);
    const int key = key0 + jj / (D / 4), d = (jj % (D / 4)) * 4;
    *reinterpret_cast<u16x4_t*>((which ? a.dv : a.dk) + ((int64_t)key * a.Hkv + kh) * D + d) = r;
  }
}

template <int DT, int DP>
int launch_bwd(const BwdArgs& a, int n_self, int n_kv, int max_remote, int parts, hipStream_t st) {
  const int64_t rows = (int64_t)a.T * a.Hq;
  if (parts & 1) {
    hipLaunchKernelGGL(delta_kernel<DT>, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, st,
                       a.out, a.dout, a.lse, rows, a.D, a.delta, a.scale, a.lse_k);
    if (max_remote > 0 && a.R > 0)
      hipLaunchKernelGGL((dq_kernel<DT, DP, true, attn_qb<DP>()>), dim3((max_remote + 7) / 8 * 8), dim3(256), 0, st, a);
    if (n_self > 0)
      hipLaunchKernelGGL((dq_kernel<DT, DP, false, attn_qb<DP>()>), dim3((unsigned)(((int64_t)n_self * a.G + 7) / 8 * 8)), dim3(256), 0, st, a);
  }
  if ((parts & 2) && n_kv > 0) {
    // kKvTileKeys keys per workgroup in every kernel; the host's key tiles match
    const int n_wg = n_kv * a.kv_splits;
    if (a.kv_splits > 1) {
      constexpr int rows = 32 * dkdv_qb<DP>();  // query rows per tile of every key-major kernel
      hipLaunchKernelGGL(dkdv_sched_kernel<DP <= 128 ? 64 : rows>, dim3(1), dim3(1024), 0, st, a,
                         n_kv, n_wg, const_cast<int*>(a.kv_sched), const_cast<int*>(a.kv_seg));
    }
    if constexpr (DP <= 128) {
      if constexpr (DP <= 64) launch_dkdv1<DT, DP>(a, n_wg, st);
      else launch_dkdv2<DT, DP>(a, n_wg, st);
    } else {
      hipLaunchKernelGGL((dkdv_kernel<DT, DP>), dim3(n_wg), dim3(512), 0, st, a);
    }
    if (a.kv_splits > 1)
      hipLaunchKernelGGL(dkdv_reduce_kernel<DT>, dim3(n_kv, kReduceSplit), dim3(256), 0, st, a);
  }
  return moba_launch_status("prefill_bwd");
}

template <int DT>
int dispatch_bwd(const BwdArgs& a, int n_self, int n_kv, int max_remote, int parts, hipStream_t st) {
  if (a.D <= 32) return launch_bwd<DT, 32>(a, n_self, n_kv, max_remote, parts, st);
  if (a.D <= 64) return launch_bwd<DT, 64>(a, n_self, n_kv, max_remote, parts, st);
  if (a.D <= 128) return launch_bwd<DT, 128>(a, n_self, n_kv, max_remote, parts, st);
  return launch_bwd<DT, 256>(a, n_self, n_kv, max_remote, parts, st);
}

// Bytes of the schedule head of the row-split workspace (256-byte aligned).
int64_t dkdv_sched_bytes(int n_kv, int splits) {
  return ((int64_t)16 * n_kv * splits + (int64_t)8 * n_kv + 255) / 256 * 256;
}

}  // namespace

extern "C" int64_t moba_hip_prefill_bwd_work(int n_kv_tiles, int kv_splits, int D) {
  if (n_kv_tiles < 1 || kv_splits < 2 || kv_splits > 16 || D < 8 || D > 256) return 0;
  return dkdv_sched_bytes(n_kv_tiles, kv_splits) +
         (int64_t)n_kv_tiles * kv_splits * kv_slot_floats(D) * 4;
}

extern "C" int moba_hip_prefill_bwd(const void* q, const void* k, const void* v, const void* out,
                                    const void* dout, const float* lse, int dtype, int T, int Hq,
                                    int Hkv, int D, float scale, const int* cu_chunk,
                                    const int* self_tiles, int n_self_tiles, const int* kv_tiles,
                                    int n_kv_tiles, const int* sel, int R, const int* filtered,
                                    int E, const int* tile_off, const int* row_off,
                                    const int* counts, const int* rows, int max_remote_tiles,
                                    float* delta, void* part_dq, void* dq, void* dk, void* dv,
                                    int parts, int kv_splits, float* part_dkv, void* pack,
                                    void* stream) {
  if (dtype != 0 && dtype != 1) { moba_set_error("prefill_bwd: dtype must be 0 (bf16) or 1 (fp16)"); return MOBA_ERR_ARG; }
  if (D < 8 || D > 256 || D % 8) { moba_set_error("prefill_bwd: head_dim must be a multiple of 8 in [8,256]"); return MOBA_ERR_ARG; }
  if (Hq < 1 || Hkv < 1 || Hq % Hkv) { moba_set_error("prefill_bwd: Hq must be a positive multiple of Hkv"); return MOBA_ERR_ARG; }
  if (R < 0 || R > 8) { moba_set_error("prefill_bwd: remote count must be in [0,8]"); return MOBA_ERR_ARG; }
  if (Hq > 65535 || (int64_t)n_self_tiles * (Hq / Hkv) > (1 << 30)) { moba_set_error("prefill_bwd: too many heads or self tiles"); return MOBA_ERR_ARG; }
  if (parts < 1 || parts > 3) { moba_set_error("prefill_bwd: parts must be 1 (dq), 2 (dk/dv) or 3 (both)"); return MOBA_ERR_ARG; }
  if ((int64_t)T * Hq * D * 2 >= ((int64_t)1 << 32)) { moba_set_error("prefill_bwd: q / dO must be smaller than 4 GiB (32-bit buffer offsets)"); return MOBA_ERR_ARG; }
  if (kv_splits < 1 || kv_splits > 16 || (kv_splits > 1 && part_dkv == nullptr)) { moba_set_error("prefill_bwd: kv_splits must be in [1,16], with a part_dkv workspace when > 1"); return MOBA_ERR_ARG; }
  if (kv_splits > 1 && n_kv_tiles > kSchedMaxTiles) { moba_set_error("prefill_bwd: kv_splits > 1 needs n_kv_tiles <= 4096"); return MOBA_ERR_ARG; }
  if ((int64_t)n_kv_tiles * kv_splits > 0x7fffffff / 4) { moba_set_error("prefill_bwd: too many kv workgroups"); return MOBA_ERR_ARG; }
  BwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.out = (const uint16_t*)out; a.dout = (const uint16_t*)dout; a.lse = lse;
  a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv;
  a.scale = scale; a.scale_log2 = scale * kLog2e;
  a.cu_chunk = cu_chunk; a.self_tiles = self_tiles; a.kv_tiles = kv_tiles;
  a.n_self_wg = n_self_tiles * (Hq / Hkv);
  a.sel = sel; a.R = R; a.filtered = filtered; a.E = E;
  a.tile_off = tile_off; a.row_off = row_off; a.counts = counts; a.rows = rows;
  a.delta = delta; a.part_dq = (uint16_t*)part_dq; a.kv_splits = kv_splits;
  a.kv_sched = a.kv_seg = nullptr; a.part_dkv = nullptr;
  if (kv_splits > 1) {  // workspace: schedule, tile slots, then the partial slots
    char* ws = (char*)part_dkv;
    a.kv_sched = (const int*)ws;
    a.kv_seg = a.kv_sched + 4 * (int64_t)n_kv_tiles * kv_splits;
    a.part_dkv = (float*)(ws + dkdv_sched_bytes(n_kv_tiles, kv_splits));
  }
  a.dq = (uint16_t*)dq; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
  a.lse_k = delta + (int64_t)T * Hq;  // adjacent to delta (one load per row in the key-major kernels)
  a.pack_rows = (R > 0 && D <= 128) ? (int64_t)T * Hq * R : 0;
  a.pack_q = (uint16_t*)pack;
  a.pack_g = a.pack_q + a.pack_rows * D;
  a.pack_lse_k = (float*)(a.pack_g + a.pack_rows * D);
  a.pack_delta = a.pack_lse_k + a.pack_rows;
  if (a.pack_rows > 0 && pack == nullptr) { moba_set_error("prefill_bwd: the pack workspace is required when R > 0 and head_dim <= 128"); return MOBA_ERR_ARG; }
  if (a.pack_rows * D * 2 >= ((int64_t)1 << 32)) { moba_set_error("prefill_bwd: packed expert rows must be smaller than 4 GiB (32-bit buffer offsets)"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  const int mr = R > 0 ? max_remote_tiles : 0;
  return dtype == 0 ? dispatch_bwd<0>(a, n_self_tiles, n_kv_tiles, mr, parts, st)
                    : dispatch_bwd<1>(a, n_self_tiles, n_kv_tiles, mr, parts, st);
}
