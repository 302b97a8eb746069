// MoBA prefill forward on gfx950: bf16/fp16 MFMA attention tiles.
//
// Replaces the two flash-attention forwards and the merge of
// src/moba_opt/mixed_attention.py:67-112 (self branch: causal within each
// chunk; remote branch: each selected (query, head) row attends one full past
// chunk) and the atomic slot build + warp-per-row merge of
// src/moba_opt/ops/merge.cu:27-153.
//
// Two launches, no atomics, no packed copies of Q or K/V:
//  * remote launch: one workgroup per tile of 128 rows of one expert
//    (filtered chunk, kv head).  Rows are read in place from q[T,Hq,D] through
//    the expert's row list; the chunk's K/V tiles are staged in LDS once per
//    workgroup.  Each row writes a normalised partial o and its (max, sum)
//    softmax statistics into its slot
//    (s*Hq + h)*R + j, j = rank of the chunk in the row's ascending selection.
//  * self launch: one workgroup per (chunk, q head, 128 consecutive rows),
//    causal within the chunk; its epilogue merges the row's partials in
//    ascending-slot order (global softmax: m = max l, O = sum e^{l-m} o / z,
//    L = m + log z) and writes the final O (input dtype) and LSE (fp32).
//
// Tile math (per wave: 2 blocks of 32 query rows, key tiles of 64):
//   S^T = K Q^T      (A = K rows from LDS, B = Q fragment in registers)
//   O^T += V^T P^T   (A = V^T read from the row-major V tile with the gfx950
//                     transposed LDS read, B = P straight from the S^T
//                     accumulators: the D-layout of S^T is the B-layout of P^T
//                     up to a fixed key order, which the transposed read follows)
// Each K / V^T fragment read from LDS feeds the MFMAs of both query blocks, and
// the next K/V tile is prefetched into registers while the current one computes.
// so every per-query quantity (running max, sum, rescale) is lane-uniform.
#include <type_traits>

#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int T, Hq, Hkv, D, G;
  float scale_log2;
  const int* cu_chunk;
  const int* self_tiles;
  int n_self_wg;        // self workgroups: entries of self_tiles x G
  const int* sel;
  int R;
  const int* filtered;
  int E;
  const int* tile_off;
  const int* row_off;
  const int* counts;
  const int* rows;
  uint16_t* part_o;     // remote partial outputs, input dtype
  float* part_ml;
  uint16_t* out;
  float* lse;
};

constexpr int kBN = 64;   // keys per LDS tile
constexpr float kRescaleSlack = 8.0f;  // log2 headroom before O is rescaled

template <int DT, int DP, bool REMOTE, int QB>
__global__ __launch_bounds__(256, attn_occupancy<DP>()) void fwd_kernel(FwdArgs a) {
  constexpr int NKS = DP / 16;  // k-steps of the QK^T contraction
  constexpr int NDB = DP / 32;  // 32-row d blocks of O^T
  constexpr int TILE = kBN * DP;           // elements of one K or V tile
  constexpr int NB = DP / 8;                // 16-byte blocks per tile row
  constexpr int NDMA = kBN * NB / 256;      // 16-byte blocks per thread per tile
  // Two stages of K and V tiles in the swz<DP> layout, filled straight from
  // HBM by buffer loads into LDS.  Separate arrays let the compiler see that
  // reads of one stage never wait on the loads in flight into the other.
  __shared__ __attribute__((aligned(16))) uint16_t K0[TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V0[TILE];
  __shared__ __attribute__((aligned(16))) uint16_t K1[TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V1[TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int D = a.D;

  int s[QB], h[QB], slot[QB];
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

  u16x8_t qf[QB][NKS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t qrow = ((int64_t)s[qb] * a.Hq + h[qb]) * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 16 + hh * 8;
      qf[qb][ks] = (valid[qb] && d < D) ? ld8(a.q + qrow + d) : zero8();
    }
  }

  // Tile loads: block j of a tile (row j / NB, physical block j % NB) comes
  // from logical column block (j % NB) ^ f(row); thread (wave w, lane l)
  // loads blocks (n * 4 + w) * 64 + l.  Offsets are relative to key k_lo of
  // head kh, so they are the same for every tile; the tile advance goes in the
  // scalar offset.  Rows past k_hi lie beyond num_records and load zeros;
  // column blocks past D are never loaded (zeroed once below).
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
  if (D < DP) {  // column blocks past D stay zero for the whole kernel
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int j = (n * 4 + wave) * 64 + lane;
      st8(K0 + j * 8, zero8()); st8(V0 + j * 8, zero8());
      st8(K1 + j * 8, zero8()); st8(V1 + j * 8, zero8());
    }
    __syncthreads();
  }

  f32x16_t oacc[QB][NDB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = zero16();
  float m_run[QB], lsum[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) { m_run[qb] = -INFINITY; lsum[qb] = 0.0f; }
  const float c2 = a.scale_log2;

  // Lane-constant byte bases of the swizzled LDS reads.
  const uint32_t kbase0 = swz_b128_base<DP>(lane);
  const uint32_t trb0 = swz_tr_base<DP>(lane, 0), trb1 = swz_tr_base<DP>(lane, 1);

  const int ntiles = (n_keys + kBN - 1) / kBN;
  auto tile = [&](const uint16_t* Kb, const uint16_t* Vb, const int it, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int kt0 = k_lo + it * kBN;
    const uint32_t kq = opaque(kbase0), t0 = opaque(trb0), t1 = opaque(trb1);
    f32x16_t sacc[QB][2];
    wave_prio<1>();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = zero16();
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const u16x8_t av = lds8(Kb, kb * 32 * DP * 2 + swz_b128<DP>(kq, ks));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = mfma32<DT>(av, qf[qb][ks], sacc[qb][kb]);
      }
    }
    wave_prio<0>();
    if constexpr (MASK) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kt0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
            const bool ok = key < k_hi && (REMOTE || key <= s[qb]);
            sacc[qb][kb][r] = ok ? sacc[qb][kb][r] : -INFINITY;
          }
    }
    u16x8_t pv[QB][2][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[qb][kb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c2;
      // Lazy rescale: keep the running max while the new scores stay within
      // 2^8 of it (p <= 256 is exact enough in bf16/fp32); O, l and the final
      // normalisation all use the same reference so the result is unchanged.
      const bool up = mx > m_run[qb] + kRescaleSlack;
      if (__any(up)) [[unlikely]] {
        const float mn = up ? mx : m_run[qb];
        const float alpha = fast_exp2(m_run[qb] - mn);
        lsum[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[qb][db][r] *= alpha;
        m_run[qb] = mn;
        __builtin_amdgcn_sched_barrier(0);
      }
      const float nm = -m_run[qb];
      float ps = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          p[r] = fast_exp2(fmaf(sacc[qb][kb][r], c2, nm));
          ps += p[r];
        }
        pv[qb][kb][0] = pack8<DT>(p);
        pv[qb][kb][1] = pack8<DT>(p + 8);
      }
      lsum[qb] += ps;
    }
    wave_prio<1>();
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint32_t ro = (kb * 32 + t * 16) * DP * 2;
          const u16x8_t av = lds_tr8(Vb, ro + swz_tr<DP>(t0, db), ro + swz_tr<DP>(t1, db));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) oacc[qb][db] = mfma32<DT>(av, pv[qb][kb][t], oacc[qb][db]);
        }
    wave_prio<0>();
  };
  // vmcnt(0) with the other counters left alone, then a workgroup barrier:
  // this wave's tile loads have landed, and after the barrier every wave's.
  auto stage_sync = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);
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
    const float l = lsum[qb] + __shfl_xor(lsum[qb], 32, 64);
    if (!valid[qb]) continue;
    if constexpr (REMOTE) {
      const float inv = 1.0f / l;
      uint16_t* po = a.part_o + (int64_t)slot[qb] * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d0 = db * 32 + 8 * j + 4 * hh;
          if (d0 < D) {
            f32x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = oacc[qb][db][4 * j + i] * inv;
            u16x4_t ob;
#pragma unroll
            for (int i = 0; i < 4; ++i) ob[i] = from_f32<DT>(o[i]);
            *reinterpret_cast<u16x4_t*>(po + d0) = ob;
          }
        }
      // partial stored as (running max, sum) in the log2 domain: merging
      // them is exact in fp32 even when |logits| is huge (an LSE would round
      // log2(l) away next to a large max)
      if (hh == 0) {
        a.part_ml[2 * (int64_t)slot[qb]] = m_run[qb];
        a.part_ml[2 * (int64_t)slot[qb] + 1] = l;
      }
    } else {
      const int64_t row = (int64_t)s[qb] * a.Hq + h[qb];
      // Slot loads are unconditional (slots below R are in the row's
      // allocation) and masked after, so each pass costs one round trip per
      // slot: guarded loads compiled to one full wait per load.
      float M2 = m_run[qb];
      for (int jj = 0; jj < a.R; ++jj) {
        const int64_t sl = row * a.R + jj;
        const int sv = a.sel[sl];
        const float mv = a.part_ml[2 * sl];
        M2 = sv >= 0 ? fmaxf(M2, mv) : M2;
      }
      const float ws = fast_exp2(m_run[qb] - M2);
      float z = l * ws;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[qb][db][r] *= ws;
      for (int jj = 0; jj < a.R; ++jj) {
        const int64_t sl = row * a.R + jj;
        const int sv = a.sel[sl];
        const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + 2 * sl);
        const uint16_t* po = a.part_o + sl * D;
        u16x4_t o[NDB][4];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int d0 = db * 32 + 8 * j + 4 * hh;
            o[db][j] = *reinterpret_cast<const u16x4_t*>(po + (d0 < D ? d0 : 0));
          }
        // an unselected slot's data may be stale or NaN: select, never 0 * x
        const float w = sv >= 0 ? ml.y * fast_exp2(ml.x - M2) : 0.0f;
        z += w;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool ok = sv >= 0 && db * 32 + 8 * j + 4 * hh < D;
#pragma unroll
            for (int i = 0; i < 4; ++i) oacc[qb][db][4 * j + i] += ok ? w * to_f32<DT>(o[db][j][i]) : 0.0f;
          }
      }
      const float invz = 1.0f / z;
      uint16_t* orow = a.out + row * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d0 = db * 32 + 8 * j + 4 * hh;
          if (d0 < D) {
            u16x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = from_f32<DT>(oacc[qb][db][4 * j + i] * invz);
            *reinterpret_cast<u16x4_t*>(orow + d0) = o;
          }
        }
      if (hh == 0) a.lse[row] = (M2 + log2f(z)) * kLn2;
    }
  }
}

template <int DT, int DP>
int launch_fwd(const FwdArgs& a, int n_self_tiles, int max_remote_tiles, hipStream_t st) {
  if (max_remote_tiles > 0 && a.R > 0) {
    hipLaunchKernelGGL((fwd_kernel<DT, DP, true, attn_qb<DP>()>), dim3((max_remote_tiles + 7) / 8 * 8), dim3(256), 0, st, a);
    int rc = moba_launch_status("prefill_fwd(remote)");
    if (rc) return rc;
  }
  if (n_self_tiles > 0) {
    hipLaunchKernelGGL((fwd_kernel<DT, DP, false, attn_qb<DP>()>), dim3((unsigned)(((int64_t)n_self_tiles * a.G + 7) / 8 * 8)), dim3(256), 0, st, a);
    return moba_launch_status("prefill_fwd(self)");
  }
  return MOBA_OK;
}

template <int DT>
int dispatch_fwd(const FwdArgs& a, int n_self, int max_remote, hipStream_t st) {
  if (a.D <= 32) return launch_fwd<DT, 32>(a, n_self, max_remote, st);
  if (a.D <= 64) return launch_fwd<DT, 64>(a, n_self, max_remote, st);
  if (a.D <= 128) return launch_fwd<DT, 128>(a, n_self, max_remote, st);
  return launch_fwd<DT, 256>(a, n_self, max_remote, st);
}

}  // namespace

extern "C" int moba_hip_prefill_rows(int D) {
  if (D < 8 || D > 256 || D % 8) return -1;
  if (D <= 32) return 128 * attn_qb<32>();
  if (D <= 64) return 128 * attn_qb<64>();
  if (D <= 128) return 128 * attn_qb<128>();
  return 128 * attn_qb<256>();
}

extern "C" int moba_hip_prefill_fwd(const void* q, const void* k, const void* v, int dtype, int T,
                                    int Hq, int Hkv, int D, float scale, const int* cu_chunk,
                                    const int* self_tiles, int n_self_tiles, const int* sel, int R,
                                    const int* filtered, int E, const int* tile_off,
                                    const int* row_off, const int* counts, const int* rows,
                                    int max_remote_tiles, void* part_o, float* part_ml,
                                    void* out, float* lse, void* stream) {
  if (dtype != 0 && dtype != 1) { moba_set_error("prefill_fwd: dtype must be 0 (bf16) or 1 (fp16)"); return MOBA_ERR_ARG; }
  if (D < 8 || D > 256 || D % 8) { moba_set_error("prefill_fwd: head_dim must be a multiple of 8 in [8,256]"); return MOBA_ERR_ARG; }
  if (Hq < 1 || Hkv < 1 || Hq % Hkv) { moba_set_error("prefill_fwd: Hq must be a positive multiple of Hkv"); return MOBA_ERR_ARG; }
  if (R < 0 || R > 8) { moba_set_error("prefill_fwd: remote count must be in [0,8]"); return MOBA_ERR_ARG; }
  if (Hq > 65535 || (int64_t)n_self_tiles * (Hq / Hkv) > (1 << 30)) { moba_set_error("prefill_fwd: too many heads or self tiles"); return MOBA_ERR_ARG; }
  FwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv;
  a.scale_log2 = scale * kLog2e;
  a.cu_chunk = cu_chunk; a.self_tiles = self_tiles; a.n_self_wg = n_self_tiles * (Hq / Hkv);
  a.sel = sel; a.R = R; a.filtered = filtered; a.E = E;
  a.tile_off = tile_off; a.row_off = row_off; a.counts = counts; a.rows = rows;
  a.part_o = (uint16_t*)part_o; a.part_ml = part_ml;
  a.out = (uint16_t*)out; a.lse = lse;
  hipStream_t st = (hipStream_t)stream;
  return dtype == 0 ? dispatch_fwd<0>(a, n_self_tiles, R > 0 ? max_remote_tiles : 0, st)
                    : dispatch_fwd<1>(a, n_self_tiles, R > 0 ? max_remote_tiles : 0, st);
}
