// Key-major dK / dV of the MoBA prefill backward for head dims 65..128:
// wave pairs with split roles and a one-tile lag, no barrier inside a tile.
//
// Replaces the dk/dv halves of the two flash-attention backwards in
// OptMixedAttention.backward (src/moba_opt/mixed_attention.py:165-221) and the
// autograd scatter-add of the packed remote dk/dv into k/v
// (grouped_attention.py:81-89): every query row that attends a key -- the
// causal rows of the key's own chunk for all G heads of its KV group, then the
// expert rows that selected the chunk -- is visited by the one workgroup that
// owns the key, so dK / dV are summed in registers in a fixed order and
// written once (no atomics).
//
// A workgroup of 8 waves owns 128 keys of one chunk and one KV head as 4 wave
// pairs of 32 keys; the two waves of a pair share a SIMD.  For 64-row tiles
// of (Q, dO) rows, at step t:
//   role P (-K in registers, dV accumulators):
//       one MFMA block: X_t = lse_k - Q_t K^T  interleaved with  dV += P_{t-1}^T dO_{t-1}
//       then P_t = exp2(-c X_t) -> registers and LDS (input dtype)
//   role D (-V in registers, -dK accumulators):
//       -dS_{t-1} = P_{t-1} Y_{t-1}                    (P from LDS)
//       then one MFMA block: -dK += (-dS_{t-1})^T Q_{t-1}  interleaved with
//       Y_t = delta - dO_t V^T
// The row terms enter as the accumulators' start values (lse_k = lse / scale
// and delta of the tile's rows, read from LDS when the block starts), so the
// element-wise phases read no per-row values.
// Each role alternates a VALU phase and an MFMA block of two independent
// accumulator chains, in opposite order, so the SIMD's MFMA unit is fed by
// one wave while the other does its element-wise work.  Role D runs one tile
// behind role P on the P it needs, so the only synchronisation is the
// barrier where the LDS stages rotate: P_{t-1} was written before it.  Three
// stages hold tiles t - 1, t and t + 1 (loading).  The expert rows come
// packed contiguously (written by the remote dq kernel), so every tile is affine in the row
// number and is loaded HBM -> LDS by buffer loads issued from inline
// assembly (the waits are placed here): role D waves issue their share when
// the step starts, role P waves between the MFMAs of their block.
#include <type_traits>

#include "common.h"
#include "bwd_args.h"

namespace moba {
namespace {

constexpr int kPairKeys = 32;   // keys per wave pair
constexpr int kRows = 64;       // query rows per tile
// role P issues load piece k of the next tile after MFMA step kDmaAt + 2k
// of its block (the loads then overlap the block instead of stalling the
// start of the step)
constexpr int kDmaAt = 6;

template <int DT, int DP>
__global__ __launch_bounds__(512, 1) void dkdv2_kernel(BwdArgs a) {
  constexpr int NKS = DP / 16, NDB = DP / 32, QB = kRows / 32;
  constexpr int NB = DP / 8;                    // 16-byte blocks per row
  constexpr int NDMA = kRows * NB / 512;        // blocks per thread per operand
  static_assert(NDMA >= 1 && kRows * NB % 512 == 0, "one block per thread at least");
  // Q / dO tiles (swz<DP> layout) and their rows' lse_k / delta, three named
  // stages; P of the last two tiles per pair: [tile & 1][pair][qb][half][lane].
  __shared__ __attribute__((aligned(16))) uint16_t Q0[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G0[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t Q1[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G1[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t Q2[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G2[kRows * DP];
  __shared__ __attribute__((aligned(16))) float L0[2 * kRows];
  __shared__ __attribute__((aligned(16))) float L1[2 * kRows];
  __shared__ __attribute__((aligned(16))) float L2[2 * kRows];
  __shared__ __attribute__((aligned(16))) u16x8_t Px[2][4][QB][2][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int pair = wave & 3;
  const bool role_p = wave < 4;
  const int D = a.D, G = a.G;
  int ti, s_lo, s_hi, slot;
  if (!kv_work(a, ti, s_lo, s_hi, slot)) return;
  const int* tile = a.kv_tiles + 4 * ti;
  const int c = tile[0], kt0 = tile[1], f = tile[2], kh = tile[3];
  if (c < 0) return;                          // padding entry of the XCD-ordered list
  const int c_lo = a.cu_chunk[c], c_hi = a.cu_chunk[c + 1];
  const int key0 = c_lo + kt0;                // first key of the workgroup
  const int pkey0 = key0 + pair * kPairKeys;  // first key of this pair
  const int mykey = pkey0 + qi;               // this lane's key (B operand column)

  // Uninitialised LDS could hold NaN patterns that a zero probability would
  // not cancel; column blocks past D are never loaded and must read zero.
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int j = n * 512 + tid;
    st8(Q0 + j * 8, zero8()); st8(G0 + j * 8, zero8());
    st8(Q1 + j * 8, zero8()); st8(G1 + j * 8, zero8());
    st8(Q2 + j * 8, zero8()); st8(G2 + j * 8, zero8());
  }
  __syncthreads();

  // query tiles: G * n_self causal tiles (rows from key0 to the chunk end, for
  // every head of the group), then the expert's packed rows
  const int self_begin = key0;
  const int n_self = (max(0, c_hi - self_begin) + kRows - 1) / kRows;
  const int e = (f >= 0 && a.R > 0) ? f * a.Hkv + kh : -1;
  const int n_rem = e >= 0 ? a.counts[e] : 0;
  const int rbase = e >= 0 ? a.row_off[e] : 0;
  const int n_tiles = G * n_self + (n_rem + kRows - 1) / kRows;
  const int it_lo = s_lo, it_hi = min(s_hi, n_tiles);  // this workgroup's share

  // Tile loads: self tiles read q / dO / lse_k / delta in place (row stride
  // Hq), expert tiles the packed copies (row stride 1); rows past the tile's
  // valid range read past num_records, i.e. zeros, and a zero Q and dO row
  // adds nothing.  Thread t loads blocks n * 512 + t; wave w loads lse_k and
  // delta of rows 8w .. 8w + 7.
  const uint32_t qbytes = (uint32_t)((int64_t)a.T * a.Hq * D * 2);
  const uint32_t pbytes = (uint32_t)((int64_t)a.pack_rows * D * 2);
  const uint32_t lbytes = (uint32_t)((int64_t)a.T * a.Hq * 4);
  const uint32_t plbytes = (uint32_t)((int64_t)a.pack_rows * 4);
  int jrow[NDMA], jcol[NDMA];
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int j = n * 512 + tid, q = j / NB;
    jrow[n] = q;
    jcol[n] = swz<DP>(q, (j % NB) * 8) - q * DP;
  }
  // Tile cursor: tile `it` is causal tile s of head g while g < G, else
  // expert tile s; advanced by one per step (no divisions in the loop).
  struct Cur { int it, g, s; };
  auto cur_at = [&](int it) __attribute__((always_inline)) {
    return it < G * n_self ? Cur{it, it / n_self, it % n_self} : Cur{it, G, it - G * n_self};
  };
  auto cur_next = [&](Cur t) __attribute__((always_inline)) {
    ++t.it; ++t.s;
    if (t.g < G && t.s == n_self) { t.s = 0; ++t.g; }
    return t;
  };
  // A tile's loads as kPieces pieces: k < 2 NDMA loads Q (k even) or dO
  // block k / 2 of this thread, k = 2 NDMA the rows' lse_k and delta.
  struct Plan {
    const uint16_t* sq; const uint16_t* sg; const float* sl;
    uint32_t nb, lb, loff;
    uint32_t off[NDMA];
  };
  constexpr int kPieces = 2 * NDMA + 1;
  static_assert(kDmaAt + 2 * (kPieces - 1) < NKS * QB, "every piece is issued inside the block");
  auto plan = [&](Cur t) __attribute__((always_inline)) {
    const bool is_self = t.g < G;
    int r0 = 0, rstride = 1, nvalid = 0;
    if (t.it >= it_hi) {
    } else if (is_self) {
      const int s0 = self_begin + t.s * kRows;
      r0 = s0 * a.Hq + kh * G + t.g; rstride = a.Hq; nvalid = min(kRows, c_hi - s0);
    } else {
      r0 = rbase + t.s * kRows; rstride = 1; nvalid = min(kRows, n_rem - t.s * kRows);
    }
    Plan pl;
    pl.sq = is_self ? a.q : a.pack_q;
    pl.sg = is_self ? a.dout : a.pack_g;
    // delta and lse_k are adjacent arrays (delta first in place, lse_k first
    // in the pack): one load of 16 lanes brings both
    pl.sl = is_self ? a.delta : a.pack_lse_k;
    pl.nb = is_self ? qbytes : pbytes;
    pl.lb = 2 * (is_self ? lbytes : plbytes);
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int q = jrow[n], col = jcol[n];
      pl.off[n] = (q < nvalid && col < D) ? (uint32_t)(((int64_t)(r0 + q * rstride) * D + col) * 2) : pl.nb;
    }
    // lanes 0..7: lse_k of rows 8w .. 8w + 7, lanes 8..15: their delta
    const int ql = wave_s * 8 + (lane & 7);
    const uint32_t l_at = (lane < 8) == is_self ? pl.lb / 2 : 0;  // lse_k half
    pl.loff = ql < nvalid ? l_at + (uint32_t)(r0 + ql * rstride) * 4 : pl.lb;
    return pl;
  };
  auto piece = [&](const Plan& pl, int k, uint16_t* Qd, uint16_t* Gd, float* Ld) __attribute__((always_inline)) {
    if (k < 2 * NDMA) {
      const int jb = (k >> 1) * 512 + wave_s * 64;   // first block of this wave's 64
      if (k & 1) dma_lds16(make_rsrc(pl.sg, pl.nb), Gd + jb * 8, pl.off[k >> 1], 0);
      else dma_lds16(make_rsrc(pl.sq, pl.nb), Qd + jb * 8, pl.off[k >> 1], 0);
    } else if (lane < 16) {
      dma_lds4(make_rsrc(pl.sl, pl.lb), Ld + wave_s * 16, pl.loff, 0);
    }
  };
  auto dma = [&](uint16_t* Qd, uint16_t* Gd, float* Ld, Cur t) __attribute__((always_inline)) {
    const Plan pl = plan(t);
#pragma unroll
    for (int k = 0; k < kPieces; ++k) piece(pl, k, Qd, Gd, Ld);
  };

  const uint32_t kq0 = swz_b128_base<DP>(lane);
  const uint32_t trb0 = swz_tr_base<DP>(lane, 0), trb1 = swz_tr_base<DP>(lane, 1);
  const float nc2 = -a.scale_log2;

  // causal rows that end before the pair's first key contribute nothing
  auto skipped = [&](Cur t) __attribute__((always_inline)) {
    return t.g < G && t.s * kRows + kRows - 1 < pair * kPairKeys;
  };
  // One MFMA block of up to two independent chains, interleaved step by
  // step, each with its operand reads PF steps ahead (PF = 3 when both run):
  //   chain A: sp (rows x keys) = Li (row terms) + A (rows, b128 reads) x kv (keys in registers)
  //   chain B: acc (keys x d) += op^T (in registers) x B (rows, transposed reads)
  // Both chains are NKS * QB = NDB * QB * 2 MFMAs long.
  auto block = [&](auto da_tag, auto db_tag, const float* Li, const uint16_t* A, const u16x8_t (&kv)[NKS],
                   f32x16_t (&sp)[QB], const uint16_t* B, const u16x8_t (&op)[QB][2],
                   f32x16_t (&acc)[NDB], auto&& side) __attribute__((always_inline)) {
    constexpr bool DA = decltype(da_tag)::value, DB = decltype(db_tag)::value;
    constexpr int N = NKS * QB, PF = (DA && DB) ? 3 : 6;
    static_assert(N == NDB * QB * 2, "chain lengths");
    const uint32_t kq = opaque(kq0), t0 = opaque(trb0), t1 = opaque(trb1);
    // chain A step i: row block i % QB, k block i / QB
    auto rda = [&](int i) __attribute__((always_inline)) {
      return lds8(A, (i % QB) * 32 * DP * 2 + swz_b128<DP>(kq, i / QB));
    };
    // chain B step i: d block i % NDB, row block (i / NDB / 2) % QB, half (i / NDB) % 2
    // (consecutive steps feed different accumulators)
    auto rdb = [&](int i) __attribute__((always_inline)) {
      const int j = i / NDB;
      const uint32_t ro = (((j / 2) % QB) * 32 + (j % 2) * 16) * DP * 2;
      return lds_tr8(B, ro + swz_tr<DP>(t0, i % NDB), ro + swz_tr<DP>(t1, i % NDB));
    };
    u16x8_t ra[PF], rb[PF];
    if constexpr (DA) {  // D layout: lane holds rows 8j + 4hh + i of block qb
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(Li + (qb * 4 + j) * 16 + 4 * hh);
#pragma unroll
          for (int i = 0; i < 4; ++i) sp[qb][4 * j + i] = l4[i];
        }
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if constexpr (DA) ra[i] = rda(i);
      if constexpr (DB) rb[i] = rdb(i);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if constexpr (DA) {
        const u16x8_t x = ra[i % PF];
        if (i + PF < N) ra[i % PF] = rda(i + PF);
        sp[i % QB] = mfma32<DT>(x, kv[i / QB], sp[i % QB]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (DB) {
        const u16x8_t b = rb[i % PF];
        if (i + PF < N) rb[i % PF] = rdb(i + PF);
        acc[i % NDB] = mfma32<DT>(op[(i / NDB / 2) % QB][(i / NDB) % 2], b, acc[i % NDB]);
        __builtin_amdgcn_sched_barrier(0);
      }
      side(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // the block for runtime flags (chain A: current tile, chain B: previous tile)
  auto run_block = [&](bool cur, bool prev, const float* Li, const uint16_t* A, const u16x8_t (&kv)[NKS],
                       f32x16_t (&sp)[QB], const uint16_t* B, const u16x8_t (&op)[QB][2],
                       f32x16_t (&acc)[NDB], auto&& side) __attribute__((always_inline)) {
    // the wave in its MFMA block issues ahead of its partner's element-wise
    // phase on the shared SIMD
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    if (cur && prev) block(std::true_type{}, std::true_type{}, Li, A, kv, sp, B, op, acc, side);
    else if (cur) block(std::true_type{}, std::false_type{}, Li, A, kv, sp, B, op, acc, side);
    else if (prev) block(std::false_type{}, std::true_type{}, Li, A, kv, sp, B, op, acc, side);
    else {
#pragma unroll
      for (int i = 0; i < NKS * QB; ++i) side(i);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
  };

  auto body = [&](auto role_tag) __attribute__((always_inline)) {
    constexpr bool ROLE_P = decltype(role_tag)::value;
    // -K (role P) or -V (role D) rows: B operands, column = key, k = d
    u16x8_t kv[NKS];
    const uint16_t* kvsrc = ROLE_P ? a.k : a.v;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = ks * 16 + hh * 8;
      kv[ks] = neg8((mykey < c_hi && d < D) ? ld8(kvsrc + ((int64_t)mykey * a.Hkv + kh) * D + d) : zero8());
    }
    // the rows must have landed before the tile loads start: the compiler's
    // own waits for them would otherwise also drain the tile loads in flight
    __builtin_amdgcn_s_waitcnt(0x0F70);
    f32x16_t acc[NDB];                          // dV (role P) or -dK (role D)
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc[i] = zero16();
    // role P: lse_k - S of the current tile; role D: delta - dP of the last computed tile
    f32x16_t sp[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) sp[qb] = zero16();
    // role P: P of the previous tile; role D: -dS of the previous tile
    u16x8_t op[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) op[qb][0] = op[qb][1] = zero8();

    // role P, tile t in stage (Qc, Lc), previous tile's dO in Gp:
    //   X_t and dV += P_prev^T dO_prev in one block, then P_t -> op and LDS
    auto p_step = [&](const uint16_t* Qc, const float* Lc, const uint16_t* Gp, Cur t, bool cur,
                      bool prev, auto&& side) __attribute__((always_inline)) {
      run_block(cur, prev, Lc, Qc, kv, sp, Gp, op, acc, side);
      if (!cur) return;
      const bool is_self = t.g < G;
      const int sq0 = is_self ? self_begin + t.s * kRows : 0;
      const bool need_mask = (pkey0 + kPairKeys > c_hi) || (is_self && sq0 < pkey0 + kPairKeys - 1);
      auto to_p = [&](auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          uint32_t w[8];  // packed pairs (rows 8j + 4hh + 2m, + 1) at w[2j + m]
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r0 = qb * 32 + 8 * j + 4 * hh;
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              p[i] = fast_exp2(sp[qb][4 * j + i] * nc2);
              if constexpr (MASK) p[i] = (mykey < c_hi && (!is_self || mykey <= sq0 + r0 + i)) ? p[i] : 0.0f;
            }
            w[2 * j] = pack2<DT>(p[0], p[1]);
            w[2 * j + 1] = pack2<DT>(p[2], p[3]);
          }
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
            op[qb][h2] = __builtin_bit_cast(u16x8_t, (u32x4_t){w[4 * h2], w[4 * h2 + 1], w[4 * h2 + 2], w[4 * h2 + 3]});
        }
      };
      if (need_mask) to_p(std::true_type{}); else to_p(std::false_type{});
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        Px[t.it & 1][pair][qb][0][lane] = op[qb][0];
        Px[t.it & 1][pair][qb][1][lane] = op[qb][1];
      }
    };
    // role D: -dS_prev = P_prev Y_prev (P from LDS), then
    // -dK += (-dS_prev)^T Q_prev and Y_t = delta - dO_t V^T in one block
    auto d_step = [&](const uint16_t* Gc, const float* Lc, const uint16_t* Qp, Cur t, bool cur,
                      bool prev) __attribute__((always_inline)) {
      if (prev) {
        const int b = (t.it - 1) & 1;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            // word m of P row block h2: rows of sp elements 8 h2 + 2m, + 1
            const u32x4_t pw = __builtin_bit_cast(u32x4_t, Px[b][pair][qb][h2][lane]);
            uint32_t w[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              float lo, hi;
              unpack2<DT>(pw[m], lo, hi);
              w[m] = pack2<DT>(lo * sp[qb][8 * h2 + 2 * m], hi * sp[qb][8 * h2 + 2 * m + 1]);
            }
            op[qb][h2] = __builtin_bit_cast(u16x8_t, (u32x4_t){w[0], w[1], w[2], w[3]});
          }
        }
      }
      run_block(cur, prev, Lc + 8, Gc, kv, sp, Qp, op, acc, [](int) {});
    };
    // one tile: stage c holds tile tc, stage p the tile before (computed when
    // pv), stage n receives the next tile; afterwards this wave's loads of
    // the next tile have landed and the barrier makes every wave's loads and
    // P writes visible
    Cur tc = cur_at(it_lo);
    bool pv = false;
    auto step = [&](uint16_t* Qp, uint16_t* Gp, float* Lp, uint16_t* Qc, uint16_t* Gc, float* Lc,
                    uint16_t* Qn, uint16_t* Gn, float* Ln) __attribute__((always_inline)) {
      const Cur tn = cur_next(tc);
      const bool cur = tc.it < it_hi && !skipped(tc);
      if constexpr (ROLE_P) {
        // role P spreads the next tile's loads over its MFMA block
        const Plan pl = plan(tn);
        p_step(Qc, Lc, Gp, tc, cur, pv, [&](int i) __attribute__((always_inline)) {
          if (i >= kDmaAt && (i - kDmaAt) % 2 == 0 && (i - kDmaAt) / 2 < kPieces)
            piece(pl, (i - kDmaAt) / 2, Qn, Gn, Ln);
        });
      } else {
        dma(Qn, Gn, Ln, tn);
        __builtin_amdgcn_sched_barrier(0);  // the next tile's loads go out first
        d_step(Gc, Lc, Qp, tc, cur, pv);
      }
      pv = cur;
      tc = tn;
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      lds_barrier();
    };
    dma(Q0, G0, L0, tc);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    lds_barrier();
    // stages rotate with period 3: tile it lives in stage (it - it_lo) % 3;
    // the loop runs one step past it_hi so both roles finish the last tile
    for (int it = it_lo; it <= it_hi; it += 3) {
      step(Q2, G2, L2, Q0, G0, L0, Q1, G1, L1);
      if (it + 1 > it_hi) break;
      step(Q0, G0, L0, Q1, G1, L1, Q2, G2, L2);
      if (it + 2 > it_hi) break;
      step(Q1, G1, L1, Q2, G2, L2, Q0, G0, L0);
    }

    // D layout: lane holds column d = i*32 + qi, keys 8j + 4hh + r.  A row
    // split writes fp32 partials to its slot for the fixed-order reduction.
    float* pdst = a.part_dkv + (int64_t)max(slot, 0) * kv_slot_floats(D) +
                  (ROLE_P ? kKvTileKeys * D : 0);
    uint16_t* dst = ROLE_P ? a.dv : a.dk;
    const float psc = ROLE_P ? 1.0f : -1.0f, osc = ROLE_P ? 1.0f : -a.scale;
#pragma unroll
    for (int i = 0; i < NDB; ++i) {
      const int d = i * 32 + qi;
      if (d >= D) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = pkey0 + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (key >= c_hi) continue;
        const int64_t o = ((int64_t)key * a.Hkv + kh) * D + d;
        if (slot >= 0) pdst[(key - key0) * D + d] = acc[i][r] * psc;
        else dst[o] = from_f32<DT>(acc[i][r] * osc);
      }
    }
  };
  if (role_p) body(std::true_type{}); else body(std::false_type{});
}

}  // namespace

template <int DT, int DP> void launch_dkdv2(const BwdArgs& a, int n_wg, hipStream_t st) {
  hipLaunchKernelGGL((dkdv2_kernel<DT, DP>), dim3(n_wg), dim3(512), 0, st, a);
}

template void launch_dkdv2<0, 128>(const BwdArgs&, int, hipStream_t);
template void launch_dkdv2<1, 128>(const BwdArgs&, int, hipStream_t);

}  // namespace moba
