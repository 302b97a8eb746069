// Key-major dK / dV of the MoBA prefill backward, one wave per SIMD.
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
// A workgroup of 4 waves owns 128 keys of one chunk and one KV head; wave w
// owns keys 32w..32w+31 and holds their K and V rows as MFMA B operands and
// their dK, dV accumulators.  For each 64-row tile of (Q, dO) rows it runs all
// four products itself:
//   X = lse_k - Q K^T,  Y = delta - dO V^T   (A = Q / dO rows from LDS, B = -K / -V)
//   P  = exp2(-c X),  -dS = P Y
//   dV += P^T dO,  -dK += (-dS)^T Q  (B = dO / Q through transposed LDS reads)
// lse_k = lse / scale and delta start the accumulators, so the row terms cost
// no element-wise work.
// The D layout of S / dP (one key per lane) is the A layout of P^T / dS^T, so
// P and dS never leave registers and the waves never wait for each other
// inside a tile: one barrier per tile, where the LDS stages rotate.  Used for
// head dims <= 64, where the registers allow two waves per SIMD.
#include <type_traits>

#include "common.h"
#include "bwd_args.h"

namespace moba {
namespace {

constexpr int kWaveKeys = 32;   // keys per wave
constexpr int kRows = 64;       // query rows per tile
constexpr int kStages = 3;      // LDS stages of (Q, dO) tiles

// s_waitcnt vmcnt(N), other counters untouched (N < 16).
template <int N> MOBA_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

template <int DT, int DP>
__global__ __launch_bounds__(256, 1) void dkdv1_kernel(BwdArgs a) {
  constexpr int NKS = DP / 16, NDB = DP / 32, QB = kRows / 32;
  constexpr int NB = DP / 8;                    // 16-byte blocks per row
  constexpr int NDMA = kRows * NB / 256;        // blocks per thread per operand
  constexpr int NS = kStages;
  static_assert(NDMA >= 1, "tile smaller than one block per thread");
  // Q / dO tiles (swz<DP> layout) and their rows' lse_k / delta in NS named
  // stages, filled by buffer loads straight into LDS NS - 1 tiles ahead.
  __shared__ __attribute__((aligned(16))) uint16_t Q0[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G0[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t Q1[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G1[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t Q2[kRows * DP];
  __shared__ __attribute__((aligned(16))) uint16_t G2[kRows * DP];
  __shared__ __attribute__((aligned(16))) float L0[2 * kRows];
  __shared__ __attribute__((aligned(16))) float L1[2 * kRows];
  __shared__ __attribute__((aligned(16))) float L2[2 * kRows];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int D = a.D, G = a.G;
  int ti, s_lo, s_hi, slot;
  if (!kv_work(a, ti, s_lo, s_hi, slot)) return;
  const int* tile = a.kv_tiles + 4 * ti;
  const int c = tile[0], kt0 = tile[1], f = tile[2], kh = tile[3];
  if (c < 0) return;                          // padding entry of the XCD-ordered list
  const int c_lo = a.cu_chunk[c], c_hi = a.cu_chunk[c + 1];
  const int key0 = c_lo + kt0;                // first key of the workgroup
  const int wkey0 = key0 + wave * kWaveKeys;  // first key of this wave
  const int mykey = wkey0 + qi;               // this lane's key (B operand column)

  // Uninitialised LDS could hold NaN patterns that a zero probability would
  // not cancel; column blocks past D are never loaded and must read zero.
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int j = n * 256 + tid;
    st8(Q0 + j * 8, zero8()); st8(G0 + j * 8, zero8());
    st8(Q1 + j * 8, zero8()); st8(G1 + j * 8, zero8());
    st8(Q2 + j * 8, zero8()); st8(G2 + j * 8, zero8());
  }
  __syncthreads();


  // query tiles: G * n_self causal tiles (rows from key0 to the chunk end, for
  // every head of the group), then the expert's rows, which the remote dq kernel
  // laid out contiguously (row_off[e] onwards) in pack_q / pack_g / pack_ld.
  const int self_begin = key0;
  const int n_self = (max(0, c_hi - self_begin) + kRows - 1) / kRows;
  const int e = (f >= 0 && a.R > 0) ? f * a.Hkv + kh : -1;
  const int n_rem = e >= 0 ? a.counts[e] : 0;
  const int rbase = e >= 0 ? a.row_off[e] : 0;
  const int n_tiles = G * n_self + (n_rem + kRows - 1) / kRows;
  const int it_lo = s_lo, it_hi = min(s_hi, n_tiles);  // this workgroup's share

  // Every tile's rows are affine in the row number, so the loads need no row
  // indices: self tiles read q / dO / lse_k / delta in place (row stride Hq),
  // expert tiles the packed copies (row stride 1).  Rows past the tile's
  // valid range read past num_records, i.e. zeros: a zero Q and dO row adds
  // nothing to dK or dV whatever its probability.  Thread t loads blocks
  // n * 256 + t.
  const uint32_t qbytes = (uint32_t)((int64_t)a.T * a.Hq * D * 2);
  const uint32_t pbytes = (uint32_t)((int64_t)a.pack_rows * D * 2);
  const uint32_t lbytes = (uint32_t)((int64_t)a.T * a.Hq * 4);
  const uint32_t plbytes = (uint32_t)((int64_t)a.pack_rows * 4);
  int jrow[NDMA], jcol[NDMA];
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int j = n * 256 + tid, q = j / NB;
    jrow[n] = q;
    jcol[n] = swz<DP>(q, (j % NB) * 8) - q * DP;
  }
  // Per wave and tile: 2 * NDMA tile loads plus lse_k and delta of 16 rows,
  // always issued (tiles past it_hi load zeros into a stage nobody reads), so
  // the wait below is a constant.
  constexpr int kLoadsPerTile = 2 * NDMA + 2;
  auto dma = [&](uint16_t* Qd, uint16_t* Gd, float* Ld, int it) __attribute__((always_inline)) {
    const bool is_self = it < G * n_self;
    int r0 = 0, rstride = 1, nvalid = 0;
    if (it >= it_hi) {
    } else if (is_self) {
      const int g = it / n_self, s0 = self_begin + (it % n_self) * kRows;
      r0 = s0 * a.Hq + kh * G + g; rstride = a.Hq; nvalid = min(kRows, c_hi - s0);
    } else {
      const int t = it - G * n_self;
      r0 = rbase + t * kRows; rstride = 1; nvalid = min(kRows, n_rem - t * kRows);
    }
    const uint16_t* srcq = is_self ? a.q : a.pack_q;
    const uint16_t* srcg = is_self ? a.dout : a.pack_g;
    const uint32_t nb = is_self ? qbytes : pbytes;
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int q = jrow[n], col = jcol[n];
      const uint32_t off = (q < nvalid && col < D)
                               ? (uint32_t)(((int64_t)(r0 + q * rstride) * D + col) * 2) : nb;
      const int jb = n * 256 + wave_s * 64;   // first block of this wave's 64
      dma_lds16(make_rsrc(srcq, nb), Qd + jb * 8, off, 0);
      dma_lds16(make_rsrc(srcg, nb), Gd + jb * 8, off, 0);
    }
    if (lane < 16) {  // wave w: lse_k and delta of rows 16w .. 16w + 15
      const int q = wave_s * 16 + lane;
      const uint32_t lb = is_self ? lbytes : plbytes;
      const uint32_t off = q < nvalid ? (uint32_t)(r0 + q * rstride) * 4 : lb;
      dma_lds4(make_rsrc(is_self ? a.lse_k : a.pack_lse_k, lb), Ld + wave_s * 16, off, 0);
      dma_lds4(make_rsrc(is_self ? a.delta : a.pack_delta, lb), Ld + kRows + wave_s * 16, off, 0);
    }
  };
  const uint32_t kq0 = swz_b128_base<DP>(lane);
  const uint32_t trb0 = swz_tr_base<DP>(lane, 0), trb1 = swz_tr_base<DP>(lane, 1);
  const float nc2 = -a.scale_log2;

  // B operands (column = key, k = d), negated: with the accumulators started
  // at the row's lse_k and delta, the MFMAs produce lse_k - S and delta - dP
  u16x8_t kf[NKS], vf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = ks * 16 + hh * 8;
    const bool ok = mykey < c_hi && d < D;
    const int64_t off = ((int64_t)mykey * a.Hkv + kh) * D + d;
    kf[ks] = neg8(ok ? ld8(a.k + off) : zero8());
    vf[ks] = neg8(ok ? ld8(a.v + off) : zero8());
  }
  // K / V rows must have landed before the tile loads start: the compiler's
  // own waits for them would otherwise also drain the tile loads in flight
  wait_vmcnt<0>();
  f32x16_t dk[NDB], dv[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) { dk[i] = zero16(); dv[i] = zero16(); }

  auto compute = [&](const uint16_t* Qb, const uint16_t* Gb, const float* Lb, const int it,
                     auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const uint32_t kq = opaque(kq0), t0 = opaque(trb0), t1 = opaque(trb1);
    const bool is_self = it < G * n_self;
    const int sq0 = is_self ? self_begin + (it % n_self) * kRows : 0;
    // D layout: lane holds rows 8j + 4hh + i of block qb
    f32x16_t sp[QB], dp[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r0 = qb * 32 + 8 * j + 4 * hh;
        const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(Lb + r0);
        const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(Lb + kRows + r0);
#pragma unroll
        for (int i = 0; i < 4; ++i) { sp[qb][4 * j + i] = l4[i]; dp[qb][4 * j + i] = d4[i]; }
      }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const uint32_t o = qb * 32 * DP * 2 + swz_b128<DP>(kq, ks);
        sp[qb] = mfma32<DT>(lds8(Qb, o), kf[ks], sp[qb]);
        dp[qb] = mfma32<DT>(lds8(Gb, o), vf[ks], dp[qb]);
      }
    // P and -dS as A operands: P = exp2(c2 (S - lse_k)), -dS = P (delta - dP)
    u16x8_t pa[QB][2], da[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r0 = qb * 32 + 8 * j + 4 * hh;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float p = fast_exp2(sp[qb][4 * j + i] * nc2);
          if constexpr (MASK) p = (mykey < c_hi && (!is_self || mykey <= sq0 + r0 + i)) ? p : 0.0f;
          pa[qb][j >> 1][(j & 1) * 4 + i] = from_f32<DT>(p);
          da[qb][j >> 1][(j & 1) * 4 + i] = from_f32<DT>(p * dp[qb][4 * j + i]);
        }
      }
#pragma unroll
    for (int i = 0; i < NDB; ++i)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint32_t ro = (qb * 32 + t * 16) * DP * 2;
          const uint32_t x0 = ro + swz_tr<DP>(t0, i), x1 = ro + swz_tr<DP>(t1, i);
          dv[i] = mfma32<DT>(pa[qb][t], lds_tr8(Gb, x0, x1), dv[i]);
          dk[i] = mfma32<DT>(da[qb][t], lds_tr8(Qb, x0, x1), dk[i]);
        }
  };
  auto run = [&](const uint16_t* Qb, const uint16_t* Gb, const float* Lb, const int it) __attribute__((always_inline)) {
    const bool is_self = it < G * n_self;
    const int sq0 = is_self ? self_begin + (it % n_self) * kRows : 0;
    // causal rows that end before the wave's first key contribute nothing
    if (is_self && sq0 + kRows - 1 < wkey0) return;
    const bool need_mask = (wkey0 + kWaveKeys > c_hi) || (is_self && sq0 < wkey0 + kWaveKeys - 1);
    if (need_mask) compute(Qb, Gb, Lb, it, std::true_type{});
    else compute(Qb, Gb, Lb, it, std::false_type{});
  };
  // Stage k of tile it is (it - it_lo) % 3.  Loads run two tiles ahead; after
  // computing tile it, each wave waits until its loads of tile it + 1 landed
  // (the loads of tile it + 2 stay in flight), then the barrier.
  auto step = [&](uint16_t* Qc, uint16_t* Gc, float* Lc, uint16_t* Qn, uint16_t* Gn, float* Ln,
                  int it) __attribute__((always_inline)) {
    dma(Qn, Gn, Ln, it + 2);
    run(Qc, Gc, Lc, it);
    wait_vmcnt<kLoadsPerTile>();
    lds_barrier();
  };
  dma(Q0, G0, L0, it_lo);
  dma(Q1, G1, L1, it_lo + 1);
  wait_vmcnt<kLoadsPerTile>();
  lds_barrier();
  for (int it = it_lo; it < it_hi; it += 3) {
    step(Q0, G0, L0, Q2, G2, L2, it);
    if (it + 1 >= it_hi) break;
    step(Q1, G1, L1, Q0, G0, L0, it + 1);
    if (it + 2 >= it_hi) break;
    step(Q2, G2, L2, Q1, G1, L1, it + 2);
  }
  wait_vmcnt<0>();  // no loads in flight when the workgroup ends

  // D layout: lane holds column d = i*32 + qi, keys 8j + 4hh + r.  A row
  // split writes fp32 partials to its slot for the fixed-order reduction.
  float* pk = a.part_dkv + (int64_t)max(slot, 0) * kv_slot_floats(D);
  float* pv = pk + kKvTileKeys * D;
#pragma unroll
  for (int i = 0; i < NDB; ++i) {
    const int d = i * 32 + qi;
    if (d >= D) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = wkey0 + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (key >= c_hi) continue;
      const int64_t o = ((int64_t)key * a.Hkv + kh) * D + d;
      if (slot >= 0) {
        pk[(key - key0) * D + d] = -dk[i][r];
        pv[(key - key0) * D + d] = dv[i][r];
      } else {
        a.dk[o] = from_f32<DT>(dk[i][r] * -a.scale);
        a.dv[o] = from_f32<DT>(dv[i][r]);
      }
    }
  }
}

}  // namespace

template <int DT, int DP> void launch_dkdv1(const BwdArgs& a, int n_wg, hipStream_t st) {
  hipLaunchKernelGGL((dkdv1_kernel<DT, DP>), dim3(n_wg), dim3(256), 0, st, a);
}

template void launch_dkdv1<0, 32>(const BwdArgs&, int, hipStream_t);
template void launch_dkdv1<0, 64>(const BwdArgs&, int, hipStream_t);
template void launch_dkdv1<1, 32>(const BwdArgs&, int, hipStream_t);
template void launch_dkdv1<1, 64>(const BwdArgs&, int, hipStream_t);

}  // namespace moba
