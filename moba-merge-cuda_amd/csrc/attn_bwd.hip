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
#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {

struct BwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* out;
  const uint16_t* dout;
  const float* lse;
  int T, Hq, Hkv, D, G;
  float scale, scale_log2;
  const int* cu_chunk;
  const int* self_tiles;
  const int* kv_tiles;
  const int* sel;
  int R;
  const int* filtered;
  int E;
  const int* tile_off;
  const int* row_off;
  const int* counts;
  const int* rows;
  float* delta;
  float* part_dq;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
};

constexpr int kBM = 128;  // dq: query rows per workgroup
constexpr int kBN = 64;   // dq: keys per LDS tile
constexpr int kBQ = 64;   // dkdv: query rows per LDS tile

// ------------------------------------------------------------------ delta
template <int DT>
__global__ __launch_bounds__(256) void delta_kernel(const uint16_t* __restrict__ o,
                                                    const uint16_t* __restrict__ g, int64_t rows,
                                                    int D, float* __restrict__ delta) {
  const int sub = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  float acc = 0.0f;
  if (row < rows) {
    for (int d = sub * 8; d < D; d += 128) {
      const u16x8_t a = ld8(o + row * D + d), b = ld8(g + row * D + d);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += to_f32<DT>(a[e]) * to_f32<DT>(b[e]);
    }
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (row < rows && sub == 0) delta[row] = acc;
}

// --------------------------------------------------------------------- dq
template <int DT, int DP, bool REMOTE>
__global__ __launch_bounds__(256, 1) void dq_kernel(BwdArgs a) {
  constexpr int KS = DP + 8, TS = kBN + 8, NKS = DP / 16, NDB = DP / 32;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[kBN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Kt[DP * TS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int D = a.D;

  int s, h, kh, k_lo, k_hi, slot = 0;
  bool valid;
  if constexpr (REMOTE) {
    const int t = blockIdx.x;
    if (t >= a.tile_off[a.E]) return;
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
    const int local = (t - a.tile_off[e]) * kBM + wave * 32 + qi;
    valid = local < a.counts[e];
    slot = valid ? a.rows[a.row_off[e] + local] : 0;
    const int sh = slot / a.R;
    s = sh / a.Hq;
    h = sh % a.Hq;
  } else {
    const int c = a.self_tiles[2 * blockIdx.x], row0 = a.self_tiles[2 * blockIdx.x + 1];
    h = blockIdx.y;
    kh = h / a.G;
    k_lo = a.cu_chunk[c];
    const int c_end = a.cu_chunk[c + 1];
    k_hi = min(c_end, k_lo + row0 + kBM);
    s = k_lo + row0 + wave * 32 + qi;
    valid = s < c_end;
    if (!valid) s = k_hi - 1;
  }
  const int64_t row = (int64_t)s * a.Hq + h;
  u16x8_t qf[NKS], gf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = ks * 16 + hh * 8;
    const bool ok = valid && d < D;
    qf[ks] = ok ? ld8(a.q + row * D + d) : zero8();
    gf[ks] = ok ? ld8(a.dout + row * D + d) : zero8();
  }
  const float lse2 = valid ? a.lse[row] * kLog2e : INFINITY;
  const float dl = valid ? a.delta[row] : 0.0f;

  f32x16_t acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();

  for (int kt0 = k_lo; kt0 < k_hi; kt0 += kBN) {
    __syncthreads();
    for (int id = tid; id < kBN * (DP / 8); id += 256) {
      const int key = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      const int kg = kt0 + key;
      const bool ok = kg < k_hi && dc < D;
      const int64_t off = ((int64_t)kg * a.Hkv + kh) * D + dc;
      const u16x8_t kv = ok ? ld8(a.k + off) : zero8();
      const u16x8_t vv = ok ? ld8(a.v + off) : zero8();
      st8(&Ks[key * KS + dc], kv);
      st8(&Vs[key * KS + dc], vv);
      const int pos = (key & ~15) + kperm16(key & 15);
#pragma unroll
      for (int e = 0; e < 8; ++e) Kt[(dc + e) * TS + pos] = kv[e];
    }
    __syncthreads();

    u16x8_t dsv[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16_t sa = zero16(), pa = zero16();
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        sa = mfma32<DT>(ld8(&Ks[(kb * 32 + qi) * KS + ks * 16 + hh * 8]), qf[ks], sa);
        pa = mfma32<DT>(ld8(&Vs[(kb * 32 + qi) * KS + ks * 16 + hh * 8]), gf[ks], pa);
      }
      float tmp[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
        const bool ok = key < k_hi && (REMOTE || key <= s);
        const float p = ok ? exp2f(sa[r] * a.scale_log2 - lse2) : 0.0f;
        tmp[r] = p * (pa[r] - dl);
      }
      dsv[kb][0] = pack8<DT>(tmp);
      dsv[kb][1] = pack8<DT>(tmp + 8);
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          acc[db] = mfma32<DT>(ld8(&Kt[(db * 32 + qi) * TS + kb * 32 + t * 16 + hh * 8]),
                               dsv[kb][t], acc[db]);
  }
  if (!valid) return;

  if constexpr (REMOTE) {
    float* po = a.part_dq + (int64_t)slot * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = db * 32 + 8 * j + 4 * hh;
        if (d0 < D) {
          f32x4_t o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = acc[db][4 * j + i] * a.scale;
          *reinterpret_cast<f32x4_t*>(po + d0) = o;
        }
      }
  } else {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= a.scale;
    for (int jj = 0; jj < a.R; ++jj) {
      if (a.sel[row * a.R + jj] < 0) continue;
      const float* po = a.part_dq + (row * a.R + jj) * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d0 = db * 32 + 8 * j + 4 * hh;
          if (d0 < D) {
            const f32x4_t o = *reinterpret_cast<const f32x4_t*>(po + d0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[db][4 * j + i] += o[i];
          }
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
          for (int i = 0; i < 4; ++i) o[i] = from_f32<DT>(acc[db][4 * j + i]);
          *reinterpret_cast<u16x4_t*>(orow + d0) = o;
        }
      }
  }
}

// ------------------------------------------------------------------- dkdv
// DSPLIT waves share one 32-key block and split its d range (DP = 256 only),
// so a workgroup owns 128 / DSPLIT keys.
template <int DT, int DP, int DSPLIT>
__global__ __launch_bounds__(256, 1) void dkdv_kernel(BwdArgs a) {
  constexpr int QS = DP + 8, TS = kBQ + 8, NKS = DP / 16, NDB = DP / 32 / DSPLIT;
  constexpr int BK = 128 / DSPLIT;
  __shared__ __attribute__((aligned(16))) uint16_t Qs[kBQ * QS];
  __shared__ __attribute__((aligned(16))) uint16_t Gs[kBQ * QS];
  __shared__ __attribute__((aligned(16))) uint16_t Qt[DP * TS];
  __shared__ __attribute__((aligned(16))) uint16_t Gt[DP * TS];
  __shared__ float lse2s[kBQ], dels[kBQ];
  __shared__ int qpos[kBQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = lane & 31, hh = lane >> 5;
  const int kblk = wave / DSPLIT, dpart = wave % DSPLIT;
  const int D = a.D, G = a.G;
  const int c = a.kv_tiles[3 * blockIdx.x], kt0 = a.kv_tiles[3 * blockIdx.x + 1];
  const int f = a.kv_tiles[3 * blockIdx.x + 2];
  const int kh = blockIdx.y;
  const int c_lo = a.cu_chunk[c], c_hi = a.cu_chunk[c + 1];
  const int key0 = c_lo + kt0;                 // first key of the workgroup
  const int mykey = key0 + kblk * 32 + qi;     // this lane's key (B operand)
  const bool key_ok = mykey < c_hi;

  u16x8_t kf[NKS], vf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = ks * 16 + hh * 8;
    const int64_t off = ((int64_t)mykey * a.Hkv + kh) * D + d;
    kf[ks] = (key_ok && d < D) ? ld8(a.k + off) : zero8();
    vf[ks] = (key_ok && d < D) ? ld8(a.v + off) : zero8();
  }
  f32x16_t dka[NDB], dva[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) { dka[i] = zero16(); dva[i] = zero16(); }

  // query tiles: G * n_self causal tiles, then the expert's rows
  const int self_begin = key0;  // queries before the first key see none of them
  const int n_self_rows = max(0, c_hi - self_begin);
  const int n_self = (n_self_rows + kBQ - 1) / kBQ;
  const int e = (f >= 0 && a.R > 0) ? f * a.Hkv + kh : -1;
  const int n_rem_rows = e >= 0 ? a.counts[e] : 0;
  const int rbase = e >= 0 ? a.row_off[e] : 0;
  const int n_tiles = G * n_self + (n_rem_rows + kBQ - 1) / kBQ;

  for (int it = 0; it < n_tiles; ++it) {
    const bool is_self = it < G * n_self;
    __syncthreads();
    if (tid < kBQ) {
      int s = 0, h = 0;
      bool ok;
      if (is_self) {
        const int g = it / n_self, r0 = (it % n_self) * kBQ;
        s = self_begin + r0 + tid;
        h = kh * G + g;
        ok = s < c_hi;
      } else {
        const int local = (it - G * n_self) * kBQ + tid;
        ok = local < n_rem_rows;
        if (ok) {
          const int sh = a.rows[rbase + local] / a.R;
          s = sh / a.Hq;
          h = sh % a.Hq;
        }
      }
      const int64_t row = (int64_t)s * a.Hq + h;
      qpos[tid] = ok ? (int)row : -1;
      lse2s[tid] = ok ? a.lse[row] * kLog2e : INFINITY;
      dels[tid] = ok ? a.delta[row] : 0.0f;
    }
    __syncthreads();
    for (int id = tid; id < kBQ * (DP / 8); id += 256) {
      const int qr = id / (DP / 8), dc = (id % (DP / 8)) * 8;
      const int row = qpos[qr];
      const bool ok = row >= 0 && dc < D;
      const u16x8_t qv = ok ? ld8(a.q + (int64_t)row * D + dc) : zero8();
      const u16x8_t gv = ok ? ld8(a.dout + (int64_t)row * D + dc) : zero8();
      st8(&Qs[qr * QS + dc], qv);
      st8(&Gs[qr * QS + dc], gv);
      const int pos = (qr & ~15) + kperm16(qr & 15);
#pragma unroll
      for (int ee = 0; ee < 8; ++ee) {
        Qt[(dc + ee) * TS + pos] = qv[ee];
        Gt[(dc + ee) * TS + pos] = gv[ee];
      }
    }
    __syncthreads();
    const int sq0 = is_self ? self_begin + ((it % n_self) * kBQ) : 0;

    u16x8_t pv[2][2], dsv[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      f32x16_t sa = zero16(), pa = zero16();
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        sa = mfma32<DT>(ld8(&Qs[(qb * 32 + qi) * QS + ks * 16 + hh * 8]), kf[ks], sa);
        pa = mfma32<DT>(ld8(&Gs[(qb * 32 + qi) * QS + ks * 16 + hh * 8]), vf[ks], pa);
      }
      float pt[16], dt[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ql = qb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
        const bool ok = key_ok && (!is_self || mykey <= sq0 + ql);
        const float p = ok ? exp2f(sa[r] * a.scale_log2 - lse2s[ql]) : 0.0f;
        pt[r] = p;
        dt[r] = p * (pa[r] - dels[ql]);
      }
      pv[qb][0] = pack8<DT>(pt);
      pv[qb][1] = pack8<DT>(pt + 8);
      dsv[qb][0] = pack8<DT>(dt);
      dsv[qb][1] = pack8<DT>(dt + 8);
    }
#pragma unroll
    for (int i = 0; i < NDB; ++i) {
      const int db = dpart * NDB + i;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = (db * 32 + qi) * TS + qb * 32 + t * 16 + hh * 8;
          dva[i] = mfma32<DT>(pv[qb][t], ld8(&Gt[col]), dva[i]);
          dka[i] = mfma32<DT>(dsv[qb][t], ld8(&Qt[col]), dka[i]);
        }
    }
  }

  // dK/dV D-layout: lane holds column d = db*32 + qi, keys 8j + 4hh + i.
#pragma unroll
  for (int i = 0; i < NDB; ++i) {
    const int d = (dpart * NDB + i) * 32 + qi;
    if (d >= D) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = key0 + kblk * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (key < c_hi) {
        const int64_t off = ((int64_t)key * a.Hkv + kh) * D + d;
        a.dk[off] = from_f32<DT>(dka[i][r] * a.scale);
        a.dv[off] = from_f32<DT>(dva[i][r]);
      }
    }
  }
}

template <int DT, int DP>
int launch_bwd(const BwdArgs& a, int n_self, int n_kv, int max_remote, hipStream_t st) {
  const int64_t rows = (int64_t)a.T * a.Hq;
  hipLaunchKernelGGL(delta_kernel<DT>, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, st,
                     a.out, a.dout, rows, a.D, a.delta);
  if (max_remote > 0 && a.R > 0)
    hipLaunchKernelGGL((dq_kernel<DT, DP, true>), dim3(max_remote), dim3(256), 0, st, a);
  if (n_self > 0)
    hipLaunchKernelGGL((dq_kernel<DT, DP, false>), dim3(n_self, a.Hq), dim3(256), 0, st, a);
  if (n_kv > 0) {
    if constexpr (DP > 128)
      hipLaunchKernelGGL((dkdv_kernel<DT, DP, 2>), dim3(n_kv, a.Hkv), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((dkdv_kernel<DT, DP, 1>), dim3(n_kv, a.Hkv), dim3(256), 0, st, a);
  }
  return moba_launch_status("prefill_bwd");
}

template <int DT>
int dispatch_bwd(const BwdArgs& a, int n_self, int n_kv, int max_remote, hipStream_t st) {
  if (a.D <= 32) return launch_bwd<DT, 32>(a, n_self, n_kv, max_remote, st);
  if (a.D <= 64) return launch_bwd<DT, 64>(a, n_self, n_kv, max_remote, st);
  if (a.D <= 128) return launch_bwd<DT, 128>(a, n_self, n_kv, max_remote, st);
  return launch_bwd<DT, 256>(a, n_self, n_kv, max_remote, st);
}

}  // namespace

extern "C" int moba_hip_prefill_bwd(const void* q, const void* k, const void* v, const void* out,
                                    const void* dout, const float* lse, int dtype, int T, int Hq,
                                    int Hkv, int D, float scale, const int* cu_chunk,
                                    const int* self_tiles, int n_self_tiles, const int* kv_tiles,
                                    int n_kv_tiles, const int* sel, int R, const int* filtered,
                                    int E, const int* tile_off, const int* row_off,
                                    const int* counts, const int* rows, int max_remote_tiles,
                                    float* delta, float* part_dq, void* dq, void* dk, void* dv,
                                    void* stream) {
  if (dtype != 0 && dtype != 1) { moba_set_error("prefill_bwd: dtype must be 0 (bf16) or 1 (fp16)"); return MOBA_ERR_ARG; }
  if (D < 8 || D > 256 || D % 8) { moba_set_error("prefill_bwd: head_dim must be a multiple of 8 in [8,256]"); return MOBA_ERR_ARG; }
  if (Hq < 1 || Hkv < 1 || Hq % Hkv) { moba_set_error("prefill_bwd: Hq must be a positive multiple of Hkv"); return MOBA_ERR_ARG; }
  if (R < 0 || R > 8) { moba_set_error("prefill_bwd: remote count must be in [0,8]"); return MOBA_ERR_ARG; }
  BwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.out = (const uint16_t*)out; a.dout = (const uint16_t*)dout; a.lse = lse;
  a.T = T; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.G = Hq / Hkv;
  a.scale = scale; a.scale_log2 = scale * kLog2e;
  a.cu_chunk = cu_chunk; a.self_tiles = self_tiles; a.kv_tiles = kv_tiles;
  a.sel = sel; a.R = R; a.filtered = filtered; a.E = E;
  a.tile_off = tile_off; a.row_off = row_off; a.counts = counts; a.rows = rows;
  a.delta = delta; a.part_dq = part_dq;
  a.dq = (uint16_t*)dq; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
  hipStream_t st = (hipStream_t)stream;
  const int mr = R > 0 ? max_remote_tiles : 0;
  return dtype == 0 ? dispatch_bwd<0>(a, n_self_tiles, n_kv_tiles, mr, st)
                    : dispatch_bwd<1>(a, n_self_tiles, n_kv_tiles, mr, st);
}
