// Argument block of the prefill backward kernels (attn_bwd.hip, attn_dkdv.hip,
// attn_dkdv2.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moba {

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
  int n_self_wg;        // self workgroups: entries of self_tiles x G
  const int* kv_tiles;
  const int* sel;
  int R;
  const int* filtered;
  int E;
  const int* tile_off;
  const int* row_off;
  const int* counts;
  const int* rows;
  // delta and lse_k are one allocation, lse_k = delta + T*Hq (the key-major
  // kernels fetch both of a row with one load); likewise pack_delta =
  // pack_lse_k + pack_rows
  float* delta;      // [T*Hq] rowsum(dO * O)
  float* lse_k;      // [T*Hq] lse / scale: the row's log-sum-exp in q.k units
  uint16_t* part_dq;  // remote dQ slots, input dtype
  // Row-split schedule (kv_splits > 1, built on the device by
  // dkdv_sched_kernel): kv_sched[4 * workgroup] = (kv tile, first row tile,
  // end row tile, partial slot or -1 to write dK / dV directly), tile -1 for
  // an idle workgroup; kv_seg[2 * kv tile] = (first slot, slots).  part_dkv
  // holds per slot [dK | dV][128 keys][D] fp32, summed by dkdv_reduce_kernel.
  const int* kv_sched;
  const int* kv_seg;
  float* part_dkv;
  int kv_splits;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  // Expert rows packed contiguously in row_off order for the key-major
  // kernel: pack_rows (= T*Hq*R) rows of q, dO, lse_k and delta, written by
  // the remote dq kernel.
  uint16_t* pack_q;
  uint16_t* pack_g;
  float* pack_lse_k;
  float* pack_delta;
  int64_t pack_rows;
};

// Key-major dK/dV launches over n_wg workgroups: one per kv tile of 128 keys,
// or, with a row-split schedule, one per schedule entry.
// dkdv1 (attn_dkdv.hip): all four products per wave, head dims <= 64.
// dkdv2 (attn_dkdv2.hip): wave pairs with split roles, head dims 65..128.
template <int DT, int DP> void launch_dkdv1(const BwdArgs& a, int n_wg, hipStream_t st);
template <int DT, int DP> void launch_dkdv2(const BwdArgs& a, int n_wg, hipStream_t st);

// Keys per dK/dV workgroup (every key-major kernel) and the size of one
// partial slot in floats.
constexpr int kKvTileKeys = 128;
__host__ __device__ inline int64_t kv_slot_floats(int D) { return (int64_t)2 * kKvTileKeys * D; }

// Work of one dK/dV workgroup: its kv tile entry and row-tile range, and the
// partial slot it writes (-1: dK / dV directly).  Returns false for an idle
// workgroup.  Unscheduled launches take tile blockIdx.x and all its rows.
__device__ inline bool kv_work(const BwdArgs& a, int& tile, int& lo, int& hi, int& slot) {
  if (a.kv_sched == nullptr) {
    tile = blockIdx.x; lo = 0; hi = 0x7fffffff; slot = -1;
    return true;
  }
  const int* w = a.kv_sched + 4 * blockIdx.x;
  tile = w[0]; lo = w[1]; hi = w[2]; slot = w[3];
  return tile >= 0;
}

}  // namespace moba
