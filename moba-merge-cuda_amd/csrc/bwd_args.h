// Argument block of the prefill backward kernels (attn_bwd.hip, attn_dkdv.hip).
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
  const int* kv_tiles;
  const int* sel;
  int R;
  const int* filtered;
  int E;
  const int* tile_off;
  const int* row_off;
  const int* counts;
  const int* rows;
  float* delta;      // [T*Hq] rowsum(dO * O)
  float* lse2;       // [T*Hq] lse * log2(e)
  float* part_dq;
  float* part_dkv;   // [kv_splits][2][T, Hkv, D] fp32 when kv_splits > 1
  int kv_splits;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  // Expert rows packed contiguously in row_off order for the key-major
  // kernel: pack_rows (= T*Hq*R) rows of q, dO, lse2 and delta.
  uint16_t* pack_q;
  uint16_t* pack_g;
  float* pack_lse2;
  float* pack_delta;
  int64_t pack_rows;
};

// Key-major dK/dV with all four products per wave (attn_dkdv.hip), head dims <= 64:
// launches the kernel over n_kv key tiles of 128 keys x kv_splits row splits.
template <int DT, int DP> void launch_dkdv1(const BwdArgs& a, int n_kv, hipStream_t st);
template <int DT, int DP> void launch_dkdv2(const BwdArgs& a, int n_kv, hipStream_t st);

}  // namespace moba
