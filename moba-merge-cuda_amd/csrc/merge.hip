// Standalone deterministic global-softmax merge of caller-owned partials.
//
// Replaces merge_forward (src/moba_opt/ops/bindings.cpp:6-22,
// src/moba_opt/ops/merge.cu:187-288): row p of the output combines the self
// partial (self_out[p], self_lse[p]) with every remote partial j whose
// mapping[j] == p,
//     m = max(l_self, l_j),  w = exp(l - m),  z = sum_j w_j + w_self,
//     O = (w_self o_self + sum_j w_j o_j) / z,  L = m + log z,
// O in the input dtype, L fp32 natural log.  The reference builds per-row
// slot lists with atomic tickets (order depends on timing) and, in its
// deterministic mode, sorts each row's slots afterwards.  Here there are no
// atomics anywhere: the contributions are ordered by a stable LSD radix sort
// on the row key (8-bit digits; stable ranks from wave ballots, per-wave and
// per-tile counts combined in wave / tile order), so each row's remote
// partials form one contiguous run in ascending j, found by a binary search
// per row.  The merge runs one wave64 per row with wave reductions (shuffle
// xor, lowered to DPP / ds_swizzle) for the max and the weight sum; lanes
// cover D with 4 consecutive elements each.  Results are bitwise repeatable.
//
// Launch sequence on the stream (all sizes from the arguments; the host
// never waits): init (status words, keys) -> per digit pass: tile
// histograms, one-workgroup exclusive scan, stable scatter -> run starts
// (binary search per row) -> merge.  status[0] = 1 when a mapping entry is
// outside [0, T*H) (such entries are ignored), status[1] = 1 when a row has
// more than kmax remote partials (only the first kmax, in j order, are used);
// the caller reads them after the stream reaches them.
#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {

constexpr int kTile = 1024;        // contributions per radix tile
constexpr int kRadixThreads = 256; // 4 waves, 4 sub-rounds of 256 per tile
constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(256) void merge_init_kernel(const int64_t* __restrict__ mapping,
                                                         int64_t n, int64_t P, int* keys,
                                                         int* vals, int* status) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j == 0) { status[0] = 0; status[1] = 0; }
  if (j >= n) return;
  const int64_t p = mapping[j];
  keys[j] = (p >= 0 && p < P) ? (int)p : (int)P;  // out of range: sorted past every row
  vals[j] = (int)j;
}

// Stable ranks of the 256 elements of one sub-round: `peers` = lanes of this
// wave holding the same digit (lanes without an element hold none), built
// from 8 ballots over the digit bits.
MOBA_DEV uint64_t digit_peers(int digit, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (digit >> b) & 1;
    const uint64_t bal = __ballot(bit);
    peers &= bit ? bal : ~bal;
  }
  return valid ? peers : 0ull;
}

// One tile's per-digit counts (HIST) or stable scatter (SCATTER).
template <bool SCATTER>
__global__ __launch_bounds__(kRadixThreads) void radix_tile_kernel(
    const int* __restrict__ keys, const int* __restrict__ vals, int64_t n, int shift, int nb,
    int* __restrict__ hist, int* __restrict__ out_keys, int* __restrict__ out_vals) {
  __shared__ int wcount[4][256];   // per-wave digit counts of the current sub-round
  __shared__ int before[256];      // digit counts of the tile's earlier sub-rounds
  __shared__ int base[256];        // SCATTER: global start of (digit, tile)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, b = blockIdx.x;
  before[tid] = 0;
  if (SCATTER) base[tid] = hist[(int64_t)tid * nb + b];
  for (int r = 0; r < kTile / kRadixThreads; ++r) {
    const int64_t e = (int64_t)b * kTile + r * kRadixThreads + tid;
    const bool valid = e < n;
    const int key = valid ? keys[e] : 0;
    const int digit = (key >> shift) & 255;
#pragma unroll
    for (int i = 0; i < 4; ++i) wcount[i][tid] = 0;
    __syncthreads();
    const uint64_t peers = digit_peers(digit, valid);
    const int lower = __popcll(peers & ((1ull << lane) - 1ull));
    if (valid && lower == 0) wcount[w][digit] = __popcll(peers);  // one writer per digit
    __syncthreads();
    if (SCATTER && valid) {
      int rank = base[digit] + before[digit] + lower;
      for (int i = 0; i < w; ++i) rank += wcount[i][digit];
      out_keys[rank] = key;
      out_vals[rank] = vals[e];
    }
    __syncthreads();
    before[tid] += wcount[0][tid] + wcount[1][tid] + wcount[2][tid] + wcount[3][tid];
    __syncthreads();
  }
  if (!SCATTER) hist[(int64_t)tid * nb + b] = before[tid];
}

// Exclusive scan of hist[count] in place, one workgroup: each thread sums a
// contiguous run, the run totals are scanned in LDS, then each run is
// rewritten with its offsets.
__global__ __launch_bounds__(kScanThreads) void radix_scan_kernel(int* hist, int64_t count) {
  __shared__ int tot[kScanThreads];
  const int tid = threadIdx.x;
  const int64_t per = (count + kScanThreads - 1) / kScanThreads;
  const int64_t lo = min(count, tid * per), hi = min(count, lo + per);
  int s = 0;
  for (int64_t i = lo; i < hi; ++i) s += hist[i];
  tot[tid] = s;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {  // Hillis-Steele inclusive scan
    const int x = tid >= off ? tot[tid - off] : 0;
    __syncthreads();
    tot[tid] += x;
    __syncthreads();
  }
  int run = tot[tid] - s;
  for (int64_t i = lo; i < hi; ++i) {
    const int c = hist[i];
    hist[i] = run;
    run += c;
  }
}

// start[r] = first sorted position whose key >= r, for r in [0, P]; flags
// out-of-range keys (sorted last, key P).
__global__ __launch_bounds__(256) void run_starts_kernel(const int* __restrict__ keys, int64_t n,
                                                         int64_t P, int* __restrict__ start,
                                                         int* status) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r > P) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < r) lo = mid + 1; else hi = mid;
  }
  start[r] = (int)lo;
  if (r == P && lo < n) status[0] = 1;
}

template <int DT>
MOBA_DEV void load4(const void* base, int64_t off, float (&x)[4]) {
  if constexpr (DT == 2) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = v[e];
  } else {
    const u16x4_t v = *reinterpret_cast<const u16x4_t*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = to_f32<DT>(v[e]);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void merge_rows_kernel(
    const void* __restrict__ self_out, const float* __restrict__ self_lse,
    const void* __restrict__ remote_out, const float* __restrict__ remote_lse,
    const int* __restrict__ sorted_vals, const int* __restrict__ start, int64_t P, int D,
    int kmax, int* status, void* __restrict__ out, float* __restrict__ lse) {
  const int lane = threadIdx.x & 63;
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // one wave per row
  if (p >= P) return;
  const int lo = start[p], n_all = start[p + 1] - lo;
  if (n_all > kmax && lane == 0) status[1] = 1;
  const int cnt = min(n_all, kmax);  // kmax <= 8 <= 64 lanes
  const float l_self = self_lse[p];
  int idx = 0;
  float l_j = -INFINITY;
  if (lane < cnt) {
    idx = sorted_vals[lo + lane];
    l_j = remote_lse[idx];
  }
  const float m = wave_max(fmaxf(l_self, l_j));
  const float w_self = expf(l_self - m);
  const float w_j = lane < cnt ? expf(l_j - m) : 0.0f;
  const float z = wave_sum(w_j) + w_self;  // remote weights first, then self
  const int d = lane * 4;
  const bool dok = d < D;
  const int dl = dok ? d : 0;
  float acc[4], x[4];
  load4<DT>(self_out, p * D + dl, x);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = x[e] * w_self;
  for (int j = 0; j < cnt; ++j) {
    const float wb = __shfl(w_j, j, 64);
    const int ib = __shfl(idx, j, 64);
    load4<DT>(remote_out, (int64_t)ib * D + dl, x);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += wb * x[e];
  }
  const float iz = 1.0f / z;
  if (dok) {
    if constexpr (DT == 2) {
      f32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = acc[e] * iz;
      *reinterpret_cast<f32x4_t*>(static_cast<float*>(out) + p * D + d) = o;
    } else {
      u16x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = from_f32<DT>(acc[e] * iz);
      *reinterpret_cast<u16x4_t*>(static_cast<uint16_t*>(out) + p * D + d) = o;
    }
  }
  if (lane == 0) lse[p] = m + logf(z);
}

struct MergeWork {
  int *ka, *va, *kb, *vb, *hist, *start;
  int64_t bytes;
};

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

MergeWork carve(void* base, int64_t P, int64_t n) {
  const int64_t nb = (n + kTile - 1) / kTile;
  const int64_t e = align256(4 * std::max<int64_t>(n, 1));
  MergeWork w;
  char* c = static_cast<char*>(base);
  w.ka = (int*)c; w.va = (int*)(c + e); w.kb = (int*)(c + 2 * e); w.vb = (int*)(c + 3 * e);
  w.hist = (int*)(c + 4 * e);
  const int64_t h = align256(4 * 256 * std::max<int64_t>(nb, 1));
  w.start = (int*)(c + 4 * e + h);
  w.bytes = 4 * e + h + align256(4 * (P + 1));
  return w;
}

}  // namespace

extern "C" int64_t moba_hip_merge_work(int64_t P, int64_t M) {
  if (P < 1 || M < 0 || P >= INT32_MAX || M >= INT32_MAX) return -1;
  char dummy;
  return carve(&dummy, P, M).bytes;
}

extern "C" int moba_hip_merge(const void* self_out, const float* self_lse, const void* remote_out,
                              const float* remote_lse, const int64_t* mapping, int dtype,
                              int64_t T, int H, int D, int64_t M, int kmax, void* work,
                              int* status, void* out, float* lse, void* stream) {
  if (dtype < 0 || dtype > 2) { moba_set_error("merge: dtype must be 0 (bf16), 1 (fp16) or 2 (fp32)"); return MOBA_ERR_ARG; }
  if (T < 1 || H < 1) { moba_set_error("merge: nonempty T,H required"); return MOBA_ERR_ARG; }
  if (D < 8 || D > 256 || D % 8) { moba_set_error("merge: head_dim must be a multiple of 8 in [8,256]"); return MOBA_ERR_ARG; }
  if (kmax < 1 || kmax > 8) { moba_set_error("merge: kmax must be in [1,8]"); return MOBA_ERR_ARG; }
  const int64_t P = T * H;
  if (P >= INT32_MAX || M < 0 || M >= INT32_MAX) { moba_set_error("merge: mapping exceeds int32 indexing capacity"); return MOBA_ERR_ARG; }
  if (!self_out || !self_lse || !out || !lse || !status || !work || (M > 0 && (!remote_out || !remote_lse || !mapping))) {
    moba_set_error("merge: null buffer");
    return MOBA_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  MergeWork w = carve(work, P, M);
  const int64_t nb = (M + kTile - 1) / kTile;
  hipLaunchKernelGGL(merge_init_kernel, dim3((unsigned)std::max<int64_t>(1, (M + 255) / 256)),
                     dim3(256), 0, st, mapping, M, P, w.ka, w.va, status);
  int *k = w.ka, *v = w.va, *k2 = w.kb, *v2 = w.vb;
  if (M > 0) {
    int bits = 1;
    while (bits < 31 && (P >> bits) != 0) ++bits;  // keys lie in [0, P]
    for (int shift = 0; shift < bits; shift += 8) {
      hipLaunchKernelGGL((radix_tile_kernel<false>), dim3((unsigned)nb), dim3(kRadixThreads), 0,
                         st, k, v, M, shift, (int)nb, w.hist, nullptr, nullptr);
      hipLaunchKernelGGL(radix_scan_kernel, dim3(1), dim3(kScanThreads), 0, st, w.hist, 256 * nb);
      hipLaunchKernelGGL((radix_tile_kernel<true>), dim3((unsigned)nb), dim3(kRadixThreads), 0,
                         st, k, v, M, shift, (int)nb, w.hist, k2, v2);
      std::swap(k, k2);
      std::swap(v, v2);
    }
  }
  hipLaunchKernelGGL(run_starts_kernel, dim3((unsigned)((P + 1 + 255) / 256)), dim3(256), 0, st,
                     k, M, P, w.start, status);
  const dim3 grid((unsigned)((P + 3) / 4));
  if (dtype == 0)
    hipLaunchKernelGGL(merge_rows_kernel<0>, grid, dim3(256), 0, st, self_out, self_lse,
                       remote_out, remote_lse, v, w.start, P, D, kmax, status, out, lse);
  else if (dtype == 1)
    hipLaunchKernelGGL(merge_rows_kernel<1>, grid, dim3(256), 0, st, self_out, self_lse,
                       remote_out, remote_lse, v, w.start, P, D, kmax, status, out, lse);
  else
    hipLaunchKernelGGL(merge_rows_kernel<2>, grid, dim3(256), 0, st, self_out, self_lse,
                       remote_out, remote_lse, v, w.start, P, D, kmax, status, out, lse);
  return moba_launch_status("merge");
}
