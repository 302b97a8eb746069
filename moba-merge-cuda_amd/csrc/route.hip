// Prefill routing: chunk-mean key pooling, FP32 gate scores, stable top-k, and
// the expert-major packing of the selected (query, head) rows.
//
// Replaces the torch routing ops of src/moba_opt/grouped_attention.py:48-94
// (stack/index_select, mean, einsum, mask, topk/argmax loop, nonzero packing).
// The arithmetic order is the canonical one of the CPU oracle, so the selected
// block sets are bit-identical to it:
//   mean  = canonical fp32 sum over the chunk's tokens (64 strided partial
//           sums + fixed pairwise tree), / C  (optionally rounded to the
//           input dtype: route_precision "upstream")
//   gate  = fma chain over d = 0..D-1 in fp32
//   top-k = descending gate, exact ties -> lowest chunk, -inf never chosen.
#include "common.h"
#include "../../include/moba_hip.h"

using namespace moba;

namespace {

constexpr int kMaxRemote = 8;

// One wave per (filtered chunk, kv head, 8 consecutive d): lane j sums the
// tokens j, j+64, ... (16-byte loads), then the canonical tree.
template <int DT>
__global__ __launch_bounds__(64) void chunk_means_kernel(const uint16_t* __restrict__ k, int Hkv,
                                                         int D, const int* __restrict__ chunk_start,
                                                         int C, int precision,
                                                         float* __restrict__ means) {
  const int nd8 = D / 8;
  const int db = blockIdx.x % nd8;
  const int kh = (blockIdx.x / nd8) % Hkv;
  const int f = blockIdx.x / (nd8 * Hkv);
  const int lane = threadIdx.x;
  const uint16_t* p = k + ((int64_t)chunk_start[f] * Hkv + kh) * D + db * 8;
  const int64_t stride = (int64_t)Hkv * D;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  for (int t = lane; t < C; t += 64) {
    const u16x8_t x = ld8(p + t * stride);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = acc[e] + to_f32<DT>(x[e]);
  }
  float out[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float m = canon_tree(acc[e]) / (float)C;
    if (precision == 0) m = to_f32<DT>(from_f32<DT>(m));
    out[e] = m;
  }
  if (lane == 0) {
    float* dst = means + ((int64_t)f * Hkv + kh) * D + db * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e] = out[e];
  }
}

// One thread per (token, q head); heads fastest so a wave reads adjacent q rows.
template <int DT>
__global__ void route_kernel(const uint16_t* __restrict__ q, int T, int Hq, int Hkv, int D,
                             const float* __restrict__ means, const int* __restrict__ cu_chunk,
                             int nchunk, const int* __restrict__ chunk_batch,
                             const int* __restrict__ first_chunk, int R, int F,
                             int* __restrict__ sel, float* __restrict__ gate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)T * Hq) return;
  const int s = (int)(idx / Hq), h = (int)(idx % Hq);
  const int G = Hq / Hkv, kh = h / G;
  // chunk containing s
  int lo = 0, hi = nchunk - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu_chunk[mid] <= s) lo = mid; else hi = mid - 1;
  }
  const int cs = lo, b = chunk_batch[cs], c0 = first_chunk[cs];
  const uint16_t* qr = q + idx * D;

  float val[kMaxRemote];
  int ix[kMaxRemote];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kMaxRemote; ++j) { val[j] = -INFINITY; ix[j] = -1; }

  for (int c = c0; c < cs; ++c) {
    const float* mr = means + ((int64_t)(c - b) * Hkv + kh) * D;
    float acc = 0.0f;
    for (int d = 0; d < D; d += 8) {
      u16x8_t qv = ld8(qr + d);
      f32x4_t m0 = *reinterpret_cast<const f32x4_t*>(mr + d);
      f32x4_t m1 = *reinterpret_cast<const f32x4_t*>(mr + d + 4);
      acc = fmaf(m0[0], to_f32<DT>(qv[0]), acc);
      acc = fmaf(m0[1], to_f32<DT>(qv[1]), acc);
      acc = fmaf(m0[2], to_f32<DT>(qv[2]), acc);
      acc = fmaf(m0[3], to_f32<DT>(qv[3]), acc);
      acc = fmaf(m1[0], to_f32<DT>(qv[4]), acc);
      acc = fmaf(m1[1], to_f32<DT>(qv[5]), acc);
      acc = fmaf(m1[2], to_f32<DT>(qv[6]), acc);
      acc = fmaf(m1[3], to_f32<DT>(qv[7]), acc);
    }
    if (gate) gate[((int64_t)(c - b) * Hq + h) * T + s] = acc;
    // stable insertion into the descending list: equal scores stay behind the
    // earlier (lower) chunk, so exact ties resolve to the lowest index.
    if (cnt == R && !(acc > val[R - 1])) continue;
    int pos = 0;
#pragma unroll
    for (int j = 0; j < kMaxRemote; ++j) pos += (j < cnt && val[j] >= acc);
#pragma unroll
    for (int j = kMaxRemote - 1; j >= 1; --j)
      if (j > pos && j < R) { val[j] = val[j - 1]; ix[j] = ix[j - 1]; }
#pragma unroll
    for (int j = 0; j < kMaxRemote; ++j)
      if (j == pos) { val[j] = acc; ix[j] = c; }
    if (cnt < R) cnt++;
  }
  // ascending chunk order for the slot list (static sorting network)
#pragma unroll
  for (int pass = 0; pass < kMaxRemote; ++pass) {
#pragma unroll
    for (int j = 0; j + 1 < kMaxRemote; ++j) {
      if (j + 1 < cnt && ix[j] > ix[j + 1]) { int t = ix[j]; ix[j] = ix[j + 1]; ix[j + 1] = t; }
    }
  }
  int* out = sel + idx * R;
  for (int j = 0; j < R; ++j) out[j] = j < cnt ? ix[j] : -1;
}

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---- expert packing ------------------------------------------------------
// Expert e = f*Hkv + kvh (reference order: (chunk, kv head)).  Its candidate
// rows are (g, s) for g in the kv group and s from the chunk end to the
// sequence end, enumerated g-major like the reference's nonzero over
// [F*Hkv, G*T] (grouped_attention.py:78-80).

MOBA_DEV int find_slot(const int* __restrict__ sel, int64_t row, int R, int c) {
  const int* p = sel + row * R;
  for (int j = 0; j < R; ++j) if (p[j] == c) return j;
  return -1;
}

struct ExpertRange { int c, kh, s0, ns, G; };

MOBA_DEV ExpertRange expert_range(int e, int Hq, int Hkv, const int* cu_chunk,
                                  const int* chunk_batch, const int* cu_seqlens,
                                  const int* filtered) {
  ExpertRange r;
  const int f = e / Hkv;
  r.kh = e % Hkv;
  r.c = filtered[f];
  r.s0 = cu_chunk[r.c + 1];
  r.ns = cu_seqlens[chunk_batch[r.c] + 1] - r.s0;
  r.G = Hq / Hkv;
  return r;
}

__global__ __launch_bounds__(256) void expert_count_kernel(
    const int* __restrict__ sel, int Hq, int Hkv, int R, const int* __restrict__ cu_chunk,
    const int* __restrict__ chunk_batch, const int* __restrict__ cu_seqlens,
    const int* __restrict__ filtered, int* __restrict__ counts) {
  const int e = blockIdx.x;
  ExpertRange x = expert_range(e, Hq, Hkv, cu_chunk, chunk_batch, cu_seqlens, filtered);
  const int64_t n = (int64_t)x.G * x.ns;
  int cnt = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const int g = (int)(i / x.ns), s = x.s0 + (int)(i % x.ns);
    cnt += find_slot(sel, (int64_t)s * Hq + x.kh * x.G + g, R, x.c) >= 0;
  }
  __shared__ int part[4];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) part[w] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) counts[e] = part[0] + part[1] + part[2] + part[3];
}

// Exclusive scans of row counts and tile counts (one workgroup).
__global__ __launch_bounds__(1024) void expert_scan_kernel(const int* __restrict__ counts, int E,
                                                         int block_rows, int* __restrict__ row_off,
                                                         int* __restrict__ tile_off) {
  __shared__ int wr[16], wt[16];
  __shared__ int carry_r, carry_t;
  if (threadIdx.x == 0) { carry_r = 0; carry_t = 0; }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int base = 0; base < E; base += 1024) {
    const int e = base + threadIdx.x;
    int r = e < E ? counts[e] : 0;
    int t = (r + block_rows - 1) / block_rows;
    // inclusive wave scan
    int ir = r, it = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int yr = __shfl_up(ir, o, 64), yt = __shfl_up(it, o, 64);
      if (lane >= o) { ir += yr; it += yt; }
    }
    if (lane == 63) { wr[w] = ir; wt[w] = it; }
    __syncthreads();
    int pr = carry_r, pt = carry_t;
    for (int i = 0; i < w; ++i) { pr += wr[i]; pt += wt[i]; }
    if (e < E) { row_off[e] = pr + ir - r; tile_off[e] = pt + it - t; }
    __syncthreads();
    if (threadIdx.x == 1023) { carry_r = pr + ir; carry_t = pt + it; }
    __syncthreads();
  }
  if (threadIdx.x == 0) { row_off[E] = carry_r; tile_off[E] = carry_t; }
}

// Ordered compaction: rows[row_off[e] + rank] = ((s*Hq + h) << 3) | j (R <= 8).
__global__ __launch_bounds__(256) void expert_fill_kernel(
    const int* __restrict__ sel, int Hq, int Hkv, int R, const int* __restrict__ cu_chunk,
    const int* __restrict__ chunk_batch, const int* __restrict__ cu_seqlens,
    const int* __restrict__ filtered, const int* __restrict__ row_off, int* __restrict__ rows) {
  const int e = blockIdx.x;
  ExpertRange x = expert_range(e, Hq, Hkv, cu_chunk, chunk_batch, cu_seqlens, filtered);
  const int64_t n = (int64_t)x.G * x.ns;
  __shared__ int wtot[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int out = row_off[e];
  for (int64_t base = 0; base < n; base += 256) {
    const int64_t i = base + threadIdx.x;
    int slot = -1, h = 0, s = 0;
    if (i < n) {
      const int g = (int)(i / x.ns);
      s = x.s0 + (int)(i % x.ns);
      h = x.kh * x.G + g;
      slot = find_slot(sel, (int64_t)s * Hq + h, R, x.c);
    }
    const uint64_t mask = __ballot(slot >= 0);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wtot[w] = __popcll(mask);
    __syncthreads();
    int off = out;
    for (int k2 = 0; k2 < w; ++k2) off += wtot[k2];
    if (slot >= 0) rows[off + before] = (((s * Hq) + h) << 3) | slot;
    const int tot = wtot[0] + wtot[1] + wtot[2] + wtot[3];
    __syncthreads();
    out += tot;
  }
}

}  // namespace

extern "C" int moba_hip_chunk_means(const void* k, int dtype, int T, int Hkv, int D,
                                    const int* chunk_start, int F, int chunk, int precision,
                                    float* means, void* stream) {
  (void)T;
  if (F <= 0) return MOBA_OK;
  if (dtype != 0 && dtype != 1) { moba_set_error("chunk_means: dtype must be 0 (bf16) or 1 (fp16)"); return MOBA_ERR_ARG; }
  if (D < 8 || D % 8 || Hkv < 1 || chunk < 1) { moba_set_error("chunk_means: bad shape"); return MOBA_ERR_ARG; }
  dim3 grid((unsigned)((int64_t)F * Hkv * (D / 8))), block(64);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == 0)
    hipLaunchKernelGGL(chunk_means_kernel<0>, grid, block, 0, st, (const uint16_t*)k, Hkv, D,
                       chunk_start, chunk, precision, means);
  else
    hipLaunchKernelGGL(chunk_means_kernel<1>, grid, block, 0, st, (const uint16_t*)k, Hkv, D,
                       chunk_start, chunk, precision, means);
  return moba_launch_status("chunk_means");
}

extern "C" int moba_hip_route_prefill(const void* q, int dtype, int T, int Hq, int Hkv, int D,
                                      const float* means, const int* cu_chunk, int nchunk,
                                      const int* chunk_batch, const int* first_chunk, int R,
                                      int F, int* sel, float* gate, void* stream) {
  if (R < 1 || R > kMaxRemote) { moba_set_error("route_prefill: remote count must be in [1,8]"); return MOBA_ERR_ARG; }
  if (D % 8 || D < 8) { moba_set_error("route_prefill: head_dim must be a multiple of 8"); return MOBA_ERR_ARG; }
  if (Hq % Hkv) { moba_set_error("route_prefill: Hq must be a multiple of Hkv"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  if (gate) {
    const int64_t n = (int64_t)F * Hq * T;
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gate,
                       n, -INFINITY);
  }
  const int64_t n = (int64_t)T * Hq;
  dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (dtype == 0)
    hipLaunchKernelGGL(route_kernel<0>, grid, block, 0, st, (const uint16_t*)q, T, Hq, Hkv, D,
                       means, cu_chunk, nchunk, chunk_batch, first_chunk, R, F, sel, gate);
  else
    hipLaunchKernelGGL(route_kernel<1>, grid, block, 0, st, (const uint16_t*)q, T, Hq, Hkv, D,
                       means, cu_chunk, nchunk, chunk_batch, first_chunk, R, F, sel, gate);
  return moba_launch_status("route_prefill");
}

extern "C" int moba_hip_pack_experts(const int* sel, int T, int Hq, int Hkv, int R,
                                     const int* cu_chunk, const int* chunk_batch,
                                     const int* cu_seqlens, const int* filtered, int F,
                                     int block_rows, int* counts, int* row_off, int* tile_off,
                                     int* rows, void* stream) {
  (void)T;
  if (F <= 0) return MOBA_OK;
  if ((int64_t)T * Hq * R >= (1ll << 31) || (int64_t)T * Hq >= (1ll << 28)) { moba_set_error("pack_experts: T*Hq*R exceeds int32 or T*Hq exceeds 2^28"); return MOBA_ERR_ARG; }
  if (R > 8) { moba_set_error("pack_experts: at most 8 remote chunks per query"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  const int E = F * Hkv;
  hipLaunchKernelGGL(expert_count_kernel, dim3(E), dim3(256), 0, st, sel, Hq, Hkv, R, cu_chunk,
                     chunk_batch, cu_seqlens, filtered, counts);
  hipLaunchKernelGGL(expert_scan_kernel, dim3(1), dim3(1024), 0, st, counts, E, block_rows,
                     row_off, tile_off);
  hipLaunchKernelGGL(expert_fill_kernel, dim3(E), dim3(256), 0, st, sel, Hq, Hkv, R, cu_chunk,
                     chunk_batch, cu_seqlens, filtered, row_off, rows);
  return moba_launch_status("pack_experts");
}
