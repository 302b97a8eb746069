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

// One workgroup per (filtered chunk, kv head).  The mean of dim d is the
// canonical sum: 64 partial sums s_j over the tokens j, j+64, j+128, ... in
// increasing order, then the fixed tree canon_tree over j.  Work item
// (j, column block b) of 8 dims is p = j * nd8 + b, so a wave's loads cover
// whole rows (coalesced); thread t owns items t, t + 256, ...  The partials
// go through LDS to one wave per dim, lane j holding s_j, for the tree.
template <int DT, int NP>
__global__ __launch_bounds__(256) void chunk_means_kernel(const uint16_t* __restrict__ k, int Hkv,
                                                          int D, const int* __restrict__ chunk_start,
                                                          int C, int precision,
                                                          float* __restrict__ means) {
  extern __shared__ float part[];  // [64][D]
  const int nd8 = D / 8, np = 64 * nd8;
  const int kh = blockIdx.x % Hkv, f = blockIdx.x / Hkv;
  const int tid = threadIdx.x;
  const int64_t stride = (int64_t)Hkv * D;
  const uint16_t* base = k + ((int64_t)chunk_start[f] * Hkv + kh) * D;
  float acc[NP][8];
  int jj[NP], bb[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = tid + 256 * i;
    jj[i] = p < np ? p / nd8 : C;  // items past np load nothing
    bb[i] = p % nd8;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.0f;
  }
  for (int t0 = 0; t0 < C; t0 += 64) {
    u16x8_t x[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int t = t0 + jj[i];
      x[i] = t < C ? ld8(base + t * stride + bb[i] * 8) : zero8();
    }
#pragma unroll
    for (int i = 0; i < NP; ++i)
      if (t0 + jj[i] < C) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i][e] = acc[i][e] + to_f32<DT>(x[i][e]);
      }
  }
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = tid + 256 * i;
    if (p < np) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[jj[i] * D + bb[i] * 8 + e] = acc[i][e];
    }
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6;
  float* dst = means + ((int64_t)f * Hkv + kh) * D;
  for (int d = w; d < D; d += 4) {
    float m = canon_tree(part[lane * D + d]) / (float)C;
    if (precision == 0) m = to_f32<DT>(from_f32<DT>(m));
    if (lane == 0) dst[d] = m;
  }
}

// One thread per (token, q head): a workgroup takes 256 consecutive tokens of
// one head, so the means rows read in the candidate loop are the same for the
// whole wave, and the token's q row is read once into registers.
template <int DT, int DP>
__global__ __launch_bounds__(256) void route_kernel(const uint16_t* __restrict__ q, int T, int Hq,
                                                    int Hkv, int D,
                                                    const float* __restrict__ means,
                                                    const int* __restrict__ cu_chunk, int nchunk,
                                                    const int* __restrict__ chunk_batch,
                                                    const int* __restrict__ first_chunk, int R,
                                                    int F, int* __restrict__ sel,
                                                    float* __restrict__ gate) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  const int h = blockIdx.y;
  if (s >= T) return;
  const int G = Hq / Hkv, kh = h / G;
  // chunk containing s
  int lo = 0, hi = nchunk - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu_chunk[mid] <= s) lo = mid; else hi = mid - 1;
  }
  const int cs = lo, b = chunk_batch[cs], c0 = first_chunk[cs];
  const int64_t idx = (int64_t)s * Hq + h;
  constexpr int NQ = DP / 8;
  u16x8_t qv[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) qv[i] = i * 8 < D ? ld8(q + idx * D + i * 8) : zero8();

  float val[kMaxRemote];
  int ix[kMaxRemote];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kMaxRemote; ++j) { val[j] = -INFINITY; ix[j] = -1; }

  for (int c = c0; c < cs; ++c) {
    const float* mr = means + ((int64_t)(c - b) * Hkv + kh) * D;
    // sequential fma chain over d = 0 .. D-1
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      if (i * 8 >= D) break;
      const f32x4_t m0 = *reinterpret_cast<const f32x4_t*>(mr + i * 8);
      const f32x4_t m1 = *reinterpret_cast<const f32x4_t*>(mr + i * 8 + 4);
      acc = fmaf(m0[0], to_f32<DT>(qv[i][0]), acc);
      acc = fmaf(m0[1], to_f32<DT>(qv[i][1]), acc);
      acc = fmaf(m0[2], to_f32<DT>(qv[i][2]), acc);
      acc = fmaf(m0[3], to_f32<DT>(qv[i][3]), acc);
      acc = fmaf(m1[0], to_f32<DT>(qv[i][4]), acc);
      acc = fmaf(m1[1], to_f32<DT>(qv[i][5]), acc);
      acc = fmaf(m1[2], to_f32<DT>(qv[i][6]), acc);
      acc = fmaf(m1[3], to_f32<DT>(qv[i][7]), acc);
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

// Candidates of an expert are split in blocks of kCandBlock; workgroup
// (e, b) handles block b of expert e.  Block counts go to work[e * nbmax + b]
// and become exclusive offsets within the expert in the scan, so the fill is
// an ordered compaction with no atomics.
constexpr int kCandBlock = 2048;

__global__ __launch_bounds__(256) void expert_count_kernel(
    const int* __restrict__ sel, int Hq, int Hkv, int R, const int* __restrict__ cu_chunk,
    const int* __restrict__ chunk_batch, const int* __restrict__ cu_seqlens,
    const int* __restrict__ filtered, int nbmax, int* __restrict__ work) {
  const int e = blockIdx.x, b = blockIdx.y;
  ExpertRange x = expert_range(e, Hq, Hkv, cu_chunk, chunk_batch, cu_seqlens, filtered);
  const int64_t n = (int64_t)x.G * x.ns;
  const int64_t i1 = min(n, (int64_t)(b + 1) * kCandBlock);
  int cnt = 0;
  for (int64_t i = (int64_t)b * kCandBlock + threadIdx.x; i < i1; i += 256) {
    const int g = (int)(i / x.ns), s = x.s0 + (int)(i % x.ns);
    cnt += find_slot(sel, (int64_t)s * Hq + x.kh * x.G + g, R, x.c) >= 0;
  }
  __shared__ int part[4];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) part[w] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) work[(int64_t)e * nbmax + b] = part[0] + part[1] + part[2] + part[3];
}

// Per expert: block counts -> exclusive block offsets and the row count; then
// exclusive scans of row counts and tile counts over the experts (one workgroup).
__global__ __launch_bounds__(1024) void expert_scan_kernel(int* __restrict__ work, int nbmax, int E,
                                                         int block_rows, int* __restrict__ counts,
                                                         int* __restrict__ row_off,
                                                         int* __restrict__ tile_off) {
  __shared__ int wr[16], wt[16];
  __shared__ int carry_r, carry_t;
  if (threadIdx.x == 0) { carry_r = 0; carry_t = 0; }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int base = 0; base < E; base += 1024) {
    const int e = base + threadIdx.x;
    int r = 0;
    if (e < E) {
      int* wb = work + (int64_t)e * nbmax;
      for (int b = 0; b < nbmax; ++b) { const int c = wb[b]; wb[b] = r; r += c; }
      counts[e] = r;
    }
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
    const int* __restrict__ filtered, const int* __restrict__ row_off, int nbmax,
    const int* __restrict__ work, int* __restrict__ rows) {
  const int e = blockIdx.x, b = blockIdx.y;
  ExpertRange x = expert_range(e, Hq, Hkv, cu_chunk, chunk_batch, cu_seqlens, filtered);
  const int64_t n = (int64_t)x.G * x.ns;
  const int64_t i0 = (int64_t)b * kCandBlock, i1 = min(n, i0 + kCandBlock);
  if (i0 >= i1) return;
  __shared__ int wtot[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int out = row_off[e] + work[(int64_t)e * nbmax + b];
  for (int64_t base = i0; base < i1; base += 256) {
    const int64_t i = base + threadIdx.x;
    int slot = -1, h = 0, s = 0;
    if (i < i1) {
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

int64_t expert_blocks(int T, int Hq, int Hkv) {
  return ((int64_t)(Hq / Hkv) * T + kCandBlock - 1) / kCandBlock;
}

}  // namespace

extern "C" int moba_hip_chunk_means(const void* k, int dtype, int T, int Hkv, int D,
                                    const int* chunk_start, int F, int chunk, int precision,
                                    float* means, void* stream) {
  (void)T;
  if (F <= 0) return MOBA_OK;
  if (dtype != 0 && dtype != 1) { moba_set_error("chunk_means: dtype must be 0 (bf16) or 1 (fp16)"); return MOBA_ERR_ARG; }
  if (D < 8 || D % 8 || Hkv < 1 || chunk < 1) { moba_set_error("chunk_means: bad shape"); return MOBA_ERR_ARG; }
  if (D > 256) { moba_set_error("chunk_means: head_dim must be at most 256"); return MOBA_ERR_ARG; }
  dim3 grid((unsigned)((int64_t)F * Hkv)), block(256);
  const size_t lds = (size_t)64 * D * sizeof(float);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* kp = (const uint16_t*)k;
#define MOBA_MEANS(DT_, NP_) \
  hipLaunchKernelGGL((chunk_means_kernel<DT_, NP_>), grid, block, lds, st, kp, Hkv, D, chunk_start, \
                     chunk, precision, means)
  const int nd8 = D / 8;
  if (dtype == 0) {
    if (nd8 <= 4) MOBA_MEANS(0, 1); else if (nd8 <= 8) MOBA_MEANS(0, 2);
    else if (nd8 <= 16) MOBA_MEANS(0, 4); else MOBA_MEANS(0, 8);
  } else {
    if (nd8 <= 4) MOBA_MEANS(1, 1); else if (nd8 <= 8) MOBA_MEANS(1, 2);
    else if (nd8 <= 16) MOBA_MEANS(1, 4); else MOBA_MEANS(1, 8);
  }
#undef MOBA_MEANS
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
  if (D > 256) { moba_set_error("route_prefill: head_dim must be at most 256"); return MOBA_ERR_ARG; }
  dim3 grid((unsigned)((T + 255) / 256), (unsigned)Hq), block(256);
  const uint16_t* qp = (const uint16_t*)q;
#define MOBA_ROUTE(DT_, DP_) \
  hipLaunchKernelGGL((route_kernel<DT_, DP_>), grid, block, 0, st, qp, T, Hq, Hkv, D, means, \
                     cu_chunk, nchunk, chunk_batch, first_chunk, R, F, sel, gate)
  if (dtype == 0) {
    if (D <= 64) MOBA_ROUTE(0, 64); else if (D <= 128) MOBA_ROUTE(0, 128); else MOBA_ROUTE(0, 256);
  } else {
    if (D <= 64) MOBA_ROUTE(1, 64); else if (D <= 128) MOBA_ROUTE(1, 128); else MOBA_ROUTE(1, 256);
  }
#undef MOBA_ROUTE
  return moba_launch_status("route_prefill");
}

extern "C" int64_t moba_hip_pack_experts_work(int T, int Hq, int Hkv, int F) {
  if (T < 0 || Hq < 1 || Hkv < 1 || Hq % Hkv || F < 0) return -1;
  return (int64_t)F * Hkv * expert_blocks(T, Hq, Hkv);
}

extern "C" int moba_hip_pack_experts(const int* sel, int T, int Hq, int Hkv, int R,
                                     const int* cu_chunk, const int* chunk_batch,
                                     const int* cu_seqlens, const int* filtered, int F,
                                     int block_rows, int* counts, int* row_off, int* tile_off,
                                     int* rows, int* work, void* stream) {
  if (F <= 0) return MOBA_OK;
  if ((int64_t)T * Hq * R >= (1ll << 31) || (int64_t)T * Hq >= (1ll << 28)) { moba_set_error("pack_experts: T*Hq*R exceeds int32 or T*Hq exceeds 2^28"); return MOBA_ERR_ARG; }
  if (R > 8) { moba_set_error("pack_experts: at most 8 remote chunks per query"); return MOBA_ERR_ARG; }
  if (Hkv < 1 || Hq % Hkv) { moba_set_error("pack_experts: Hq must be a multiple of Hkv"); return MOBA_ERR_ARG; }
  if (work == nullptr) { moba_set_error("pack_experts: the work buffer (moba_hip_pack_experts_work ints) is required"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  const int E = F * Hkv;
  const int nbmax = (int)expert_blocks(T, Hq, Hkv);
  if (nbmax < 1) return MOBA_OK;
  hipLaunchKernelGGL(expert_count_kernel, dim3(E, nbmax), dim3(256), 0, st, sel, Hq, Hkv, R,
                     cu_chunk, chunk_batch, cu_seqlens, filtered, nbmax, work);
  hipLaunchKernelGGL(expert_scan_kernel, dim3(1), dim3(1024), 0, st, work, nbmax, E, block_rows,
                     counts, row_off, tile_off);
  hipLaunchKernelGGL(expert_fill_kernel, dim3(E, nbmax), dim3(256), 0, st, sel, Hq, Hkv, R,
                     cu_chunk, chunk_batch, cu_seqlens, filtered, row_off, nbmax, work, rows);
  return moba_launch_status("pack_experts");
}
