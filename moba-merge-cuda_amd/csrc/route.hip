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

// One workgroup per (filtered chunk, kv head, dim slice of D / ds).  The mean of dim d is the
// canonical sum: 64 partial sums s_j over the tokens j, j+64, j+128, ... in
// increasing order, then the fixed tree canon_tree over j.  Work item
// (j, column block b) of 8 dims is p = j * nd8 + b, so a wave's loads cover
// whole rows (coalesced); thread t owns items t, t + 256, ...  The partials
// go through LDS to one wave per dim, lane j holding s_j, for the tree.
template <int DT, int NP>
__global__ __launch_bounds__(256) void chunk_means_kernel(const uint16_t* __restrict__ k, int Hkv,
                                                          int D, const int* __restrict__ chunk_start,
                                                          int C, int precision, int ds,
                                                          float* __restrict__ means) {
  extern __shared__ float part[];  // [64][D]
  const int nd8 = D / 8 / ds, np = 64 * nd8;  // this workgroup's 8-dim blocks
  const int sub = blockIdx.x % ds, fk = blockIdx.x / ds;
  const int kh = fk % Hkv, f = fk / Hkv;
  const int tid = threadIdx.x;
  const int64_t stride = (int64_t)Hkv * D;
  const uint16_t* base = k + ((int64_t)chunk_start[f] * Hkv + kh) * D;
  float acc[NP][8];
  int jj[NP], bb[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = tid + 256 * i;
    jj[i] = p < np ? p / nd8 : C;  // items past np load nothing
    bb[i] = sub * nd8 + p % nd8;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.0f;
  }
  // KU row groups of 64 tokens per pass: all their loads are issued before
  // the adds, which then run in token order (one load latency per pass, not
  // per group)
  constexpr int KU = NP <= 2 ? 8 : 4;
  for (int t0 = 0; t0 < C; t0 += 64 * KU) {
    u16x8_t x[KU][NP];
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int t = t0 + 64 * u + jj[i];
        x[u][i] = t < C ? ld8(base + t * stride + bb[i] * 8) : zero8();
      }
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int i = 0; i < NP; ++i)
        if (t0 + 64 * u + jj[i] < C) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[i][e] = acc[i][e] + to_f32<DT>(x[u][i][e]);
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
  for (int d = sub * nd8 * 8 + w; d < (sub + 1) * nd8 * 8; d += 4) {
    float m = canon_tree(part[lane * D + d]) / (float)C;
    if (precision == 0) m = to_f32<DT>(from_f32<DT>(m));
    if (lane == 0) dst[d] = m;
  }
}

// One thread per (token, q head): a workgroup takes 256 consecutive tokens of
// one head.  The means rows its tokens score (filtered indices [flo, fhi) of
// the head's kv head) go through LDS in tiles of kRouteTile rows.  A wave
// walks the union of its lanes' candidate ranges in a wave-uniform loop:
// each 16-lane row of the wave reads 16 values of the candidate's means row
// into one register per 16 dims, and the fma chain takes dim d from lane
// d % 16 of its row by a DPP row broadcast (an operand modifier of the fma),
// so a means row costs DP / 16 LDS reads per wave instead of DP / 4
// broadcast 16-byte reads; lanes outside a candidate's range discard its
// score.  The token's q row is held in registers (fp32 up to 128 dims, the
// input dtype above).  The fma chain of each candidate is the canonical
// order, unchanged.
constexpr int kRouteTile = 32;

// DE: the head dim when it is DP exactly (no per-piece bound checks), else 0.
template <int DT, int DP, int DE>
__global__ __launch_bounds__(256) void route_kernel(const uint16_t* __restrict__ q, int T, int Hq,
                                                    int Hkv, int D,
                                                    const float* __restrict__ means,
                                                    const int* __restrict__ cu_chunk, int nchunk,
                                                    const int* __restrict__ chunk_batch,
                                                    const int* __restrict__ first_chunk, int R,
                                                    int F, int* __restrict__ sel,
                                                    float* __restrict__ gate) {
  __shared__ __attribute__((aligned(16))) float mt[kRouteTile * DP];
  __shared__ int red[2][4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int s = blockIdx.x * 256 + tid;
  const int h = blockIdx.y;
  const bool live = s < T;
  const int G = Hq / Hkv, kh = h / G;
  // the q row first: its loads overlap the chunk search below
  const int64_t idx = (int64_t)s * Hq + h;
  constexpr int NQ = DP / 8;
  u16x8_t qv[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) qv[i] = (live && i * 8 < D) ? ld8(q + idx * D + i * 8) : zero8();
  // chunk containing s (the last token's for the threads past T)
  const int sc = live ? s : T - 1;
  // search once per wave for its first token (uniform loads), then per lane
  // only when the wave straddles a chunk boundary
  const int sw = __builtin_amdgcn_readfirstlane(sc);
  int lo = 0, hi = nchunk - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu_chunk[mid] <= sw) lo = mid; else hi = mid - 1;
  }
  if (__ballot(sc >= cu_chunk[lo + 1]) != 0) {
    lo = 0; hi = nchunk - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (cu_chunk[mid] <= sc) lo = mid; else hi = mid - 1;
    }
  }
  const int cs = lo, b = chunk_batch[cs], c0 = first_chunk[cs];
  // this thread's candidates are filtered rows [c0 - b, cs - b)
  const int f0 = c0 - b, f1 = cs - b;
  int mn = live && f1 > f0 ? f0 : 0x7fffffff, mx = live && f1 > f0 ? f1 : 0;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    mn = min(mn, __shfl_xor(mn, o, 64));
    mx = max(mx, __shfl_xor(mx, o, 64));
  }
  const int wlo = __builtin_amdgcn_readfirstlane(mn), whi = __builtin_amdgcn_readfirstlane(mx);
  if (lane == 0) { red[0][tid >> 6] = wlo; red[1][tid >> 6] = whi; }
  __syncthreads();
  const int flo = min(min(red[0][0], red[0][1]), min(red[0][2], red[0][3]));
  const int fhi = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));

  constexpr bool QF32 = DP <= 128;      // q row as fp32 registers
  float qf[QF32 ? DP : 1];
  if constexpr (QF32) {
#pragma unroll
    for (int i = 0; i < NQ; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[i * 8 + e] = to_f32<DT>(qv[i][e]);
  }

  float val[kMaxRemote];
  int ix[kMaxRemote];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kMaxRemote; ++j) { val[j] = -INFINITY; ix[j] = -1; }

  // LDS tile: rows of DP floats, columns past D zero (so are q's), and
  // fma(0, 0, acc) == acc keeps the chain exact over the padding
  constexpr int NST = (kRouteTile * DP / 4 + 255) / 256;
  constexpr int NM = DP / 16;  // registers of a means row per lane
  for (int t0 = flo; t0 < fhi; t0 += kRouteTile) {
    const int nt = min(kRouteTile, fhi - t0);
    f32x4_t stg[NST];
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int x = tid + 256 * i, r = x / (DP / 4), d = (x % (DP / 4)) * 4;
      stg[i] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
      if (r < nt && d < D)
        stg[i] = *reinterpret_cast<const f32x4_t*>(means + ((int64_t)(t0 + r) * Hkv + kh) * D + d);
    }
    __syncthreads();  // the previous tile is consumed
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int x = tid + 256 * i;
      if (x < kRouteTile * DP / 4) *reinterpret_cast<f32x4_t*>(mt + x * 4) = stg[i];
    }
    __syncthreads();
    const int fa = max(wlo, t0), fb = min(whi, t0 + nt);
    for (int f = fa; f < fb; ++f) {
      const float* mr = mt + (f - t0) * DP + (lane & 15);
      float mv[NM];
#pragma unroll
      for (int i = 0; i < NM; ++i) mv[i] = mr[16 * i];
      // sequential fma chain over d = 0 .. DP-1 (zero past D)
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        float qa[8], qb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qa[e] = QF32 ? qf[16 * i + e] : to_f32<DT>(qv[2 * i][e]);
          qb[e] = QF32 ? qf[16 * i + 8 + e] : to_f32<DT>(qv[2 * i + 1][e]);
        }
        acc = fma8_bcast<0>(acc, mv[i], qa);
        acc = fma8_bcast<8>(acc, mv[i], qb);
      }
      if (!(live && f >= f0 && f < f1)) continue;
      const int c = f + b;
      if (gate) gate[((int64_t)f * Hq + h) * T + s] = acc;
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
  }
  if (!live) return;
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

// Selection bitmasks: word w of row (s, h) has bit f % 64 set when (s, h)
// selected the chunk of filtered index f, f / 64 == w; laid out
// mask[(h * NW + w) * T + s], so the candidate scans of the experts, which
// walk s for a fixed (h, w), read 8 consecutive bytes per candidate instead
// of a strided R-int row of sel.  One thread per (s, h).
__global__ __launch_bounds__(256) void sel_mask_kernel(const int* __restrict__ sel, int T, int Hq,
                                                       int R, const int* __restrict__ chunk_batch,
                                                       int NW, uint64_t* __restrict__ mask) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;  // s * Hq + h
  if (row >= (int64_t)T * Hq) return;
  const int s = (int)(row / Hq), h = (int)(row % Hq);
  int fs[kMaxRemote];
#pragma unroll
  for (int j = 0; j < kMaxRemote; ++j) {
    const int c = j < R ? sel[row * R + j] : -1;
    fs[j] = c >= 0 ? c - chunk_batch[c] : -1;
  }
  for (int w = 0; w < NW; ++w) {
    uint64_t m = 0;
#pragma unroll
    for (int j = 0; j < kMaxRemote; ++j)
      if (fs[j] >= 0 && (fs[j] >> 6) == w) m |= 1ull << (fs[j] & 63);
    mask[((int64_t)h * NW + w) * T + s] = m;
  }
}

struct ExpertRange { int c, f, kh, s0, ns, G; };

MOBA_DEV ExpertRange expert_range(int e, int Hq, int Hkv, const int* cu_chunk,
                                  const int* chunk_batch, const int* cu_seqlens,
                                  const int* filtered) {
  ExpertRange r;
  const int f = e / Hkv;
  r.kh = e % Hkv;
  r.f = f;
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
    const uint64_t* __restrict__ mask, int T, int NW, int Hq, int Hkv,
    const int* __restrict__ cu_chunk, const int* __restrict__ chunk_batch,
    const int* __restrict__ cu_seqlens, const int* __restrict__ filtered, int nbmax,
    int* __restrict__ work) {
  const int e = blockIdx.x, b = blockIdx.y;
  ExpertRange x = expert_range(e, Hq, Hkv, cu_chunk, chunk_batch, cu_seqlens, filtered);
  const int64_t n = (int64_t)x.G * x.ns;
  const int64_t i1 = min(n, (int64_t)(b + 1) * kCandBlock);
  const int mw = x.f >> 6, bit = x.f & 63;
  int cnt = 0;
  for (int64_t i = (int64_t)b * kCandBlock + threadIdx.x; i < i1; i += 256) {
    const int g = (int)(i / x.ns), s = x.s0 + (int)(i % x.ns);
    cnt += (int)((mask[((int64_t)(x.kh * x.G + g) * NW + mw) * T + s] >> bit) & 1);
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
    const uint64_t* __restrict__ mask, int T, int NW, int Hq, int Hkv,
    const int* __restrict__ cu_chunk, const int* __restrict__ chunk_batch,
    const int* __restrict__ cu_seqlens, const int* __restrict__ filtered,
    const int* __restrict__ row_off, int nbmax, const int* __restrict__ work,
    int* __restrict__ rows) {
  const int e = blockIdx.x, b = blockIdx.y;
  ExpertRange x = expert_range(e, Hq, Hkv, cu_chunk, chunk_batch, cu_seqlens, filtered);
  const int mw = x.f >> 6, bit = x.f & 63;
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
      const uint64_t* mh = mask + (int64_t)h * NW * T + s;
      const uint64_t m = mh[(int64_t)mw * T];
      if ((m >> bit) & 1) {
        // slot = the selected chunks before this one (sel is ascending)
        slot = __popcll(m & ((1ull << bit) - 1ull));
        for (int w2 = 0; w2 < mw; ++w2) slot += __popcll(mh[(int64_t)w2 * T]);
      }
    }
    const uint64_t hits = __ballot(slot >= 0);
    const int before = __popcll(hits & ((1ull << lane) - 1ull));
    if (lane == 0) wtot[w] = __popcll(hits);
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
  // dim slices per (chunk, kv head), until the grid has about 512 workgroups,
  // each slice at least 128 bytes of a key row (whole 128-byte lines; 64 when
  // there are fewer than 64 (chunk, kv head) pairs)
  int ds = 1;
  const int64_t wgs = (int64_t)F * Hkv;
  while ((D / 8) % (2 * ds) == 0 && D / 8 / (2 * ds) >= (wgs < 64 ? 4 : 8) && wgs * ds < 512) ds *= 2;
  dim3 grid((unsigned)((int64_t)F * Hkv * ds)), block(256);
  const size_t lds = (size_t)64 * D * sizeof(float);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* kp = (const uint16_t*)k;
#define MOBA_MEANS(DT_, NP_) \
  hipLaunchKernelGGL((chunk_means_kernel<DT_, NP_>), grid, block, lds, st, kp, Hkv, D, chunk_start, \
                     chunk, precision, ds, means)
  const int nd8 = D / 8 / ds;
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
#define MOBA_ROUTE(DT_, DP_, DE_) \
  hipLaunchKernelGGL((route_kernel<DT_, DP_, DE_>), grid, block, 0, st, qp, T, Hq, Hkv, D, means, \
                     cu_chunk, nchunk, chunk_batch, first_chunk, R, F, sel, gate)
#define MOBA_ROUTE_DT(DT_) \
  if (D == 64) MOBA_ROUTE(DT_, 64, 64); else if (D < 64) MOBA_ROUTE(DT_, 64, 0); \
  else if (D == 128) MOBA_ROUTE(DT_, 128, 128); else if (D < 128) MOBA_ROUTE(DT_, 128, 0); \
  else if (D == 256) MOBA_ROUTE(DT_, 256, 256); else MOBA_ROUTE(DT_, 256, 0);
  if (dtype == 0) {
    MOBA_ROUTE_DT(0)
  } else {
    MOBA_ROUTE_DT(1)
  }
#undef MOBA_ROUTE_DT
#undef MOBA_ROUTE
  return moba_launch_status("route_prefill");
}

// Work ints of moba_hip_pack_experts: the selection bitmasks (2 ints per
// 64-bit word), then the per-(expert, block) counts.
int64_t mask_ints(int T, int Hq, int F) { return (int64_t)T * Hq * ((F + 63) / 64) * 2; }

extern "C" int64_t moba_hip_pack_experts_work(int T, int Hq, int Hkv, int F) {
  if (T < 0 || Hq < 1 || Hkv < 1 || Hq % Hkv || F < 0) return -1;
  return mask_ints(T, Hq, F) + (int64_t)F * Hkv * expert_blocks(T, Hq, Hkv);
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
  if (work == nullptr || ((uintptr_t)work & 7)) { moba_set_error("pack_experts: the work buffer (moba_hip_pack_experts_work ints, 8-byte aligned) is required"); return MOBA_ERR_ARG; }
  hipStream_t st = (hipStream_t)stream;
  const int E = F * Hkv;
  const int nbmax = (int)expert_blocks(T, Hq, Hkv);
  if (nbmax < 1) return MOBA_OK;
  const int NW = (F + 63) / 64;
  uint64_t* mask = reinterpret_cast<uint64_t*>(work);  // 8-byte aligned: the work buffer's start
  int* cwork = work + mask_ints(T, Hq, F);
  hipLaunchKernelGGL(sel_mask_kernel, dim3((unsigned)(((int64_t)T * Hq + 255) / 256)), dim3(256),
                     0, st, sel, T, Hq, R, chunk_batch, NW, mask);
  hipLaunchKernelGGL(expert_count_kernel, dim3(E, nbmax), dim3(256), 0, st, mask, T, NW, Hq, Hkv,
                     cu_chunk, chunk_batch, cu_seqlens, filtered, nbmax, cwork);
  hipLaunchKernelGGL(expert_scan_kernel, dim3(1), dim3(1024), 0, st, cwork, nbmax, E, block_rows,
                     counts, row_off, tile_off);
  hipLaunchKernelGGL(expert_fill_kernel, dim3(E, nbmax), dim3(256), 0, st, mask, T, NW, Hq, Hkv,
                     cu_chunk, chunk_batch, cu_seqlens, filtered, row_off, nbmax, cwork, rows);
  return moba_launch_status("pack_experts");
}
