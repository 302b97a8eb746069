// Shared device helpers for the gfx950 MoBA kernels.
//
// Element storage is raw 16-bit (bf16 = dtype 0, fp16 = dtype 1).  MFMA tiles
// use v_mfma_f32_32x32x16_{bf16,f16}; the operand layouts (verified on gfx950):
//   A[m][k] : lane l supplies row m = l%32, k = (l/32)*8 + e, e = 0..7
//   B[k][n] : lane l supplies col n = l%32, k = (l/32)*8 + e
//   D[m][n] : lane l holds   col n = l%32, rows m = 8*j + 4*(l/32) + i  (value j*4+i)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MOBA_DEV __device__ __forceinline__

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

namespace moba {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

MOBA_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even float -> bf16 (same bit recipe as the CPU oracle).
MOBA_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

MOBA_DEV float f16_to_f32(uint16_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, h);
  return (float)x;
}
MOBA_DEV uint16_t f32_to_f16(float f) {
  _Float16 x = (_Float16)f;  // v_cvt_f16_f32, round-to-nearest-even
  return __builtin_bit_cast(uint16_t, x);
}

template <int DT> MOBA_DEV float to_f32(uint16_t v) {
  if constexpr (DT == 0) return bf16_to_f32(v); else return f16_to_f32(v);
}
// Hardware conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32, round to nearest
// even; identical to f32_to_bf16 for every non-NaN input).
template <int DT> MOBA_DEV uint16_t from_f32(float v) {
  if constexpr (DT == 0) return __builtin_bit_cast(uint16_t, (__bf16)v);
  else return f32_to_f16(v);
}

// Two floats to two packed 16-bit values, a in the low half: one
// v_cvt_pk_* instruction (same rounding as from_f32).
template <int DT> MOBA_DEV uint32_t pack2(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  if constexpr (DT == 0) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
  } else {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
  }
}
// The two 16-bit values of a packed word as floats (low half first).
template <int DT> MOBA_DEV void unpack2(uint32_t w, float& lo, float& hi) {
  if constexpr (DT == 0) {
    lo = __uint_as_float(w << 16);
    hi = __uint_as_float(w & 0xffff0000u);
  } else {
    lo = to_f32<1>((uint16_t)(w & 0xffffu));
    hi = to_f32<1>((uint16_t)(w >> 16));
  }
}

// 32x32x16 MFMA on 8 packed 16-bit elements per lane.
template <int DT>
MOBA_DEV f32x16_t mfma32(const u16x8_t& a, const u16x8_t& b, const f32x16_t& c) {
  if constexpr (DT == 0) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// 16x16x32 MFMA (A: row l%16, k (l/16)*8+e; D: column l%16, rows 4(l/16)+i).
template <int DT>
MOBA_DEV f32x4_t mfma16(const u16x8_t& a, const u16x8_t& b, const f32x4_t& c) {
  if constexpr (DT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

MOBA_DEV f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

MOBA_DEV u16x8_t zero8() {
  u16x8_t z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = 0;
  return z;
}

// sign flip of 8 bf16 / fp16 values (exact)
MOBA_DEV u16x8_t neg8(u16x8_t x) {
  const u32x4_t m = {0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
  return __builtin_bit_cast(u16x8_t, __builtin_bit_cast(u32x4_t, x) ^ m);
}

MOBA_DEV u16x8_t ld8(const uint16_t* p) { return *reinterpret_cast<const u16x8_t*>(p); }
MOBA_DEV void st8(uint16_t* p, const u16x8_t& v) { *reinterpret_cast<u16x8_t*>(p) = v; }

// Position of key r (0..15) of a 16-key MFMA k-group inside a transposed LDS
// row.  A 32-key score block held as D-layout gives lane half h the keys
// {4h..4h+3, 8+4h..8+4h+3} of each 16-key group; storing key r at this
// position makes those 8 keys contiguous at offset 8h.
MOBA_DEV int kperm16(int r) { return ((r >> 2) & 1) * 8 + ((r >> 3) & 1) * 4 + (r & 3); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// gfx950 transposed LDS read (ds_read_b64_tr_b16).  In each 16-lane group,
// lane i receives column (cbase + i) of 4 consecutive rows k0..k0+3 of a
// row-major LDS tile when lane i' of the group addresses
// row k0 + i'/4, columns cbase + 4*(i'%4) .. +3.
MOBA_DEV u16x4_t ld_tr4(const uint16_t* p) {
  s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p));
  return __builtin_bit_cast(u16x4_t, v);
}

// MFMA 32x32x16 operand whose contraction index runs over ROWS of a row-major
// LDS tile X (stride ld elements): lane (col = l%32, half hh) gets
// X[g16 + 4hh + 0..3][c0 + l%32] and X[g16 + 8 + 4hh + 0..3][c0 + l%32], i.e.
// the same key order as the P/dS operands built from a D-layout accumulator.
MOBA_DEV u16x8_t ld_tr_operand(const uint16_t* X, int ld, int g16, int c0, int lane) {
  const int hh = lane >> 5, sub = lane & 15, cb = c0 + ((lane >> 4) & 1) * 16;
  const uint16_t* p0 = X + (g16 + 4 * hh + (sub >> 2)) * ld + cb + 4 * (sub & 3);
  const u16x4_t a = ld_tr4(p0), b = ld_tr4(p0 + 8 * ld);
  u16x8_t r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// XOR-swizzled row-major LDS tiles of DP-element rows (no padding).  The
// 16-byte block b of row r is stored at block b ^ f(r), f(r) = bitrev4(r % 16)
// masked to the row's block count.  With 64 four-byte banks this keeps both
// access patterns of the attention kernels conflict-free:
//   * ds_read_b128 of one block from 16 consecutive rows (16 lanes per cycle);
//   * ds_read_b64_tr_b16 of 4 consecutive rows x 4 consecutive blocks
//     (32 lanes per cycle).
template <int DP> MOBA_DEV int swz(int r, int col) {
  constexpr int NBM = (DP / 8 < 16 ? DP / 8 : 16) - 1;
  const int f = (int)(__builtin_bitreverse32((uint32_t)r) >> 28) & NBM;
  return r * DP + ((((col >> 3) ^ f) << 3) | (col & 7));
}

// Byte-offset form of the swizzled reads.  The bank-spreading XOR f(r)
// depends on r % 16 only, so a lane's rows (its own row plus multiples of 16)
// share one lane-constant base.  A row starts at a multiple of 16 * NB bytes,
// so adding block blk to a base is one XOR on the low block bits the swizzle
// owns plus an add of the rest.
template <int DP> constexpr int swz_nbm() { return (DP / 8 < 16 ? DP / 8 : 16) - 1; }
template <int DP> MOBA_DEV uint32_t swz_add(uint32_t base, int blk) {
  constexpr int NBM = swz_nbm<DP>();
  return (base ^ (uint32_t)((blk & NBM) << 4)) + (uint32_t)((blk & ~NBM) << 4);
}
// ds_read_b128 operand of rows (lane % 32) + 16m, k-step ks: base for ks = 0.
template <int DP> MOBA_DEV uint32_t swz_b128_base(int lane) {
  return (uint32_t)swz<DP>(lane & 31, (lane >> 5) * 8) * 2;
}
template <int DP> MOBA_DEV uint32_t swz_b128(uint32_t base, int ks) { return swz_add<DP>(base, 2 * ks); }
// Transposed-read pieces (rows g16 + 4hh + (l%16)/4 + 8*half, columns
// 32*db + 16*((l/16)%2) + 4*(l%4)): base for g16 = 0, db = 0.
template <int DP> MOBA_DEV uint32_t swz_tr_base(int lane, int half) {
  const int sub = lane & 15;
  return (uint32_t)swz<DP>(4 * (lane >> 5) + (sub >> 2) + 8 * half,
                           ((lane >> 4) & 1) * 16 + 4 * (sub & 3)) * 2;
}
template <int DP> MOBA_DEV uint32_t swz_tr(uint32_t base, int db) { return swz_add<DP>(base, 4 * db); }

// Hides a value from the optimiser so that addresses derived from it are
// recomputed where they are used instead of being held in registers.
MOBA_DEV uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

MOBA_DEV u16x8_t lds8(const uint16_t* base, uint32_t byte_off) {
  return *reinterpret_cast<const u16x8_t*>(reinterpret_cast<const char*>(base) + byte_off);
}
// MFMA operand from two transposed reads at byte offsets a and b of base.
MOBA_DEV u16x8_t lds_tr8(const uint16_t* base, uint32_t a, uint32_t b) {
  const char* p = reinterpret_cast<const char*>(base);
  const u16x4_t x = ld_tr4(reinterpret_cast<const uint16_t*>(p + a));
  const u16x4_t y = ld_tr4(reinterpret_cast<const uint16_t*>(p + b));
  u16x8_t o;
  o[0] = x[0]; o[1] = x[1]; o[2] = x[2]; o[3] = x[3];
  o[4] = y[0]; o[5] = y[1]; o[6] = y[2]; o[7] = y[3];
  return o;
}

// ld_tr_operand on a swizzled tile (same lane/key order).
template <int DP>
MOBA_DEV u16x8_t ld_tr_operand_swz(const uint16_t* X, int g16, int c0, int lane) {
  const int hh = lane >> 5, sub = lane & 15, cb = c0 + ((lane >> 4) & 1) * 16;
  const int r = g16 + 4 * hh + (sub >> 2), col = cb + 4 * (sub & 3);
  const u16x4_t a = ld_tr4(X + swz<DP>(r, col)), b = ld_tr4(X + swz<DP>(r + 8, col));
  u16x8_t o;
  o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
  o[4] = b[0]; o[5] = b[1]; o[6] = b[2]; o[7] = b[3];
  return o;
}

// Buffer resource over [base, base + bytes) for raw buffer loads (stride 0;
// offsets at or past `bytes` read as zero).
MOBA_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, bytes, 0x00020000);
}

// One 16-byte buffer load per lane straight into LDS: lane l's 16 bytes land
// at lds + 16 * l (lds must be wave-uniform).
MOBA_DEV void load_lds16(__amdgpu_buffer_rsrc_t r, uint16_t* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           voff, soff, 0, 0);
}

// The same LDS loads issued from inline assembly, out of the compiler's
// sight.  An LDS-DMA load reads M0 and needs one wait state after the SALU
// write of M0 (the s_nop the compiler itself places in that position).  Out
// of sight, it inserts no waits for them (its alias tracking of LDS loads would
// otherwise wait on loads into a stage other than the one being read).  The
// caller orders them itself: s_waitcnt vmcnt plus a barrier before the LDS is
// read, and a barrier after the last read of a stage before it is reloaded.
MOBA_DEV uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
MOBA_DEV void dma_lds16(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds_addr(lds)), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
MOBA_DEV void dma_lds4(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :: "s"(lds_addr(lds)), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

// Workgroup barriers for kernels whose LDS tiles arrive by buffer loads.
// The empty asm statements keep the compiler from moving memory accesses
// across the barrier; the explicit waits are visible to its wait-count pass.
//   stage_barrier: this wave's buffer loads (and LDS accesses) complete, then
//                  the barrier: every wave's loads have landed after it.
//   lds_barrier:   LDS accesses complete, then the barrier; buffer loads in
//                  flight stay in flight.
MOBA_DEV void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
MOBA_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 32-row query blocks per wave in the query-major attention kernels (forward
// and dQ); a workgroup of 4 waves covers 128 * attn_qb rows.  One block per
// wave leaves room for two waves per SIMD.
template <int DP> constexpr int attn_qb() { return 1; }
template <int DP> constexpr int attn_occupancy() { return attn_qb<DP>() == 1 ? 2 : 1; }

// Workgroup L of a 1-D grid runs on XCD L % 8 (8 XCDs, each with its own L2).
// Maps L to a work index so that every XCD takes one contiguous eighth of
// [0, total) in order: neighbouring work items, which share K/V tiles, stay in
// one L2.  The grid must hold at least 8 * ceil(total / 8) workgroups; surplus
// workgroups get -1.
MOBA_DEV int xcd_contiguous(int L, int total) {
  const int per = (total + 7) >> 3;
  const int i = L >> 3, t = (L & 7) * per + i;
  return (i < per && t < total) ? t : -1;
}

// Wave issue priority (0 or 1): a wave in an MFMA-heavy phase is set ahead of
// a wave in an element-wise phase on the same SIMD, which keeps the matrix
// unit fed.  No scheduling fences: the compiler keeps s_setprio in order with
// the MFMAs and transcendental ops around it and may interleave other work.
template <int P> MOBA_DEV void wave_prio() { __builtin_amdgcn_s_setprio(P); }

MOBA_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int DT> MOBA_DEV u16x8_t pack8(const float* v) {
  u16x8_t r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = from_f32<DT>(v[e]);
  return r;
}

// Canonical fp32 reduction shared with the CPU oracle: lane j of a wave holds
// the sequential sum of elements j, j+64, j+128, ...; the partials are then
// added by the fixed tree part[j] += part[j+off], off = 32..1.  Lane 0 returns
// the result (other lanes return partial values).
MOBA_DEV float canon_tree(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = v + __shfl_down(v, off, 64);
  return v;
}

MOBA_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
MOBA_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}


// acc = fma(b_j, m[j], acc) for j = 0..7 in order, b_j = lane (row base + J0
// + j) of b: the fma reads b through a DPP row broadcast (row_newbcast, one
// source lane for each 16-lane row), which the compiler does not form on its
// own.  A 16-lane row then holds 16 dims of a row vector in one register, and
// a whole wave streams a sequential fma chain against it with no LDS reads.
// The leading s_nop covers the DPP read-after-VALU-write hazard on b (the
// compiler does not look inside the block).
template <int J0>
MOBA_DEV float fma8_bcast(float acc, float b, const float (&m)[8]) {
  static_assert(J0 == 0 || J0 == 8, "row lanes 0..7 or 8..15");
  if constexpr (J0 == 0) {
    asm volatile(
        "s_nop 1\n"
        "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
        : "+v"(acc)
        : "v"(b), "v"(m[0]), "v"(m[1]), "v"(m[2]), "v"(m[3]), "v"(m[4]), "v"(m[5]), "v"(m[6]),
          "v"(m[7]));
  } else {
    asm volatile(
        "s_nop 1\n"
        "v_fmac_f32_dpp %0, %1, %2 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
        : "+v"(acc)
        : "v"(b), "v"(m[0]), "v"(m[1]), "v"(m[2]), "v"(m[3]), "v"(m[4]), "v"(m[5]), "v"(m[6]),
          "v"(m[7]));
  }
  return acc;
}

// Four chains interleaved: acc[k] = fma(lane (row base + J0 + j) of b[k],
// m[j], acc[k]) for j = 0..7 in order, chain k independent of the others (so
// consecutive instructions do not wait on each other).  Hazard as above.
#define MOBA_F4(J, MJ)                                                                         \
  "v_fmac_f32_dpp %0, %4, " MJ " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n"             \
  "v_fmac_f32_dpp %1, %5, " MJ " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n"             \
  "v_fmac_f32_dpp %2, %6, " MJ " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n"             \
  "v_fmac_f32_dpp %3, %7, " MJ " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n"
template <int J0>
MOBA_DEV void fma8_bcast4(float (&acc)[4], const float (&b)[4], const float (&m)[8]) {
  static_assert(J0 == 0 || J0 == 8, "row lanes 0..7 or 8..15");
  if constexpr (J0 == 0) {
    asm volatile("s_nop 1\n" MOBA_F4(0, "%8") MOBA_F4(1, "%9") MOBA_F4(2, "%10") MOBA_F4(3, "%11")
                 MOBA_F4(4, "%12") MOBA_F4(5, "%13") MOBA_F4(6, "%14") MOBA_F4(7, "%15")
                 : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
                 : "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(m[0]), "v"(m[1]), "v"(m[2]),
                   "v"(m[3]), "v"(m[4]), "v"(m[5]), "v"(m[6]), "v"(m[7]));
  } else {
    asm volatile("s_nop 1\n" MOBA_F4(8, "%8") MOBA_F4(9, "%9") MOBA_F4(10, "%10") MOBA_F4(11, "%11")
                 MOBA_F4(12, "%12") MOBA_F4(13, "%13") MOBA_F4(14, "%14") MOBA_F4(15, "%15")
                 : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
                 : "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(m[0]), "v"(m[1]), "v"(m[2]),
                   "v"(m[3]), "v"(m[4]), "v"(m[5]), "v"(m[6]), "v"(m[7]));
  }
}
#undef MOBA_F4

// Order-preserving 64-bit key of a route score: larger key = higher score,
// then lower chunk (the stable top-k order); 0 for -inf / NaN, which are never
// selected.  -0 and +0 compare equal, as the float comparison does.
MOBA_DEV uint64_t route_key(float v, int c) {
  if (!(v > -INFINITY)) return 0;
  uint32_t u = __float_as_uint(v + 0.0f);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(0x7fffffff - c);
}

}  // namespace moba

// Error reporting shared by the C-ABI entry points.
void moba_set_error(const char* fmt, ...);
int moba_launch_status(const char* what);
