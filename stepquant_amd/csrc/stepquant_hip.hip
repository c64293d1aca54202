// MI355X (gfx950) kernels for STEPQuant's packed-state recurrent update.
//
// One workgroup owns one (request, value-head) tile of K x V state values.
// The tile's packed code region (contiguous per head in the page layout of
// stepquant/kernels/pool.py:19-66) is staged through LDS with 16-byte
// loads, every lane then owns RPT key rows x 4 adjacent value columns, so
// each lane's codes are one whole byte run of 4*b bits in every row.
//
//   sq_encode        dense fp32 -> page, bit-identical to the CPU fit_state
//                    (quantization.py:54-98): exact IEEE division/sqrt and
//                    PyTorch's CPU float32 summation order.
//   sq_decode_dense  page -> dense fp32 (kernels/fused.py:18-59).
//   sq_decode_step   fused read + gated delta update + readout + requantise +
//                    store (pool.py:200-331), one HBM pass over the page.
//   sq_decode_readout / sq_writeback  the same step split over a foreground
//                    and a writeback stream (pool.py:284-316).
//
// Register math of the decode step uses reciprocals of per-row and
// per-column scales (computed with IEEE division); the encode path uses
// IEEE division per element.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "stepquant_hip.h"

namespace {

// ------------------------------------------------------------------ fp16

// IEEE half <-> float by the hardware conversions (v_cvt_f32_f16,
// v_cvt_f16_f32): exact one way, round to nearest even the other, subnormal
// halves kept (f16 denormals are on in these kernels), overflow to infinity:
// torch's .half() for every non-NaN input.
__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
// The empty asm keeps the conversion apart from the operation that produced
// f: merged into one v_fma_mixlo_f16 the pair would round once instead of to
// fp32 first and then to half, as the fp32 reference does.
__device__ __forceinline__ uint32_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// quantization.py:49-51: clamp(2^-24, 65504).half().float()
__device__ __forceinline__ float fp16_scale(float x, uint32_t *hbits) {
  float c = x < 5.9604644775390625e-08f ? 5.9604644775390625e-08f : x;
  c = c > 65504.0f ? 65504.0f : c;
  uint32_t h = f2h(c);
  if (hbits) *hbits = h;
  return h2f(h);
}

// x / d rounded to nearest for a divisor d that is an fp16 value (at most 11
// significant bits), from d's correctly rounded reciprocal inv = 1 / d:
// q0 = x inv, then one correction with the exact residual x - q0 d.  For
// every pair of significands (x any of the 2^23, d any of the 2^10) the
// result equals the IEEE quotient (checked exhaustively on the CPU);
// exponents only scale it, so it is exact while x, the residual and the
// quotient stay normal: |x| >= 2^-100 and |q0| <= 2^126.  x = 0 gives a
// zero of either sign.
__device__ __forceinline__ float div_half(float x, float d, float inv) {
  const float q0 = x * inv;
  const float r = fmaf(-q0, d, x);
  return fmaf(r, inv, q0);
}

// compile-time switch for the two forms of a loop
template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

// float -> bfloat16 bits by v_cvt_pk_bf16_f32 (round to nearest even, as
// torch's .bfloat16() for every non-NaN input)
__device__ __forceinline__ uint32_t f2bf(float f) {
  asm("" : "+v"(f));  // a separate rounding step, as for f2h
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
// two floats rounded to bf16 (nearest even, as f2bf) in one packed
// conversion; a in the low half
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v){a, b}, bf16x2_v));
}

__device__ __forceinline__ float load_val(const void *p, int dtype, int64_t idx) {
  if (dtype == SQ_F32) return ((const float *)p)[idx];
  if (dtype == SQ_BF16) return __uint_as_float((uint32_t)((const uint16_t *)p)[idx] << 16);
  return h2f(((const uint16_t *)p)[idx]);
}

__device__ __forceinline__ void store_val(void *p, int dtype, int64_t idx, float v) {
  if (dtype == SQ_F32) ((float *)p)[idx] = v;
  else if (dtype == SQ_BF16) ((uint16_t *)p)[idx] = (uint16_t)f2bf(v);
  else ((uint16_t *)p)[idx] = (uint16_t)f2h(v);
}

// four consecutive elements (one dtype test for all four)
__device__ __forceinline__ void load4(const void *p, int dtype, int64_t idx, float o[4]) {
  if (dtype == SQ_F32) {
    const float *f = (const float *)p + idx;
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = f[c];
  } else if (dtype == SQ_BF16) {
    const uint16_t *u = (const uint16_t *)p + idx;
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = __uint_as_float((uint32_t)u[c] << 16);
  } else {
    const uint16_t *u = (const uint16_t *)p + idx;
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = h2f(u[c]);
  }
}

__device__ __forceinline__ void store4(void *p, int dtype, int64_t idx, const float v[4]) {
  if (dtype == SQ_F32) {
    float *f = (float *)p + idx;
#pragma unroll
    for (int c = 0; c < 4; c++) f[c] = v[c];
  } else if (dtype == SQ_BF16) {
    uint16_t *u = (uint16_t *)p + idx;
#pragma unroll
    for (int c = 0; c < 4; c++) u[c] = (uint16_t)f2bf(v[c]);
  } else {
    uint16_t *u = (uint16_t *)p + idx;
#pragma unroll
    for (int c = 0; c < 4; c++) u[c] = (uint16_t)f2h(v[c]);
  }
}

// four consecutive elements starting at a multiple of 4 of an 8-byte aligned
// array: 16-bit values go out as one 8-byte store instead of four 2-byte ones
__device__ __forceinline__ void store4_aligned(void *p, int dtype, int64_t idx, const float v[4]) {
  if (dtype == SQ_F32) {
    *(float4 *)((float *)p + idx) = make_float4(v[0], v[1], v[2], v[3]);
    return;
  }
  if (dtype == SQ_BF16) {
    float w[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
    for (int c = 0; c < 4; c++) asm("" : "+v"(w[c]));  // a separate rounding step, as for f2bf
    *(uint2 *)((uint16_t *)p + idx) = make_uint2(bf16x2_bits(w[0], w[1]), bf16x2_bits(w[2], w[3]));
    return;
  }
  uint32_t e[4];
#pragma unroll
  for (int c = 0; c < 4; c++) e[c] = f2h(v[c]);
  *(uint2 *)((uint16_t *)p + idx) = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
}

__device__ __forceinline__ int64_t load_slot(const void *p, int dtype, int64_t idx) {
  return dtype == SQ_I64 ? ((const int64_t *)p)[idx] : (int64_t)((const int32_t *)p)[idx];
}

// A workgroup-uniform read of memory that no kernel writes while it runs
// (tables, slot lists, inputs), through the constant address space so that
// it becomes a scalar load: its wait does not wait for the vector loads.
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)p;
}

__device__ __forceinline__ int64_t load_slot_uniform(const void *p, int dtype, int64_t idx) {
  return dtype == SQ_I64 ? ld_uniform((const int64_t *)p + idx) : (int64_t)ld_uniform((const int32_t *)p + idx);
}

__device__ __forceinline__ uint32_t page_half(const uint8_t *page, int64_t byte) {
  return (uint32_t)page[byte] | ((uint32_t)page[byte + 1] << 8);
}

__device__ __forceinline__ void put_page_half(uint8_t *page, int64_t byte, uint32_t h) {
  *(uint16_t *)(page + byte) = (uint16_t)h;  // byte offsets of scales are even
}

// ------------------------------------------------ LDS staging of a region

// Stage global bytes [gstart, gend) (2-byte aligned) into LDS.  The LDS copy
// starts at the enclosing 16-byte boundary: lds byte (a - w16) holds global
// byte a.  Returns the offset of gstart inside the staged window.
__device__ __forceinline__ int stage_in(const uint8_t *gstart, int64_t nbytes, uint8_t *lds, int tid,
                                        int nthreads) {
  // pointer arithmetic (not integer casts) keeps the global address space
  const int shift = (int)((uintptr_t)gstart & 15);
  const uint4 *src = (const uint4 *)(gstart - shift);
  const int n16 = (int)((shift + nbytes + 15) >> 4);
  uint4 *dst = (uint4 *)lds;
  for (int c = tid; c < n16; c += nthreads) dst[c] = src[c];
  return shift;
}

// Write LDS back to [gstart, gstart + nbytes): whole 16-byte chunks inside
// the region use 16-byte stores, edge chunks store only the region's 2-byte
// units (from one 16-byte LDS read).  `lds` is the staged window as returned
// by stage_in (global byte a lives at lds + (a - floor16(gstart))).
__device__ __forceinline__ void stage_out(uint8_t *gstart, int64_t nbytes, const uint8_t *lds, int tid,
                                          int nthreads) {
  const int shift = (int)((uintptr_t)gstart & 15);
  uint8_t *w16 = gstart - shift;
  const int64_t end = shift + nbytes;  // region end relative to w16
  const int n16 = (int)((end + 15) >> 4);
  for (int c = tid; c < n16; c += nthreads) {
    const int64_t a = 16 * (int64_t)c;
    const uint4 v = ((const uint4 *)lds)[c];
    if (a >= shift && a + 16 <= end) {
      *(uint4 *)(w16 + a) = v;
    } else {
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int64_t b = a + 2 * u;
        if (b >= shift && b + 2 <= end) *(uint16_t *)(w16 + b) = (uint16_t)(wv[u >> 1] >> (16 * (u & 1)));
      }
    }
  }
}

// 32 bits little-endian starting at an arbitrary LDS byte (4 spare bytes
// after the staged window keep the second dword in bounds).
__device__ __forceinline__ uint32_t lds_word(const uint8_t *lds, int p) {
  const uint32_t *w = (const uint32_t *)(lds + (p & ~3));
  uint32_t lo = w[0], hi = w[1];
  return __builtin_amdgcn_alignbit(hi, lo, (uint32_t)(p & 3) * 8u);
}

__device__ __forceinline__ void lds_put_bytes(uint8_t *lds, int p, uint32_t word, int nbytes) {
  for (int b = 0; b < nbytes; b++) lds[p + b] = (uint8_t)(word >> (8 * b));
}

// ---------------------------------------- PyTorch CPU summation order (f32)

// Streaming form of aten SumKernel.cpp multi_row_sum: terms arrive in row-
// major order (row ii, column k); R accumulators per level; 16-row cascade.
template <int R>
struct TorchCascade {
  float acc[4][R];
  int64_t size, ii;
  int k;
  __device__ void init(int64_t rows) {
    size = rows;
    ii = 0;
    k = 0;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int c = 0; c < R; c++) acc[a][c] = 0.0f;
  }
  __device__ void push(float t) {
    // caller guarantees (ii, k) is inside size x R
#pragma unroll
    for (int c = 0; c < R; c++)
      if (c == k) acc[0][c] += t;
    if (++k == R) {
      k = 0;
      ++ii;
      if ((ii & 15) == 0 && ii <= size) {
        for (int j = 1; j < 4; j++) {
#pragma unroll
          for (int c = 0; c < R; c++) {
            acc[j][c] += acc[j - 1][c];
            acc[j - 1][c] = 0.0f;
          }
          if (ii & ((int64_t)15 << (4 * j))) break;
        }
      }
    }
  }
  __device__ void finish(float *out) {
#pragma unroll
    for (int c = 0; c < R; c++) {
      float a = acc[0][c];
      a += acc[1][c];
      a += acc[2][c];
      a += acc[3][c];
      out[c] = a;
    }
  }
};

// row_sum with ilp factor 4 over n terms given by f(i), i ascending.
template <typename F>
__device__ float torch_row_sum_ilp4(int64_t n, F f) {
  TorchCascade<4> cas;
  const int64_t size_ilp = n / 4;
  cas.init(size_ilp);
  for (int64_t i = 0; i < size_ilp * 4; i++) cas.push(f(i));
  float p[4];
  cas.finish(p);
  for (int64_t i = size_ilp * 4; i < n; i++) p[0] += f(i);
  p[0] += p[1];
  p[0] += p[2];
  p[0] += p[3];
  return p[0];
}

// x.sum(-1) order for n contiguous values f(0..n-1) (8-wide vectors).
template <typename F>
__device__ float torch_inner_sum(int64_t n, F f) {
  if (n < 8) return torch_row_sum_ilp4(n, f);
  const int64_t nvec = n / 8;
  float total = 0.0f;
  for (int64_t t = nvec * 8; t < n; t++) total += f(t);
  for (int l = 0; l < 8; l++) total += torch_row_sum_ilp4(nvec, [&](int64_t m) { return f(8 * m + l); });
  return total;
}

// torch_inner_sum of row[0..n-1], one vector lane at a time: the same
// operations in the same order, with the lanes' loads not all in flight at
// once (fully unrolled, they would hold n registers)
__device__ float inner_sum_lanewise(const float *row, int n) {
  if (n < 8) return torch_row_sum_ilp4(n, [&](int64_t t) { return row[t]; });
  const int nvec = n / 8;
  float total = 0.0f;
  for (int t = nvec * 8; t < n; t++) total += row[t];
#pragma unroll 1
  for (int l = 0; l < 8; l++) total += torch_row_sum_ilp4(nvec, [&](int64_t m) { return row[8 * m + l]; });
  return total;
}

// -------------------------------------------------------- pool metadata

struct PoolDev {
  uint8_t *data;
  int64_t page_bytes;
  int64_t num_slots;
  const int32_t *bits, *offsets, *rows, *columns, *head_meta;
  const float *impact;
  int H, K, V, G, kda;
  int ng, ngsh;  // K=V=128 kernels: row-scale groups of a 2-bit row (128 / G) and its log2
  int stage;   // bytes of LDS staging per workgroup (largest head window)
  int rstage;  // bytes of LDS for one head's row scales (fast path)
  int fast;    // SQ_POOL_FAST_* bits: which K=V=128 kernel the pool qualifies for
  int storage; // 0: packed codes; 1: int8 carriers, plane value (i, j) at base + i + j*K
  int hrot;    // K=V=128 step kernels: H - 1 when H is a power of two (head of block (x, y) is (x + y) & hrot), else 0
};

__device__ __forceinline__ int tile_of(const PoolDev &P) { return P.kda ? (P.V < 4 ? P.V : 4) : (P.V < 16 ? P.V : 16); }

// Byte position (relative to the head's code region) of the 4-value group
// starting at column j0 in row i; pivots use width 16.
__device__ __forceinline__ int group_pos(int off_rel, int stride, int tile, int j0, int width) {
  return off_rel + (j0 / tile) * stride + ((j0 % tile) * width) / 8;
}

// Byte position of FP16 pivot value j of a row: tiled with the codes in
// packed pages, a contiguous row of V halves in byte pages (pool.py:33-40).
__device__ __forceinline__ int pivot_pos(const PoolDev &P, int off_rel, int stride, int tile, int j) {
  return P.storage ? off_rel + 2 * j : group_pos(off_rel, stride, tile, j, 16);
}

// int8 carrier of value (i, j) in a byte page: the head's plane starts at
// offsets[H*K + h] (relative: plane_rel) and holds value (i, j) at i + j*K;
// the carrier is z (KDA: z * 2^(8 - b), so that x = r c carrier).
__device__ __forceinline__ int carrier_pos(int plane_rel, int K, int i, int j) { return plane_rel + i + j * K; }

__device__ __forceinline__ int colbase_of(const PoolDev &P, int h) { return P.columns[h]; }

// Cross-lane moves without the LDS crossbar (DPP): the value of lane i + N
// of the same 16-lane row, and a permutation within each group of four lanes.
template <int N>
__device__ __forceinline__ float row_shl(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x100 + N, 0xF, 0xF, true));
}
template <int PERM>
__device__ __forceinline__ uint32_t quad_perm(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, PERM, 0xF, 0xF, true);
}

// =====================================================================
// Encode, GDN heads of one width (no FP16 pivots), K = V = 128, packed,
// NTH threads (512: 16 row groups of 32 lanes, 4 threads per column).
// Every value of the tile is loaded once per layout, both batches issued
// together before any arithmetic: row layout for the row scales (row group
// rw = tid / 32 takes rows rw + (NTH / 32) p, lane (l, k) = (lane / 4,
// lane % 4) the values 32u + 8k + l), column layout (thread j + 128 hf: rows
// CR hf .. CR hf + CR - 1 of column j, CR = 128 * 128 / NTH) for the column
// scales and codes.  The operations and their order are those of the
// general path below (the sums in PyTorch's order).
// =====================================================================
// Four codes b0..b3 (< 2^W), one per byte of x, as consecutive W-bit
// fields (b0 lowest): the packed 4-value group of a row.
template <int W>
__device__ __forceinline__ uint32_t pack_bytes(uint32_t x) {
  if (W == 8) return x;
  if (W == 4) return __builtin_amdgcn_perm(0u, x | (x >> 4), 0x0c0c0200u);  // bytes 0 and 2 of b0|b1<<4, b2|b3<<4
  if (W == 2) {
    const uint32_t y = x | (x >> 6);  // byte 0: b0 | b1 << 2, byte 2: b2 | b3 << 2
    return (y & 0xfu) | ((y >> 12) & 0xf0u);
  }
  // W == 6: b0, b1 at bits 0 and 6, b2, b3 at bits 16 and 22, then bits
  // [16, 28) moved down to [12, 24) by one bitfield insert
  const uint32_t y = (x & 0x003f003fu) | ((x >> 2) & 0x0fc00fc0u);
  uint32_t w;
  __asm__("v_bfi_b32 %0, %1, %2, %3" : "=v"(w) : "s"(0xfffu), "v"(y), "v"(y >> 4));
  return w;
}

template <int W, int NTH>
__device__ __forceinline__ void encode_fast128(const PoolDev &P, const float *__restrict__ X, uint8_t *page,
                                               uint8_t *smem, int h) {
#pragma clang fp contract(off)
  constexpr int K = 128, V = 128;
  const int tid = threadIdx.x;
  constexpr bool two = W == 2;
  const int NG = two ? V / 32 : 1;
  const int ngrp = two ? 32 : V;
  const int32_t *hm = P.head_meta + 4 * h;
  const int code_start = hm[0], code_bytes = hm[1];
  const int stride = P.offsets[(int64_t)P.H * K + h];
  const int shift = (int)((uintptr_t)(page + code_start) & 15);
  uint8_t *stage = smem;
  float *rsc = (float *)(smem + P.stage);  // [K][NG]
  float *wl = rsc + K * 4;                 // [K] squared fit weights w^2
  int *orel = (int *)(wl + K);             // [K] row offsets within the code region
  constexpr int HALVES = NTH / 32, RP = K / HALVES;  // 32-lane row groups, rows per group
  constexpr int CT = NTH / V, CR = K / CT;             // threads per column, rows per thread
  static_assert(RP * 4 <= 32 && CR % 16 == 0, "row groups hold at most 8 rows, columns whole 16-row blocks");
  float *cmax = (float *)(orel + K);       // [CT][V]
  float *bsum = cmax + CT * V;             // [K/16][2][V]
  float *rinv = bsum + (K / 16) * 2 * V;   // [K][NG] 1 / row scale, correctly rounded

  // The column phase divides by fp16 scales (row scales, c0, c): with their
  // correctly rounded reciprocals, div_half gives the IEEE quotient when
  // every value is 0 or 2^-76 <= |x| <= 2^60 (scales lie in [2^-24, 65504],
  // so the quotients stay within [2^-92, 2^108]).  Tiles with a value
  // outside (or a NaN or infinity) divide with IEEE division.
  uint32_t lo_bits = 0xffffffffu, hi_bits = 0u;  // min of |x| bits - 1 (zeros wrap), max of |x| bits
  // this thread's CR values of column j (the column phase's layout), loaded
  // together with the row layout's values below: one wait for memory
  const int j = tid & (V - 1), hf = tid >> 7, i0 = CR * hf;
  float xs[CR], sc[CR];
#pragma unroll
  for (int r = 0; r < CR; r++) xs[r] = X[(i0 + r) * V + j];
  // ---- row phase.  Each 32-lane half takes rows rw + HALVES p; its row
  // sums (in PyTorch's order) land in lane 0 and go through LDS to lane
  // p NG + g, so the scale arithmetic of the half's RP NG (row, group) pairs
  // runs once, side by side, instead of once per pair on lane 0.
  {
    const int lane = tid & 31, l = lane >> 2, k = lane & 3, rw = tid >> 5;
    float v[RP][4];
    // lane e < RP NG: the inputs of pair (p, g) = (e / NG, e % NG)
    const int pe = lane / NG, ge = lane % NG, ie = rw + HALVES * (pe & (RP - 1));
    const float wie = P.impact[(int64_t)h * K + ie];
    const int roe = P.rows[(int64_t)h * K + ie], ofe = P.offsets[(int64_t)h * K + ie];
#pragma unroll
    for (int p = 0; p < RP; p++) {
      const int i = rw + HALVES * p;
#pragma unroll
      for (int u = 0; u < 4; u++) v[p][u] = X[i * V + 32 * u + 8 * k + l];
    }
#pragma unroll
    for (int p = 0; p < RP; p++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const uint32_t a = __float_as_uint(v[p][u]) & 0x7fffffffu;
        lo_bits = min(lo_bits, a - 1u);
        hi_bits = max(hi_bits, a);
      }
    float *tot = cmax + 32 * rw;  // the half's row sums (cmax is free until the column phase)
#pragma unroll
    for (int p = 0; p < RP; p++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        if (g >= NG) break;
        // 2-bit: one term per lane and group; otherwise four (ii ascending)
        float acc = 0.0f;
        if (two) {
          acc += fabsf(v[p][g]);
        } else {
#pragma unroll
          for (int u = 0; u < 4; u++) acc += fabsf(v[p][u]);
        }
        // lanes 4q of each half: sl = acc(4q) + acc(4q+1) + acc(4q+2) + acc(4q+3);
        // lane 0 of each half: total = sl(0) + sl(4) + ... + sl(28), in order
        float sl = acc;
        sl += row_shl<1>(acc);
        sl += row_shl<2>(acc);
        sl += row_shl<3>(acc);
        const float up = __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(sl), __float_as_uint(sl),
                                                                          false, false)[1]);  // lane + 16
        float total = 0.0f;
        total += sl;
        total += row_shl<4>(sl);
        total += row_shl<8>(sl);
        total += row_shl<12>(sl);
        total += up;
        total += row_shl<4>(up);
        total += row_shl<8>(up);
        total += row_shl<12>(up);
        if (lane == 0) tot[p * NG + g] = total;
      }
    }
    // (the LDS accesses of one wave complete in order: lane e reads what lane 0 wrote)
    if (lane < RP * NG) {
      const int i = ie, g = ge;
      float m = tot[lane] / (float)ngrp;
      m = m < 1e-20f ? 1e-20f : m;
      uint32_t hb;
      const float r = fp16_scale(__builtin_sqrtf(m / wie), &hb);
      rsc[i * NG + g] = r;
      rinv[i * NG + g] = 1.0f / r;
      put_page_half(page, roe + 2 * g, hb);
      if (g == 0) {
        wl[i] = wie * wie;
        orel[i] = ofe - code_start;
      }
    }
  }
  // ---- column phase: the thread's values of column j, raw and scaled
  const int g = two ? j / 32 : 0;
  const bool ieee = __syncthreads_or(lo_bits < 0x19800000u - 1u || hi_bits > 0x5d800000u);
  auto columns = [&](auto fast_tag) {
  constexpr bool FAST = decltype(fast_tag)::value;
  float amax = 0.0f;
#pragma unroll
  for (int r = 0; r < CR; r++) {
    const int ig = (i0 + r) * NG + g;
    sc[r] = FAST ? div_half(xs[r], rsc[ig], rinv[ig]) : xs[r] / rsc[ig];
    const float a = fabsf(sc[r]);
    amax = a > amax ? a : amax;
  }
  cmax[hf * V + j] = amax;
  __syncthreads();
  float am = 0.0f;
#pragma unroll
  for (int u = 0; u < CT; u++) {
    const float a = cmax[u * V + j];
    am = a > am ? a : am;
  }
  const float qmax = two ? 3.0f : (float)((1 << (W - 1)) - 1);
  const float t0 = am / (qmax * 1.0f);
  const float c0 = fp16_scale(t0 > 0.0f ? t0 : 0.0f, nullptr);
  const float c0inv = 1.0f / c0;
  auto zq = [&](float s, float cdiv, float cinv) -> float {
    const float y = FAST ? div_half(s, cdiv, cinv) : s / cdiv;
    if (two) return (y >= 0.0f ? 1.0f : -1.0f) * (fabsf(y) >= 2.0f ? 3.0f : 1.0f);
    return __builtin_amdgcn_fmed3f(__builtin_rintf(y), -qmax, qmax);
  };
  // refit sums: CR / 16 blocks of 16 rows per thread, each from zero
#pragma unroll
  for (int mb = 0; mb < CR / 16; mb++) {
    float bn = 0.0f, bd = 0.0f;
#pragma unroll
    for (int rr = 0; rr < 16; rr++) {
      const int r = 16 * mb + rr, i = i0 + r;
      const float wsq = wl[i];  // (w w) 1 of integer rows: the factor 1 is exact
      const float z = zq(sc[r], c0, c0inv);
      const float v = (rsc[i * NG + g] * 1.0f) * z;
      bn += (wsq * v) * xs[r];
      bd += wsq * (v * v);
    }
    const int m = (CR / 16) * hf + mb;
    bsum[(2 * m) * V + j] = bn;
    bsum[(2 * m + 1) * V + j] = bd;
  }
  __syncthreads();
  float num = 0.0f, den = 0.0f;
#pragma unroll
  for (int m = 0; m < K / 16; m++) {
    num += bsum[(2 * m) * V + j];
    den += bsum[(2 * m + 1) * V + j];
  }
  const float denc = den < 1e-30f ? 1e-30f : den;
  uint32_t chb;
  const float c = fp16_scale(den > 0.0f ? num / denc : c0, &chb);
  const float cinv = 1.0f / c;
  const int colbase = P.columns[h];
  if (hf == 0 && colbase >= 0) put_page_half(page, colbase + 2 * (int64_t)j, chb);
  // final codes: each lane converts its column's codes of rows 4t .. 4t + 3
  // into the bytes of one dword; a 4 x 4 byte transpose within the quad of
  // lanes j & ~3 .. j | 3 (two lane exchanges, two byte permutes) leaves lane
  // q with the four codes of row 4t + q in the quad's 4-value group, which it
  // packs into W-bit fields and stores (the rows of a head of one width
  // follow each other 2W bytes apart)
  const float L = two ? 3.0f : (float)((1 << (W - 1)) - 1);
  const int q = j & 3;
  const uint32_t sel1 = (q & 1) ? 0x03070105u : 0x06020400u;  // [nb1 own1 nb3 own3] / [own0 nb0 own2 nb2]
  const uint32_t sel2 = (q & 2) ? 0x03020706u : 0x05040100u;  // [nb2 nb3 own2 own3] / [own0 own1 nb0 nb1]
  const int pos0 = shift + group_pos(orel[i0], stride, 16, j & ~3, W) + q * 2 * W;
#pragma unroll
  for (int t = 0; t < CR / 4; t++) {
    uint32_t w4 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float z = zq(sc[4 * t + k], c, cinv);
      const float code = two ? (z + 3.0f) * 0.5f : z + L;  // an exact small integer
      w4 = __builtin_amdgcn_cvt_pk_u8_f32(code, k, w4);
    }
    w4 = __builtin_amdgcn_perm(quad_perm<0xB1>(w4), w4, sel1);  // lane ^ 1
    w4 = __builtin_amdgcn_perm(quad_perm<0x4E>(w4), w4, sel2);  // lane ^ 2
    lds_put_bytes(stage, pos0 + 4 * t * 2 * W, pack_bytes<W>(w4), W / 2);
  }
  };
  if (ieee) columns(BoolTag<false>{});
  else columns(BoolTag<true>{});
  __syncthreads();
  stage_out(page + code_start, code_bytes, stage, tid, NTH);
}

// GDN pools with K = V = 128 (packed, 2-bit groups of 32): the fast form
// above, FP16 pivot heads as halves of every value.
// 512 threads per tile, 4 waves per SIMD (1024 threads at 8 waves per SIMD
// measured the same)
#ifndef ENC128_NT
#define ENC128_NT 512
#endif
#ifndef ENC128_WAVES
#define ENC128_WAVES 4
#endif
__global__ __launch_bounds__(ENC128_NT) __attribute__((amdgpu_waves_per_eu(ENC128_WAVES))) void encode128_kernel(
    PoolDev P, const float *__restrict__ state, const void *slots, int slots_dtype) {
  constexpr int NTH = ENC128_NT;
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = P.H;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int64_t slot = load_slot(slots, slots_dtype, b);
  if (slot <= 0 || slot >= P.num_slots) return;  // masked (or outside the pool)
  uint8_t *page = P.data + slot * P.page_bytes;
  const float *X = state + ((int64_t)b * H + h) * 128 * 128;
  const int W = P.bits[(int64_t)h * 128];
  switch (W) {  // the width as a compile-time constant: code packing without loops or branches
    case 2: encode_fast128<2, NTH>(P, X, page, smem, h); return;
    case 4: encode_fast128<4, NTH>(P, X, page, smem, h); return;
    case 6: encode_fast128<6, NTH>(P, X, page, smem, h); return;
    case 8: encode_fast128<8, NTH>(P, X, page, smem, h); return;
    default: break;
  }
  // pivot head: value (i, j) as a half at its tiled position
  const int code_start = P.head_meta[4 * h];
  const int stride = P.offsets[(int64_t)H * 128 + h];
  for (int e = threadIdx.x; e < 128 * 128; e += NTH) {
    const int i = e >> 7, j = e & 127;
    const int off = P.offsets[(int64_t)h * 128 + i];
    put_page_half(page, (int64_t)code_start + (off - code_start) + (j / 16) * stride + (j % 16) * 2, f2h(X[e]));
  }
}

// =====================================================================
// Encode, KDA pools with K = V = 128, packed: per-row widths (2, 4, 6, 8)
// and FP16 pivot rows, 4-value tiles, 512 threads.  The operations and
// their order are those of encode_kernel's split path (four threads per
// column, 16-row blocks of the refit sums), with every value of the tile
// loaded once per layout into registers (row layout for the row scales,
// column layout for the rest), so a tile waits for memory twice rather than
// once per row and pass, and the divisions by fp16 scales use their
// correctly rounded reciprocals (div_half) when the tile's values allow it.
// =====================================================================
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void encode_kda128_kernel(
    PoolDev P, const float *__restrict__ state, const void *slots, int slots_dtype) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int K = 128, V = 128;
  const int H = P.H;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int tid = threadIdx.x;
  const int64_t slot = load_slot(slots, slots_dtype, b);
  if (slot <= 0 || slot >= P.num_slots) return;  // masked (or outside the pool)
  uint8_t *page = P.data + slot * P.page_bytes;
  const float *X = state + ((int64_t)b * H + h) * K * V;
  const int32_t *hm = P.head_meta + 4 * h;
  const int code_start = hm[0], code_bytes = hm[1];
  const int stride = P.offsets[(int64_t)H * K + h];
  const int shift = (int)((uintptr_t)(page + code_start) & 15);
  uint8_t *stage = smem;
  float *rsc = (float *)(smem + P.stage);  // [K] row scales (1 for pivots)
  float *rinv = rsc + K;                   // [K] 1 / row scale
  float *wl = rinv + K;                    // [K] fit weights
  int *bl = (int *)(wl + K);               // [K] widths
  int *orel = bl + K;                      // [K] row offsets within the code region
  float *cmax = (float *)(orel + K);       // [4 parts][4 widths][V]
  float *bsum = cmax + 16 * V;             // [K/16][2][V]
  // per row: qmax, 1 / norm, r norm, w^2 (0 for pivots) | width, L, row offset, width class
  float4 *rowc = (float4 *)(bsum + (K / 16) * 2 * V);
  int4 *rowi = (int4 *)(rowc + K);
  uint32_t lo_bits = 0xffffffffu, hi_bits = 0u;  // min of |x| bits - 1 (zeros wrap), max of |x| bits
  // ---- row phase: r = fp16(sqrt(max(mean|x|, 1e-20) / w)) in PyTorch's
  // summation order (as encode_fast128); pivot rows as halves.  Each 32-lane
  // half takes rows rw + 16 p; lane 0's row sums reach lane p through LDS,
  // and the scale arithmetic of the half's 8 rows runs side by side.
  {
    const int lane = tid & 31, l = lane >> 2, k = lane & 3, rw = tid >> 5;
    float v[8][4];
    int of[8], bi[8];
    const int ie = rw + 16 * (lane & 7);  // lane p < 8: row rw + 16 p
    const float wie = P.impact[(int64_t)h * K + ie];
    const int roe = P.rows[(int64_t)h * K + ie];
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const int i = rw + 16 * p;
#pragma unroll
      for (int u = 0; u < 4; u++) v[p][u] = X[i * V + 32 * u + 8 * k + l];
      of[p] = P.offsets[(int64_t)h * K + i];
      bi[p] = P.bits[(int64_t)h * K + i];
    }
    // the existing code region (padding bytes before pivot rows keep their
    // contents, as in encode_kernel), staged after the tile's loads
    stage_in(page + code_start, code_bytes, stage, tid, 512);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 8; p++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const uint32_t a = __float_as_uint(v[p][u]) & 0x7fffffffu;
        lo_bits = min(lo_bits, a - 1u);
        hi_bits = max(hi_bits, a);
      }
    float *tot = cmax + 8 * rw;  // the half's row sums (cmax is free until the column phase)
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const int off_rel = of[p] - code_start;
      if (bi[p] == 16) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int j = 32 * u + 8 * k + l;
          const int pos = shift + group_pos(off_rel, stride, 4, j, 16);
          const uint32_t hb = f2h(v[p][u]);
          stage[pos] = (uint8_t)hb;
          stage[pos + 1] = (uint8_t)(hb >> 8);
        }
      }
      float acc = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; u++) acc += fabsf(v[p][u]);
      float sl = acc;
      sl += row_shl<1>(acc);
      sl += row_shl<2>(acc);
      sl += row_shl<3>(acc);
      const float up = __uint_as_float(
          __builtin_amdgcn_permlane16_swap(__float_as_uint(sl), __float_as_uint(sl), false, false)[1]);
      float total = 0.0f;
      total += sl;
      total += row_shl<4>(sl);
      total += row_shl<8>(sl);
      total += row_shl<12>(sl);
      total += up;
      total += row_shl<4>(up);
      total += row_shl<8>(up);
      total += row_shl<12>(up);
      if (lane == 0) tot[p] = total;
    }
    // (the LDS accesses of one wave complete in order: lane p reads what lane 0 wrote)
    if (lane < 8) {
      const int i = ie, bw = P.bits[(int64_t)h * K + i];
      const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
      float r = 1.0f;
      if (bw == 16) {
        rsc[i] = 1.0f;
        rinv[i] = 1.0f;
      } else {
        float m = tot[lane] / (float)V;
        m = m < 1e-20f ? 1e-20f : m;
        uint32_t hb;
        r = fp16_scale(__builtin_sqrtf(m / wie), &hb);
        rsc[i] = r;
        rinv[i] = 1.0f / r;
        put_page_half(page, roe, hb);
      }
      wl[i] = wie;
      bl[i] = bw;
      orel[i] = off_rel;
      // the column phase's per-row factors, formed as it would form them
      const int bc = bw < 8 ? bw : 8;
      const float norm = (float)(1 << (8 - bc));
      rowc[i] = make_float4((float)((1 << (bc - 1)) - 1), 1.0f / norm, r * norm, (wie * wie) * (bw != 16 ? 1.0f : 0.0f));
      rowi[i] = make_int4(bw, (1 << (bc - 1)) - 1, off_rel, bc / 2 - 1);
    }
  }
  // ---- column phase: this thread's 32 values of column j (rows 32 hf ..)
  const int j = tid & (V - 1), hf = tid >> 7, i0 = 32 * hf;
  float xs[32], sc[32];
#pragma unroll
  for (int r = 0; r < 32; r++) xs[r] = X[(i0 + r) * V + j];
  const bool ieee = __syncthreads_or(lo_bits < 0x19800000u - 1u || hi_bits > 0x5d800000u);
  // Every lane of a wave works on the same row at a time (rows i0 + r, i0
  // wave-uniform), so a row's factors are read into scalar registers: the
  // width-dependent choices become scalar branches and the per-value work
  // is the arithmetic alone.
  auto ufl = [](float x) { return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x))); };
  auto columns = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
    float amax[4] = {0.f, 0.f, 0.f, 0.f};  // widths 2, 4, 6, 8
#pragma unroll
    for (int r = 0; r < 32; r++) {
      if (r % 8 == 0) __builtin_amdgcn_sched_barrier(0);  // row factors loaded 8 rows at a time
      const int i = i0 + r;
      sc[r] = FAST ? div_half(xs[r], ufl(rsc[i]), ufl(rinv[i])) : xs[r] / ufl(rsc[i]);
      const int w = __builtin_amdgcn_readfirstlane(rowi[i].x);
      if (w == 16) continue;
      const float a = fabsf(sc[r]);
      const int wsel = (w < 8 ? w : 8) / 2 - 1;
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (q == wsel) amax[q] = a > amax[q] ? a : amax[q];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) cmax[(hf * 4 + q) * V + j] = amax[q];
    __syncthreads();
    float mx = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float am = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float a = cmax[(u * 4 + q) * V + j];
        am = a > am ? a : am;
      }
      const int bc = 2 * q + 2;
      const float qmax = (float)((1 << (bc - 1)) - 1);
      const float norm = (float)(1 << (8 - bc));
      const float t = am / (qmax * norm);
      mx = t > mx ? t : mx;
    }
    const float c0 = fp16_scale(mx, nullptr);
    const float c0inv = 1.0f / c0;
    // level of a scaled value in a row of quantisation range qmax (1 / norm: the row's power of two)
    auto zq = [&](float s, float cdiv, float cinv, float qmax, float inv_norm) -> float {
      float y = FAST ? div_half(s, cdiv, cinv) : s / cdiv;
      y = y * inv_norm;  // exact: norm is a power of two
      float z = __builtin_rintf(y);
      z = z > -qmax ? z : -qmax;
      z = z < qmax ? z : qmax;
      return z;
    };
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
      float bn = 0.0f, bd = 0.0f;
#pragma unroll
      for (int rr = 0; rr < 16; rr++) {
        const int r = 16 * mb + rr, i = i0 + r;
        if (rr % 8 == 0) __builtin_amdgcn_sched_barrier(0);
        const float wsq = ufl(rowc[i].w);
        const float z = zq(sc[r], c0, c0inv, ufl(rowc[i].x), ufl(rowc[i].y));
        const float v = ufl(rowc[i].z) * z;
        bn += (wsq * v) * xs[r];
        bd += wsq * (v * v);
      }
      const int m = 2 * hf + mb;
      bsum[(2 * m) * V + j] = bn;
      bsum[(2 * m + 1) * V + j] = bd;
    }
    __syncthreads();
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int m = 0; m < K / 16; m++) {
      num += bsum[(2 * m) * V + j];
      den += bsum[(2 * m + 1) * V + j];
    }
    const float denc = den < 1e-30f ? 1e-30f : den;
    uint32_t chb;
    const float c = fp16_scale(den > 0.0f ? num / denc : c0, &chb);
    const float cinv = 1.0f / c;
    const int colbase = P.columns[h];
    if (hf == 0 && colbase >= 0) put_page_half(page, colbase + 2 * (int64_t)j, chb);
    // final codes: each lane converts its column's codes of rows 4t .. 4t + 3
    // into the bytes of one dword; a 4 x 4 byte transpose within the quad of
    // lanes j & ~3 .. j | 3 (two lane exchanges, two byte permutes) leaves
    // lane q with the four codes of row 4t + q in the quad's 4-value tile,
    // which it packs with that row's width and stores (pivot rows: nothing)
    const int q = j & 3;
    const uint32_t sel1 = (q & 1) ? 0x03070105u : 0x06020400u;  // [nb1 own1 nb3 own3] / [own0 nb0 own2 nb2]
    const uint32_t sel2 = (q & 2) ? 0x03020706u : 0x05040100u;  // [nb2 nb3 own2 own3] / [own0 own1 nb0 nb1]
    const int blk = shift + (j >> 2) * stride;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      if (t % 2 == 0) __builtin_amdgcn_sched_barrier(0);
      uint32_t w4 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int r = 4 * t + k, i = i0 + r;
        // pivot rows give an unused byte (their lane stores nothing)
        const float z = zq(sc[r], c, cinv, ufl(rowc[i].x), ufl(rowc[i].y));
        const float code = z + (float)__builtin_amdgcn_readfirstlane(rowi[i].y);
        w4 = __builtin_amdgcn_cvt_pk_u8_f32(code, k, w4);  // code >= 0: z + L with z in [-L, L]
      }
      w4 = __builtin_amdgcn_perm(quad_perm<0xB1>(w4), w4, sel1);  // lane ^ 1
      w4 = __builtin_amdgcn_perm(quad_perm<0x4E>(w4), w4, sel2);  // lane ^ 2
      const int4 ri = rowi[i0 + 4 * t + q];  // this lane's row: width, L, row offset, width class
      const int w = ri.x;
      if (w != 16) {
        const uint32_t word = (w4 & 0xffu) | (((w4 >> 8) & 0xffu) << w) | (((w4 >> 16) & 0xffu) << (2 * w)) |
                              ((w4 >> 24) << (3 * w));
        uint8_t *dst = stage + blk + ri.z;
        dst[0] = (uint8_t)word;
        if (w >= 4) dst[1] = (uint8_t)(word >> 8);
        if (w >= 6) dst[2] = (uint8_t)(word >> 16);
        if (w == 8) dst[3] = (uint8_t)(word >> 24);
      }
    }
  };
  if (ieee) columns(BoolTag<false>{});
  else columns(BoolTag<true>{});
  __syncthreads();
  stage_out(page + code_start, code_bytes, stage, tid, 512);
}

// =====================================================================
// Encode: dense fp32 -> page, bit-exact fit_state.  Thread j owns column j
// (NT >= V); rows are processed by thread i in the row phase.
// =====================================================================
__global__ __launch_bounds__(512) void encode_kernel(PoolDev P, const float *__restrict__ state,
                                                     const void *slots, int slots_dtype, int split) {
  // Every product and sum rounds separately, as PyTorch's CPU ops do.
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = P.H, K = P.K, V = P.V;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int tid = threadIdx.x, NT = blockDim.x;
  const int64_t slot = load_slot(slots, slots_dtype, b);
  if (slot <= 0 || slot >= P.num_slots) return;  // masked (or outside the pool)
  uint8_t *page = P.data + slot * P.page_bytes;
  const int32_t *hm = P.head_meta + 4 * h;
  const int code_start = hm[0], code_bytes = hm[1];
  const int32_t *hbits = P.bits + (int64_t)h * K;
  const float *hw = P.impact + (int64_t)h * K;
  const int two = !P.kda && hbits[0] == 2;
  const int NG = two ? V / P.G : 1;
  const int Geff = two ? P.G : V;
  const int tile = tile_of(P);
  const int stride = P.offsets[(int64_t)H * K + h];
  const float *X = state + ((int64_t)b * H + h) * K * V;
  // LDS: staging window | row scale per (row, group) f32 [K * NG] | with a
  // row split: per-part column maxima [split][4][V] and 16-row block sums [K/16][2][V]
  uint8_t *stage = smem;
  float *rsc = (float *)(smem + P.stage);
  float *cmax = rsc + ((K * NG + 3) & ~3);
  float *bsum = cmax + split * 4 * V;

  int shift = 0;
  if (code_bytes > 0) shift = stage_in(page + code_start, code_bytes, stage, tid, NT);
  __syncthreads();

  // ---- row phase: r (and GDN 2-bit group r), pivots.
  // Fast form for rows summed in groups of n = 32..256 values (n a multiple
  // of 32): 32 lanes per row, lane (l, k) = (lane / 4, lane % 4) adds
  // |x[8(4 ii + k) + l]| for ii ascending, exactly PyTorch's vectorised
  // inner sum (8 vector lanes, 4 accumulators each, no cascade level below
  // 512 values); the partial sums are then combined in PyTorch's order:
  // s_l = ((a_l0 + a_l1) + a_l2) + a_l3, total = (...(s_0 + s_1) + ...) + s_7.
  // Loads of a row are coalesced.
  const int ngrp = two ? Geff : V;
  if (ngrp >= 32 && ngrp <= 256 && (ngrp & 31) == 0 && (NT & 31) == 0) {
    const int lane = tid & 31, l = lane >> 2, k = lane & 3;
    const int per_pass = NT >> 5;
    for (int i = tid >> 5; i < K; i += per_pass) {
      const float *xr = X + (int64_t)i * V;
      const int bi = hbits[i];
      if (bi == 16) {
        const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
        for (int j = lane; j < V; j += 32) {
          int p = shift + pivot_pos(P, off_rel, stride, tile, j);
          uint32_t hb = f2h(xr[j]);
          stage[p] = (uint8_t)hb;
          stage[p + 1] = (uint8_t)(hb >> 8);
        }
        if (lane == 0) rsc[i * NG] = 1.0f;
        continue;
      }
      const float wi = hw[i];
      const int64_t ro = P.rows[(int64_t)h * K + i];
      const int ng = two ? NG : 1;
      for (int g = 0; g < ng; g++) {
        const float *xg = xr + g * ngrp;
        float acc = 0.0f;
        for (int ii = 0; ii < ngrp / 32; ii++) acc += fabsf(xg[8 * (4 * ii + k) + l]);
        // combine within the quad (k = 0..3) and then over l, in order
        const float a1 = __shfl_down(acc, 1, 32), a2 = __shfl_down(acc, 2, 32), a3 = __shfl_down(acc, 3, 32);
        float sl = acc;
        sl += a1;
        sl += a2;
        sl += a3;
        float total = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) total += __shfl(sl, 4 * q, 32);
        if (lane == 0) {
          float m = total / (float)ngrp;
          m = m < 1e-20f ? 1e-20f : m;
          uint32_t hb;
          float r = fp16_scale(__builtin_sqrtf(m / wi), &hb);
          rsc[i * NG + g] = r;
          put_page_half(page, ro + 2 * g, hb);
        }
      }
    }
  } else
  for (int i = tid; i < K; i += NT) {
    const float *xr = X + (int64_t)i * V;
    const int bi = hbits[i];
    const float wi = hw[i];
    if (bi == 16) {
      const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
      for (int j = 0; j < V; j++) {
        int p = shift + pivot_pos(P, off_rel, stride, tile, j);
        uint32_t hb = f2h(xr[j]);
        stage[p] = (uint8_t)hb;
        stage[p + 1] = (uint8_t)(hb >> 8);
      }
      rsc[i * NG] = 1.0f;
      continue;
    }
    const int64_t ro = P.rows[(int64_t)h * K + i];
    if (two) {
      for (int g = 0; g < NG; g++) {
        float s = torch_inner_sum(Geff, [&](int64_t t) { return fabsf(xr[g * Geff + t]); });
        float m = s / (float)Geff;
        m = m < 1e-20f ? 1e-20f : m;
        uint32_t hb;
        float r = fp16_scale(__builtin_sqrtf(m / wi), &hb);
        rsc[i * NG + g] = r;
        put_page_half(page, ro + 2 * g, hb);
      }
    } else {
      float s = torch_inner_sum(V, [&](int64_t t) { return fabsf(xr[t]); });
      float m = s / (float)V;
      m = m < 1e-20f ? 1e-20f : m;
      uint32_t hb;
      float r = fp16_scale(__builtin_sqrtf(m / wi), &hb);
      rsc[i * NG] = r;
      put_page_half(page, ro, hb);
    }
  }
  __syncthreads();

  // ---- column phase with the rows of every column split over `split`
  // threads (thread j + V*hf owns rows [hf*K/split, (hf+1)*K/split) of column
  // j; K is a multiple of 16*split).  PyTorch's key-axis sum of the refit
  // (V >= 32) adds rows in 16-row blocks, each block from zero, and the block
  // sums in order; below 512 rows no other level changes the value, so the
  // blocks are summed in parallel and combined in order.
  if (split > 1) {
    const int j = tid % V, hf = tid / V;
    const int rows = K / split, i0 = hf * rows;
    const int g = two ? j / P.G : 0;
    float amax[4] = {0.f, 0.f, 0.f, 0.f};  // widths 2, 4, 6, 8
    for (int i = i0; i < i0 + rows; i++) {
      const int bi = hbits[i];
      if (bi == 16) continue;
      const float a = fabsf(X[(int64_t)i * V + j] / rsc[i * NG + g]);
      const int wsel = (bi < 8 ? bi : 8) / 2 - 1;
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (q == wsel) amax[q] = a > amax[q] ? a : amax[q];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) cmax[(hf * 4 + q) * V + j] = amax[q];
    __syncthreads();
    float mx = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float am = 0.0f;
      for (int u = 0; u < split; u++) {
        const float a = cmax[(u * 4 + q) * V + j];
        am = a > am ? a : am;
      }
      const int bc = 2 * q + 2;
      const float qmax = two ? 3.0f : (float)((1 << (bc - 1)) - 1);
      const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      const float t = am / (qmax * norm);
      mx = t > mx ? t : mx;
    }
    const float c0 = fp16_scale(mx, nullptr);
    auto z_at = [&](int i, float cdiv) -> float {
      const int bi = hbits[i];
      const int bc = bi < 8 ? bi : 8;
      const float qmax = (float)((1 << (bc - 1)) - 1);
      const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      const float sc = X[(int64_t)i * V + j] / rsc[i * NG + (bi == 16 ? 0 : g)];
      float y = sc / cdiv;
      if (P.kda) y = y * (1.0f / norm);  // exact: norm is a power of two
      if (two) return (y >= 0.0f ? 1.0f : -1.0f) * (fabsf(y) >= 2.0f ? 3.0f : 1.0f);
      float z = __builtin_rintf(y);
      z = z > -qmax ? z : -qmax;
      z = z < qmax ? z : qmax;
      return z;
    };
    for (int m = i0 / 16; m < (i0 + rows) / 16; m++) {
      float bn = 0.0f, bd = 0.0f;
      for (int i = 16 * m; i < 16 * m + 16; i++) {
        const int bi = hbits[i];
        const int bc = bi < 8 ? bi : 8;
        const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
        const float wsq = (hw[i] * hw[i]) * (bi != 16 ? 1.0f : 0.0f);
        const float z = z_at(i, c0);
        const float v = (rsc[i * NG + (bi == 16 ? 0 : g)] * norm) * z;
        bn += (wsq * v) * X[(int64_t)i * V + j];
        bd += wsq * (v * v);
      }
      bsum[(2 * m) * V + j] = bn;
      bsum[(2 * m + 1) * V + j] = bd;
    }
    __syncthreads();
    float num = 0.0f, den = 0.0f;
    for (int m = 0; m < K / 16; m++) {
      num += bsum[(2 * m) * V + j];
      den += bsum[(2 * m + 1) * V + j];
    }
    const float denc = den < 1e-30f ? 1e-30f : den;
    uint32_t chb;
    const float c = fp16_scale(den > 0.0f ? num / denc : c0, &chb);
    if (hf == 0 && colbase_of(P, h) >= 0) put_page_half(page, colbase_of(P, h) + 2 * (int64_t)j, chb);
    // final codes of this thread's rows; quads of lanes assemble 4-value groups
    for (int i = i0; i < i0 + rows; i++) {
      const int bi = hbits[i];
      uint32_t code = 0;
      if (bi != 16) {
        const int bc = bi < 8 ? bi : 8;
        const float z = z_at(i, c);
        if (P.storage) {
          const int carrier = P.kda ? (int)z * (1 << (8 - bc)) : (int)z;
          stage[shift + carrier_pos(stride - code_start, K, i, j)] = (uint8_t)(int8_t)carrier;
          continue;
        }
        code = two ? (uint32_t)(((int)z + 3) / 2) : (uint32_t)((int)z + ((1 << (bc - 1)) - 1));
      } else if (P.storage) {
        continue;
      }
      const uint32_t c1 = __shfl_xor(code, 1), c2 = __shfl_xor(code, 2), c3 = __shfl_xor(code, 3);
      if (bi != 16 && (tid & 3) == 0) {
        const uint32_t word = code | (c1 << bi) | (c2 << (2 * bi)) | (c3 << (3 * bi));
        const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
        lds_put_bytes(stage, shift + group_pos(off_rel, stride, tile, j, bi), word, bi / 2);
      }
    }
    __syncthreads();
    if (code_bytes > 0) stage_out(page + code_start, code_bytes, stage, tid, NT);
    return;
  }

  // ---- column phase (thread j <-> column j; lanes of a quad are adjacent columns)
  const int colbase = P.columns[h];
  for (int jb = 0; jb < V; jb += NT) {
    const int j = jb + tid;
    const bool act = j < V;
    const int jj = act ? j : V - 1;
    const int g = two ? jj / P.G : 0;
    // pass 1: c0 = fp16(max_i where(int, |x/r|/(qmax*norm), 0)).  Division
    // by a positive constant is monotone, so the maximum of the quotients is
    // the quotient of the largest |x/r| among the rows of each width.
    float amax[4] = {0.f, 0.f, 0.f, 0.f};  // widths 2, 4, 6, 8
    for (int i = 0; i < K; i++) {
      const int bi = hbits[i];
      if (bi == 16) continue;
      const float a = fabsf(X[(int64_t)i * V + jj] / rsc[i * NG + g]);
      const int wsel = (bi < 8 ? bi : 8) / 2 - 1;
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (q == wsel) amax[q] = a > amax[q] ? a : amax[q];
    }
    float mx = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int bc = 2 * q + 2;
      const float qmax = two ? 3.0f : (float)((1 << (bc - 1)) - 1);
      const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      const float t = amax[q] / (qmax * norm);
      mx = t > mx ? t : mx;
    }
    const float c0 = fp16_scale(mx, nullptr);
    // pass 2: z = encode(c0); weighted sums in torch's key-axis order
    auto z_of = [&](int i, float cdiv) -> float {
      int bi = hbits[i];
      int bc = bi < 8 ? bi : 8;
      float qmax = (float)((1 << (bc - 1)) - 1);
      float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      float sc = X[(int64_t)i * V + jj] / rsc[i * NG + (bi == 16 ? 0 : g)];
      float y = sc / cdiv;
      if (P.kda) y = y * (1.0f / norm);  // exact: norm is a power of two
      if (two) return (y >= 0.0f ? 1.0f : -1.0f) * (fabsf(y) >= 2.0f ? 3.0f : 1.0f);
      float z = __builtin_rintf(y);
      z = z > -qmax ? z : -qmax;
      z = z < qmax ? z : qmax;
      return z;
    };
    auto term = [&](int64_t i, bool numerator) -> float {
      int bi = hbits[i];
      int bc = bi < 8 ? bi : 8;
      float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      float wsq = (hw[i] * hw[i]) * (bi != 16 ? 1.0f : 0.0f);
      float z = z_of((int)i, c0);
      float v = (rsc[i * NG + (bi == 16 ? 0 : g)] * norm) * z;
      return numerator ? (wsq * v) * X[i * V + jj] : wsq * (v * v);
    };
    float num, den;
    if (V >= 32) {
      TorchCascade<1> cn, cd;
      cn.init(K);
      cd.init(K);
      for (int i = 0; i < K; i++) {
        // term(i, true) and term(i, false) with one z
        const int bi = hbits[i];
        const int bc = bi < 8 ? bi : 8;
        const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
        const float wsq = (hw[i] * hw[i]) * (bi != 16 ? 1.0f : 0.0f);
        const float z = z_of(i, c0);
        const float v = (rsc[i * NG + (bi == 16 ? 0 : g)] * norm) * z;
        cn.push((wsq * v) * X[(int64_t)i * V + jj]);
        cd.push(wsq * (v * v));
      }
      cn.finish(&num);
      cd.finish(&den);
    } else {
      num = torch_row_sum_ilp4(K, [&](int64_t i) { return term(i, true); });
      den = torch_row_sum_ilp4(K, [&](int64_t i) { return term(i, false); });
    }
    const float denc = den < 1e-30f ? 1e-30f : den;
    uint32_t chb;
    const float c = fp16_scale(den > 0.0f ? num / denc : c0, &chb);
    if (act && colbase >= 0) put_page_half(page, colbase + 2 * (int64_t)j, chb);
    // pass 3: final codes; quads of lanes assemble each 4-value group
    for (int i = 0; i < K; i++) {
      int bi = hbits[i];
      uint32_t code = 0;
      if (bi != 16) {
        int bc = bi < 8 ? bi : 8;
        float z = z_of(i, c);
        if (P.storage) {
          // int8 carrier at plane value (i, j)
          if (act) {
            const int carrier = P.kda ? (int)z * (1 << (8 - bc)) : (int)z;
            stage[shift + carrier_pos(stride - code_start, K, i, j)] = (uint8_t)(int8_t)carrier;
          }
          continue;
        }
        code = two ? (uint32_t)(((int)z + 3) / 2) : (uint32_t)((int)z + ((1 << (bc - 1)) - 1));
      } else if (P.storage) {
        continue;
      }
      const int lane = tid & 3;
      uint32_t c1 = __shfl_xor(code, 1);
      uint32_t c2 = __shfl_xor(code, 2);
      uint32_t c3 = __shfl_xor(code, 3);
      if (bi != 16 && act && lane == 0) {
        uint32_t word = code | (c1 << bi) | (c2 << (2 * bi)) | (c3 << (3 * bi));
        int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
        lds_put_bytes(stage, shift + group_pos(off_rel, stride, tile, j, bi), word, bi / 2);
      }
    }
  }
  __syncthreads();
  if (code_bytes > 0) stage_out(page + code_start, code_bytes, stage, tid, NT);
}

// =====================================================================
// Decode step.  Lane t: column group cg = t / RG (4 columns), row group
// rg = t % RG; rows rg, rg+RG, ... (RPT of them).
// =====================================================================
enum { MODE_FUSED = 0, MODE_READ = 1, MODE_WRITE = 2, MODE_DECODE = 3 };

struct StepDev {
  const void *q, *k, *v, *g, *beta, *a_log, *dt_bias;
  void *out;
  const void *slots;
  int64_t q_stride, k_stride, v_stride;
  int HK, qkv_dtype, gate_dtype, out_dtype, slots_dtype, normalize;
  int hk_mul;  // K=V=128 kernels: key head of value head h = (h * hk_mul) >> 20
  float scale;
  float *s_key, *s_decay, *s_delta;
  int64_t *s_slots;
  float *dense;  // MODE_DECODE output
};

template <int RG>
__device__ __forceinline__ float rg_sum(float x) {
#pragma unroll
  for (int m = 1; m < RG; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

template <int RG>
__device__ __forceinline__ float rg_max(float x) {
#pragma unroll
  for (int m = 1; m < RG; m <<= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}

template <int RPT, int RG, int MODE>
__global__ __launch_bounds__(512) void step_kernel(PoolDev P, StepDev S) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = P.H, K = P.K, V = P.V;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int tid = threadIdx.x, NT = blockDim.x;
  const int CG = V / 4;
  const int cg = tid / RG, rg = tid % RG;
  const bool act = cg < CG;
  const int j0 = (act ? cg : 0) * 4;

  int64_t slot;
  if (MODE == MODE_WRITE) {
    slot = S.s_slots[b];
  } else {
    slot = load_slot(S.slots, S.slots_dtype, b);
    if (MODE == MODE_READ && h == 0 && tid == 0) S.s_slots[b] = slot;
  }
  if (slot <= 0 || slot >= P.num_slots) {  // masked (or outside the pool): zero readout, no page access
    if (MODE == MODE_FUSED || MODE == MODE_READ) {
      for (int j = tid; j < V; j += NT) store_val(S.out, S.out_dtype, ((int64_t)b * H + h) * V + j, 0.0f);
    }
    if (MODE == MODE_DECODE) {
      float *d = S.dense + ((int64_t)b * H + h) * K * V;
      for (int e = tid; e < K * V; e += NT) d[e] = 0.0f;
    }
    return;
  }
  uint8_t *page = P.data + slot * P.page_bytes;
  const int32_t *hm = P.head_meta + 4 * h;
  const int code_start = hm[0], code_bytes = hm[1];
  const int32_t *hbits = P.bits + (int64_t)h * K;
  const int two = !P.kda && hbits[0] == 2;
  const int tile = tile_of(P);
  const int stride = P.offsets[(int64_t)H * K + h];
  const int colbase = P.columns[h];

  // LDS layout: staging window | red [CG][K] f32 (requantising modes) |
  // prepared q, k, retention per row | 3 scalars
  uint8_t *stage = smem;
  float *red = (float *)(smem + P.stage);
  float *qv = red + ((MODE == MODE_FUSED || MODE == MODE_WRITE) ? CG * K : 0);
  float *kv = qv + K;
  float *dv = kv + K;
  float *misc = dv + K;

  // ---- stage the code region (16-byte loads)
  int shift = 0;
  if (code_bytes > 0) shift = stage_in(page + code_start, code_bytes, stage, tid, NT);

  // ---- per-row inputs: prepared q, k, retention
  float beta = 0.0f;
  if (MODE == MODE_FUSED || MODE == MODE_READ) {
    const int hk = h / (H / S.HK);
    const int64_t qb = (int64_t)b * S.q_stride + (int64_t)hk * K;
    const int64_t kb = (int64_t)b * S.k_stride + (int64_t)hk * K;
    // wave 0 computes the norms
    if (tid < 64) {
      float sq = 0.0f, sk = 0.0f;
      for (int i = tid; i < K; i += 64) {
        float a = load_val(S.q, S.qkv_dtype, qb + i), c = load_val(S.k, S.qkv_dtype, kb + i);
        sq += a * a;
        sk += c * c;
      }
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) {
        sq += __shfl_xor(sq, m);
        sk += __shfl_xor(sk, m);
      }
      if (tid == 0) {
        misc[0] = S.normalize ? 1.0f / __builtin_sqrtf(sq + 1e-6f) : 1.0f;
        misc[1] = S.normalize ? 1.0f / __builtin_sqrtf(sk + 1e-6f) : 1.0f;
        float bt = load_val(S.beta, S.gate_dtype, (int64_t)b * H + h);
        if (S.a_log) bt = 1.0f / (1.0f + __expf(-bt));
        misc[2] = bt;
      }
    }
    __syncthreads();
    const float nq = misc[0], nk = misc[1];
    beta = misc[2];
    float alog = S.a_log ? __expf(load_val(S.a_log, S.gate_dtype, h)) : 0.0f;
    for (int i = tid; i < K; i += NT) {
      qv[i] = (load_val(S.q, S.qkv_dtype, qb + i) * nq) * S.scale;
      kv[i] = load_val(S.k, S.qkv_dtype, kb + i) * nk;
      int64_t gi = P.kda ? ((int64_t)b * H + h) * K + i : (int64_t)b * H + h;
      float gv = load_val(S.g, S.gate_dtype, gi);
      if (S.a_log) {
        float u = gv + load_val(S.dt_bias, S.gate_dtype, P.kda ? (int64_t)h * K + i : (int64_t)h);
        float sp = u > 20.0f ? u : __logf(1.0f + __expf(u < 20.0f ? u : 20.0f));
        gv = -alog * sp;
      }
      dv[i] = __expf(gv);
    }
  } else if (MODE == MODE_WRITE) {
    const int64_t base = ((int64_t)b * H + h) * K;
    for (int i = tid; i < K; i += NT) {
      kv[i] = S.s_key[base + i];
      dv[i] = S.s_decay[base + i];
    }
  }
  __syncthreads();

  // ---- unpack this lane's RPT x 4 values: x = r*c*z (pivots: fp16)
  float x[RPT][4];
  float cj[4] = {0.f, 0.f, 0.f, 0.f};
  if (act && colbase >= 0) {
#pragma unroll
    for (int c = 0; c < 4; c++) cj[c] = h2f(page_half(page, colbase + 2 * (j0 + c)));
  }
#pragma unroll
  for (int r = 0; r < RPT; r++) {
    const int i = rg + RG * r;
    const int bi = hbits[i];
    const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
    if (bi == 16) {
      const int p = shift + pivot_pos(P, off_rel, stride, tile, j0);
      uint32_t w0 = lds_word(stage, p), w1 = lds_word(stage, p + 4);
      float d = (MODE == MODE_DECODE) ? 1.0f : dv[i];
      x[r][0] = h2f(w0 & 0xffffu) * d;
      x[r][1] = h2f(w0 >> 16) * d;
      x[r][2] = h2f(w1 & 0xffffu) * d;
      x[r][3] = h2f(w1 >> 16) * d;
    } else {
      const int p = shift + (P.storage ? carrier_pos(stride - code_start, K, i, j0) : group_pos(off_rel, stride, tile, j0, bi));
      const uint32_t word = P.storage ? 0u : lds_word(stage, p);
      const int bc = bi < 8 ? bi : 8;
      const int L = (1 << (bc - 1)) - 1;
      const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      const int64_t ro = P.rows[(int64_t)h * K + i];
      const float rr = h2f(page_half(page, ro + (two ? 2 * (j0 / P.G) : 0)));
#pragma unroll
      for (int c = 0; c < 4; c++) {
        uint32_t code = (word >> (c * bi)) & ((1u << bi) - 1u);
        float z = P.storage ? (float)(int8_t)stage[p + c * K]
                            : (two ? 2.0f * (float)code - 3.0f : (float)((int)code - L) * norm);
        if (MODE == MODE_DECODE) x[r][c] = (rr * cj[c]) * z;
        else x[r][c] = ((rr * dv[i]) * cj[c]) * z;
      }
    }
  }

  if (MODE == MODE_DECODE) {
    if (act) {
      float *d = S.dense + ((int64_t)b * H + h) * K * V;
#pragma unroll
      for (int r = 0; r < RPT; r++) {
        const int i = rg + RG * r;
        *(float4 *)(d + (int64_t)i * V + j0) = make_float4(x[r][0], x[r][1], x[r][2], x[r][3]);
      }
    }
    return;
  }

  // ---- delta = beta (v - k^T S_retained);  S' = S_retained + k delta^T
  float delta[4];
  if (MODE == MODE_WRITE) {
#pragma unroll
    for (int c = 0; c < 4; c++) delta[c] = act ? S.s_delta[((int64_t)b * H + h) * V + j0 + c] : 0.0f;
  } else {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float s = 0.0f;
#pragma unroll
      for (int r = 0; r < RPT; r++) s += kv[rg + RG * r] * x[r][c];
      s = rg_sum<RG>(s);
      float vv = act ? load_val(S.v, S.qkv_dtype, (int64_t)b * S.v_stride + (int64_t)h * V + j0 + c) : 0.0f;
      delta[c] = beta * (vv - s);
    }
  }
#pragma unroll
  for (int r = 0; r < RPT; r++) {
    const float kk = kv[rg + RG * r];
#pragma unroll
    for (int c = 0; c < 4; c++) x[r][c] += kk * delta[c];
  }
  if (MODE == MODE_FUSED || MODE == MODE_READ) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float o = 0.0f;
#pragma unroll
      for (int r = 0; r < RPT; r++) o += qv[rg + RG * r] * x[r][c];
      o = rg_sum<RG>(o);
      if (act && rg == 0) store_val(S.out, S.out_dtype, ((int64_t)b * H + h) * V + j0 + c, o);
    }
  }
  if (MODE == MODE_READ) {
    if (act && rg == 0) {
#pragma unroll
      for (int c = 0; c < 4; c++) S.s_delta[((int64_t)b * H + h) * V + j0 + c] = delta[c];
    }
    const int64_t base = ((int64_t)b * H + h) * K;
    for (int i = tid; i < K; i += NT) {
      S.s_key[base + i] = kv[i];
      S.s_decay[base + i] = dv[i];
    }
    return;
  }

  // ================= requantise (FUSED / WRITE) =================
  // pivot rows: fp16 of the updated values, in place
#pragma unroll
  for (int r = 0; r < RPT; r++) {
    const int i = rg + RG * r;
    if (hbits[i] == 16 && act) {
      const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
      const int p = shift + pivot_pos(P, off_rel, stride, tile, j0);
      uint16_t *d16 = (uint16_t *)(stage + p);
#pragma unroll
      for (int c = 0; c < 4; c++) d16[c] = (uint16_t)f2h(x[r][c]);
    }
  }
  const bool any_int = colbase >= 0;
  if (any_int) {
    // row |x| partial sums per lane -> red[cg][i]
    if (act) {
#pragma unroll
      for (int r = 0; r < RPT; r++) {
        const int i = rg + RG * r;
        red[cg * K + i] = fabsf(x[r][0]) + fabsf(x[r][1]) + fabsf(x[r][2]) + fabsf(x[r][3]);
      }
    }
    __syncthreads();
    // r' per (row, group); stored in red[first cg of group][i]
    const int NG = two ? V / P.G : 1;
    const int Geff = two ? P.G : V;
    const int cg_per = Geff / 4;
    for (int e = tid; e < K * NG; e += NT) {
      const int i = e / NG, gq = e % NG;
      const int bi = hbits[i];
      if (bi == 16) continue;
      float s = 0.0f;
      for (int q = 0; q < cg_per; q++) s += red[(gq * cg_per + q) * K + i];
      float m = s / (float)Geff;
      m = m < 1e-20f ? 1e-20f : m;
      uint32_t hb;
      float rn = fp16_scale(__builtin_sqrtf(m / P.impact[(int64_t)h * K + i]), &hb);
      put_page_half(page, P.rows[(int64_t)h * K + i] + 2 * gq, hb);
      red[gq * cg_per * K + i] = rn;
    }
    __syncthreads();
    // scaled values s = x / (r' norm), column statistics
    const int gq = two ? j0 / P.G : 0;
    float U[RPT], iL[RPT];
    float mx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      const int i = rg + RG * r;
      const int bi = hbits[i];
      if (bi == 16) {
        U[r] = 0.0f;
        iL[r] = 0.0f;
        continue;
      }
      const int bc = bi < 8 ? bi : 8;
      const float norm = P.kda ? (float)(1 << (8 - bc)) : 1.0f;
      const float rn = red[gq * (two ? P.G / 4 : CG) * K + i] * norm;
      const float inv = 1.0f / rn;
      const float w = P.impact[(int64_t)h * K + i];
      U[r] = (w * w) * (rn * rn);
      iL[r] = two ? (1.0f / 3.0f) : 1.0f / (float)((1 << (bc - 1)) - 1);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        x[r][c] *= inv;
        mx[c] = fmaxf(mx[c], fabsf(x[r][c]) * iL[r]);
      }
    }
    float ic0[4], c0[4], num[4], den[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      c0[c] = fp16_scale(rg_max<RG>(mx[c]), nullptr);
      ic0[c] = 1.0f / c0[c];
      num[c] = 0.0f;
      den[c] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      if (iL[r] == 0.0f) continue;
      const float Lf = two ? 3.0f : 1.0f / iL[r];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        float y = x[r][c] * ic0[c];
        float z;
        if (two) z = (y >= 0.0f ? 1.0f : -1.0f) * (fabsf(y) >= 2.0f ? 3.0f : 1.0f);
        else z = fminf(fmaxf(__builtin_rintf(y), -Lf), Lf);
        float t = U[r] * z;
        num[c] += t * x[r][c];
        den[c] += t * z;
      }
    }
    float icn[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float n = rg_sum<RG>(num[c]), d = rg_sum<RG>(den[c]);
      float dc = d < 1e-30f ? 1e-30f : d;
      uint32_t hb;
      float cc = fp16_scale(d > 0.0f ? n / dc : c0[c], &hb);
      icn[c] = 1.0f / cc;
      if (act && rg == 0) put_page_half(page, colbase + 2 * (j0 + c), hb);
    }
    // final codes -> staging
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      const int i = rg + RG * r;
      const int bi = hbits[i];
      if (bi == 16 || !act) continue;
      const int bc = bi < 8 ? bi : 8;
      const int L = (1 << (bc - 1)) - 1;
      uint32_t word = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        float y = x[r][c] * icn[c];
        uint32_t code;
        int carrier;
        if (two) {
          code = y >= 0.0f ? (fabsf(y) >= 2.0f ? 3u : 2u) : (fabsf(y) >= 2.0f ? 0u : 1u);
          carrier = 2 * (int)code - 3;
        } else {
          float z = fminf(fmaxf(__builtin_rintf(y), -(float)L), (float)L);
          code = (uint32_t)((int)z + L);
          carrier = P.kda ? (int)z * (1 << (8 - bc)) : (int)z;
        }
        if (P.storage) stage[shift + carrier_pos(stride - code_start, K, i, j0 + c)] = (uint8_t)(int8_t)carrier;
        word |= code << (c * bi);
      }
      if (!P.storage) {
        const int off_rel = P.offsets[(int64_t)h * K + i] - code_start;
        lds_put_bytes(stage, shift + group_pos(off_rel, stride, tile, j0, bi), word, bi / 2);
      }
    }
  }
  __syncthreads();
  if (code_bytes > 0) stage_out(page + code_start, code_bytes, stage, tid, NT);
}


// =====================================================================
// GDN fast path: K = V = 128 and one width per head (2/4/6/8-bit codes or
// an FP16 pivot head), every region 16-byte aligned.  The width is uniform
// per workgroup, so it is a scalar branch into a body compiled for that
// width.  Lane layout: tid = 8*cg + rg, rg = row group in lane bits 0-2, so
// reductions over the 8 row groups (column statistics) are DPP quad and
// half-row exchanges; wave w holds column groups 8w..8w+7.
//
// Readout algebra: with x_ij = a_i c_j (code_ij - L), a_i = r_i * decay,
//   k^T x  = c_j (sum_i k_i a_i code_ij - L sum_i k_i a_i)
//   q^T x' = c_j (sum_i q_i a_i code_ij - L sum_i q_i a_i) + delta_j q^T k
// so the foreground needs two FMAs per value and no dequantised tile.
// The writer works on inner_ij = x'_ij / c_j = a_i z_ij + k_i delta_j / c_j.
// =====================================================================
// Four waves per SIMD (128 VGPRs): four workgroups per CU hide the page and
// input latency of each tile behind the others' arithmetic.
#ifndef GDN128_WAVES
#define GDN128_WAVES 4
#endif
#ifndef SCHED_ROWS
#define SCHED_ROWS 16  // rows between scheduling fences: the whole tile (no spills at 4 waves per SIMD)
#endif
#ifndef KDA_SCHED_ROWS
#define KDA_SCHED_ROWS 16  // the KDA tile: all 16 rows in one window (no spills at 4 waves per SIMD)
#endif

namespace fast {

constexpr int FK = 128, FV = 128, FNT = 256, FRPT = 16;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xF, 0xF, true);
}
// sum / max over the 8 row-group lanes (lane bits 0-2)
__device__ __forceinline__ float rg8_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  return x;
}
// max of non-negative floats, compared as integers (no NaN canonicalisation)
__device__ __forceinline__ float rg8_max_nonneg(float x) {
  uint32_t u = __float_as_uint(x);
  u = max(u, dpp_u<0xB1>(u));
  u = max(u, dpp_u<0x4E>(u));
  u = max(u, dpp_u<0x141>(u));
  return __uint_as_float(u);
}

// Reduce-scatter of four per-column values over the 8 row-group lanes: every
// lane ends with the full reduction of column (rg >> 1) of its four.  Lane
// partners rg ^ 7 (row_half_mirror, other bit 2), rg ^ 2 and rg ^ 1: after
// each exchange a lane keeps the half of its columns that matches its bit.
template <class OP>
__device__ __forceinline__ uint32_t rs4(const uint32_t v[4], int rg, OP op) {
  const bool b2 = rg & 4, b1 = rg & 2;
  const uint32_t m0 = op(b2 ? v[2] : v[0], dpp_u<0x141>(b2 ? v[0] : v[2]));
  const uint32_t m1 = op(b2 ? v[3] : v[1], dpp_u<0x141>(b2 ? v[1] : v[3]));
  const uint32_t m = op(b1 ? m1 : m0, dpp_u<0x4E>(b1 ? m0 : m1));
  return op(m, dpp_u<0xB1>(m));
}
__device__ __forceinline__ float rs4_sum(const float v[4], int rg) {
  const uint32_t u[4] = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  return __uint_as_float(
      rs4(u, rg, [](uint32_t a, uint32_t b) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); }));
}
// maximum of non-negative floats, compared as integers
__device__ __forceinline__ float rs4_max_nonneg(const float v[4], int rg) {
  const uint32_t u[4] = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  return __uint_as_float(rs4(u, rg, [](uint32_t a, uint32_t b) { return a > b ? a : b; }));
}
// the value of column c (held by row-group lanes 2c, 2c + 1) in every lane
// of the group: ds_swizzle in bit mode reads lane (lane & 0x18) | 2c of each
// 32-lane half, on the LDS crossbar (no VALU work)
template <int c>
__device__ __forceinline__ float from_col(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x18 | ((2 * c) << 5)));
}

__device__ __forceinline__ float hw_h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// clamp(2^-24, 65504) then round to half (v_cvt_f16_f32, round to nearest
// even; f16 denormals are preserved in this kernel's float mode).
__device__ __forceinline__ float hw_fp16_scale(float x, uint32_t *hbits) {
  const float c = __builtin_amdgcn_fmed3f(x, 5.9604644775390625e-08f, 65504.0f);
  const _Float16 h = (_Float16)c;
  if (hbits) *hbits = __builtin_bit_cast(uint16_t, h);
  return (float)h;
}

// hardware reciprocal (1 ulp); the decode step's requantisation only needs
// quotients accurate to a few ulp
__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }

struct Ctx {
  uint8_t *page;
  uint8_t *code;   // staged code region
  uint8_t *rst;    // staged row scales
  uint8_t *cst;    // staged column scales
  float *qraw, *kraw, *wv, *misc, *red;
  float *ks, *qs;  // per-row prepared k, q
  float4 *rc;      // per (group, row), at [g*128 + i]: k*a, q*a, ZS*a, a with a = r * retention
  float2 *iu;      // per (group, row), at [g*128 + i]: 1/r', w^2 r'^2
  int b, h, tid, rg, cg, wave, j0, blk, sub;
  int code_start, code_bytes, row_start, row_bytes, colbase;
};

// misc[] slots: 0 beta, 1 retention, 8..11 squared norms of q/k halves,
// 16.. and 32.. per-wave partial sums of k*a (per group), q*a (per group), q*k
constexpr int MISC_FLOATS = 48;
constexpr int KDA_COL_STAGE = 288;  // staged column-scale window (2V bytes + alignment)
constexpr int SUM_KA = 0, SUM_QA = 4, SUM_QK = 8;

// sum over the 64 lanes of a wave, result in every lane: 16-lane rows by
// DPP, then row pairs and wave halves by lane swaps
__device__ __forceinline__ float wave_sum(float x) {
  x = rg8_sum(x);
  x += dpp<0x140>(x);  // row_mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Per-row constants of the integer bodies, row i = tid mod 128: threads
// 0..127 write rc[i, g] (and the prepared k); for the readout, threads
// 128..255 form the same products of their row and reduce the sums over
// rows of k*a, q*a and q*k, in parallel with the first two waves.
template <int MODE>
__device__ __forceinline__ void row_setup_int(const StepDev &S, const Ctx &C, int NG, float ZS) {
  const bool sums = C.tid >= FK;
  if (MODE == MODE_WRITE && sums) return;
  const int i = C.tid & (FK - 1);
  float nq = 1.0f, nk = 1.0f;
  if (MODE != MODE_WRITE && S.normalize) {
    nq = __builtin_amdgcn_rsqf((C.misc[8] + C.misc[10]) + 1e-6f);
    nk = __builtin_amdgcn_rsqf((C.misc[9] + C.misc[11]) + 1e-6f);
  }
  const float k = MODE == MODE_WRITE ? C.kraw[i] : C.kraw[i] * nk;
  const float q = MODE == MODE_WRITE ? 0.0f : (C.qraw[i] * nq) * S.scale;
  const uint16_t *r16 = (const uint16_t *)C.rst;
  const float retention = C.misc[1];
  if (!sums) {
    C.ks[i] = k;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      if (g < NG) {
        const float a = hw_h2f(r16[i * NG + g]) * retention;
        C.rc[g * FK + i] = make_float4(k * a, q * a, ZS * a, a);
      }
    }
  } else if (MODE != MODE_WRITE) {
    float *part = C.misc + 16 + 16 * (i >> 6);
#pragma unroll
    for (int g = 0; g < 4; g++) {
      if (g < NG) {
        const float a = hw_h2f(r16[i * NG + g]) * retention;
        const float s1 = wave_sum(k * a), s2 = wave_sum(q * a);
        if ((i & 63) == 0) {
          part[SUM_KA + g] = s1;
          part[SUM_QA + g] = s2;
        }
      }
    }
    const float s3 = wave_sum(q * k);
    if ((i & 63) == 0) part[SUM_QK] = s3;
  }
}

// Per-row inputs of FP16 pivot heads, once per workgroup into LDS (threads
// 0..127, row i = tid): prepared q (scaled) and prepared k.
template <int MODE>
__device__ __forceinline__ void row_setup(const StepDev &S, const Ctx &C) {
  if (C.tid < FK) {
    const int i = C.tid;
    float nq = 1.0f, nk = 1.0f;
    if (MODE != MODE_WRITE && S.normalize) {
      nq = __builtin_amdgcn_rsqf((C.misc[8] + C.misc[10]) + 1e-6f);
      nk = __builtin_amdgcn_rsqf((C.misc[9] + C.misc[11]) + 1e-6f);
    }
    const float k = MODE == MODE_WRITE ? C.kraw[i] : C.kraw[i] * nk;
    C.ks[i] = k;
    C.qs[i] = MODE == MODE_WRITE ? 0.0f : (C.qraw[i] * nq) * S.scale;
  }
}

template <int MODE>
__device__ __forceinline__ void store_out(const PoolDev &P, const StepDev &S, const Ctx &C, const float *o,
                                          const float *delta) {
  const int64_t base = ((int64_t)C.b * P.H + C.h) * FV + C.j0;
  if (C.rg == 0) {
    if (MODE == MODE_FUSED || MODE == MODE_READ) store4(S.out, S.out_dtype, base, o);
    if (MODE == MODE_READ) {
#pragma unroll
      for (int c = 0; c < 4; c++) S.s_delta[base + c] = delta[c];
    }
  }
}

// The head's regions are staged into LDS with direct global-to-LDS loads
// (no registers, no waits until the barrier that follows): CH 16-byte chunks
// per lane of the code region (a W-bit head has 128*W chunks, W/2 per lane;
// FP16 pivot heads: 2048 chunks, 8 per lane), row scales on lanes
// 0..row_chunks-1, column scales on lanes 240..255.  Each wave's chunks are
// 64 consecutive 16-byte units, so one LDS base per wave addresses them.
typedef const __attribute__((address_space(1))) void *gptr_t;
typedef __attribute__((address_space(3))) void *lptr_t;

template <int CH>
__device__ __forceinline__ void stage_async(const Ctx &C, int row_chunks, bool cols) {
  const int wv = C.tid >> 6;
  const uint4 *src = (const uint4 *)(C.page + C.code_start) + C.tid;
#pragma unroll
  for (int k = 0; k < CH; k++)
    __builtin_amdgcn_global_load_lds((gptr_t)(src + FNT * k), (lptr_t)(C.code + 16 * (FNT * k + 64 * wv)), 16, 0, 0);
  if (C.tid < row_chunks)
    __builtin_amdgcn_global_load_lds((gptr_t)((const uint4 *)(C.page + C.row_start) + C.tid),
                                     (lptr_t)(C.rst + 16 * 64 * wv), 16, 0, 0);
  if (cols && C.tid >= FNT - 16)
    __builtin_amdgcn_global_load_lds((gptr_t)((const uint4 *)(C.page + C.colbase) + (C.tid - (FNT - 16))),
                                     (lptr_t)(C.cst + 16 * (64 * wv - (FNT - 16))), 16, 0, 0);
}

// Per-head inputs into LDS (raw q, k rows, their squared norms per wave,
// beta and the head's retention, the fit weights), and this lane's 4 values
// of v (the writer: delta) as raw bits in registers.  Issued after the
// page's global-to-LDS loads; every vector load is issued before any value
// is used (the q/k/v element width QW is a compile-time choice), so all
// their latencies overlap in one round trip.  F32 gate scalars are scalar
// loads.
template <int MODE, bool QW4, bool COLV = false>
__device__ __forceinline__ void prologue(const PoolDev &P, const StepDev &S, const Ctx &C, uint32_t vraw[4]) {
  const int64_t bh = (int64_t)C.b * P.H + C.h;
  const float w = P.impact[(int64_t)C.h * FK + (C.tid & (FK - 1))];
  if (MODE == MODE_WRITE) {
    __builtin_memcpy(vraw, S.s_delta + bh * FV + C.j0, 16);
    const float k = S.s_key[bh * FK + (C.tid & (FK - 1))];
    const float d = ld_uniform(S.s_decay + bh * FK);
    if (C.tid < FK) C.kraw[C.tid] = k;
    if (C.tid == FK) C.misc[1] = d;
  } else {
    const int hk = (C.h * S.hk_mul) >> 20;
    const int i = C.tid & (FK - 1);  // every wave reads rows (no divergence); threads >= 128 keep them
    const int64_t qi = (int64_t)C.b * S.q_stride + (int64_t)hk * FK + i;
    const int64_t ki = (int64_t)C.b * S.k_stride + (int64_t)hk * FK + i;
    // COLV: only this lane's readout column j0 + (rg >> 1), in vraw[0]
    const int64_t vi = (int64_t)C.b * S.v_stride + (int64_t)C.h * FV + C.j0 + (COLV ? C.rg >> 1 : 0);
    uint32_t qr, kr;
    if (QW4) {
      if (COLV) vraw[0] = ((const uint32_t *)S.v)[vi];
      else __builtin_memcpy(vraw, (const float *)S.v + vi, 16);
      qr = ((const uint32_t *)S.q)[qi];
      kr = ((const uint32_t *)S.k)[ki];
    } else {
      if (COLV) vraw[0] = ((const uint16_t *)S.v)[vi];
      else __builtin_memcpy(vraw, (const uint16_t *)S.v + vi, 8);
      qr = ((const uint16_t *)S.q)[qi];
      kr = ((const uint16_t *)S.k)[ki];
    }
    float bt, gv, dtb = 0.0f, al = 0.0f;
    if (S.gate_dtype == SQ_F32) {
      bt = __uint_as_float(ld_uniform((const uint32_t *)S.beta + bh));
      gv = __uint_as_float(ld_uniform((const uint32_t *)S.g + bh));
      if (S.a_log) {
        dtb = __uint_as_float(ld_uniform((const uint32_t *)S.dt_bias + C.h));
        al = __uint_as_float(ld_uniform((const uint32_t *)S.a_log + C.h));
      }
    } else {
      // the raw bits of all four before any conversion: one wait covers them
      // (without A_log, its reads fall on the gate and beta and are unused)
      const bool has_a = S.a_log != nullptr;
      const uint32_t br = ((const uint16_t *)S.beta)[bh], gr = ((const uint16_t *)S.g)[bh];
      const uint32_t dr = ((const uint16_t *)(has_a ? S.dt_bias : S.g))[has_a ? (int64_t)C.h : bh];
      const uint32_t ar = ((const uint16_t *)(has_a ? S.a_log : S.beta))[has_a ? (int64_t)C.h : bh];
      auto cv = [&](uint32_t u) { return S.gate_dtype == SQ_BF16 ? __uint_as_float(u << 16) : hw_h2f(u); };
      bt = cv(br);
      gv = cv(gr);
      if (has_a) {
        dtb = cv(dr);
        al = cv(ar);
      }
    }
    const float qv = QW4 ? __uint_as_float(qr) : S.qkv_dtype == SQ_BF16 ? __uint_as_float(qr << 16) : hw_h2f(qr);
    const float kv = QW4 ? __uint_as_float(kr) : S.qkv_dtype == SQ_BF16 ? __uint_as_float(kr << 16) : hw_h2f(kr);
    // waves 2 and 3 store the rows and their norms, wave 0 the gates: waves
    // 0 and 1 set up the rows after the barrier, waves 2 and 3 fit r'
    if (C.tid >= FK) {
      C.qraw[i] = qv;
      C.kraw[i] = kv;
      const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
      if ((C.tid & 63) == 0) {
        C.misc[8 + 2 * ((C.tid - FK) >> 6)] = sq;
        C.misc[9 + 2 * ((C.tid - FK) >> 6)] = sk;
      }
    } else if (C.tid == 0) {
      if (S.a_log) {
        bt = __builtin_amdgcn_rcpf(1.0f + __expf(-bt));
        const float u = gv + dtb;
        const float sp = u > 20.0f ? u : __logf(1.0f + __expf(u < 20.0f ? u : 20.0f));
        gv = -__expf(al) * sp;
      }
      C.misc[0] = bt;
      C.misc[1] = __expf(gv);
    }
  }
  if (C.tid < FK) C.wv[C.tid] = w;
}

// this lane's v (the writer: delta) from its raw bits
template <int MODE, bool QW4>
__device__ __forceinline__ void raw_v(const StepDev &S, const uint32_t vraw[4], float v[4]) {
#pragma unroll
  for (int c = 0; c < 4; c++) {
    if (MODE == MODE_WRITE || QW4) {
      v[c] = __uint_as_float(vraw[c]);
    } else {
      const uint32_t h = (vraw[c >> 1] >> (16 * (c & 1))) & 0xffffu;
      v[c] = S.qkv_dtype == SQ_BF16 ? __uint_as_float(h << 16) : hw_h2f(h);
    }
  }
}

// one value of v from its raw bits (the prologue's COLV load)
template <bool QW4>
__device__ __forceinline__ float raw_v1(const StepDev &S, uint32_t bits) {
  if (QW4) return __uint_as_float(bits);
  return S.qkv_dtype == SQ_BF16 ? __uint_as_float(bits << 16) : hw_h2f(bits);
}

// Writer hand-off of the readout pass: prepared key rows and per-row retention.
template <int MODE>
__device__ __forceinline__ void handoff(const PoolDev &P, const StepDev &S, const Ctx &C) {
  if (MODE == MODE_READ && C.tid < FK) {
    const int64_t bh = (int64_t)C.b * P.H + C.h;
    float nk = 1.0f;
    if (S.normalize) nk = __builtin_amdgcn_rsqf((C.misc[9] + C.misc[11]) + 1e-6f);
    S.s_key[bh * FK + C.tid] = C.kraw[C.tid] * nk;
    S.s_decay[bh * FK + C.tid] = C.misc[1];
  }
}

template <int CODE_CHUNKS_PER_LANE>
__device__ __forceinline__ void stage_back_fast(const Ctx &C, int row_chunks, bool cols) {
  // the offset re-read as a wave-uniform value: the store address is then
  // formed here from the scalar page base instead of being kept in vector
  // registers since the loads at the start of the tile
  const int cs = __builtin_amdgcn_readfirstlane(C.code_start);
  uint4 *dst = (uint4 *)(C.page + cs);
  const uint4 *src = (const uint4 *)C.code;
#pragma unroll
  for (int k = 0; k < CODE_CHUNKS_PER_LANE; k++) dst[C.tid + FNT * k] = src[C.tid + FNT * k];
  if (C.tid < row_chunks) ((uint4 *)(C.page + C.row_start))[C.tid] = ((const uint4 *)C.rst)[C.tid];
  if (cols && C.tid >= FNT - 16)
    ((uint4 *)(C.page + C.colbase))[C.tid - (FNT - 16)] = ((const uint4 *)C.cst)[C.tid - (FNT - 16)];
}

// x through an empty asm: the compiler cannot reuse an earlier value derived
// from it, so addresses formed from it late are not kept in registers (or
// spilled) across the whole tile
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// w + w + [bit set for this lane] in one add with carry-in: the lane mask
// (a compare's ballot) is the carry, so a bit is shifted in without a select
__device__ __forceinline__ uint32_t shift_in(uint32_t w, uint64_t mask) {
  uint32_t r;
  uint64_t carry;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(carry) : "v"(w), "s"(mask));
  return r;
}

// byte offset of this lane's first code row segment in the staged region:
// rows rg + 8r follow 8 * 2W bytes apart
template <int W>
__device__ __forceinline__ int code_pos0(int tid) {
  const int cg = tid >> 3;
  return (cg >> 2) * (FK * 2 * W) + (tid & 7) * (2 * W) + (cg & 3) * (W / 2);
}

// signed W-bit field c of a word (sign-extended)
template <int W>
__device__ __forceinline__ int sfield(uint32_t word, int c) {
  return (int)(word << (32 - W * (c + 1))) >> (32 - W);
}

// Final codes of four values from v = y + L: level(y) = rint(y) + L
// saturated to [0, 2L].  v_cvt_pk_u8_f32 converts with round-to-nearest-even
// into one byte lane, so the saturated v converts straight into place; the
// W-bit fields are then gathered with one shift-or and a byte permute or
// bitfield insert.  Fields: column c at bits [cW, cW + W).
template <int W>
__device__ __forceinline__ uint32_t pack_codes(const float v[4]) {
  constexpr float TOP = (float)(2 * ((1 << (W - 1)) - 1));
  auto lvl = [](float x) { return __builtin_amdgcn_fmed3f(x, 0.0f, TOP); };
  if (W == 8) {
    uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(lvl(v[0]), 0, 0u);
    w = __builtin_amdgcn_cvt_pk_u8_f32(lvl(v[1]), 1, w);
    w = __builtin_amdgcn_cvt_pk_u8_f32(lvl(v[2]), 2, w);
    return __builtin_amdgcn_cvt_pk_u8_f32(lvl(v[3]), 3, w);
  }
  // even columns in bytes 0 and 2, odd columns in bytes 0 and 2 of a second
  // word; the conversion saturates at 0 and the upper clamp to 2L is one
  // packed 16-bit minimum per word (each byte sits alone in its 16-bit half)
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const u16x2 top2 = {(unsigned short)TOP, (unsigned short)TOP};
  uint32_t e = __builtin_amdgcn_cvt_pk_u8_f32(v[0], 0, 0u);
  e = __builtin_amdgcn_cvt_pk_u8_f32(v[2], 2, e);
  uint32_t o = __builtin_amdgcn_cvt_pk_u8_f32(v[1], 0, 0u);
  o = __builtin_amdgcn_cvt_pk_u8_f32(v[3], 2, o);
  e = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, e), top2));
  o = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, o), top2));
  const uint32_t x = e | (o << W);  // columns 0,1 at bit 0; columns 2,3 at bit 16
  if (W == 4) return __builtin_amdgcn_perm(0u, x, 0x0c0c0200u);  // bytes 0 and 2
  // W == 6: bits [0,12) from x, bits [12,24) from x >> 4, as one bitfield
  // insert (the compiler otherwise rewrites the expression into three ops)
  uint32_t w;
  __asm__("v_bfi_b32 %0, %1, %2, %3" : "=v"(w) : "s"(0xfffu), "v"(x), "v"(x >> 4));
  return w;
}

// Wave priority of a step's short serial phases (the page and input
// loads with the set-up that follows them, the readout's reductions, the
// row-sum reduce-scatter and r' fit, the column scales): one level above the
// long per-value passes, so a tile's loads are issued, and a workgroup whose
// waves wait at a barrier on such a phase gets it done, before the SIMD's
// other waves take their next pass instructions.
template <int MODE, bool ON>
__device__ __forceinline__ void serial_phase() {
  if (MODE != MODE_DECODE) __builtin_amdgcn_s_setprio(ON ? 1 : 0);
}

template <int W, int MODE, bool QW4>
__device__ __forceinline__ void int_body(const PoolDev &P, const StepDev &S, Ctx &C) {
#pragma clang fp contract(off)
  constexpr int L = W == 2 ? 3 : (1 << (W - 1)) - 1;
  // Codes are offset binary (code = z + L; 2-bit: code = (z + 3) / 2).  With
  // the field's top bit flipped they read as a signed W-bit integer
  // s = code - 2^(W-1), and z = ZS*s + 1.  Sums over s instead of over the
  // unsigned code keep the cancelled offset at 1 instead of L, so columns
  // whose codes sit near the middle of the range lose no precision.
  constexpr float ZS = W == 2 ? 2.0f : 1.0f;
  constexpr uint32_t XM = W == 8 ? 0x80808080u : W == 6 ? 0x820820u : W == 4 ? 0x8888u : 0xAAu;
  constexpr int SEG = 2 * W;                   // bytes of one row's 16-value segment
  const int NG = W == 2 ? P.ng : 1;
  const int g = W == 2 ? (C.j0 * P.ng) >> 7 : 0;  // j0 / G with G = 128 / NG
  const uint16_t *c16 = (const uint16_t *)C.cst;
  serial_phase<MODE, true>();  // the loads issue first, the set-up follows
  stage_async<W / 2>(C, 16 * NG, true);
  uint32_t vraw[4];
  prologue<MODE, QW4, MODE != MODE_WRITE>(P, S, C, vraw);
  __syncthreads();
  const float beta = C.misc[0];
  handoff<MODE>(P, S, C);
  row_setup_int<MODE>(S, C, NG, ZS);
  __syncthreads();
  serial_phase<MODE, false>();

  float cj[4];
#pragma unroll
  for (int c = 0; c < 4; c++) cj[c] = hw_h2f(c16[C.j0 + c]);

  // per-lane row pointers: row rg + 8r of this lane's value group
  const float4 *rcl = C.rc + g * FK + C.rg;
  const float2 *iul = C.iu + g * FK + C.rg;
  const float *ksl = C.ks + C.rg;
  const int RS8 = 8;  // row stride of rcl / iul for 8 rows (group-major [g][i]: no bank conflicts)

  // ---- foreground: codes, k^T x and q^T x sums
  float cf[FRPT][4];
  float aK[4] = {0.f, 0.f, 0.f, 0.f}, aQ[4] = {0.f, 0.f, 0.f, 0.f};
  // rows rg + 8r are 8*SEG bytes apart: one base address, immediate offsets
  const int pos0 = code_pos0<W>(C.tid);
  const uint32_t *w32 = (const uint32_t *)(C.code + (pos0 & ~3));
  const uint32_t sh = (uint32_t)(pos0 & 3) * 8u;
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % SCHED_ROWS) == SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    uint32_t word;
    if (W == 8) word = w32[r * 4 * W];  // 8 rows = 16W bytes = 4W dwords
    else if (W == 4) word = *(const uint16_t *)(C.code + pos0 + r * 8 * SEG);
    else if (W == 2) word = C.code[pos0 + r * 8 * SEG];
    else word = __builtin_amdgcn_alignbit(w32[r * 4 * W + 1], w32[r * 4 * W], sh);
    word ^= XM;
#pragma unroll
    for (int c = 0; c < 4; c++) cf[r][c] = (float)sfield<W>(word, c);
    const float4 rc = rcl[r * RS8];
    if (MODE != MODE_WRITE) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        aK[c] = fmaf(rc.x, cf[r][c], aK[c]);
        aQ[c] = fmaf(rc.y, cf[r][c], aQ[c]);
      }
    }
    // the writer's a z = ZS a s + a, which does not wait for the readout's
    // delta (a*z first: exact zero for z = 0; the rank-1 term comes later)
    if (MODE != MODE_READ) {
#pragma unroll
      for (int c = 0; c < 4; c++) cf[r][c] = fmaf(rc.z, cf[r][c], rc.w);
    }
  }
  // the whole tile completes here: the compiler would otherwise sink these
  // products past the readout and keep the row constants live across it
  if (MODE != MODE_READ) {
#pragma unroll
    for (int r = 0; r < FRPT; r++)
#pragma unroll
      for (int c = 0; c < 4; c++) asm volatile("" : "+v"(cf[r][c]));
  }
  serial_phase<MODE, true>();
  // Per-column work runs once per column: the row-group lanes 2c, 2c + 1
  // finish column c of their four (reduce-scatter), and results every lane
  // needs come back by swizzle.
  const int cl = C.rg >> 1;
  const float cjc = hw_h2f(c16[C.j0 + cl]);
  float dj[4];  // delta / c
  if (MODE == MODE_WRITE) {
    float vv[4];
    raw_v<MODE, QW4>(S, vraw, vv);
#pragma unroll
    for (int c = 0; c < 4; c++) dj[c] = vv[c] * rcp(cj[c]);
  } else {
    const float sKA = C.misc[16 + SUM_KA + g] + C.misc[32 + SUM_KA + g];
    const float sQA = C.misc[16 + SUM_QA + g] + C.misc[32 + SUM_QA + g];
    const float sQK = C.misc[16 + SUM_QK] + C.misc[32 + SUM_QK];
    const float kS = cjc * fmaf(ZS, rs4_sum(aK, C.rg), sKA);
    const float delta = beta * (raw_v1<QW4>(S, vraw[0]) - kS);
    const float o = fmaf(delta, sQK, cjc * fmaf(ZS, rs4_sum(aQ, C.rg), sQA));
    if ((C.rg & 1) == 0) {
      const int64_t at = ((int64_t)C.b * P.H + C.h) * FV + C.j0 + cl;
      store_val(S.out, S.out_dtype, at, o);
      if (MODE == MODE_READ) S.s_delta[at] = delta;
    }
    if (MODE == MODE_READ) return;
    const float djc = delta * rcp(cjc);
    dj[0] = from_col<0>(djc);
    dj[1] = from_col<1>(djc);
    dj[2] = from_col<2>(djc);
    dj[3] = from_col<3>(djc);
  }

  serial_phase<MODE, false>();
  // ---- writer: inner = x'/c = a z + k delta/c, row sums of |x'|
  float rowp[FRPT];
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % SCHED_ROWS) == SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const float k = ksl[8 * r];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      // the rank-1 term on a z (no offset is cancelled against k*delta/c)
      const float inner = fmaf(k, dj[c], cf[r][c]);
      cf[r][c] = inner;
      acc = fmaf(cj[c], fabsf(inner), acc);
    }
    rowp[r] = acc;
  }
  serial_phase<MODE, true>();
  // reduce-scatter over the wave's 8 column groups (lane bits 3,4,5):
  // lane halves exchange with v_permlane32_swap (lanes 32-63 of the first
  // operand trade places with lanes 0-31 of the second), 16-lane rows with
  // v_permlane16_swap (odd rows of the first with even rows of the second),
  // so one add leaves row r in the lower and row r + half in the upper lanes
  const int b3 = (C.tid >> 3) & 1, b4 = (C.tid >> 4) & 1, b5 = (C.tid >> 5) & 1;
  float p8[8], p4[4], p2[2];
#pragma unroll
  for (int r = 0; r < 8; r++) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(rowp[r]), __float_as_uint(rowp[r + 8]),
                                                     false, false);
    p8[r] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(p8[r]), __float_as_uint(p8[r + 4]),
                                                     false, false);
    p4[r] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const float keep = b3 ? p4[r + 2] : p4[r], send = b3 ? p4[r] : p4[r + 2];
    p2[r] = keep + dpp<0x128>(send);  // row_ror:8 == lane xor 8 within 16
  }
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int r = 8 * b5 + 4 * b4 + 2 * b3 + q;
    C.red[C.wave * FK + C.rg + 8 * r] = p2[q];
  }
  __syncthreads();
  {
    const int Geff = W == 2 ? P.G : FV;
    const int wpg = Geff / 32;  // waves per value group
    const int ngsh = W == 2 ? P.ngsh : 0;
    // 1 / Geff, a power of two (Geff = 128 >> ngsh): the mean's division is
    // this exact multiplication
    const float ginv = __builtin_amdgcn_ldexpf(1.0f, ngsh - 7);
    for (int e = C.tid ^ FK; e < FK * NG; e += FNT) {  // rows on waves 2, 3 first
      const int i = e >> ngsh, gq = e & (NG - 1);
      float sum = C.red[(gq * wpg) * FK + i];
      for (int w = 1; w < wpg; w++) sum += C.red[(gq * wpg + w) * FK + i];
      float m = sum * ginv;
      m = m < 1e-20f ? 1e-20f : m;
      uint32_t hb;
      const float wi = C.wv[i];
      const float rn = hw_fp16_scale(__builtin_sqrtf(m / wi), &hb);
      C.iu[gq * FK + i] = make_float2(rcp(rn), (wi * wi) * (rn * rn));
      ((uint16_t *)C.rst)[e] = (uint16_t)hb;
    }
  }
  __syncthreads();
  serial_phase<MODE, false>();
  // ---- t = x'/(r' c) (the scaled value s = x'/r' is t*c), column max of |t|
  float mx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % SCHED_ROWS) == SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const float ir = iul[r * RS8].x;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float t = cf[r][c] * ir;
      cf[r][c] = t;
      mx[c] = fmaxf(mx[c], fabsf(t));
    }
  }
  serial_phase<MODE, true>();
  // c0 = fp16(max|s| / L); y = s/c0 = t * (c/c0)
  float f0[4], num[4] = {0.f, 0.f, 0.f, 0.f}, den[4] = {0.f, 0.f, 0.f, 0.f};
  const float c0 = hw_fp16_scale((cjc * rs4_max_nonneg(mx, C.rg)) * (1.0f / (float)L), nullptr);
  const bool top = c0 >= 65504.0f;
  {
    const float f0c = cjc * rcp(c0);
    f0[0] = from_col<0>(f0c);
    f0[1] = from_col<1>(f0c);
    f0[2] = from_col<2>(f0c);
    f0[3] = from_col<3>(f0c);
  }
  serial_phase<MODE, false>();
  // Unless c0 saturated at the fp16 maximum, |y| <= L (1 + 2^-11) and
  // rint(y) needs no clamp to [-L, L].
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % SCHED_ROWS) == SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const float U = iul[r * RS8].y;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float y = cf[r][c] * f0[c];
      if (W == 2) {
        // z = +-mag carries the sign of t (f0 > 0, and y = -0 gives +mag for
        // t = -0, whose term is zero either way), so U z t = (U mag) |t| and
        // U z z = (U mag) mag with the same roundings: no sign select needed
        const float mag = fabsf(y) >= 2.0f ? 3.0f : 1.0f;
        const float t = U * mag;
        num[c] = fmaf(t, fabsf(cf[r][c]), num[c]);
        den[c] = fmaf(t, mag, den[c]);
      } else {
        const float z = __builtin_rintf(y);
        const float t = U * z;
        num[c] = fmaf(t, cf[r][c], num[c]);
        den[c] = fmaf(t, z, den[c]);
      }
    }
  }
  if (W != 2 && __any(top)) {
    // Saturated c0 (states beyond the fp16 range): redo the sums with the
    // clamp, recomputing t from the staged old codes and the row constants
    // with the same operations, so the register tile is left untouched.
#pragma unroll
    for (int c = 0; c < 4; c++) num[c] = den[c] = 0.f;
    const int p0 = code_pos0<W>(opaque(C.tid));
    const uint32_t *w32s = (const uint32_t *)(C.code + (p0 & ~3));
#pragma unroll 1
    for (int r = 0; r < FRPT; r++) {
      const int i = C.rg + 8 * r;
      uint32_t word;
      if (W == 8) word = w32s[r * 4 * W];
      else if (W == 4) word = *(const uint16_t *)(C.code + p0 + r * 8 * SEG);
      else word = __builtin_amdgcn_alignbit(w32s[r * 4 * W + 1], w32s[r * 4 * W], (uint32_t)(p0 & 3) * 8u);
      const float4 rc = C.rc[g * FK + i];
      const float k = C.ks[i];
      const float2 iu = C.iu[g * FK + i];
      word ^= XM;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float code = (float)sfield<W>(word, c);
        const float t = fmaf(k, dj[c], fmaf(rc.z, code, rc.w)) * iu.x;
        const float z = __builtin_amdgcn_fmed3f(__builtin_rintf(t * f0[c]), -(float)L, (float)L);
        const float uz = iu.y * z;
        num[c] = fmaf(uz, t, num[c]);
        den[c] = fmaf(uz, z, den[c]);
      }
    }
  }
  serial_phase<MODE, true>();
  float f[4];
  {
    const float n = cjc * rs4_sum(num, C.rg), d = rs4_sum(den, C.rg);
    const float dc = d < 1e-30f ? 1e-30f : d;
    uint32_t hb;
    const float cc = hw_fp16_scale(d > 0.0f ? n * rcp(dc) : c0, &hb);
    const float fc = cjc * rcp(cc);
    const int tl = opaque(C.tid);  // column 4 (tid >> 3) + (rg >> 1), address formed here
    if ((tl & 1) == 0) ((uint16_t *)C.cst)[4 * (tl >> 3) + ((tl & 7) >> 1)] = (uint16_t)hb;
    f[0] = from_col<0>(fc);
    f[1] = from_col<1>(fc);
    f[2] = from_col<2>(fc);
    f[3] = from_col<3>(fc);
  }
  serial_phase<MODE, false>();
  // ---- final codes, packed back into the staged region
  const int pend = code_pos0<W>(opaque(C.tid));
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % SCHED_ROWS) == SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    uint32_t word;
    if (W == 2) {
      // code = 2 [y >= 0] + [(y >= 0) == (|y| >= 2)] ({0,1,2,3} for levels
      // -3, -1, 1, 3), shifted in from the last column: one add with carry-in
      // per bit
      word = 0;
#pragma unroll
      for (int c = 3; c >= 0; c--) {
        const float y = cf[r][c] * f[c];
        const uint64_t pos = __builtin_amdgcn_ballot_w64(y >= 0.0f);
        const uint64_t big = __builtin_amdgcn_ballot_w64(fabsf(y) >= 2.0f);
        word = shift_in(shift_in(word, pos), ~(pos ^ big));
      }
    } else {
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = fmaf(cf[r][c], f[c], (float)L);
      word = pack_codes<W>(v);
    }
    const int pos = pend + r * 8 * SEG;
    if (W == 8) *(uint32_t *)(C.code + pos) = word;
    else if (W == 4) *(uint16_t *)(C.code + pos) = (uint16_t)word;
    else if (W == 2) C.code[pos] = (uint8_t)word;
    else {
      // 3 bytes at an odd or even offset, one byte store each
      C.code[pos] = (uint8_t)word;
      C.code[pos + 1] = (uint8_t)(word >> 8);
      C.code[pos + 2] = (uint8_t)(word >> 16);
    }
  }
  __syncthreads();
  stage_back_fast<W / 2>(C, 16 * NG, true);
}

template <int MODE, bool QW4>
__device__ __forceinline__ void pivot_body(const PoolDev &P, const StepDev &S, Ctx &C) {
#pragma clang fp contract(off)
  constexpr int SEG = 32, BLK = FK * SEG;
  stage_async<8>(C, 0, false);
  uint32_t vraw[4];
  prologue<MODE, QW4>(P, S, C, vraw);
  __syncthreads();
  const float beta = C.misc[0], decay = C.misc[1];
  handoff<MODE>(P, S, C);
  row_setup<MODE>(S, C);
  __syncthreads();
  float qi[FRPT], ki[FRPT];
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    qi[r] = C.qs[C.rg + 8 * r];
    ki[r] = C.ks[C.rg + 8 * r];
  }
  float x[FRPT][4];
  float sk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    const int i = C.rg + 8 * r;
    const uint2 hv = *(const uint2 *)(C.code + C.blk * BLK + i * SEG + C.sub * 8);
    x[r][0] = hw_h2f(hv.x & 0xffffu) * decay;
    x[r][1] = hw_h2f(hv.x >> 16) * decay;
    x[r][2] = hw_h2f(hv.y & 0xffffu) * decay;
    x[r][3] = hw_h2f(hv.y >> 16) * decay;
#pragma unroll
    for (int c = 0; c < 4; c++) sk[c] = fmaf(ki[r], x[r][c], sk[c]);
  }
  float delta[4], o[4], vv[4];
  raw_v<MODE, QW4>(S, vraw, vv);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    if (MODE == MODE_WRITE) delta[c] = vv[c];
    else delta[c] = beta * (vv[c] - rg8_sum(sk[c]));
  }
  float oq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < FRPT; r++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      x[r][c] = fmaf(ki[r], delta[c], x[r][c]);
      oq[c] = fmaf(qi[r], x[r][c], oq[c]);
    }
  if (MODE != MODE_WRITE) {
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = rg8_sum(oq[c]);
    store_out<MODE>(P, S, C, o, delta);
  }
  if (MODE == MODE_READ) return;
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    const int i = C.rg + 8 * r;
    uint2 hv;
    hv.x = f2h(x[r][0]) | (f2h(x[r][1]) << 16);
    hv.y = f2h(x[r][2]) | (f2h(x[r][3]) << 16);
    *(uint2 *)(C.code + C.blk * BLK + i * SEG + C.sub * 8) = hv;
  }
  __syncthreads();
  stage_back_fast<8>(C, 0, false);
}

// Page -> dense fp32 of one W-bit head (decode): x = (r_i c_j) z_ij with
// z = code - L (2-bit: 2 code - 3), the operations and order of the general
// kernel, so both give the same bits.
template <int W>
__device__ __forceinline__ void decode_body(const PoolDev &P, const StepDev &S, const Ctx &C) {
#pragma clang fp contract(off)
  constexpr float ZS = W == 2 ? 2.0f : 1.0f;
  constexpr uint32_t XM = W == 8 ? 0x80808080u : W == 6 ? 0x820820u : W == 4 ? 0x8888u : 0xAAu;
  constexpr int SEG = 2 * W;
  const int NG = W == 2 ? P.ng : 1;
  const int g = W == 2 ? (C.j0 * P.ng) >> 7 : 0;
  stage_async<W / 2>(C, 16 * NG, true);
  __syncthreads();
  const uint16_t *c16 = (const uint16_t *)C.cst, *r16 = (const uint16_t *)C.rst;
  float cj[4];
#pragma unroll
  for (int c = 0; c < 4; c++) cj[c] = hw_h2f(c16[C.j0 + c]);
  const int pos0 = code_pos0<W>(C.tid);
  const uint32_t *w32 = (const uint32_t *)(C.code + (pos0 & ~3));
  const uint32_t sh = (uint32_t)(pos0 & 3) * 8u;
  float *d = S.dense + ((int64_t)C.b * P.H + C.h) * FK * FV + C.j0;
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    uint32_t word;
    if (W == 8) word = w32[r * 4 * W];
    else if (W == 4) word = *(const uint16_t *)(C.code + pos0 + r * 8 * SEG);
    else if (W == 2) word = C.code[pos0 + r * 8 * SEG];
    else word = __builtin_amdgcn_alignbit(w32[r * 4 * W + 1], w32[r * 4 * W], sh);
    word ^= XM;
    const int i = C.rg + 8 * r;
    const float rr = hw_h2f(r16[i * NG + g]);
    float x[4];
#pragma unroll
    for (int c = 0; c < 4; c++) x[c] = (rr * cj[c]) * fmaf(ZS, (float)sfield<W>(word, c), 1.0f);
    *(float4 *)(d + (int64_t)i * FV) = make_float4(x[0], x[1], x[2], x[3]);
  }
}

// Page -> dense fp32 of an FP16 pivot head (decode).
__device__ __forceinline__ void decode_pivot(const PoolDev &P, const StepDev &S, const Ctx &C) {
  constexpr int SEG = 32, BLK = FK * SEG;
  stage_async<8>(C, 0, false);
  __syncthreads();
  float *d = S.dense + ((int64_t)C.b * P.H + C.h) * FK * FV + C.j0;
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    const int i = C.rg + 8 * r;
    const uint2 hv = *(const uint2 *)(C.code + C.blk * BLK + i * SEG + C.sub * 8);
    *(float4 *)(d + (int64_t)i * FV) =
        make_float4(hw_h2f(hv.x & 0xffffu), hw_h2f(hv.x >> 16), hw_h2f(hv.y & 0xffffu), hw_h2f(hv.y >> 16));
  }
}

}  // namespace fast

template <int MODE, bool QW4>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GDN128_WAVES))) void gdn128_kernel(PoolDev P,
                                                                                                       StepDev S) {
  using namespace fast;
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = P.H;
  Ctx C;
  C.b = blockIdx.y;  // grid (heads, requests): no division
  // The dispatcher deals consecutive blocks to the 8 XCDs in turn, so with
  // heads in block order an XCD would run the same H/8 heads for every
  // request (and their widths set its load); rotating the head by the request
  // gives every XCD every head.
  C.h = P.hrot ? (int)((blockIdx.x + blockIdx.y) & (unsigned)P.hrot) : (int)blockIdx.x;
  C.tid = threadIdx.x;
  C.rg = C.tid & 7;
  C.cg = C.tid >> 3;
  C.wave = C.tid >> 6;
  C.j0 = 4 * C.cg;
  C.blk = C.cg >> 2;
  C.sub = C.cg & 3;
  // The slot and the head's metadata are scalar loads; the page's
  // global-to-LDS loads are issued as soon as they arrive, the per-head
  // inputs after them (int_body), so all those latencies overlap.
  int64_t slot;
  if (MODE == MODE_WRITE) slot = ld_uniform(S.s_slots + C.b);
  else slot = load_slot_uniform(S.slots, S.slots_dtype, C.b);
  const int32_t *hm = P.head_meta + 4 * C.h;
  const int W = ld_uniform(P.bits + (int64_t)C.h * FK);
  const int code_start = ld_uniform(hm), code_bytes = ld_uniform(hm + 1);
  const int row_start = ld_uniform(hm + 2), row_bytes = ld_uniform(hm + 3);
  const int colbase = ld_uniform(P.columns + C.h);
  if (MODE == MODE_READ && C.h == 0 && C.tid == 0) S.s_slots[C.b] = slot;
  if (slot <= 0 || slot >= P.num_slots) {
    if (MODE == MODE_FUSED || MODE == MODE_READ)
      for (int j = C.tid; j < FV; j += FNT) store_val(S.out, S.out_dtype, ((int64_t)C.b * H + C.h) * FV + j, 0.0f);
    if (MODE == MODE_DECODE) {  // masked: a zero state
      float4 *d = (float4 *)(S.dense + ((int64_t)C.b * H + C.h) * FK * FV);
      for (int e = C.tid; e < FK * FV / 4; e += FNT) d[e] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return;
  }
  C.page = P.data + slot * P.page_bytes;
  C.code_start = code_start;
  C.code_bytes = code_bytes;
  C.row_start = row_start;
  C.row_bytes = row_bytes;
  C.colbase = colbase;
  C.code = smem;
  C.rst = smem + P.stage;
  C.cst = C.rst + P.rstage;
  C.qraw = (float *)(C.cst + 2 * FV);
  C.kraw = C.qraw + FK;
  C.wv = C.kraw + FK;
  C.misc = C.wv + FK;
  C.red = C.misc + MISC_FLOATS;
  C.ks = C.red + 4 * FK;
  C.qs = C.ks + FK;
  const int ngm = P.ng;
  C.rc = (float4 *)(C.qs + FK);
  C.iu = (float2 *)(C.rc + FK * ngm);
  if constexpr (MODE == MODE_DECODE) {
    switch (W) {
      case 2: decode_body<2>(P, S, C); break;
      case 4: decode_body<4>(P, S, C); break;
      case 6: decode_body<6>(P, S, C); break;
      case 8: decode_body<8>(P, S, C); break;
      default: decode_pivot(P, S, C); break;
    }
  } else {
    switch (W) {
      case 2: int_body<2, MODE, QW4>(P, S, C); break;
      case 4: int_body<4, MODE, QW4>(P, S, C); break;
      case 6: int_body<6, MODE, QW4>(P, S, C); break;
      case 8: int_body<8, MODE, QW4>(P, S, C); break;
      default: pivot_body<MODE, QW4>(P, S, C); break;
    }
  }
}

// =====================================================================
// KDA, K = V = 128: per key-row widths (2/4/6/8-bit codes, FP16 pivot rows),
// one 4-value tile per row per block, per-channel retention.  One
// workgroup per (request, head); lane (rg, cg) owns rows rg + 8r (r < 16)
// and block cg (columns 4cg .. 4cg+3), as the GDN kernel.  Row widths vary
// per lane, so code fields are extracted and packed with run-time widths.
// Integer rows use x = a_i c_j z_ij with a_i = r_i * retention_i * norm_i,
// norm_i = 2^(8 - b_i); pivot rows (x = fp16 * retention, no scales) are
// handled in a separate pass over the head's pivot rows.
// =====================================================================
namespace kfast {
using namespace fast;

struct KCtx {
  uint8_t *page, *code, *rst, *cst;
  int lbase, shift_r, shift_col;  // lbase: this lane's block in the staged code
  float *qraw, *kraw, *wv, *gv, *misc, *red, *ks, *qs;
  float4 *rc;   // per row: k*a, q*a, a, top-bit mask (float bits)  (zeros for pivot rows)
  float4 *rl;   // per row: L, 1/L, 1/(r' norm), w^2 r'^2 norm^2 (zeros for pivots)
  int4 *rm;     // per row: byte position within a block, width w (0: pivot), 2w, 3w
  int4 *rk;     // per row: top-bit mask, tile byte mask, L + 1/2, 2L + 1/2 (float bits; zeros for pivots)
                // (the foreground reads rm and rc only: the mask rides in rc.w)
  uint32_t *pmask;  // 128-bit mask of pivot rows
  int b, h, tid, rg, cg, wave, j0;
  int code_start, code_bytes, row_start, row_bytes, colbase, stride;
};

// The code region is staged block by block (32 blocks of `stride` bytes, one
// per 4 columns), each block in its own 16-byte aligned LDS window of
// `pitch` bytes, pitch = 32 (mod 64): the eight blocks a wave reads at once
// start in different LDS banks.
__host__ __device__ __forceinline__ int block_chunks(int stride) { return (stride + 15 + 8 + 15) / 16; }
__host__ __device__ __forceinline__ int block_pitch(int stride) {
  return 64 * ((16 * block_chunks(stride) - 32 + 63) / 64) + 32;
}

// Staging with direct global-to-LDS loads (no registers, no waits until the
// next barrier): wave w copies blocks 8w..8w+7, one instruction
// per block and 64 chunks (a block's window is contiguous in LDS).
__device__ __forceinline__ void stage_blocks_async(const uint8_t *g0, int stride, int pitch, uint8_t *lds, int tid) {
  const int nc = block_chunks(stride);
  const int gmod = (int)((uintptr_t)g0 & 15);
  // the wave index in a scalar register: block addresses are wave-uniform
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int c0 = 0; c0 < nc; c0 += 64) {
#pragma unroll
    for (int bb = 0; bb < 8; bb++) {
      const int blk = 8 * w + bb;
      const int off = blk * stride;
      const uintptr_t bs = (uintptr_t)(g0 + (off - ((gmod + off) & 15)));
      const uint8_t *block = (const uint8_t *)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(bs >> 32)) << 32) |
                                               (uint32_t)__builtin_amdgcn_readfirstlane((int)bs));
      const uint4 *src = (const uint4 *)(block + 16u * (uint32_t)(c0 + lane));
      if (c0 + lane < nc)
        __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)(lds + blk * pitch + 16 * c0), 16, 0, 0);
    }
  }
}

// stage_in with direct global-to-LDS loads; returns the offset of gstart in
// the staged window (chunk c of the aligned window lands at lds + 16c)
__device__ __forceinline__ int stage_region_async(const uint8_t *gstart, int64_t nbytes, uint8_t *lds, int tid) {
  const int shift = (int)((uintptr_t)gstart & 15);
  const uint4 *src = (const uint4 *)(gstart - shift);
  const int n16 = (int)((shift + nbytes + 15) >> 4);
  const int wbase = tid & ~63;
  for (int c0 = 0; c0 < n16; c0 += FNT)
    if (c0 + tid < n16)
      __builtin_amdgcn_global_load_lds((gptr_t)(src + c0 + tid), (lptr_t)(lds + 16 * (c0 + wbase)), 16, 0, 0);
  return shift;
}

// Write the staged blocks back: per block, 16-byte chunks inside the block
// with one store, the chunks at its two edges in 2-byte units from one LDS
// read (block bounds are even; neighbouring blocks write the other units of
// shared chunks).
__device__ __forceinline__ void stage_out_blocks(uint8_t *g0, int stride, int pitch, const uint8_t *lds, int tid) {
  const int nc = block_chunks(stride);
  const int gmod = (int)((uintptr_t)g0 & 15);
  for (int f = tid; f < 32 * nc; f += FNT) {
    const int blk = f & 31, ch = f >> 5;
    const int off = blk * stride;
    const int sb = (gmod + off) & 15;
    uint8_t *w = g0 + (off - sb);
    const int a = 16 * ch;
    const uint4 v = *(const uint4 *)(lds + blk * pitch + a);
    if (a >= sb && a + 16 <= sb + stride) {
      *(uint4 *)(w + a) = v;
    } else if (a < sb + stride && a + 16 > sb) {
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int bb = a + 2 * u;
        if (bb >= sb && bb + 2 <= sb + stride) *(uint16_t *)(w + bb) = (uint16_t)(wv[u >> 1] >> (16 * (u & 1)));
      }
    }
  }
}

// LDS dwords at address a and a + 4: keep the bits outside `mask`, set those of
// `bits` (bits within mask), each dword as one atomic read-modify-write
__device__ __forceinline__ void lds_mskor2(uint32_t a, uint64_t mask, uint64_t bits) {
  asm volatile("ds_mskor_b32 %0, %1, %2\n\tds_mskor_b32 %0, %3, %4 offset:4" ::"v"(a), "v"((uint32_t)mask),
               "v"((uint32_t)bits), "v"((uint32_t)(mask >> 32)), "v"((uint32_t)(bits >> 32))
               : "memory");
}

// sign-extended field of run-time width w at bit offset o
__device__ __forceinline__ int sbfe(uint32_t word, uint32_t o, uint32_t w) {
  return __builtin_amdgcn_sbfe((int)word, o, w);
}

// the 32 bits starting at staged byte p
__device__ __forceinline__ uint32_t word_at(const uint8_t *lds, int p) {
  const uint32_t *w = (const uint32_t *)(lds + (p & ~3));
  return __builtin_amdgcn_alignbit(w[1], w[0], (uint32_t)(p & 3) * 8u);
}

typedef __attribute__((address_space(3))) const uint32_t lds_word_t;

// LDS address of a byte of the dynamic shared window
__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) { return (uint32_t)(uintptr_t)(lptr_t)p; }

// the 32 bits starting at LDS byte address a (alignbit takes the shift mod 32)
__device__ __forceinline__ uint32_t word_at_addr(uint32_t a) {
  lds_word_t *w = (lds_word_t *)(uintptr_t)(a & ~3u);
  return __builtin_amdgcn_alignbit(w[1], w[0], a << 3);
}

// The row's plan entries (width, code offset, row-scale offset) of row
// tid mod 128, loaded with the tile's inputs before the first barrier.
struct RowPlan {
  int bits, offset, row;
};

__device__ __forceinline__ RowPlan row_plan(const PoolDev &P, int h, int tid) {
  const int64_t hi = (int64_t)h * FK + (tid & (FK - 1));
  return RowPlan{P.bits[hi], P.offsets[hi], P.rows[hi]};
}

// Per-row constants, row i = tid mod 128: threads 0..127 write them and the
// pivot-row mask; for the readout, threads 128..255 form the same products
// of their row and reduce the sums over rows of k*a, q*a (integer rows) and
// q*k (all rows), in parallel with the first two waves.
template <int MODE>
__device__ __forceinline__ void row_setup(const StepDev &S, const KCtx &C, const RowPlan rp) {
  const bool sums = C.tid >= FK;
  if (MODE == MODE_WRITE && sums) return;
  {
    const int i = C.tid & (FK - 1);
    const int bi = rp.bits;
    const bool piv = bi == 16;
    float nq = 1.0f, nk = 1.0f;
    if (MODE != MODE_WRITE && S.normalize) {
      nq = __builtin_amdgcn_rsqf((C.misc[8] + C.misc[10]) + 1e-6f);
      nk = __builtin_amdgcn_rsqf((C.misc[9] + C.misc[11]) + 1e-6f);
    }
    const float k = MODE == MODE_WRITE ? C.kraw[i] : C.kraw[i] * nk;
    const float q = MODE == MODE_WRITE ? 0.0f : (C.qraw[i] * nq) * S.scale;
    const float retention = C.gv[i];
    float ka = 0.f, qa = 0.f, a = 0.f;
    if (!piv) {
      const float norm = (float)(1 << (8 - bi));
      const float r = hw_h2f(*(const uint16_t *)(C.rst + C.shift_r + (rp.row - C.row_start)));
      a = (r * retention) * norm;
      ka = k * a;
      qa = q * a;
    }
    if (sums) {
      float *part = C.misc + 16 + 16 * (i >> 6);
      const float s1 = wave_sum(ka), s2 = wave_sum(qa), s3 = wave_sum(q * k);
      if ((i & 63) == 0) {
        part[SUM_KA] = s1;
        part[SUM_QA] = s2;
        part[SUM_QK] = s3;
      }
      return;
    }
    C.ks[i] = k;
    C.qs[i] = q;
    const int pos = rp.offset - C.code_start;  // within a block
    if (piv) {
      C.rc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      C.rl[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      C.rm[i] = make_int4(pos, 0, 0, 0);  // width 0: no code fields
      C.rk[i] = make_int4(0, 0, 0, 0);
    } else {
      const int L = (1 << (bi - 1)) - 1;
      uint32_t xm = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) xm |= 1u << (c * bi + bi - 1);
      C.rc[i] = make_float4(ka, qa, a, __uint_as_float(xm));
      C.rl[i] = make_float4((float)L, 1.0f / (float)L, 0.f, 0.f);
      C.rm[i] = make_int4(pos, bi, 2 * bi, 3 * bi);
      C.rk[i] = make_int4((int)xm, (int)(0xffffffffu >> (32 - 4 * bi)), __float_as_int((float)L + 0.5f),
                          __float_as_int(2.0f * (float)L + 0.5f));
    }
    const uint64_t pb = __ballot(piv);
    if ((i & 63) == 0) {
      C.pmask[2 * (i >> 6)] = (uint32_t)pb;
      C.pmask[2 * (i >> 6) + 1] = (uint32_t)(pb >> 32);
    }
  }
}

// four FP16 values of pivot row p in this lane's block, times `scale`
__device__ __forceinline__ void pivot_load(const KCtx &C, int p, float scale, float x[4]) {
  const int pos = C.rm[p].x + C.lbase;
  const uint32_t lo = word_at(C.code, pos), hi = word_at(C.code, pos + 4);
  x[0] = hw_h2f(lo & 0xffffu) * scale;
  x[1] = hw_h2f(lo >> 16) * scale;
  x[2] = hw_h2f(hi & 0xffffu) * scale;
  x[3] = hw_h2f(hi >> 16) * scale;
}

// Next pivot row of the head from the (wave-uniform) 128-bit mask, cleared
// from the mask; -1 when none is left.
__device__ __forceinline__ int next_pivot(uint64_t &lo, uint64_t &hi) {
  if (lo) {
    const int p = __builtin_ctzll(lo);
    lo &= lo - 1u;
    return p;
  }
  if (hi) {
    const int p = 64 + __builtin_ctzll(hi);
    hi &= hi - 1u;
    return p;
  }
  return -1;
}

template <int MODE, bool QW4>
__device__ __forceinline__ void body(const PoolDev &P, const StepDev &S, KCtx &C, uint32_t vraw) {
#pragma clang fp contract(off)
  const float beta = C.misc[0];
  const bool has_cols = C.colbase >= 0;
  float cj[4];
#pragma unroll
  for (int c = 0; c < 4; c++)
    cj[c] = has_cols ? hw_h2f(*(const uint16_t *)(C.cst + C.shift_col + 2 * (C.j0 + c))) : 1.0f;
  const uint64_t pm_lo = ((uint64_t)__builtin_amdgcn_readfirstlane(C.pmask[1]) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane(C.pmask[0]);
  const uint64_t pm_hi = ((uint64_t)__builtin_amdgcn_readfirstlane(C.pmask[3]) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane(C.pmask[2]);
  const int base = C.lbase;
  const uint32_t cb = lds_addr(C.code) + (uint32_t)base;  // this lane's block

  // ---- foreground: signed code fields s = code - 2^(b-1) (z = s + 1)
  float cf[FRPT][4];
  float aK[4] = {0.f, 0.f, 0.f, 0.f}, aQ[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % KDA_SCHED_ROWS) == KDA_SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const int i = C.rg + 8 * r;
    const int4 m = C.rm[i];
    const float4 rc = C.rc[i];
    const uint32_t word = word_at_addr(cb + (uint32_t)m.x) ^ __float_as_uint(rc.w);
    const uint32_t w = (uint32_t)m.y;
    cf[r][0] = (float)sbfe(word, 0, w);
    cf[r][1] = (float)sbfe(word, w, w);
    cf[r][2] = (float)sbfe(word, (uint32_t)m.z, w);
    cf[r][3] = (float)sbfe(word, (uint32_t)m.w, w);
    if (MODE != MODE_WRITE) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        aK[c] = fmaf(rc.x, cf[r][c], aK[c]);
        aQ[c] = fmaf(rc.y, cf[r][c], aQ[c]);
      }
    }
    // the writer's a z = a s + a, which does not wait for the readout's delta
    if (MODE != MODE_READ) {
#pragma unroll
      for (int c = 0; c < 4; c++) cf[r][c] = fmaf(rc.z, cf[r][c], rc.z);
    }
  }
  // the readout sums and the tile complete here: the compiler would
  // otherwise sink the last rows' field extraction past the pivot loop and
  // keep their code words (spilled) across it
  if (MODE != MODE_WRITE) {
#pragma unroll
    for (int c = 0; c < 4; c++) asm volatile("" : "+v"(aK[c]), "+v"(aQ[c]));
  }
  if (MODE != MODE_READ) {
#pragma unroll
    for (int r = 0; r < FRPT; r++)
#pragma unroll
      for (int c = 0; c < 4; c++) asm volatile("" : "+v"(cf[r][c]));
  }
  serial_phase<MODE, true>();
  // Per-column work runs once per column: row-group lanes 2c, 2c + 1 finish
  // column c of their four (reduce-scatter), results come back by swizzle.
  const int cl = C.rg >> 1;
  const float cjc = has_cols ? hw_h2f(*(const uint16_t *)(C.cst + C.shift_col + 2 * (C.j0 + cl))) : 1.0f;
  const bool pivots = (pm_lo | pm_hi) != 0;  // wave-uniform
  float dj[4];            // delta / c per column
  float dlc = 0.0f;       // this lane's column delta (the pivot rows' update)
  if (MODE == MODE_WRITE) {
    const int64_t bi = ((int64_t)C.b * P.H + C.h) * FV + C.j0;
#pragma unroll
    for (int c = 0; c < 4; c++) dj[c] = S.s_delta[bi + c] * rcp(cj[c]);
  } else {
    // pivot rows owned by this lane (row % 8 == rg)
    float pK[4] = {0.f, 0.f, 0.f, 0.f}, pQ[4] = {0.f, 0.f, 0.f, 0.f};
    uint64_t lo = pm_lo, hi = pm_hi;
    for (int p = next_pivot(lo, hi); p >= 0; p = next_pivot(lo, hi)) {
      if ((p & 7) == C.rg) {
        float x[4];
        pivot_load(C, p, C.gv[p], x);
        const float k = C.ks[p], q = C.qs[p];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          pK[c] = fmaf(k, x[c], pK[c]);
          pQ[c] = fmaf(q, x[c], pQ[c]);
        }
      }
    }
    const float sKA = C.misc[16 + SUM_KA] + C.misc[32 + SUM_KA];
    const float sQA = C.misc[16 + SUM_QA] + C.misc[32 + SUM_QA];
    const float sQK = C.misc[16 + SUM_QK] + C.misc[32 + SUM_QK];
    const float vc = QW4 ? __uint_as_float(vraw)
                         : S.qkv_dtype == SQ_BF16 ? __uint_as_float(vraw << 16) : hw_h2f(vraw);
    const float pKc = pivots ? rs4_sum(pK, C.rg) : 0.0f, pQc = pivots ? rs4_sum(pQ, C.rg) : 0.0f;
    const float kS = fmaf(cjc, rs4_sum(aK, C.rg) + sKA, pKc);
    const float dl = beta * (vc - kS);
    const float o = fmaf(dl, sQK, fmaf(cjc, rs4_sum(aQ, C.rg) + sQA, pQc));
    if ((C.rg & 1) == 0) {
      const int64_t at = ((int64_t)C.b * P.H + C.h) * FV + C.j0 + cl;
      store_val(S.out, S.out_dtype, at, o);
      if (MODE == MODE_READ) S.s_delta[at] = dl;
    }
    if (MODE == MODE_READ) return;
    const float djc = dl * rcp(cjc);
    dj[0] = from_col<0>(djc);
    dj[1] = from_col<1>(djc);
    dj[2] = from_col<2>(djc);
    dj[3] = from_col<3>(djc);
    dlc = dl;
  }

  serial_phase<MODE, false>();
  // ---- writer: inner = x'/c = a z + k delta/c; row sums of |x'|
  float rowp[FRPT];
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % KDA_SCHED_ROWS) == KDA_SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const int i = C.rg + 8 * r;
    const float k = C.ks[i];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float inner = fmaf(k, dj[c], cf[r][c]);
      cf[r][c] = inner;
      acc = fmaf(cj[c], fabsf(inner), acc);
    }
    rowp[r] = acc;
  }
  serial_phase<MODE, true>();
  float p8[8], p4[4], p2[2];
#pragma unroll
  for (int r = 0; r < 8; r++) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(rowp[r]), __float_as_uint(rowp[r + 8]),
                                                     false, false);
    p8[r] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(p8[r]), __float_as_uint(p8[r + 4]),
                                                     false, false);
    p4[r] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  const int b3 = (C.tid >> 3) & 1, b4 = (C.tid >> 4) & 1, b5 = (C.tid >> 5) & 1;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const float keep = b3 ? p4[r + 2] : p4[r], send = b3 ? p4[r] : p4[r + 2];
    p2[r] = keep + dpp<0x128>(send);
  }
#pragma unroll
  for (int q = 0; q < 2; q++) C.red[C.wave * FK + C.rg + 8 * (8 * b5 + 4 * b4 + 2 * b3 + q)] = p2[q];
  __syncthreads();
  if (C.tid >= FK) {  // waves 2, 3 (0 and 1 did the row set-up)
    const int i = C.tid - FK;
    const int4 m = C.rm[i];
    if (m.y != 0) {
      const float sum = ((C.red[i] + C.red[FK + i]) + C.red[2 * FK + i]) + C.red[3 * FK + i];
      float mean = sum / (float)FV;
      mean = mean < 1e-20f ? 1e-20f : mean;
      const float wi = C.wv[i];
      uint32_t hb;
      const float rn = hw_fp16_scale(__builtin_sqrtf(mean / wi), &hb);
      const float norm = (float)(1 << (8 - m.y));
      const float rnn = rn * norm;
      C.rl[i].z = rcp(rnn);
      C.rl[i].w = (wi * wi) * (rnn * rnn);
      *(uint16_t *)(C.rst + C.shift_r + (P.rows[(int64_t)C.h * FK + i] - C.row_start)) = (uint16_t)hb;
    }
  }
  __syncthreads();
  serial_phase<MODE, false>();
  // ---- t = x'/(r' norm c); column max of |t| / L (c0 = fp16(c * max))
  float mx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % KDA_SCHED_ROWS) == KDA_SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const float4 rl = C.rl[C.rg + 8 * r];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float t = cf[r][c] * rl.z;
      cf[r][c] = t;
      mx[c] = fmaxf(mx[c], fabsf(t) * rl.y);
    }
  }
  serial_phase<MODE, true>();
  float f0[4], num[4] = {0.f, 0.f, 0.f, 0.f}, den[4] = {0.f, 0.f, 0.f, 0.f};
  const float c0 = hw_fp16_scale(cjc * rs4_max_nonneg(mx, C.rg), nullptr);
  const bool top = c0 >= 65504.0f;
  {
    const float f0c = cjc * rcp(c0);
    f0[0] = from_col<0>(f0c);
    f0[1] = from_col<1>(f0c);
    f0[2] = from_col<2>(f0c);
    f0[3] = from_col<3>(f0c);
  }
  serial_phase<MODE, false>();
  // |y| <= L_i (1 + 2^-11) unless c0 saturated: rint needs no clamp
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % KDA_SCHED_ROWS) == KDA_SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const float U = C.rl[C.rg + 8 * r].w;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float z = __builtin_rintf(cf[r][c] * f0[c]);
      const float t = U * z;
      num[c] = fmaf(t, cf[r][c], num[c]);
      den[c] = fmaf(t, z, den[c]);
    }
  }
  if (__any(top)) {
    // Saturated c0 (states beyond the fp16 range): redo the sums with the
    // clamp to [-L, L], recomputing t from the staged old codes and the row
    // constants with the same operations (the register tile stays as is).
#pragma unroll
    for (int c = 0; c < 4; c++) num[c] = den[c] = 0.f;
#pragma unroll 1
    for (int r = 0; r < FRPT; r++) {
      const int i = C.rg + 8 * r;
      const int4 m = C.rm[i];
      const float4 rc = C.rc[i];
      const float4 rl = C.rl[i];
      const float k = C.ks[i];
      const uint32_t word = word_at_addr(cb + (uint32_t)m.x) ^ __float_as_uint(rc.w);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float s = (float)sbfe(word, c * (uint32_t)m.y, (uint32_t)m.y);
        const float t = fmaf(k, dj[c], fmaf(rc.z, s, rc.z)) * rl.z;
        const float z = __builtin_amdgcn_fmed3f(__builtin_rintf(t * f0[c]), -rl.x, rl.x);
        const float u = rl.w * z;
        num[c] = fmaf(u, t, num[c]);
        den[c] = fmaf(u, z, den[c]);
      }
    }
  }
  serial_phase<MODE, true>();
  float f[4];
  {
    const float n = cjc * rs4_sum(num, C.rg), d = rs4_sum(den, C.rg);
    const float dc = d < 1e-30f ? 1e-30f : d;
    uint32_t hb;
    const float cc = hw_fp16_scale(d > 0.0f ? n * rcp(dc) : c0, &hb);
    const float fc = cjc * rcp(cc);
    const int tl = opaque(C.tid);  // column 4 (tid >> 3) + (rg >> 1), address formed here
    if ((tl & 1) == 0 && has_cols)
      *(uint16_t *)(C.cst + C.shift_col + 2 * (4 * (tl >> 3) + ((tl & 7) >> 1))) = (uint16_t)hb;
    f[0] = from_col<0>(fc);
    f[1] = from_col<1>(fc);
    f[2] = from_col<2>(fc);
    f[3] = from_col<3>(fc);
  }
  serial_phase<MODE, false>();
  // ---- final codes: level = rint(y) + L saturated to [0, 2L], packed with the row's width
#pragma unroll
  for (int r = 0; r < FRPT; r++) {
    if ((r % KDA_SCHED_ROWS) == KDA_SCHED_ROWS - 1) __builtin_amdgcn_sched_barrier(0);
    const int i = C.rg + 8 * r;
    const int4 m = C.rm[i];
    const int4 k = C.rk[i];
    const float lh = __int_as_float(k.z), top = __int_as_float(k.w);
    uint32_t code[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      // floor(y + L + 1/2) on [0, 2L]: the level of rint(y) + L
      code[c] = (uint32_t)__builtin_amdgcn_fmed3f(fmaf(cf[r][c], f[c], lh), 0.0f, top);
    }
    const uint32_t word = code[0] | (code[1] << (uint32_t)m.y) | (code[2] << (uint32_t)m.z) | (code[3] << (uint32_t)m.w);
    // the tile's bytes (mask k.y; none for pivot rows) merged into the two
    // dwords they can span; neighbouring rows share those dwords
    const uint32_t a = cb + (uint32_t)m.x;
    const uint32_t sh = (a << 3) & 24u;
    lds_mskor2(a & ~3u, (uint64_t)(uint32_t)k.y << sh, (uint64_t)word << sh);
  }
  // the masked merges are not tracked by the compiler's wait counts
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // ---- pivot rows: x' = x retention + k delta, stored as FP16
  if (pivots) {
    float delta[4];
    if (MODE == MODE_WRITE) {
      const int64_t bi = ((int64_t)C.b * P.H + C.h) * FV + C.j0;
#pragma unroll
      for (int c = 0; c < 4; c++) delta[c] = S.s_delta[bi + c];
    } else {
      delta[0] = from_col<0>(dlc);
      delta[1] = from_col<1>(dlc);
      delta[2] = from_col<2>(dlc);
      delta[3] = from_col<3>(dlc);
    }
    uint64_t lo = pm_lo, hi = pm_hi;
    for (int p = next_pivot(lo, hi); p >= 0; p = next_pivot(lo, hi)) {
      if ((p & 7) == C.rg) {
        float x[4];
        pivot_load(C, p, C.gv[p], x);
        const float k = C.ks[p];
        uint16_t *dst = (uint16_t *)(C.code + C.rm[p].x + base);
#pragma unroll
        for (int c = 0; c < 4; c++) dst[c] = (uint16_t)f2h(fmaf(k, delta[c], x[c]));
      }
    }
  }
  __syncthreads();
  stage_out_blocks(C.page + C.code_start, C.stride, block_pitch(C.stride), C.code, C.tid);
  // the row and column regions from waves 1 and 2 (wave 0 writes the first
  // edge chunks of the blocks)
  if (C.row_bytes > 0) stage_out(C.page + C.row_start, C.row_bytes, C.rst, (C.tid - 64) & (FNT - 1), FNT);
  if (has_cols) stage_out(C.page + C.colbase, 2 * FV, C.cst, (C.tid - 128) & (FNT - 1), FNT);
}

// Page -> dense fp32 (decode): per-row tables of the rows this workgroup
// stages (threads 0..127, row i = tid: the code field layout, r, and 2^(8-b)
// of integer rows; width 0 marks pivot rows), then x = (r c) ((code - L) 2^(8-b))
// per value, FP16 halves for pivot rows: the operations of the general
// kernel's decode mode.
__device__ __forceinline__ void decode_rows(const KCtx &C, const RowPlan rp) {
  if (C.tid >= FK) return;
  const int i = C.tid, bi = rp.bits;
  const int pos = rp.offset - C.code_start;  // within a block
  if (bi == 16) {
    C.rm[i] = make_int4(pos, 0, 0, 0);
    C.rc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    return;
  }
  const float r = hw_h2f(*(const uint16_t *)(C.rst + C.shift_r + (rp.row - C.row_start)));
  uint32_t xm = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) xm |= 1u << (c * bi + bi - 1);
  C.rm[i] = make_int4(pos, bi, 2 * bi, 3 * bi);
  C.rc[i] = make_float4(r, (float)(1 << (8 - bi)), 0.f, __uint_as_float(xm));
}

__device__ __forceinline__ void decode_body(const PoolDev &P, const StepDev &S, const KCtx &C) {
#pragma clang fp contract(off)
  const bool has_cols = C.colbase >= 0;
  float cj[4];
#pragma unroll
  for (int c = 0; c < 4; c++)
    cj[c] = has_cols ? hw_h2f(*(const uint16_t *)(C.cst + C.shift_col + 2 * (C.j0 + c))) : 1.0f;
  const uint32_t cb = lds_addr(C.code) + (uint32_t)C.lbase;  // this lane's block
  float *d = S.dense + ((int64_t)C.b * P.H + C.h) * FK * FV + C.j0;
#pragma unroll 4
  for (int r = 0; r < FRPT; r++) {
    const int i = C.rg + 8 * r;
    const int4 m = C.rm[i];
    float x[4];
    if (m.y == 0) {
      pivot_load(C, i, 1.0f, x);
    } else {
      const float4 rc = C.rc[i];
      const uint32_t word = word_at_addr(cb + (uint32_t)m.x) ^ __float_as_uint(rc.w);
      const uint32_t w = (uint32_t)m.y;
      // signed fields s = code - 2^(b-1), so code - L = s + 1
      const int s[4] = {sbfe(word, 0, w), sbfe(word, w, w), sbfe(word, (uint32_t)m.z, w), sbfe(word, (uint32_t)m.w, w)};
#pragma unroll
      for (int c = 0; c < 4; c++) x[c] = (rc.x * cj[c]) * ((float)(s[c] + 1) * rc.y);
    }
    *(float4 *)(d + (int64_t)i * FV) = make_float4(x[0], x[1], x[2], x[3]);
  }
}

}  // namespace kfast

// Per-head inputs of the KDA kernel into LDS: raw q, k rows and their squared
// norms, per-row retention, beta, the fit weights (the writer: prepared k and
// retention).  Every vector load is issued before any value is used (q/k
// width QW4 and gate width are branch-free runs), after the page's
// global-to-LDS loads, so all latencies overlap.
template <int MODE, bool QW4>
__device__ __forceinline__ void kda_prologue(const PoolDev &P, const StepDev &S, const kfast::KCtx &C,
                                             uint32_t &vraw) {
  using namespace kfast;
  const int64_t bh = (int64_t)C.b * P.H + C.h;
  const int i = C.tid & (FK - 1);
  const float w = P.impact[(int64_t)C.h * FK + i];
  if (MODE == MODE_WRITE) {
    const float k = S.s_key[bh * FK + i], d = S.s_decay[bh * FK + i];
    if (C.tid < FK) C.kraw[C.tid] = k;
    else C.gv[i] = d;
  } else {
    const int hk = (C.h * S.hk_mul) >> 20;
    const int64_t qi = (int64_t)C.b * S.q_stride + (int64_t)hk * FK + i;
    const int64_t ki = (int64_t)C.b * S.k_stride + (int64_t)hk * FK + i;
    // this lane's readout column j0 + (rg >> 1) of v, raw
    const int64_t vi = (int64_t)C.b * S.v_stride + (int64_t)C.h * FV + C.j0 + (C.rg >> 1);
    uint32_t qr, kr, gr, dr = 0u;
    if (QW4) {
      qr = ((const uint32_t *)S.q)[qi];
      kr = ((const uint32_t *)S.k)[ki];
      vraw = ((const uint32_t *)S.v)[vi];
    } else {
      qr = ((const uint16_t *)S.q)[qi];
      kr = ((const uint16_t *)S.k)[ki];
      vraw = ((const uint16_t *)S.v)[vi];
    }
    float bt, al = 0.0f;
    const bool g4 = S.gate_dtype == SQ_F32;
    if (g4) {
      gr = ((const uint32_t *)S.g)[bh * FK + i];
      if (S.a_log) dr = ((const uint32_t *)S.dt_bias)[(int64_t)C.h * FK + i];
      bt = __uint_as_float(ld_uniform((const uint32_t *)S.beta + bh));
      if (S.a_log) al = __uint_as_float(ld_uniform((const uint32_t *)S.a_log + C.h));
    } else {
      // The raw bits of all four 16-bit inputs before any conversion, so
      // one wait covers them (a conversion next to its load would wait
      // there and put a second memory round trip after the page's).
      // Without A_log, its two reads fall on the gate and beta, unused.
      const bool has_a = S.a_log != nullptr;
      gr = ((const uint16_t *)S.g)[bh * FK + i];
      dr = ((const uint16_t *)(has_a ? S.dt_bias : S.g))[has_a ? (int64_t)C.h * FK + i : bh * FK + i];
      const uint32_t br = ((const uint16_t *)S.beta)[bh];
      const uint32_t ar = ((const uint16_t *)(has_a ? S.a_log : S.beta))[has_a ? (int64_t)C.h : bh];
      auto cv = [&](uint32_t u) { return S.gate_dtype == SQ_BF16 ? __uint_as_float(u << 16) : hw_h2f(u); };
      bt = cv(br);
      if (has_a) al = cv(ar);
    }
    const float qv = QW4 ? __uint_as_float(qr) : S.qkv_dtype == SQ_BF16 ? __uint_as_float(qr << 16) : hw_h2f(qr);
    const float kv = QW4 ? __uint_as_float(kr) : S.qkv_dtype == SQ_BF16 ? __uint_as_float(kr << 16) : hw_h2f(kr);
    if (C.tid < FK) {
      C.qraw[C.tid] = qv;
      C.kraw[C.tid] = kv;
      const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
      if ((C.tid & 63) == 0) {
        C.misc[8 + 2 * (C.tid >> 6)] = sq;
        C.misc[9 + 2 * (C.tid >> 6)] = sk;
      }
    } else {
      auto gate_val = [&](uint32_t u) {
        return g4 ? __uint_as_float(u) : S.gate_dtype == SQ_BF16 ? __uint_as_float(u << 16) : hw_h2f(u);
      };
      float gv = gate_val(gr);
      if (S.a_log) {
        const float u = gv + gate_val(dr);
        const float sp = u > 20.0f ? u : __logf(1.0f + __expf(u < 20.0f ? u : 20.0f));
        gv = -__expf(al) * sp;
      }
      C.gv[i] = __expf(gv);
      if (i == 0) C.misc[0] = S.a_log ? 1.0f / (1.0f + __expf(-bt)) : bt;
    }
  }
  if (C.tid >= FK) C.wv[i] = w;
}

// Four waves per SIMD: the fused kernel fits 128 VGPRs with no scratch (the
// readout sums finish before the pivot loop, one delta register is kept
// instead of four); a fourth wave hides the tile's LDS and input latency.
#ifndef KDA128_WAVES
#define KDA128_WAVES 4
#endif
template <int MODE, bool QW4>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KDA128_WAVES))) void kda128_kernel(PoolDev P,
                                                                                                      StepDev S) {
  using namespace kfast;
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = P.H;
  KCtx C;
  C.b = blockIdx.y;  // grid (heads, requests): no division
  // The dispatcher deals consecutive blocks to the 8 XCDs in turn, so with
  // heads in block order an XCD would run the same H/8 heads for every
  // request (and their widths set its load); rotating the head by the request
  // gives every XCD every head.
  C.h = P.hrot ? (int)((blockIdx.x + blockIdx.y) & (unsigned)P.hrot) : (int)blockIdx.x;
  C.tid = threadIdx.x;
  C.rg = C.tid & 7;
  C.cg = C.tid >> 3;
  C.wave = C.tid >> 6;
  C.j0 = 4 * C.cg;
  // slot and head metadata as scalar loads; the page's global-to-LDS loads
  // go out as soon as they arrive, the per-head inputs after them
  int64_t slot;
  if (MODE == MODE_WRITE) slot = ld_uniform(S.s_slots + C.b);
  else slot = load_slot_uniform(S.slots, S.slots_dtype, C.b);
  const int32_t *hm = P.head_meta + 4 * C.h;
  const int code_start = ld_uniform(hm), code_bytes = ld_uniform(hm + 1);
  const int row_start = ld_uniform(hm + 2), row_bytes = ld_uniform(hm + 3);
  const int colbase = ld_uniform(P.columns + C.h);
  const int stride = ld_uniform(P.offsets + (int64_t)H * FK + C.h);
  if (MODE == MODE_READ && C.h == 0 && C.tid == 0) S.s_slots[C.b] = slot;
  if (slot <= 0 || slot >= P.num_slots) {
    if (MODE == MODE_FUSED || MODE == MODE_READ)
      for (int j = C.tid; j < FV; j += FNT) store_val(S.out, S.out_dtype, ((int64_t)C.b * H + C.h) * FV + j, 0.0f);
    if (MODE == MODE_DECODE) {  // masked: a zero state
      float4 *d = (float4 *)(S.dense + ((int64_t)C.b * H + C.h) * FK * FV);
      for (int e = C.tid; e < FK * FV / 4; e += FNT) d[e] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return;
  }
  C.page = P.data + slot * P.page_bytes;
  C.code_start = code_start;
  C.code_bytes = code_bytes;
  C.row_start = row_start;
  C.row_bytes = row_bytes;
  C.colbase = colbase;
  C.stride = stride;
  C.code = smem;
  C.rst = smem + P.stage;
  C.cst = C.rst + P.rstage;
  C.qraw = (float *)(C.cst + KDA_COL_STAGE);
  C.kraw = C.qraw + FK;
  C.wv = C.kraw + FK;
  C.gv = C.wv + FK;
  C.misc = C.gv + FK;
  C.red = C.misc + MISC_FLOATS;
  C.ks = C.red + 4 * FK;
  C.qs = C.ks + FK;
  C.rc = (float4 *)(C.qs + FK);
  C.rl = C.rc + FK;
  C.rm = (int4 *)(C.rl + FK);
  C.rk = C.rm + FK;
  C.pmask = (uint32_t *)(C.rk + FK);

  // stage the head's code, row-scale and column-scale regions
  serial_phase<MODE, true>();  // the loads issue first, the set-up follows
  const int pitch = block_pitch(C.stride);
  stage_blocks_async(C.page + C.code_start, C.stride, pitch, C.code, C.tid);
  C.lbase = C.cg * pitch + (int)((uintptr_t)(C.page + C.code_start + (int64_t)C.cg * C.stride) & 15);
  C.shift_r = C.row_bytes > 0 ? stage_region_async(C.page + C.row_start, C.row_bytes, C.rst, C.tid) : 0;
  C.shift_col = C.colbase >= 0 ? stage_region_async(C.page + C.colbase, 2 * FV, C.cst, C.tid) : 0;
  uint32_t vraw = 0u;
  const RowPlan rp = row_plan(P, C.h, C.tid);
  if constexpr (MODE == MODE_DECODE) {
    __syncthreads();
    decode_rows(C, rp);
    __syncthreads();
    decode_body(P, S, C);
    return;
  }
  kda_prologue<MODE, QW4>(P, S, C, vraw);
  __syncthreads();
  if (MODE == MODE_READ && C.tid < FK) {
    const int64_t bh = (int64_t)C.b * H + C.h;
    float nk = 1.0f;
    if (S.normalize) nk = __builtin_amdgcn_rsqf((C.misc[9] + C.misc[11]) + 1e-6f);
    S.s_key[bh * FK + C.tid] = C.kraw[C.tid] * nk;
    S.s_decay[bh * FK + C.tid] = C.gv[C.tid];
  }
  row_setup<MODE>(S, C, rp);
  __syncthreads();
  serial_phase<MODE, false>();
  body<MODE, QW4>(P, S, C, vraw);
}

// =====================================================================
// Chunked GDN prefill, K = V = 128, chunks of 64 tokens, bf16 MFMA
// (v_mfma_f32_16x16x32_bf16) with fp32 accumulation.
//
// For a chunk with start state S0 [K, V], Gamma_t = prod_{s<=t} g_s:
//   A_ts  = beta_t (Gamma_t/Gamma_s) k_t.k_s  (s < t)
//   Delta = (I + A)^{-1} R,  R = diag(beta) (V - diag(Gamma) K S0)
//   O     = diag(Gamma) Q S0 + (M o Q K^T) Delta,        M_ts = Gamma_t/Gamma_s (s <= t)
//   S_C   = Gamma_C S0 + (diag(Gamma_C/Gamma) K)^T Delta
// (q, k L2-normalised and q scaled: the norms multiply into the products).
// One workgroup per (sequence, head): 8 waves, chunks in order.
// Delta comes from 16-token blocks: D_i = T_ii (R_i - sum_{k<i} A_ik D_k),
// T_ii = (I + A_ii)^{-1}.
// Operands with a single rounding to bf16 would lose precision (T_ii, A, P,
// Delta, S); they are split as x = hi + lo (two bf16) and multiplied as
// hi*hi + hi*lo + lo*hi, leaving ~2^-16 relative error per product; q, k, v
// are bf16 inputs and enter exactly.
// MFMA operand layout (checked on gfx950): lane l holds A[l % 16][8(l/16)..+7]
// and B[8(l/16)..+7][l % 16]; the result lane l holds D[4(l/16)..+3][l % 16].
// =====================================================================
namespace pf {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

constexpr int PC = 64, PKD = 128, PV = 128;
constexpr int NW = 8, NT = 64 * NW;            // waves and threads of a workgroup
constexpr int P136 = 136, P72 = 72, PA = 68;  // row pitches (elements) of the LDS arrays
constexpr int OFF_KC = 0;                          // bf16 [64 t][136]   k rows (d contiguous)
constexpr int OFF_QC = OFF_KC + PC * P136 * 2;     // bf16 [64 t][136]   q rows
constexpr int OFF_KT = OFF_QC + PC * P136 * 2;     // bf16 [128 d][72]   k columns (t contiguous, swizzled)
constexpr int OFF_VC = OFF_KT + PKD * P72 * 2;     // bf16 [64 t][136]   v rows
constexpr int OFF_AT = OFF_VC + PC * P136 * 2;     // f32  [64 t][68]    A (diagonal blocks read)
constexpr int OFF_P = OFF_AT + PC * PA * 4;        // bf16 2 x [64 t][72] masked, scaled Q K^T (hi, lo)
constexpr int OFF_T = OFF_P + 2 * PC * P72 * 2;    // bf16 2 x [64 t][72] M (hi, lo): T_ii, -A_ik (i > k), 0
constexpr int OFF_SM = OFF_T + 2 * PC * P72 * 2;   // f32 [10][64] per-token scalars
constexpr int LDS_BYTES = OFF_SM + 10 * 64 * 4;
constexpr int MAX_CK = 64;                          // checkpoints per sequence (one per lane)
enum { SM_LC = 0, SM_BETA, SM_NK, SM_NQ, SM_GK, SM_QG, SM_KD, SM_KSQ, SM_QSQ };

// The pool's pages, for a kernel that reads the initial states itself.
struct PageInit {
  const uint8_t *data;
  int64_t page_bytes, num_slots;
  const int32_t *bits, *head_meta, *columns, *offsets, *rows;
  const void *slots;  // [batch] initial slots
  int slots_dtype, ng;
};

struct PrefillDev {
  const void *q, *k, *v, *g, *beta, *a_log, *dt_bias;
  void *out;
  const int32_t *cu, *ckpt;
  const float *init;  // dense initial states, unless page_init
  float *ck_state;
  int64_t q_stride, k_stride, v_stride;
  int H, HK, NC, gate_dtype, out_dtype, normalize, beta_logits;
  float scale;
  int page_init;  // 1: initial states decoded from the pages of pi.slots inside the kernel
  PageInit pi;
};

// Element (r, t) of the transposed k tile sits in row r at column
// tcol(r, t): the 8-token block index is XORed with bits 3-5 of r, so rows
// 8 apart start in different banks; runs of 4 or 8 consecutive tokens
// (t % 4 == 0) stay contiguous.
__device__ __forceinline__ int tcol(int r, int t) { return (((t >> 3) ^ (r >> 3)) & 7) * 8 + (t & 7); }

// Position of index c (a key column of the k and q tiles, a token column of
// the k-column, P and M tiles) within its 32-wide block: the runs c = 16 a +
// 4 b .. + 3 are stored at 8 b + 4 a, so the 8 entries at 32 m + 8 b .. + 7
// are indices 32 m + 4 b .. + 3 and 32 m + 16 + 4 b .. + 3 -- the k-slot
// order in which an operand built from two accumulator tiles lists them
// (split8), read with one 16-byte load.  Runs of 4 stay contiguous.
__device__ __forceinline__ int pcol(int c) { return (c & ~31) + 8 * ((c >> 2) & 3) + 4 * ((c >> 4) & 1) + (c & 3); }

// Four consecutive tokens of one column of a token-major bf16 tile
// [t][P136], with gfx950's transposing LDS load (ds_read_b64_tr_b16).
// Within each 16-lane row of the wave the instruction reads 8 bytes at
// every lane's address, as a 16 x 4 matrix M (row i: lane i's four halves),
// and returns to lane j the column j % 4 of rows j / 4 + 4k, k = 0..3 (lane
// layout checked on gfx950).  Lane i addressing token t0 + i / 4 at column
// c0 + 4 (i % 4) therefore receives column c0 + j of tokens t0 .. t0 + 3.
typedef short tr4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ tr4_t col4(const uint8_t *tile, int t0, int c0, int lane16) {
  const int byte = ((t0 + (lane16 >> 2)) * P136 + c0 + 4 * (lane16 & 3)) * 2;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) tr4_t *)(uintptr_t)(fast::lptr_t)(tile + byte));
}

// 4 x 4 transpose of dwords between the four 16-lane rows of a wave: row r
// enters with x[m] = M[r][m] and leaves with x[m] = M[m][r] (v_permlane32_swap
// trades the upper half of its first operand with the lower half of its
// second, v_permlane16_swap the odd rows of the first with the even rows of
// the second)
__device__ __forceinline__ void rows_transpose4(uint32_t x[4]) {
  const auto s02 = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
  const auto s13 = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
  const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  x[0] = s01[0];
  x[1] = s01[1];
  x[2] = s23[0];
  x[3] = s23[1];
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp0(float v) {  // DPP move, 0 where the source lane is outside the row
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}
// inclusive prefix sum over the 64 lanes: 16-lane rows by DPP shifts with
// zero fill, then rows 1, 3 add lane 15 of the row before, rows 2, 3 lane 31
__device__ __forceinline__ float wave_scan(float x) {
  x += dpp0<0x111, 0xF>(x);  // row_shr:1
  x += dpp0<0x112, 0xF>(x);  // row_shr:2
  x += dpp0<0x114, 0xF>(x);  // row_shr:4
  x += dpp0<0x118, 0xF>(x);  // row_shr:8
  x += dpp0<0x142, 0xA>(x);  // row_bcast:15 into rows 1, 3
  x += dpp0<0x143, 0xC>(x);  // row_bcast:31 into rows 2, 3
  return x;
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// 16 x 16 x 16 product: lane l holds A[l % 16][4 (l / 16) + j] and
// B[4 (l / 16) + j][l % 16], j = 0..3, and gets D[4 (l / 16) + j][l % 16]:
// an accumulator tile is a B operand as it is, and the A operand of its
// transpose
typedef short bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 ld8(const uint8_t *lds, int byte) { return *(const bf16x8 *)(lds + byte); }
__device__ __forceinline__ bf16x4 ld4(const uint8_t *lds, int byte) { return *(const bf16x4 *)(lds + byte); }
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf2f(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// two values rounded to bf16 (nearest even) and packed, a in the low half:
// one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack2(float a, float b) { return bf16x2_bits(a, b); }
// hi/lo bf16 halves of a pair (x = hi + lo to ~2^-16 relative): the hi pair
// is one packed conversion, its two values come back by shift and mask
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
  hi = bf16x2_bits(a, b);
  lo = bf16x2_bits(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}
// hi/lo halves of four values as two packed bf16 x 4
__device__ __forceinline__ void split4(const float x[4], uint2 &hi, uint2 &lo) {
  split2(x[0], x[1], hi.x, lo.x);
  split2(x[2], x[3], hi.y, lo.y);
}
// an accumulator tile's four values as hi/lo 16 x 16 x 16 operands
__device__ __forceinline__ void split4x(const f32x4 &x, bf16x4 &hi, bf16x4 &lo) {
  uint2 h, l;
  split2(x[0], x[1], h.x, l.x);
  split2(x[2], x[3], h.y, l.y);
  hi = __builtin_bit_cast(bf16x4, h);
  lo = __builtin_bit_cast(bf16x4, l);
}
// The 32 k-slots of a 16 x 16 x 32 product are summed in any order, so both
// operands may list them in the same permuted order.  Here slot e of lane
// group q4 = l / 16 is row 4 q4 + e of a 32-row block for e < 4 and row
// 16 + 4 q4 + e - 4 for e >= 4: a block held as two accumulator tiles x0
// (rows 0-15) and x1 (rows 16-31) is then an operand as it is (split into
// hi/lo bf16, no lane exchange), and the other operand's LDS tile stores
// its columns in that order (pcol).
__device__ __forceinline__ void split8(const f32x4 &x0, const f32x4 &x1, bf16x8 &hi, bf16x8 &lo) {
  uint32_t h[4], l[4];
  split2(x0[0], x0[1], h[0], l[0]);
  split2(x0[2], x0[3], h[1], l[1]);
  split2(x1[0], x1[1], h[2], l[2]);
  split2(x1[2], x1[3], h[3], l[3]);
  hi = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
}
__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
  return __builtin_bit_cast(bf16x8, make_uint4(__builtin_bit_cast(uint2, a).x, __builtin_bit_cast(uint2, a).y,
                                               __builtin_bit_cast(uint2, b).x, __builtin_bit_cast(uint2, b).y));
}

// lane Q's value of each quad in all four of its lanes (DPP quad_perm [Q,Q,Q,Q])
template <int Q>
__device__ __forceinline__ float quad_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), Q * 0x55, 0xF, 0xF, false));
}
// step ST.. of the diagonal-block forward substitution: the quad's lane
// ST % 4 holds x_ST (its row slot ST / 4); every lane's rows r = g + 4k take
// -A[r][ST] x_ST (rows[4 k PA + ST] is A[g + 4k][ST])
template <int ST>
__device__ __forceinline__ void tsolve_step(float acc[4], const float *rows) {
  if constexpr (ST < 16) {
    const float xs = quad_bcast<ST & 3>(acc[ST >> 2]);
#pragma unroll
    for (int k = 0; k < 4; k++) acc[k] = fmaf(-rows[4 * k * PA + ST], xs, acc[k]);
    tsolve_step<ST + 1>(acc, rows);
  }
}

// sum over the 16 lanes of a DPP row
__device__ __forceinline__ float row16_sum(float x) {
  x = fast::rg8_sum(x);
  return x + fast::dpp<0x140>(x);  // row_mirror
}

// Raw inputs of one chunk, fetched into registers one chunk ahead so the
// global loads overlap the previous chunk's arithmetic.
struct Fetch {
  uint4 k[2], q[2], v[2];
  uint32_t lg, bt;  // raw gate and beta bits (an f32 word or a 16-bit value)
  int n;
  int64_t tb;
};

// Workgroup barrier ordering LDS accesses only: the prefetched global loads
// of the next chunk stay in flight across it (a full __syncthreads would
// wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Initial state of one (sequence, head) read from its page, for GDN pools
// with K = V = 128, one width per head and 16-byte aligned regions (the
// pools the K = V = 128 decode kernels take).  The head's code, row-scale
// and column-scale regions are copied into LDS (the chunk tiles' space,
// unused until the first chunk); each lane then decodes the 32 values of its
// column j = 16 w + c16 (code block w) with the page decode's operations in
// its order, x = (r_d c_j)(ZS s + 1) with s the field with its top bit
// flipped, sign-extended (2-bit heads: z = 2 s + 1 and the row scale of j's
// value group), so the state is the dense decode's to the bit.
constexpr int INIT_ROWS = 32768, INIT_COLS = INIT_ROWS + 1024;  // LDS offsets of the staged scale regions
static_assert(INIT_COLS + 2 * PV <= OFF_P, "the staged page must not overlap the T and P tiles cleared at the start");

template <int W>
__device__ __forceinline__ void init_from_codes(const uint8_t *lds, int w, int q4, int c16, int ng, f32x4 S[8]) {
#pragma clang fp contract(off)
  constexpr float ZS = W == 2 ? 2.0f : 1.0f;
  constexpr int SEG = 2 * W;  // bytes of a row's 16-value segment
  const int j = 16 * w + c16;
  const float cj = fast::hw_h2f(((const uint16_t *)(lds + INIT_COLS))[j]);
  const uint16_t *rows = (const uint16_t *)(lds + INIT_ROWS);
  const int NG = W == 2 ? ng : 1;  // row scales per row: the value groups of a 2-bit head
  const int g = W == 2 ? (j * ng) >> 7 : 0;
  const int bit = c16 * W, sh = bit & 7;
  const uint8_t *base = lds + w * (PKD * SEG) + (bit >> 3);
#pragma unroll
  for (int dt = 0; dt < 8; dt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int d = 16 * dt + 4 * q4 + r;
      const uint8_t *p = base + d * SEG;
      uint32_t u = p[0];
      if (sh + W > 8) u |= (uint32_t)p[1] << 8;  // a 6-bit field across two bytes
      const uint32_t f = ((u >> sh) & ((1u << W) - 1u)) ^ (1u << (W - 1));
      const int sv = (int)(f << (32 - W)) >> (32 - W);
      const float rr = fast::hw_h2f(rows[d * NG + g]);
      S[dt][r] = (rr * cj) * fmaf(ZS, (float)sv, 1.0f);
    }
}

// FP16 pivot head: row d's 16-value segment of block w holds fp16 values
__device__ __forceinline__ void init_from_pivots(const uint8_t *lds, int w, int q4, int c16, f32x4 S[8]) {
#pragma unroll
  for (int dt = 0; dt < 8; dt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int d = 16 * dt + 4 * q4 + r;
      S[dt][r] = fast::hw_h2f(((const uint16_t *)(lds + w * (PKD * 32) + d * 32))[c16]);
    }
}

__device__ __forceinline__ void init_from_page(const PageInit &pi, int b, int h, uint8_t *lds, int tid, f32x4 S[8]) {
  const int w = tid >> 6, q4 = (tid >> 4) & 3, c16 = tid & 15;
  const int64_t slot = pi.slots_dtype == SQ_I64 ? ld_uniform((const int64_t *)pi.slots + b)
                                                 : (int64_t)ld_uniform((const int32_t *)pi.slots + b);
  if (slot <= 0 || slot >= pi.num_slots) {  // whole workgroup: a zero state
#pragma unroll
    for (int dt = 0; dt < 8; dt++) S[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  const int W = ld_uniform(pi.bits + (int64_t)h * PKD);
  const int32_t *hm = pi.head_meta + 4 * h;
  const int code_start = ld_uniform(hm), code_bytes = ld_uniform(hm + 1);
  const int row_start = ld_uniform(hm + 2), row_bytes = ld_uniform(hm + 3);
  const uint8_t *page = pi.data + slot * pi.page_bytes;
  for (int e = tid; e < code_bytes / 16; e += NT) ((uint4 *)lds)[e] = ((const uint4 *)(page + code_start))[e];
  if (W != 16) {
    for (int e = tid; e < row_bytes / 16; e += NT)
      ((uint4 *)(lds + INIT_ROWS))[e] = ((const uint4 *)(page + row_start))[e];
    if (tid < 2 * PV / 16)
      ((uint4 *)(lds + INIT_COLS))[tid] = ((const uint4 *)(page + ld_uniform(pi.columns + h)))[tid];
  }
  __syncthreads();
  switch (W) {
    case 2: init_from_codes<2>(lds, w, q4, c16, pi.ng, S); break;
    case 4: init_from_codes<4>(lds, w, q4, c16, pi.ng, S); break;
    case 6: init_from_codes<6>(lds, w, q4, c16, pi.ng, S); break;
    case 8: init_from_codes<8>(lds, w, q4, c16, pi.ng, S); break;
    default: init_from_pivots(lds, w, q4, c16, S); break;
  }
}

// One workgroup of 8 waves per (sequence, head), chunks in order.  Wave w
// owns the 16 state columns j = 16 w .. 16 w + 15 for all 128 rows d (in
// registers, accumulator layout); R, Delta and Delta' of its columns stay in
// registers too and reach the next product through to_operand.  The chunk's
// k, q, v, A, T and P are shared through LDS.  Transposed products keep every
// operand in a layout it already has: O^T = S0^T Q^T + Delta^T P^T gives
// each lane 4 consecutive output columns for one token.
__global__ __launch_bounds__(NT) void prefill_kernel(PrefillDev D) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = D.H;
  // Workgroups are dealt to the 8 XCDs round-robin (x mod 8).  The G value
  // heads that share a key head read the same q and k rows, so they are
  // placed on one XCD (x, x + 8, ..., one L2) when the grid divides evenly.
  int x = blockIdx.x;
  const int G = H / D.HK;
  if (G > 1 && gridDim.x % (8 * G) == 0) {
    const int slot = x >> 3;
    x = ((x & 7) + 8 * (slot / G)) * G + slot % G;
  }
  const int h = x % H;
  const int b = x / H;
  const int hk = h / G;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, q4 = l >> 4, c16 = l & 15;
  // sequence bounds as wave-uniform values (addresses formed from them stay scalar)
  const int t0 = __builtin_amdgcn_readfirstlane(D.cu[b]), len = __builtin_amdgcn_readfirstlane(D.cu[b + 1]) - t0;
  if (len <= 0) return;  // whole workgroup: an empty sequence has no chunk and no checkpoint
  float *sm = (float *)(smem + OFF_SM);
  uint8_t *Kc = smem + OFF_KC, *Qc = smem + OFF_QC, *Kt = smem + OFF_KT, *Vc = smem + OFF_VC;
  float *AT = (float *)(smem + OFF_AT);
  uint8_t *Pl = smem + OFF_P, *Tb = smem + OFF_T;
  const __bf16 *qg = (const __bf16 *)D.q, *kg = (const __bf16 *)D.k, *vg = (const __bf16 *)D.v;
  const int jw = 16 * w;  // this wave's first state column
  // one store per 4 output values when the output array's alignment allows
  // it (16 bytes for fp32, 8 for 16-bit values)
  const bool out_aligned = ((uintptr_t)D.out & (D.out_dtype == SQ_F32 ? 15 : 7)) == 0;
  // T and P in bf16 hi/lo: blocks above the diagonal stay zero, the others
  // are rewritten every chunk
  for (int e = tid; e < 2 * PC * P72 / 2; e += NT) ((uint32_t *)Tb)[e] = ((uint32_t *)Pl)[e] = 0u;
  // T entry (t, s) as hi/lo bf16 next to its fp32 value
  auto put_t = [&](int t, int s, float x) {
    const __bf16 hi = (__bf16)x;
    ((__bf16 *)Tb)[t * P72 + pcol(s)] = hi;
    ((__bf16 *)Tb)[PC * P72 + t * P72 + pcol(s)] = (__bf16)(x - (float)hi);
  };

  // ---- state S[d][j] of this wave's columns: tile dt holds rows d = 16 dt + 4 q4 + r, column jw + c16
  f32x4 S[8];
  if (D.page_init) {
    init_from_page(D.pi, b, h, smem, tid, S);
    __syncthreads();  // the staged page is read before the first chunk's tiles overwrite it
  } else {
    const float *src = D.init + ((int64_t)b * H + h) * PKD * PV + jw + c16;
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
      for (int r = 0; r < 4; r++) S[dt][r] = src[(int64_t)(16 * dt + 4 * q4 + r) * PV];
  }
  // this sequence's checkpoints (ascending), one per lane
  const int ckv = l < D.NC ? D.ckpt[(int64_t)b * D.NC + l] : 0x7fffffff;
  // tokens of the segment starting at c: up to the first listed checkpoint
  // past c (within the sequence), the sequence end, or one chunk
  auto segment = [&](int c) {
    const uint64_t m = __ballot(ckv > c && ckv <= len);
    const int stop = m ? __builtin_amdgcn_readlane(ckv, __builtin_ctzll(m)) : len;
    return stop - c < PC ? stop - c : PC;
  };
  lds_barrier();
  // The loads are unconditional, from rows clamped into the sequence (tokens
  // past the segment are zeroed when staged): nothing computed from a loaded
  // value may sit here, or the wait for the load would too.
  auto fetch = [&](Fetch &F, int c) {
    F.n = c < len ? segment(c) : 0;
    F.tb = (int64_t)t0 + c;
    // the chunk's first row (the sequence's last past its end) as a
    // wave-uniform base; rows within the chunk, clamped into the sequence,
    // as 32-bit byte offsets (one 24-bit multiply-add: rows below 64, row
    // strides below 2^23 elements)
    const int rb = __builtin_amdgcn_readfirstlane(c < len ? c : len - 1), lim = len - 1 - rb;
    const uint8_t *kb = (const uint8_t *)(kg + ((int64_t)t0 + rb) * D.k_stride + hk * PKD);
    const uint8_t *qb = (const uint8_t *)(qg + ((int64_t)t0 + rb) * D.q_stride + hk * PKD);
    const uint8_t *vb = (const uint8_t *)(vg + ((int64_t)t0 + rb) * D.v_stride + h * PV);
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int idx = tid + NT * it, t = idx >> 4, d8 = (idx & 15) * 8;
      const uint32_t tr = (uint32_t)(t < lim ? t : lim), db = 2u * (uint32_t)d8;
      F.k[it] = *(const uint4 *)(kb + (__umul24(tr, 2u * (uint32_t)D.k_stride) + db));
      F.q[it] = *(const uint4 *)(qb + (__umul24(tr, 2u * (uint32_t)D.q_stride) + db));
      F.v[it] = *(const uint4 *)(vb + (__umul24(tr, 2u * (uint32_t)D.v_stride) + db));
    }
    if (w == 0) {
      const int64_t at = ((int64_t)t0 + (c + l < len ? c + l : len - 1)) * H + h;
      if (D.gate_dtype == SQ_F32) {
        F.lg = ((const uint32_t *)D.g)[at];
        F.bt = ((const uint32_t *)D.beta)[at];
      } else {
        F.lg = ((const uint16_t *)D.g)[at];
        F.bt = ((const uint16_t *)D.beta)[at];
      }
    } else {
      F.lg = F.bt = 0u;  // read by wave 0 only
    }
  };

  // the head's gate constants, once: dt_bias and e^{A_log}
  const float dt_h = D.a_log ? load_val(D.dt_bias, D.gate_dtype, h) : 0.0f;
  const float ea_h = D.a_log ? __expf(load_val(D.a_log, D.gate_dtype, h)) : 0.0f;
  Fetch F;
  fetch(F, 0);
  int ci = 0;  // next checkpoint index
  for (int c0 = 0; c0 < len;) {
    const int n = F.n;
    const int64_t tb = F.tb;
    // lane indices re-derived each chunk through an empty asm: the LDS
    // addresses formed from them (swizzled, not base + offset) are then
    // computed where used instead of being held across the loop
    const int tid = fast::opaque(threadIdx.x), l = tid & 63, q4 = l >> 4, c16 = l & 15;

    // ---- stage the fetched chunk: k, q and v rows, k columns, squared norms, decays
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int idx = tid + NT * it, t = idx >> 4, d8 = (idx & 15) * 8;
      const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
      const uint4 kv = t < n ? F.k[it] : zero, qv = t < n ? F.q[it] : zero, vv = t < n ? F.v[it] : zero;
      // key columns d8 .. d8 + 3 and d8 + 4 .. d8 + 7 at their permuted places
      *(uint2 *)(Kc + (t * P136 + pcol(d8)) * 2) = make_uint2(kv.x, kv.y);
      *(uint2 *)(Kc + (t * P136 + pcol(d8 + 4)) * 2) = make_uint2(kv.z, kv.w);
      *(uint2 *)(Qc + (t * P136 + pcol(d8)) * 2) = make_uint2(qv.x, qv.y);
      *(uint2 *)(Qc + (t * P136 + pcol(d8 + 4)) * 2) = make_uint2(qv.z, qv.w);
      *(uint4 *)(Vc + (t * P136 + d8) * 2) = vv;
      // squared norms of the 8 values, two bf16 products per v_dot2_f32_bf16
      float sk = 0.f, sq = 0.f;
      {
        const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          sk = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kw[e]), __builtin_bit_cast(bf16x2, kw[e]),
                                               sk, false);
          sq = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, qw[e]), __builtin_bit_cast(bf16x2, qw[e]),
                                               sq, false);
        }
      }
      {
        // k columns: the wave's four 16-lane rows hold tokens t0 .. t0 + 3
        // (row r = t - t0); after the transpose row r holds value pair r
        // (key rows d8 + 2r, d8 + 2r + 1) of all four tokens, stored as two
        // 8-byte runs of consecutive tokens
        const int rr = (tid >> 4) & 3, t0 = t - rr, d = d8 + 2 * rr;
        const int o0 = (d * P72 + tcol(d, pcol(t0))) * 2;
        uint32_t x[4] = {kv.x, kv.y, kv.z, kv.w};
        rows_transpose4(x);
        *(uint2 *)(Kt + o0) = make_uint2(__builtin_amdgcn_perm(x[1], x[0], 0x05040100u),
                                         __builtin_amdgcn_perm(x[3], x[2], 0x05040100u));
        *(uint2 *)(Kt + o0 + P72 * 2) = make_uint2(__builtin_amdgcn_perm(x[1], x[0], 0x07060302u),
                                                   __builtin_amdgcn_perm(x[3], x[2], 0x07060302u));
      }
      sk = row16_sum(sk);
      sq = row16_sum(sq);
      if ((idx & 15) == 0) {
        sm[SM_KSQ * 64 + t] = sk;
        sm[SM_QSQ * 64 + t] = sq;
      }
    }
    if (w == 0) {
      auto gate = [&](uint32_t x) {
        if (l >= n) return 0.0f;
        if (D.gate_dtype == SQ_F32) return __uint_as_float(x);
        return D.gate_dtype == SQ_BF16 ? __uint_as_float(x << 16) : h2f((uint16_t)x);
      };
      float lg = gate(F.lg), bt = gate(F.bt);
      if (D.a_log && l < n) {
        const float u = lg + dt_h;
        const float sp = u > 20.0f ? u : __logf(1.0f + __expf(u < 20.0f ? u : 20.0f));
        lg = -ea_h * sp;
      }
      if (D.beta_logits && l < n) bt = __builtin_amdgcn_rcpf(1.0f + __expf(-bt));
      lg = wave_scan(lg);  // inclusive prefix sum of the log decays over the 64 tokens
      sm[SM_LC * 64 + l] = lg;
      sm[SM_BETA * 64 + l] = bt;
    }
    // the next segment's inputs are in flight while this one is computed
    const int c_next = c0 + n;
    fetch(F, c_next);
    lds_barrier();
    if (tid < 64) {
      const int t = tid;
      const float nk = D.normalize ? __builtin_amdgcn_rsqf(sm[SM_KSQ * 64 + t] + 1e-6f) : 1.0f;
      const float nq = (D.normalize ? __builtin_amdgcn_rsqf(sm[SM_QSQ * 64 + t] + 1e-6f) : 1.0f) * D.scale;
      const float lc = sm[SM_LC * 64 + t], lcC = sm[SM_LC * 64 + 63];
      const float gam = __expf(lc);
      sm[SM_NK * 64 + t] = nk;
      sm[SM_NQ * 64 + t] = nq;
      sm[SM_GK * 64 + t] = gam * nk;  // Gamma_t nk_t
      sm[SM_QG * 64 + t] = nq * gam;
      sm[SM_KD * 64 + t] = nk * __expf(lcC - lc);
    }
    lds_barrier();

    f32x4 R[4], oq[4];
    // ---- A and P tiles (t-tile tw, s-tile ns) with ns <= tw:
    // A_ts = beta_t nk_t nk_s (Gamma_t/Gamma_s) k_t.k_s (s < t), P_ts likewise with q_t (s <= t).
    // The ten tiles go at most two to a wave; tiles above the diagonal stay
    // zero.
    {
      // (the A or the P half alone when doA / doP is false)
      auto ap_tile = [&](int tw, int ns, bool doA = true, bool doP = true) {
        const int t = 16 * tw + c16;
        bf16x8 bk[4], bq[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
          if (doA) bk[ks] = ld8(Kc, (t * P136 + 8 * q4 + 32 * ks) * 2);
          if (doP) bq[ks] = ld8(Qc, (t * P136 + 8 * q4 + 32 * ks) * 2);
        }
        const float lct = sm[SM_LC * 64 + t], bnt = sm[SM_BETA * 64 + t] * sm[SM_NK * 64 + t];
        const float nqt = sm[SM_NQ * 64 + t];
        f32x4 aA = {0.f, 0.f, 0.f, 0.f}, aP = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
          const bf16x8 a = ld8(Kc, ((16 * ns + c16) * P136 + 8 * q4 + 32 * ks) * 2);
          if (doA) aA = mfma(a, bk[ks], aA);
          if (doP) aP = mfma(a, bq[ks], aP);
        }
        const int s0 = 16 * ns + 4 * q4;
        const float4 lcs = *(const float4 *)(sm + SM_LC * 64 + s0);
        const float4 nks = *(const float4 *)(sm + SM_NK * 64 + s0);
        const float lc4[4] = {lcs.x, lcs.y, lcs.z, lcs.w}, nk4[4] = {nks.x, nks.y, nks.z, nks.w};
        float av[4], pv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int s = s0 + r;
          const float e = s <= t ? __expf(lct - lc4[r]) : 0.0f;
          av[r] = s < t ? (bnt * nk4[r]) * e * aA[r] : 0.0f;
          pv[r] = s <= t ? (nqt * nk4[r]) * e * aP[r] : 0.0f;
        }
        if (doA && ns == tw) {
          *(float4 *)(AT + t * PA + s0) = make_float4(av[0], av[1], av[2], av[3]);
        } else if (doA && ns < tw) {  // -A of the block below the diagonal, as hi/lo
          const float na[4] = {-av[0], -av[1], -av[2], -av[3]};
          uint2 ah, al;
          split4(na, ah, al);
          *(uint2 *)(Tb + (t * P72 + pcol(s0)) * 2) = ah;
          *(uint2 *)(Tb + PC * P72 * 2 + (t * P72 + pcol(s0)) * 2) = al;
        }
        if (doP) {
          uint2 hi, lo;
          split4(pv, hi, lo);
          *(uint2 *)(Pl + (t * P72 + pcol(s0)) * 2) = hi;
          *(uint2 *)(Pl + PC * P72 * 2 + (t * P72 + pcol(s0)) * 2) = lo;
        }
      };
      // T_ii = (I + A_ii)^{-1}, diagonal block i by forward substitution on
      // the wave that computed A_ii (no barrier: the block is its own).
      // Column j of the block is solved by the four lanes 4j .. 4j + 3; lane
      // g of them holds rows g, g + 4, g + 8, g + 12.  At step s the lane
      // holding row s has its final x_s, which a quad broadcast (DPP) gives
      // the other three, and every row takes its term -A_rs x_s: each row's
      // sum runs over s in ascending order as in a row-by-row solve
      // (A_rs = 0 for s >= r adds nothing), and the dependent chain is 16
      // steps instead of 120 multiply-adds.
      auto diag_solve = [&](int i) {
        const float *blk = AT + 16 * i * PA + 16 * i;
        const int jc = l >> 2, g = l & 3;
        const float *rows = blk + g * PA;  // rows g + 4 k at rows[4 k PA]
        float acc[4];
#pragma unroll
        for (int k = 0; k < 4; k++) acc[k] = 4 * k + g == jc ? 1.0f : 0.0f;
        tsolve_step<0>(acc, rows);
#pragma unroll
        for (int k = 0; k < 4; k++) put_t(16 * i + 4 * k + g, 16 * i + jc, acc[k]);
      };
      // ---- K S0 (rows t, this wave's columns), consumed at once by
      // R = beta (V - Gamma nk K S0), and diag(nq Gamma) (S0^T Q^T), the
      // first term of O^T; S0 (hi/lo, key rows in the permuted slot order of
      // split8) is the shared operand, k and q enter exactly.  Independent
      // of the A/P tiles, so each wave's tiles and these products share one
      // scheduling region and their latencies overlap.
      bf16x8 sh[4], sl[4];
#pragma unroll
      for (int kc = 0; kc < 4; kc++) split8(S[2 * kc], S[2 * kc + 1], sh[kc], sl[kc]);
      // key-slot blocks outermost: the four token tiles' accumulators are
      // independent, so each block's loads are in flight while the previous
      // block's products run
      auto ks_part = [&]() {
        f32x4 ak[4];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) ak[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
          bf16x8 kr[4];
#pragma unroll
          for (int tt = 0; tt < 4; tt++) kr[tt] = ld8(Kc, ((16 * tt + c16) * P136 + 32 * kc + 8 * q4) * 2);
#pragma unroll
          for (int tt = 0; tt < 4; tt++) ak[tt] = mfma(kr[tt], sh[kc], ak[tt]);
#pragma unroll
          for (int tt = 0; tt < 4; tt++) ak[tt] = mfma(kr[tt], sl[kc], ak[tt]);
        }
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
          const int ta = 16 * tt + 4 * q4;
          const float4 be = *(const float4 *)(sm + SM_BETA * 64 + ta), gk = *(const float4 *)(sm + SM_GK * 64 + ta);
          const float be4[4] = {be.x, be.y, be.z, be.w}, gk4[4] = {gk.x, gk.y, gk.z, gk.w};
          const tr4_t vr = col4(Vc, ta, jw, c16);  // v of tokens ta .. ta + 3, column jw + c16
          const float v4[4] = {bf2f((uint16_t)vr[0]), bf2f((uint16_t)vr[1]), bf2f((uint16_t)vr[2]),
                               bf2f((uint16_t)vr[3])};
#pragma unroll
          for (int r = 0; r < 4; r++) R[tt][r] = be4[r] * (v4[r] - gk4[r] * ak[tt][r]);
        }
      };
      auto qs_part = [&]() {
        f32x4 aq[4];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) aq[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
          bf16x8 qr[4];
#pragma unroll
          for (int tt = 0; tt < 4; tt++) qr[tt] = ld8(Qc, ((16 * tt + c16) * P136 + 32 * kc + 8 * q4) * 2);
#pragma unroll
          for (int tt = 0; tt < 4; tt++) aq[tt] = mfma(sh[kc], qr[tt], aq[tt]);
#pragma unroll
          for (int tt = 0; tt < 4; tt++) aq[tt] = mfma(sl[kc], qr[tt], aq[tt]);
        }
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
          const float qgt = sm[SM_QG * 64 + 16 * tt + c16];
#pragma unroll
          for (int r = 0; r < 4; r++) oq[tt][r] = aq[tt][r] * qgt;
        }
      };
      // waves 0-3: diagonal tile i = w and its T_ii; waves 4-7: the six
      // tiles below the diagonal, two of them split into their A and P
      // halves, so that each SIMD (waves w and w + 4) holds two and a half
      // tile pairs and one diagonal solve
      switch (__builtin_amdgcn_readfirstlane(w)) {
        case 0: ap_tile(0, 0); ks_part(); diag_solve(0); qs_part(); break;
        case 1: ap_tile(1, 1); ks_part(); diag_solve(1); qs_part(); break;
        case 2: ap_tile(2, 2); ks_part(); diag_solve(2); qs_part(); break;
        case 3: ap_tile(3, 3); ks_part(); diag_solve(3); qs_part(); break;
        case 4: ap_tile(3, 0); ks_part(); ap_tile(3, 1, true, false); qs_part(); break;
        case 5: ap_tile(3, 2); ks_part(); ap_tile(1, 0, true, false); qs_part(); break;
        case 6: ap_tile(2, 0); ks_part(); ap_tile(3, 1, false, true); qs_part(); break;
        default: ap_tile(2, 1); ks_part(); ap_tile(1, 0, false, true); qs_part(); break;
      }
    }
    lds_barrier();

    // ---- Delta by blocks of 16 tokens, in this wave's registers (no barrier):
    // D_i = T_ii (R_i + sum_{k<i} (-A_ik) D_k), both products from M = [T_ii
    // on the diagonal, -A_ik below it].  A block that is solved is split
    // into hi/lo bf16 once, in place: as the B operand of 16 x 16 x 16
    // products (rows 4 q4 .. 4 q4 + 3 of column c16: the accumulator layout
    // itself) and, paired with its neighbour, of 16 x 16 x 32 products in
    // the permuted slot order.  Delta' = diag(nk Gamma_C / Gamma) Delta.
    f32x4 dp[4];
    bf16x8 ph01, pl01, ph23, pl23;  // [D_0; D_1] and [D_2; D_3] (hi, lo), permuted slots
    {
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      bf16x4 xh[4], xl[4];
      // acc + M[16 i .. 16 i + 15][16 k .. 16 k + 15] x (hi/lo pairs hi*hi + hi*lo + lo*hi)
      auto mone = [&](int i, int k, bf16x4 bh, bf16x4 bl, f32x4 acc) {
        const int o = ((16 * i + c16) * P72 + pcol(16 * k + 4 * q4)) * 2;
        const bf16x4 mh = ld4(Tb, o), ml = ld4(Tb, PC * P72 * 2 + o);
        acc = mfma16(mh, bh, acc);
        acc = mfma16(mh, bl, acc);
        return mfma16(ml, bh, acc);
      };
      // acc + M[16 i .. 16 i + 15][0 .. 31] [D_0; D_1]
      auto mpair = [&](int i, f32x4 acc) {
        const int o = ((16 * i + c16) * P72 + 8 * q4) * 2;
        const bf16x8 mh = ld8(Tb, o), ml = ld8(Tb, PC * P72 * 2 + o);
        acc = mfma(mh, ph01, acc);
        acc = mfma(mh, pl01, acc);
        return mfma(ml, ph01, acc);
      };
#pragma unroll
      for (int i = 0; i < 4; i++) {
        f32x4 acc = R[i];
        if (i == 1) acc = mone(1, 0, xh[0], xl[0], acc);
        if (i >= 2) acc = mpair(i, acc);
        if (i == 3) acc = mone(3, 2, xh[2], xl[2], acc);
        bf16x4 ah, al;
        split4x(acc, ah, al);
        const f32x4 d = mone(i, i, ah, al, zero);
        split4x(d, xh[i], xl[i]);
        if (i == 1) {
          ph01 = cat8(xh[0], xh[1]);
          pl01 = cat8(xl[0], xl[1]);
        }
        if (i == 3) {
          ph23 = cat8(xh[2], xh[3]);
          pl23 = cat8(xl[2], xl[3]);
        }
        const float4 kd = *(const float4 *)(sm + SM_KD * 64 + 16 * i + 4 * q4);
        dp[i][0] = d[0] * kd.x;
        dp[i][1] = d[1] * kd.y;
        dp[i][2] = d[2] * kd.z;
        dp[i][3] = d[3] * kd.w;
      }
    }
    // ---- O^T = diag(nq Gamma) (S0^T Q^T) + Delta^T P^T: rows j of this wave,
    // column t; a split pair [D_2kc; D_2kc+1] is the A operand of its
    // transpose as it is, and token pairs past the tile are causal zeros
    // (the six tile pairs' loads first, then their products interleaved
    // across the four independent token tiles)
    {
      bf16x8 ph[6], pl[6];
#pragma unroll
      for (int e = 0; e < 6; e++) {
        const int tt = e < 2 ? e : 2 + ((e - 2) >> 1), kc = e < 2 ? 0 : (e - 2) & 1;
        const int o = ((16 * tt + c16) * P72 + 32 * kc + 8 * q4) * 2;
        ph[e] = ld8(Pl, o);
        pl[e] = ld8(Pl, PC * P72 * 2 + o);
      }
      f32x4 acc[4] = {oq[0], oq[1], oq[2], oq[3]};
#pragma unroll
      for (int pass = 0; pass < 3; pass++)
#pragma unroll
        for (int kc = 0; kc < 2; kc++)
#pragma unroll
          for (int tt = 2 * kc; tt < 4; tt++) {
            const int e = tt < 2 ? tt : 2 + 2 * (tt - 2) + kc;
            const bf16x8 x = pass < 2 ? (kc ? ph23 : ph01) : (kc ? pl23 : pl01);
            acc[tt] = mfma(x, pass == 1 ? pl[e] : ph[e], acc[tt]);
          }
#pragma unroll
      for (int tt = 0; tt < 4; tt++) {
        const int t = 16 * tt + c16;
        if (t < n) {
          const float o4[4] = {acc[tt][0], acc[tt][1], acc[tt][2], acc[tt][3]};
          // the chunk's first output row as a wave-uniform index, the token
          // and column within it as a 32-bit offset
          const int64_t ob = (tb * H + h) * PV + jw;
          const int64_t at = ob + (int64_t)(uint32_t)(t * H * PV + 4 * q4);
          if (out_aligned) store4_aligned(D.out, D.out_dtype, at, o4);
          else store4(D.out, D.out_dtype, at, o4);
        }
      }
    }
    // ---- S <- Gamma_C S0 + K^T Delta' (rows d, this wave's columns; tokens
    // in the permuted slot order, two 4-token runs of the k column each)
    {
      bf16x8 eh[2], el[2];
      split8(dp[0], dp[1], eh[0], el[0]);
      split8(dp[2], dp[3], eh[1], el[1]);
      const float gC = __expf(sm[SM_LC * 64 + 63]);
      // four row tiles at a time: their eight loads first, then the
      // products interleaved across the four independent accumulators
#pragma unroll
      for (int d4 = 0; d4 < 8; d4 += 4) {
        bf16x8 a[4][2];
#pragma unroll
        for (int dt = d4; dt < d4 + 4; dt++) {
          const int d = 16 * dt + c16;
#pragma unroll
          for (int kc = 0; kc < 2; kc++) a[dt - d4][kc] = ld8(Kt, (d * P72 + tcol(d, 32 * kc + 8 * q4)) * 2);
#pragma unroll
          for (int r = 0; r < 4; r++) S[dt][r] = S[dt][r] * gC;
        }
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
#pragma unroll
          for (int dt = d4; dt < d4 + 4; dt++) S[dt] = mfma(a[dt - d4][kc], eh[kc], S[dt]);
#pragma unroll
          for (int dt = d4; dt < d4 + 4; dt++) S[dt] = mfma(a[dt - d4][kc], el[kc], S[dt]);
        }
      }
    }
    lds_barrier();  // the next chunk's staging overwrites the shared tiles
    c0 = c_next;
    // checkpoints reached at c0
    for (; ci < D.NC; ci++) {
      const int p = __builtin_amdgcn_readlane(ckv, ci);
      if (p > c0 && p <= len) break;
      if (p == c0) {
        float *dst = D.ck_state + (((int64_t)b * D.NC + ci) * H + h) * PKD * PV + jw + c16;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
          for (int r = 0; r < 4; r++) dst[(int64_t)(16 * dt + 4 * q4 + r) * PV] = S[dt][r];
      }
    }
  }
}

}  // namespace pf



// =====================================================================
// Chunked KDA prefill (per-channel decay), K = V = 128, chunks of 32
// tokens solved as two blocks of 16, bf16 MFMA with fp32 accumulation.  The recurrence of
// stepquant/core.py:5-15 with the KDA log decay g_t in R^K (the role of the
// upstream chunk kernel behind the reference's kernel_extend,
// sglang/runtime.py:193-202, for Kimi-Linear pools).
//
// For a chunk with start state S0 [K, V] and per-channel cumulative log
// decays G_t (G_tc = sum_{s<=t} g_sc):
//   A_ts  = beta_t sum_c k_tc k_sc e^{G_tc - G_sc}      (s < t)
//   P_ts  = sum_c q_tc k_sc e^{G_tc - G_sc}              (s <= t)
//   Delta = (I + A)^{-1} R,   R_t = beta_t (v_t - (k_t o e^{G_t})^T S0)
//   O_t   = (q_t o e^{G_t})^T S0 + sum_{s<=t} P_ts Delta_s
//   S_C   = diag(e^{G_C}) S0 + (K o e^{G_C - G})^T Delta
// (q, k L2-normalised and q scaled: the norms multiply into the products).
// Every decay factor above has a non-positive exponent except inside A and
// P, where e^{G_tc - G_sc} = e^{G_tc - G_Cc} e^{G_Cc - G_sc} (G_C: the last
// token) makes A and P MFMA products (each three 16 x 128 x 16 blocks on or
// below the diagonal).  The first factor
// grows to e^{G_0c - G_Cc}, the chunk's decay; when that exceeds 2^96 for
// any channel the chunk forms A and P pair by pair and channel by channel
// instead (sub, exp2, no factor that could overflow), so any gate is
// handled exactly.  The state-side products run on MFMA with
// every fp32 operand split into hi + lo bf16 (hi*hi + hi*lo + lo*hi, ~2^-16
// relative): K S0 and Q S0 as 16 x 16 x 32 products (S0 in the permuted
// k-slot order of pf::split8), Delta^T P^T and the state update as
// 16 x 16 x 16 products whose B operands are accumulator tiles as they are
// (the update's k operand read from the token-major tile by transposing LDS
// loads).  Delta solves (I + A) Delta = R block by block by forward
// substitution in each wave's registers (fp32, tokens in ascending order; the
// solved token's row reaches the other lane rows by v_permlane16/32_swap;
// block 1's right-hand side less A10 Delta_0 as one MFMA product), so no
// wave waits on another for an inverse.  One workgroup of 8 waves per (sequence, head); wave w owns
// state columns 16 w .. 16 w + 15 for all 128 rows in registers
// (accumulator layout).
// =====================================================================
namespace kc {

using pf::bf16x4;
using pf::bf16x8;
using pf::f32x4;

constexpr int C = 32;                   // tokens per chunk: two blocks of 16
constexpr int NT = 512;                 // 8 waves
constexpr int KV = 128;                 // K = V = 128
constexpr int RP = 136;                 // bf16 row pitch of token rows
constexpr int GP = 132;                 // f32 row pitch of the decay rows
constexpr int AP = 36;                  // f32 row pitch of A (rows 16-byte aligned)
constexpr int PP = 40;                  // bf16 row pitch of P and of -A10
constexpr int NPAIR = C * (C - 1) / 2;  // strictly lower pairs (t, s)
// LDS.  The hi planes of KB and QB hold the raw k and q rows from the
// staging until each thread replaces its own entries by the scaled operand.
constexpr int OFF_VR = 0;                         // bf16 [C][RP] v
constexpr int OFF_G = OFF_VR + C * RP * 2;        // f32 [C][GP] cumulative log2 decays
constexpr int OFF_KG = OFF_G + C * GP * 4;        // bf16 2 x [C][RP] nk k e^G (hi, lo), channels in pcol order
constexpr int OFF_QG = OFF_KG + 2 * C * RP * 2;   // bf16 2 x [C][RP] nq q e^G (hi, lo), channels in pcol order
constexpr int OFF_KE = OFF_QG + 2 * C * RP * 2;   // bf16 2 x [C][RP] nk k e^{G_C - G} (hi, lo)
constexpr int OFF_KB = OFF_KE + 2 * C * RP * 2;   // bf16 2 x [C][RP] k e^{G - G_C} (hi, lo); raw k first
constexpr int OFF_QB = OFF_KB + 2 * C * RP * 2;   // bf16 2 x [C][RP] q e^{G - G_C} (hi, lo); raw q first
constexpr int OFF_A = OFF_QB + 2 * C * RP * 2;   // f32 [C][AP] A (zero on and above the diagonal)
constexpr int OFF_M = OFF_A + C * AP * 4;         // bf16 2 x [16][PP] -A10 (hi, lo): rows 16.., columns 0..15
constexpr int OFF_PM = OFF_M + 2 * 16 * PP * 2;   // bf16 2 x [C][PP] P (hi, lo), zero above the diagonal
constexpr int OFF_SM = OFF_PM + 2 * C * PP * 2;   // f32 [4][C] beta, nk, nq; flags
constexpr int OFF_EC = OFF_SM + 4 * C * 4;        // f32 [KV] e^{G_C}
constexpr int LDS_BYTES = OFF_EC + KV * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS of the KDA chunk kernel");
enum { SM_BETA = 0, SM_NK, SM_NQ, SM_FLAG };
// a chunk whose decay exceeds 2^GROW_MAX on some channel takes the pairwise path
constexpr float GROW_MAX = 96.0f;

// (t, s) of strictly-lower pair p, t > s, pairs ordered by t then s
__constant__ uint8_t pair_t[NPAIR] = {1, 2, 2, 3, 3, 3, 4, 4, 4, 4, 5, 5, 5, 5, 5, 6, 6, 6, 6, 6, 6, 7, 7, 7, 7, 7, 7, 7, 8, 8, 8, 8, 8, 8, 8, 8, 9, 9, 9, 9, 9, 9, 9, 9, 9, 10, 10, 10, 10, 10, 10, 10, 10, 10, 10, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 12, 12, 12, 12, 12, 12, 12, 12, 12, 12, 12, 12, 13, 13, 13, 13, 13, 13, 13, 13, 13, 13, 13, 13, 13, 14, 14, 14, 14, 14, 14, 14, 14, 14, 14, 14, 14, 14, 14, 15, 15, 15, 15, 15, 15, 15, 15, 15, 15, 15, 15, 15, 15, 15, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 17, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 18, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 19, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 20, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 21, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 23, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 24, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 25, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 26, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 27, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 28, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 29, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 30, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31, 31};
__constant__ uint8_t pair_s[NPAIR] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3, 0, 1, 2, 3, 4, 0, 1, 2, 3, 4, 5, 0, 1, 2, 3, 4, 5, 6, 0, 1, 2, 3, 4, 5, 6, 7, 0, 1, 2, 3, 4, 5, 6, 7, 8, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30};

// Raw inputs of one chunk for this thread, fetched one chunk ahead: token
// tid >> 4, channels 8 (tid & 15) .. + 7 of k, q, v (bf16) and, in the
// decay mapping (channel tid >> 2, tokens 8 (tid & 3) .. + 7), the raw gates.
struct Fetch {
  uint4 k, q, v;
  float g[8];
  float beta;
  int n;
};

__device__ __forceinline__ void bf8(const uint4 &x, float o[8]) {
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int e = 0; e < 4; e++) {
    o[2 * e] = __uint_as_float(w[e] << 16);
    o[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}

// hi/lo halves of eight values as two packed bf16 x 8 (natural order)
__device__ __forceinline__ void split8v(const float x[8], uint4 &hi, uint4 &lo) {
  pf::split2(x[0], x[1], hi.x, lo.x);
  pf::split2(x[2], x[3], hi.y, lo.y);
  pf::split2(x[4], x[5], hi.z, lo.z);
  pf::split2(x[6], x[7], hi.w, lo.w);
}

// the value of 16-lane row Q of the wave in every row (two lane-row swaps)
template <int Q>
__device__ __forceinline__ float row_bcast(float x) {
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const uint32_t y = (Q & 1) ? s16[1] : s16[0];  // rows (x0, x0, x2, x2) or (x1, x1, x3, x3)
  const auto s32 = __builtin_amdgcn_permlane32_swap(y, y, false, false);
  return __uint_as_float((Q & 2) ? s32[1] : s32[0]);
}

// one step of a 16-token block's substitution: token S's Delta (row S / 4,
// register S % 4) to every lane, and -A[t][S] Delta_S into every token t of
// this lane (a[r][S]: the block's A row of the lane's token r, loaded before
// the first step; A is zero on and above the diagonal, so earlier tokens
// take exact zeros)
template <int S>
__device__ __forceinline__ void delta_step(float dv[4], const float (&a)[4][16]) {
  if constexpr (S < 16) {
    const float xs = row_bcast<S / 4>(dv[S % 4]);
#pragma unroll
    for (int r = 0; r < 4; r++) dv[r] = fmaf(-a[r][S], xs, dv[r]);
    delta_step<S + 1>(dv, a);
  }
}

// Delta of one 16-token block from its right-hand side: rows t0 + 4 q4 + r
// of A, columns c0 .. c0 + 15
__device__ __forceinline__ f32x4 block_solve(const float *A, int t0, int c0, int q4, const f32x4 &rhs) {
  float a[4][16];  // all loads issued before the chain
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const float4 x = *(const float4 *)(A + (t0 + 4 * q4 + r) * AP + c0 + 4 * m);
      a[r][4 * m] = x.x;
      a[r][4 * m + 1] = x.y;
      a[r][4 * m + 2] = x.z;
      a[r][4 * m + 3] = x.w;
    }
  float dv[4] = {rhs[0], rhs[1], rhs[2], rhs[3]};
  delta_step<0>(dv, a);
  const f32x4 d = {dv[0], dv[1], dv[2], dv[3]};
  return d;
}

// acc + (16 x 16 hi/lo matrix at byte offset o of `tile`, lo plane `lo`
// bytes further) x (the hi/lo B operand xh, xl)
__device__ __forceinline__ f32x4 mm16(const uint8_t *tile, int o, int lo, bf16x4 xh, bf16x4 xl, f32x4 acc) {
  const bf16x4 mh = pf::ld4(tile, o), ml = pf::ld4(tile, lo + o);
  acc = pf::mfma16(mh, xh, acc);
  acc = pf::mfma16(mh, xl, acc);
  return pf::mfma16(ml, xh, acc);
}

// acc + (the hi/lo A operand xh, xl) x (16 x 16 hi/lo matrix at byte offset o
// of `tile`, lo plane `lo` bytes further, as the B operand)
__device__ __forceinline__ f32x4 mm16t(const uint8_t *tile, int o, int lo, bf16x4 xh, bf16x4 xl, f32x4 acc) {
  const bf16x4 mh = pf::ld4(tile, o), ml = pf::ld4(tile, lo + o);
  acc = pf::mfma16(xh, mh, acc);
  acc = pf::mfma16(xh, ml, acc);
  return pf::mfma16(xl, mh, acc);
}

// Initial state of one (sequence, head) of a KDA pool with K = V = 128
// (per-row widths, FP16 pivot rows, 4-value tiles), read from its page: the
// head's code, row-scale and column-scale regions and its rows' plan entries
// are copied into LDS (the chunk tiles' space, unused until the first
// chunk), then each lane decodes the 32 values of its column j = 16 w + c16
// (block j / 4, field j % 4) with the KDA page decode's operations in its
// order, x = (r c_j)((s + 1) 2^(8-b)) with s the field with its top bit
// flipped, sign-extended, and the stored half for pivot rows, so the state
// is the dense decode's to the bit.
constexpr int KI_ROWS = 33024, KI_COLS = KI_ROWS + 288, KI_TAB = KI_COLS + 288;  // LDS offsets past the code
static_assert(KI_TAB + 3 * KV * 4 <= OFF_A, "the staged page must not overlap A, which is cleared at the start");

__device__ __forceinline__ void kda_init_from_page(const pf::PageInit &pi, int b, int h, int H, uint8_t *lds, int tid,
                                                   pf::f32x4 S[8]) {
#pragma clang fp contract(off)
  const int w = tid >> 6, q4 = (tid >> 4) & 3, c16 = tid & 15;
  const int64_t slot = pi.slots_dtype == SQ_I64 ? ld_uniform((const int64_t *)pi.slots + b)
                                                 : (int64_t)ld_uniform((const int32_t *)pi.slots + b);
  if (slot <= 0 || slot >= pi.num_slots) {  // whole workgroup: a zero state
#pragma unroll
    for (int dt = 0; dt < 8; dt++) S[dt] = pf::f32x4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  const int32_t *hm = pi.head_meta + 4 * h;
  const int code_start = ld_uniform(hm), code_bytes = ld_uniform(hm + 1);
  const int row_start = ld_uniform(hm + 2), row_bytes = ld_uniform(hm + 3);
  const int colbase = ld_uniform(pi.columns + h);
  const int stride = ld_uniform(pi.offsets + (int64_t)H * KV + h);
  const uint8_t *page = pi.data + slot * pi.page_bytes;
  // 16-byte windows around each region (pages may start on any even byte)
  auto stage = [&](const uint8_t *g, int nbytes, uint8_t *dst) {
    const int sh = (int)((uintptr_t)g & 15);
    const uint4 *src = (const uint4 *)(g - sh);
    for (int e = tid; e < (sh + nbytes + 15) >> 4; e += NT) ((uint4 *)dst)[e] = src[e];
    return sh;
  };
  const int shc = stage(page + code_start, code_bytes, lds);
  const int shr = row_bytes > 0 ? stage(page + row_start, row_bytes, lds + KI_ROWS) : 0;
  const int shk = colbase >= 0 ? stage(page + colbase, 2 * KV, lds + KI_COLS) : 0;
  int *tab = (int *)(lds + KI_TAB);  // per row: width, code offset within a block, row-scale offset
  if (tid < KV) {
    const int64_t e = (int64_t)h * KV + tid;
    tab[tid] = pi.bits[e];
    tab[KV + tid] = pi.offsets[e] - code_start;
    tab[2 * KV + tid] = pi.rows[e] - row_start;
  }
  __syncthreads();
  const int j = 16 * w + c16, f = j & 3;
  const float cj = colbase >= 0 ? fast::hw_h2f(*(const uint16_t *)(lds + KI_COLS + shk + 2 * j)) : 1.0f;
  const int blk = shc + (j >> 2) * stride;  // this column's block within the staged window (an even byte)
#pragma unroll
  for (int dt = 0; dt < 8; dt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int d = 16 * dt + 4 * q4 + r;
      const int bw = tab[d], pos = blk + tab[KV + d];
      float x;
      if (bw == 16) {
        x = fast::hw_h2f(*(const uint16_t *)(lds + pos + 2 * f)) * 1.0f;
      } else {
        const float rr = fast::hw_h2f(*(const uint16_t *)(lds + KI_ROWS + shr + tab[2 * KV + d]));
        uint32_t xm = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) xm |= 1u << (c * bw + bw - 1);
        const uint32_t word = kfast::word_at(lds, pos) ^ xm;
        const int sv = kfast::sbfe(word, (uint32_t)(f * bw), (uint32_t)bw);
        x = (rr * cj) * ((float)(sv + 1) * (float)(1 << (8 - bw)));
      }
      S[dt][r] = x;
    }
}

__global__ __launch_bounds__(NT) void kda_chunk_kernel(pf::PrefillDev D) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = D.H;
  const int h = blockIdx.x % H, b = blockIdx.x / H;
  const int hk = h / (H / D.HK);
  const int t0 = __builtin_amdgcn_readfirstlane(D.cu[b]);
  const int len = __builtin_amdgcn_readfirstlane(D.cu[b + 1]) - t0;
  if (len <= 0) return;  // whole workgroup
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, q4 = l >> 4, c16 = l & 15;
  const int jw = 16 * w;
  uint8_t *VR = smem + OFF_VR;
  float *G = (float *)(smem + OFF_G);
  uint8_t *KG = smem + OFF_KG, *QG = smem + OFF_QG, *KE = smem + OFF_KE, *KB = smem + OFF_KB, *QB = smem + OFF_QB;
  uint8_t *M = smem + OFF_M, *PM = smem + OFF_PM;
  float *A = (float *)(smem + OFF_A);
  float *sm = (float *)(smem + OFF_SM);
  float *EC = (float *)(smem + OFF_EC);
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr int KB_LO = C * RP * 2, PLO = C * PP * 2, MLO = 16 * PP * 2;
  // A and P: entries on / above the diagonal stay zero (written once; the
  // MFMA path rewrites them with zeros); the pairwise-path flags start clear
  for (int e = tid; e < C * PP; e += NT) ((uint32_t *)PM)[e] = 0u;
  for (int e = tid; e < C * AP; e += NT) A[e] = 0.0f;
  if (tid < 2) sm[SM_FLAG * C + tid] = 0.0f;
  pf::lds_barrier();

  // ---- state S[d][j] of this wave's columns: tile dt holds rows d = 16 dt + 4 q4 + r, column jw + c16
  f32x4 S[8];
  if (D.page_init) {
    kda_init_from_page(D.pi, b, h, H, smem, tid, S);
    __syncthreads();  // the staged page is read before the first chunk's tiles overwrite it
  } else {
    const float *src = D.init + ((int64_t)b * H + h) * KV * KV + jw + c16;
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
      for (int r = 0; r < 4; r++) S[dt][r] = src[(int64_t)(16 * dt + 4 * q4 + r) * KV];
  }
  const int ckv = l < D.NC ? D.ckpt[(int64_t)b * D.NC + l] : 0x7fffffff;
  auto segment = [&](int c) {  // tokens of the chunk at c: up to the next checkpoint, the end, or C
    const uint64_t m = __ballot(ckv > c && ckv <= len);
    const int stop = m ? __builtin_amdgcn_readlane(ckv, __builtin_ctzll(m)) : len;
    return stop - c < C ? stop - c : C;
  };
  // staging mapping: token tt, channels c8 .. c8 + 7; decay mapping: channel gc, tokens 8 gq .. 8 gq + 7
  const int tt = tid >> 4, c8 = (tid & 15) * 8;
  const int gc = tid >> 2, gq = tid & 3;
  const float ea = D.a_log ? __expf(load_val(D.a_log, D.gate_dtype, h)) : 0.0f;
  const float dtb = D.a_log ? load_val(D.dt_bias, D.gate_dtype, (int64_t)h * KV + gc) : 0.0f;
  const uint8_t *qg = (const uint8_t *)D.q, *kg = (const uint8_t *)D.k, *vg = (const uint8_t *)D.v;
  auto fetch = [&](Fetch &F, int c) {
    F.n = c < len ? segment(c) : 0;
    const int last = len - 1;
    const int64_t row = (int64_t)t0 + (c + tt < len ? c + tt : last);
    F.k = *(const uint4 *)(kg + (row * D.k_stride + (int64_t)hk * KV + c8) * 2);
    F.q = *(const uint4 *)(qg + (row * D.q_stride + (int64_t)hk * KV + c8) * 2);
    F.v = *(const uint4 *)(vg + (row * D.v_stride + (int64_t)h * KV + c8) * 2);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int64_t gr = (int64_t)t0 + (c + 8 * gq + i < len ? c + 8 * gq + i : last);
      F.g[i] = load_val(D.g, D.gate_dtype, (gr * H + h) * KV + gc);
    }
    const int64_t br = (int64_t)t0 + (c + (l & 31) < len ? c + (l & 31) : last);
    F.beta = load_val(D.beta, D.gate_dtype, br * H + h);
  };

  Fetch F;
  // ---- staging of the chunk whose inputs are in F (n tokens, flag word pa): v
  // rows, raw k and q rows, norms, beta; cumulative decays per channel
  auto stage_chunk = [&](int pa) {
    const int n = F.n;
    float kf[8], qf[8];
    bf8(F.k, kf);
    bf8(F.q, qf);
    const bool live = tt < n;
    const uint32_t mk = live ? 0xffffffffu : 0u;  // tokens past the chunk's: zero rows
    *(uint4 *)(KB + (tt * RP + c8) * 2) = make_uint4(F.k.x & mk, F.k.y & mk, F.k.z & mk, F.k.w & mk);
    *(uint4 *)(QB + (tt * RP + c8) * 2) = make_uint4(F.q.x & mk, F.q.y & mk, F.q.z & mk, F.q.w & mk);
    *(uint4 *)(VR + (tt * RP + c8) * 2) = make_uint4(F.v.x & mk, F.v.y & mk, F.v.z & mk, F.v.w & mk);
    float sk = 0.f, sq = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      sk = fmaf(kf[e], kf[e], sk);
      sq = fmaf(qf[e], qf[e], sq);
    }
    sk = pf::row16_sum(sk);
    sq = pf::row16_sum(sq);
    if ((tid & 15) == 0) {
      sm[SM_NK * C + tt] = live && D.normalize ? __builtin_amdgcn_rsqf(sk + 1e-6f) : (live ? 1.0f : 0.0f);
      sm[SM_NQ * C + tt] = live ? (D.normalize ? __builtin_amdgcn_rsqf(sq + 1e-6f) : 1.0f) * D.scale : 0.0f;
    }
    if (w == 0 && l < C) {
      float bt = F.beta;
      if (D.beta_logits) bt = __builtin_amdgcn_rcpf(1.0f + __expf(-bt));
      sm[SM_BETA * C + l] = l < n ? bt : 0.0f;
    }
    // log2 decays of tokens 8 gq .. 8 gq + 7 of channel gc (0 past the
    // chunk's tokens), then the inclusive scan over the 32 tokens: within
    // the thread, then across the quad (lanes gq = 0..3 of the channel)
    float gl[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float gv = F.g[i];
      if (D.a_log) {
        const float u = gv + dtb;
        const float sp = u > 20.0f ? u : __logf(1.0f + __expf(u < 20.0f ? u : 20.0f));
        gv = -ea * sp;
      }
      gl[i] = 8 * gq + i < n ? gv * LOG2E : 0.0f;
    }
#pragma unroll
    for (int i = 1; i < 8; i++) gl[i] += gl[i - 1];
    const float tot = gl[7];
    const float t1 = pf::quad_bcast<0>(tot), t2 = pf::quad_bcast<1>(tot), t3 = pf::quad_bcast<2>(tot);
    const float pre = gq == 0 ? 0.0f : gq == 1 ? t1 : gq == 2 ? t1 + t2 : (t1 + t2) + t3;
#pragma unroll
    for (int i = 0; i < 8; i++) G[(8 * gq + i) * GP + gc] = pre + gl[i];
    // the chunk's decay of channel gc (log2): G_0 - G_C, read on lane gq = 0
    const float gC = ((t1 + t2) + t3) + pf::quad_bcast<3>(tot);
    if (gq == 0 && gl[0] - gC > GROW_MAX) sm[SM_FLAG * C + pa] = 1.0f;
    return n;
  };

  fetch(F, 0);
  int ci = 0;
  int par = 0;  // chunk parity: which flag word this chunk uses
  int n = stage_chunk(par);
  fetch(F, n);  // the next chunk's inputs are in flight while this one is computed
  pf::lds_barrier();
  for (int c0 = 0; c0 < len; par ^= 1) {
    const int c_next = c0 + n;
    const bool pairwise = sm[SM_FLAG * C + par] != 0.0f;  // workgroup-uniform
    // ---- operands of token tt, channels c8 .. c8 + 7: nk k e^G and nq q e^G
    // (hi/lo, pcol order), nk k e^{G_C - G} (hi/lo), e^{G_C}; for the MFMA path
    // k e^{G - G_C} and q e^{G - G_C} (hi/lo) in place of the raw rows
    {
      const float nk = sm[SM_NK * C + tt], nq = sm[SM_NQ * C + tt];
      float g8[8], gc8[8];
      {
        const float4 a0 = *(const float4 *)(G + tt * GP + c8), a1 = *(const float4 *)(G + tt * GP + c8 + 4);
        const float4 e0 = *(const float4 *)(G + (C - 1) * GP + c8), e1 = *(const float4 *)(G + (C - 1) * GP + c8 + 4);
        const float ga[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float ge[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
          g8[e] = ga[e];
          gc8[e] = ge[e];
        }
      }
      float kf[8], qf[8];
      bf8(*(const uint4 *)(KB + (tt * RP + c8) * 2), kf);
      bf8(*(const uint4 *)(QB + (tt * RP + c8) * 2), qf);
      float kgv[8], qgv[8], kdv[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float eg = __builtin_amdgcn_exp2f(g8[e]);
        kgv[e] = (nk * kf[e]) * eg;
        qgv[e] = (nq * qf[e]) * eg;
        kdv[e] = (nk * kf[e]) * __builtin_amdgcn_exp2f(gc8[e] - g8[e]);
      }
      {
        // channels c8 .. c8 + 3 and c8 + 4 .. c8 + 7 at their permuted places
        uint4 kh8, kl8, qh8, ql8;
        split8v(kgv, kh8, kl8);
        split8v(qgv, qh8, ql8);
        const int p0 = pf::pcol(c8), p1 = pf::pcol(c8 + 4);
        *(uint2 *)(KG + (tt * RP + p0) * 2) = make_uint2(kh8.x, kh8.y);
        *(uint2 *)(KG + (tt * RP + p1) * 2) = make_uint2(kh8.z, kh8.w);
        *(uint2 *)(KG + KB_LO + (tt * RP + p0) * 2) = make_uint2(kl8.x, kl8.y);
        *(uint2 *)(KG + KB_LO + (tt * RP + p1) * 2) = make_uint2(kl8.z, kl8.w);
        *(uint2 *)(QG + (tt * RP + p0) * 2) = make_uint2(qh8.x, qh8.y);
        *(uint2 *)(QG + (tt * RP + p1) * 2) = make_uint2(qh8.z, qh8.w);
        *(uint2 *)(QG + KB_LO + (tt * RP + p0) * 2) = make_uint2(ql8.x, ql8.y);
        *(uint2 *)(QG + KB_LO + (tt * RP + p1) * 2) = make_uint2(ql8.z, ql8.w);
      }
      uint4 h4, l4;
      split8v(kdv, h4, l4);
      *(uint4 *)(KE + (tt * RP + c8) * 2) = h4;
      *(uint4 *)(KE + KB_LO + (tt * RP + c8) * 2) = l4;
      if (!pairwise) {
        float kbv[8], qbv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float eb = __builtin_amdgcn_exp2f(g8[e] - gc8[e]);
          kbv[e] = kf[e] * eb;
          qbv[e] = qf[e] * eb;
        }
        split8v(kbv, h4, l4);
        *(uint4 *)(KB + (tt * RP + c8) * 2) = h4;  // over this thread's own raw entries
        *(uint4 *)(KB + KB_LO + (tt * RP + c8) * 2) = l4;
        split8v(qbv, h4, l4);
        *(uint4 *)(QB + (tt * RP + c8) * 2) = h4;
        *(uint4 *)(QB + KB_LO + (tt * RP + c8) * 2) = l4;
      }
      if (tt == 0) {
        *(float4 *)(EC + c8) = make_float4(__builtin_amdgcn_exp2f(gc8[0]), __builtin_amdgcn_exp2f(gc8[1]),
                                           __builtin_amdgcn_exp2f(gc8[2]), __builtin_amdgcn_exp2f(gc8[3]));
        *(float4 *)(EC + c8 + 4) = make_float4(__builtin_amdgcn_exp2f(gc8[4]), __builtin_amdgcn_exp2f(gc8[5]),
                                               __builtin_amdgcn_exp2f(gc8[6]), __builtin_amdgcn_exp2f(gc8[7]));
      }
    }
    // ---- pairwise path: A and P below the diagonal, pair by pair over 32
    // channels per lane (four lanes per pair) with the exact pairwise decays
    // from the raw rows; P's diagonal from q_t . k_t
    if (pairwise) {
      for (int task = tid; task < 4 * NPAIR + C; task += NT) {
        if (task < 4 * NPAIR) {
          const int p = task >> 2, part = task & 3;
          const int t = pair_t[p], s = pair_s[p];
          const int cb = 32 * part;
          float a = 0.f, pp = 0.f;
#pragma unroll
          for (int m = 0; m < 4; m++) {
            const int c = cb + 8 * m;
            float kt[8], qt[8], ks[8];
            bf8(*(const uint4 *)(KB + (t * RP + c) * 2), kt);
            bf8(*(const uint4 *)(QB + (t * RP + c) * 2), qt);
            bf8(*(const uint4 *)(KB + (s * RP + c) * 2), ks);
            const float4 ga0 = *(const float4 *)(G + t * GP + c), ga1 = *(const float4 *)(G + t * GP + c + 4);
            const float4 gb0 = *(const float4 *)(G + s * GP + c), gb1 = *(const float4 *)(G + s * GP + c + 4);
            const float dg[8] = {ga0.x - gb0.x, ga0.y - gb0.y, ga0.z - gb0.z, ga0.w - gb0.w,
                                 ga1.x - gb1.x, ga1.y - gb1.y, ga1.z - gb1.z, ga1.w - gb1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
              const float kse = ks[e] * __builtin_amdgcn_exp2f(dg[e]);
              a = fmaf(kt[e], kse, a);
              pp = fmaf(qt[e], kse, pp);
            }
          }
          a += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0xB1, 0xF, 0xF, false));   // lane ^ 1
          pp += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pp), 0xB1, 0xF, 0xF, false));
          a += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x4E, 0xF, 0xF, false));   // lane ^ 2
          pp += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pp), 0x4E, 0xF, 0xF, false));
          if (part == 0) {
            const float nks = sm[SM_NK * C + s];
            const float av = ((sm[SM_BETA * C + t] * sm[SM_NK * C + t]) * nks) * a;
            A[t * AP + s] = av;
            if (t >= 16 && s < 16) {  // -A10 for the second block's right-hand side
              const __bf16 hi = (__bf16)(-av);
              ((__bf16 *)M)[(t - 16) * PP + s] = hi;
              ((__bf16 *)M)[16 * PP + (t - 16) * PP + s] = (__bf16)(-av - (float)hi);
            }
            const float pv = (sm[SM_NQ * C + t] * nks) * pp;
            const __bf16 hi = (__bf16)pv;
            ((__bf16 *)PM)[t * PP + s] = hi;
            ((__bf16 *)PM)[C * PP + t * PP + s] = (__bf16)(pv - (float)hi);
          }
        } else {
          const int t = task - 4 * NPAIR;
          float d = 0.f;
#pragma unroll 4
          for (int c = 0; c < KV; c += 8) {
            float kt[8], qt[8];
            bf8(*(const uint4 *)(KB + (t * RP + c) * 2), kt);
            bf8(*(const uint4 *)(QB + (t * RP + c) * 2), qt);
#pragma unroll
            for (int e = 0; e < 8; e++) d = fmaf(qt[e], kt[e], d);
          }
          const float pv = (sm[SM_NQ * C + t] * sm[SM_NK * C + t]) * d;
          const __bf16 hi = (__bf16)pv;
          ((__bf16 *)PM)[t * PP + t] = hi;
          ((__bf16 *)PM)[C * PP + t * PP + t] = (__bf16)(pv - (float)hi);
        }
      }
    }
    pf::lds_barrier();
    if (tid == 0) sm[SM_FLAG * C + par] = 0.0f;  // read by every thread before the barrier above
    // ---- MFMA path: the three A blocks (waves 0-2) and three P blocks
    // (waves 3-5) below or on the diagonal as 16 x 128 x 16 products of the
    // growing and the decaying factors: A_ts = beta_t nk_t (k_t e^{G_t -
    // G_C}) . (nk_s k_s e^{G_C - G_s}) for s < t, P_ts = nq_t (q_t e^{G_t -
    // G_C}) . (nk_s k_s e^{G_C - G_s}) for s <= t (zero above)
    if (!pairwise && w < 6) {
      const int blk = w < 3 ? w : w - 3;
      const int ti = blk == 0 ? 0 : 1, si = blk == 2 ? 1 : 0;
      const uint8_t *X = w < 3 ? KB : QB;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 4; kc++) {
        const int ox = ((16 * ti + c16) * RP + 32 * kc + 8 * q4) * 2, oe = ((16 * si + c16) * RP + 32 * kc + 8 * q4) * 2;
        const bf16x8 xh = pf::ld8(X, ox), xl = pf::ld8(X, KB_LO + ox);
        const bf16x8 eh = pf::ld8(KE, oe), el = pf::ld8(KE, KB_LO + oe);
        acc = pf::mfma(xh, eh, acc);
        acc = pf::mfma(xh, el, acc);
        acc = pf::mfma(xl, eh, acc);
      }
      // acc[r]: token t = 16 ti + 4 q4 + r, source s = 16 si + c16
      const int s0 = 16 * si + c16;
      if (w < 3) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int t = 16 * ti + 4 * q4 + r;
          const float av = s0 < t ? (sm[SM_BETA * C + t] * sm[SM_NK * C + t]) * acc[r] : 0.0f;
          A[t * AP + s0] = av;
          if (blk == 1) {
            const __bf16 hi = (__bf16)(-av);
            ((__bf16 *)M)[(t - 16) * PP + s0] = hi;
            ((__bf16 *)M)[16 * PP + (t - 16) * PP + s0] = (__bf16)(-av - (float)hi);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int t = 16 * ti + 4 * q4 + r;
          const float pv = s0 <= t ? sm[SM_NQ * C + t] * acc[r] : 0.0f;
          const __bf16 hi = (__bf16)pv;
          ((__bf16 *)PM)[t * PP + s0] = hi;
          ((__bf16 *)PM)[C * PP + t * PP + s0] = (__bf16)(pv - (float)hi);
        }
      }
    }
    // ---- K S0 and Q S0 for this wave's columns, two 16-token tiles
    bf16x8 sh[4], sl[4];
#pragma unroll
    for (int kc = 0; kc < 4; kc++) pf::split8(S[2 * kc], S[2 * kc + 1], sh[kc], sl[kc]);
    f32x4 R[2], oq[2];
    // key-slot blocks outermost: the four accumulators (k and q, two token
    // tiles) are independent, and each product pass runs over all four
    f32x4 ak[2], aq[2];
#pragma unroll
    for (int tb = 0; tb < 2; tb++) ak[tb] = aq[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < 4; kc++) {
      bf16x8 kh[2], kl[2], qh[2], ql[2];
#pragma unroll
      for (int tb = 0; tb < 2; tb++) {
        const int o = ((16 * tb + c16) * RP + 32 * kc + 8 * q4) * 2;
        kh[tb] = pf::ld8(KG, o);
        kl[tb] = pf::ld8(KG, KB_LO + o);
        qh[tb] = pf::ld8(QG, o);
        ql[tb] = pf::ld8(QG, KB_LO + o);
      }
#pragma unroll
      for (int tb = 0; tb < 2; tb++) {
        ak[tb] = pf::mfma(kh[tb], sh[kc], ak[tb]);
        aq[tb] = pf::mfma(sh[kc], qh[tb], aq[tb]);
      }
#pragma unroll
      for (int tb = 0; tb < 2; tb++) {
        ak[tb] = pf::mfma(kh[tb], sl[kc], ak[tb]);
        aq[tb] = pf::mfma(sl[kc], qh[tb], aq[tb]);
      }
#pragma unroll
      for (int tb = 0; tb < 2; tb++) {
        ak[tb] = pf::mfma(kl[tb], sh[kc], ak[tb]);
        aq[tb] = pf::mfma(sh[kc], ql[tb], aq[tb]);
      }
    }
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
      // R_t = beta_t (v_t - (nk k e^G)_t S0), tokens 16 tb + 4 q4 .. + 3, column jw + c16
      const pf::tr4_t vr = pf::col4(VR, 16 * tb + 4 * q4, jw, c16);
      const float4 be = *(const float4 *)(sm + SM_BETA * C + 16 * tb + 4 * q4);
      const float be4[4] = {be.x, be.y, be.z, be.w};
#pragma unroll
      for (int r = 0; r < 4; r++) R[tb][r] = be4[r] * (pf::bf2f((uint16_t)vr[r]) - ak[tb][r]);
      oq[tb] = aq[tb];  // O^T first term: column 4 q4 + r, token 16 tb + c16
    }
    pf::lds_barrier();
    // ---- (I + A) Delta = R by blocks: Delta_0 from block 0, then block 1's
    // right-hand side less A10 Delta_0 (M holds -A10); O^T += Delta^T P^T;
    // S <- diag(e^{G_C}) S0 + Kd^T Delta over the 32 tokens
    const f32x4 d0 = block_solve(A, 0, 0, q4, R[0]);
    bf16x4 d0h, d0l;
    pf::split4x(d0, d0h, d0l);
    const f32x4 d1 = block_solve(A, 16, 16, q4, mm16(M, (c16 * PP + 4 * q4) * 2, MLO, d0h, d0l, R[1]));
    bf16x4 d1h, d1l;
    pf::split4x(d1, d1h, d1l);
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
      // rows of P for tokens 16 tb + c16: the blocks of source tokens 0-15 and (tb = 1) 16-31
      const int o = ((16 * tb + c16) * PP + 4 * q4) * 2;
      f32x4 acc = oq[tb];
      acc = mm16t(PM, o, PLO, d0h, d0l, acc);
      if (tb == 1) acc = mm16t(PM, o + 32, PLO, d1h, d1l, acc);
      const int t = 16 * tb + c16;
      if (t < n) {
        const float o4[4] = {acc[0], acc[1], acc[2], acc[3]};
        const int64_t at = ((int64_t)(t0 + c0 + t) * H + h) * KV + jw + 4 * q4;
        store4(D.out, D.out_dtype, at, o4);
      }
    }
    {
      bf16x8 eh, el;
      pf::split8(d0, d1, eh, el);  // the 32 tokens in the permuted slot order (pcol)
      // four row tiles at a time: their loads first, then each product pass
      // over the four independent accumulators
#pragma unroll
      for (int d4 = 0; d4 < 8; d4 += 4) {
        bf16x8 kh[4], kl[4];
#pragma unroll
        for (int dt = d4; dt < d4 + 4; dt++) {
          // Kd rows 16 dt + c16 (channels) over the 32 tokens in the slot order
          // of split8: transposing loads of tokens 4 q4 .. + 3 and 16 + 4 q4 .. + 3
          kh[dt - d4] = pf::cat8(pf::col4(KE, 4 * q4, 16 * dt, c16), pf::col4(KE, 16 + 4 * q4, 16 * dt, c16));
          kl[dt - d4] = pf::cat8(pf::col4(KE + KB_LO, 4 * q4, 16 * dt, c16),
                                 pf::col4(KE + KB_LO, 16 + 4 * q4, 16 * dt, c16));
          const float4 ec = *(const float4 *)(EC + 16 * dt + 4 * q4);
          S[dt][0] = S[dt][0] * ec.x;
          S[dt][1] = S[dt][1] * ec.y;
          S[dt][2] = S[dt][2] * ec.z;
          S[dt][3] = S[dt][3] * ec.w;
        }
#pragma unroll
        for (int dt = d4; dt < d4 + 4; dt++) S[dt] = pf::mfma(kh[dt - d4], eh, S[dt]);
#pragma unroll
        for (int dt = d4; dt < d4 + 4; dt++) S[dt] = pf::mfma(kh[dt - d4], el, S[dt]);
#pragma unroll
        for (int dt = d4; dt < d4 + 4; dt++) S[dt] = pf::mfma(kl[dt - d4], eh, S[dt]);
      }
    }
    // The next chunk's staging, issued behind the state update's products
    // (its exponentials and scan run while they do): its rows, norms, beta
    // and decays go to tiles that this chunk no longer reads (the update
    // reads KE and EC only), and the barrier below orders them before use.
    const int n_next = stage_chunk(par ^ 1);
    fetch(F, c_next + n_next);
    pf::lds_barrier();  // the next chunk's staging is complete, this chunk's tiles are read
    c0 = c_next;
    n = n_next;
    for (; ci < D.NC; ci++) {
      const int p = __builtin_amdgcn_readlane(ckv, ci);
      if (p > c0 && p <= len) break;
      if (p == c0) {
        float *dst = D.ck_state + (((int64_t)b * D.NC + ci) * H + h) * KV * KV + jw + c16;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
          for (int r = 0; r < 4; r++) dst[(int64_t)(16 * dt + 4 * q4 + r) * KV] = S[dt][r];
      }
    }
  }
}

}  // namespace kc

__global__ void fill_zero_kernel(float *p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0.0f;
}

__global__ void clear_kernel(uint8_t *data, int64_t page_bytes, int64_t num_slots, const void *slots,
                             int dtype) {
  int64_t s = load_slot(slots, dtype, blockIdx.y);
  if (s < 0) s += num_slots;
  if (s < 0 || s >= num_slots) return;
  uint8_t *p = data + s * page_bytes;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < page_bytes;
       e += (int64_t)gridDim.x * blockDim.x)
    p[e] = 0;
}

// Pages src[y] -> temp[y] (scatter == 0) or temp[y] -> dst[y] (scatter == 1).
// Negative indices wrap like Python; a pair whose source or destination
// lies outside the pool is skipped in both passes, so a destination never
// receives a temp page that the gather did not write.
__global__ void gather_kernel(const uint8_t *data, int64_t page_bytes, int64_t num_slots, const void *src,
                              const void *dst, int dtype, uint8_t *temp, int scatter) {
  int64_t s = load_slot(src, dtype, blockIdx.y);
  int64_t d = load_slot(dst, dtype, blockIdx.y);
  if (s < 0) s += num_slots;
  if (d < 0) d += num_slots;
  if (s < 0 || s >= num_slots || d < 0 || d >= num_slots) return;
  uint8_t *t = temp + (int64_t)blockIdx.y * page_bytes;
  uint8_t *p = (uint8_t *)data + (scatter ? d : s) * page_bytes;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < page_bytes;
       e += (int64_t)gridDim.x * blockDim.x) {
    if (scatter) p[e] = t[e];
    else t[e] = p[e];
  }
}

// =====================================================================
// Baseline state formats (reference kernels/format_pool.py:29-128 with the
// programs of kernels/formats.py and kernels/floating.py; CPU definitions
// formats.py:53-86 group_fit / dual_fit):
//   FP32       the page is the fp32 state: value (i, j) at offsets[hK+i] + 4j.
//   SYMMETRIC  per (row, 128-value group g): fp16 s = fp16(max|x| / L) at
//              rows[hK+i] + 4g and an fp16 zero point z = L two bytes after
//              it; codes rint(x / s) clamped to [-L, L], plus L.
//   DSQ        fp16 r_i = fp16(sqrt(max(mean_j |x_ij|, 1e-20))) at rows[hK+i];
//              fp16 c_j = fp16(max_i |x_ij / r_i| / L) and a zero half at
//              columns[h] + 4j; codes rint((x / r) / c) clamped, plus L.
// L = 2^(b-1) - 1.  Codes of a row are a little-endian bit stream at
// offsets[hK+i] (value j at bit j*b).  Decoding: (code - z) * s and
// (r * c) * (code - L).  Every product, quotient and sum rounds separately
// (IEEE division and square root), as in PyTorch's CPU ops; row means use
// PyTorch's CPU summation order, so encoding is bit-identical to the CPU
// definitions for the same fp32 input.
// One workgroup per (request, head, tile of up to 128 value columns); lane
// (rg, cg) owns rows rg + 8r and columns 4cg .. 4cg+3 of the tile.
// =====================================================================
enum { FMT_ENCODE = 0, FMT_DECODE = 1, FMT_STEP = 2 };
constexpr int FMT_TV = 128, FMT_RPT = 16, FMT_SMALL_LDS = (3 * 128 + 16 + 128) * 4;

struct FmtDev {
  uint8_t *data;
  int64_t page_bytes, num_slots;
  const int32_t *offsets, *rows, *columns;
  int H, K, V, kind, bits, kda;
  int stage;        // bytes of LDS staging for the head's code rows (0: rows read from the page)
  const float *in;  // FMT_ENCODE: dense [B, H, K, V]
  float *dense;     // FMT_DECODE: dense [B, H, K, V]
  const void *slots;
  int slots_dtype;
};

// the 4 codes of columns j0..j0+3 (j0 % 4 == 0) of a row: W/2 bytes
__device__ __forceinline__ uint32_t fmt_read_codes(const uint8_t *row, int j0, int W) {
  const uint8_t *p = row + (j0 * W) / 8;
  uint32_t w = 0;
  for (int t = 0; t < W / 2; t++) w |= (uint32_t)p[t] << (8 * t);
  return w;
}

__device__ __forceinline__ void fmt_write_codes(uint8_t *row, int j0, int W, uint32_t w) {
  uint8_t *p = row + (j0 * W) / 8;
  for (int t = 0; t < W / 2; t++) p[t] = (uint8_t)(w >> (8 * t));
}

// div_half with its range condition: `ok` is cleared when x or the
// quotient leaves the range where div_half equals the IEEE quotient.
__device__ __forceinline__ float div_fp16_divisor(float x, float d, float inv, bool &ok) {
  ok = ok && fabsf(x) >= 0x1p-100f && fabsf(x * inv) <= 0x1p+126f;
  return div_half(x, d, inv);
}


template <int MODE, int KIND>  // KIND: the format (F.kind), fixed per instantiation
__global__ __launch_bounds__(256) void format_kernel(FmtDev F, StepDev S) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) uint8_t smem[];
  const int H = F.H, K = F.K, V = F.V;
  const int TV = V < FMT_TV ? V : FMT_TV;
  const int b = blockIdx.x / H, h = blockIdx.x % H, tile = blockIdx.y;
  const int tid = threadIdx.x, rg = tid & 7, cg = tid >> 3;
  const bool act = 4 * cg < TV;
  const int j0 = tile * TV + (act ? 4 * cg : 0);
  const int64_t bh = (int64_t)b * H + h;
  const int64_t slot = load_slot(F.slots, F.slots_dtype, b);
  if (slot <= 0 || slot >= F.num_slots) {  // masked: zero readout / zero state, no page access
    if (MODE == FMT_STEP)
      for (int j = tid; j < TV; j += 256) store_val(S.out, S.out_dtype, bh * V + tile * TV + j, 0.0f);
    if (MODE == FMT_DECODE)
      for (int e = tid; e < K * TV; e += 256) F.dense[(bh * K + e / TV) * V + tile * TV + e % TV] = 0.0f;
    return;
  }
  uint8_t *page = F.data + slot * F.page_bytes;
  const int W = F.bits;
  const int L = (1 << ((W < 8 ? W : 8) - 1)) - 1;
  // LDS: staged code rows | q, k, retention per row | misc | per-row scale | reduction space
  uint8_t *stg = smem;
  float *qs = (float *)(smem + F.stage);
  float *ks = qs + 128;
  float *ds = ks + 128;
  float *misc = ds + 128;
  float *rowv = misc + 16;
  float *big = rowv + 128;

  // Code rows of the head are one contiguous region (every row has the same
  // width): staged through LDS with 16-byte loads and stores instead of
  // per-lane byte accesses.
  const bool staged = F.stage > 0;
  const int64_t code_start = staged ? F.offsets[(int64_t)h * K] : 0;
  const int64_t code_bytes = (int64_t)K * V * W / 8;
  int shift = staged ? (int)((uintptr_t)(page + code_start) & 15) : 0;
  if (staged && MODE != FMT_ENCODE) shift = stage_in(page + code_start, code_bytes, stg, tid, 256);
  if (staged) __syncthreads();

  float beta = 0.0f;
  if (MODE == FMT_STEP) {
    // input preparation as kernels/formats.py:120-146
    const int hk = h / (H / S.HK);
    const int64_t qb = (int64_t)b * S.q_stride + (int64_t)hk * K;
    const int64_t kb = (int64_t)b * S.k_stride + (int64_t)hk * K;
    if (tid < 64) {
      float sq = 0.0f, sk = 0.0f;
      for (int i = tid; i < K; i += 64) {
        const float a = load_val(S.q, S.qkv_dtype, qb + i), c = load_val(S.k, S.qkv_dtype, kb + i);
        sq += a * a;
        sk += c * c;
      }
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) {
        sq += __shfl_xor(sq, m);
        sk += __shfl_xor(sk, m);
      }
      if (tid == 0) {
        misc[0] = S.normalize ? 1.0f / __builtin_sqrtf(sq + 1e-6f) : 1.0f;
        misc[1] = S.normalize ? 1.0f / __builtin_sqrtf(sk + 1e-6f) : 1.0f;
        float bt = load_val(S.beta, S.gate_dtype, bh);
        if (S.a_log) bt = 1.0f / (1.0f + __expf(-bt));
        misc[2] = bt;
      }
    }
    __syncthreads();
    const float nq = misc[0], nk = misc[1];
    beta = misc[2];
    const float alog = S.a_log ? __expf(load_val(S.a_log, S.gate_dtype, h)) : 0.0f;
    for (int i = tid; i < K; i += 256) {
      qs[i] = (load_val(S.q, S.qkv_dtype, qb + i) * nq) * S.scale;
      ks[i] = load_val(S.k, S.qkv_dtype, kb + i) * nk;
      const int64_t gi = F.kda ? bh * K + i : bh;
      float gv = load_val(S.g, S.gate_dtype, gi);
      if (S.a_log) {
        const float u = gv + load_val(S.dt_bias, S.gate_dtype, F.kda ? (int64_t)h * K + i : (int64_t)h);
        const float sp = u > 20.0f ? u : __logf(1.0f + __expf(u < 20.0f ? u : 20.0f));
        gv = -alog * sp;
      }
      ds[i] = __expf(gv);
    }
    __syncthreads();
  }

  // ---- this lane's values
  float x[FMT_RPT][4];
  if (MODE == FMT_ENCODE) {
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
#pragma unroll
      for (int c = 0; c < 4; c++) x[r][c] = (act && i < K) ? F.in[(bh * K + i) * V + j0 + c] : 0.0f;
    }
  } else {
    float cj[4] = {0.f, 0.f, 0.f, 0.f};
    if (KIND == SQ_FMT_DSQ && act) {
#pragma unroll
      for (int c = 0; c < 4; c++) cj[c] = h2f(page_half(page, F.columns[h] + 4 * (j0 + c)));
    }
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
#pragma unroll
      for (int c = 0; c < 4; c++) x[r][c] = 0.0f;
      if (!act || i >= K) continue;
      const uint8_t *row = page + F.offsets[(int64_t)h * K + i];
      if (KIND == SQ_FMT_FP32) {
        const float *fr = (const float *)row + j0;
#pragma unroll
        for (int c = 0; c < 4; c++) x[r][c] = fr[c];
        continue;
      }
      const uint32_t word = staged ? lds_word(stg, shift + (int)(((int64_t)i * V + j0) * W / 8))
                                   : fmt_read_codes(row, j0, W);
      const int64_t ro = F.rows[(int64_t)h * K + i];
      if (KIND == SQ_FMT_SYMMETRIC) {
        const int64_t meta = ro + 4 * (j0 / FMT_TV);
        const float s = h2f(page_half(page, meta)), z = h2f(page_half(page, meta + 2));
#pragma unroll
        for (int c = 0; c < 4; c++) x[r][c] = ((float)((word >> (c * W)) & ((1u << W) - 1u)) - z) * s;
      } else {
        const float rr = h2f(page_half(page, ro));
#pragma unroll
        for (int c = 0; c < 4; c++)
          x[r][c] = (rr * cj[c]) * (float)((int)((word >> (c * W)) & ((1u << W) - 1u)) - L);
      }
    }
  }
  if (MODE == FMT_DECODE) {
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (act && i < K)
#pragma unroll
        for (int c = 0; c < 4; c++) F.dense[(bh * K + i) * V + j0 + c] = x[r][c];
    }
    return;
  }

  if (MODE == FMT_STEP) {
    // retained = S e^g; residual = v - k^T retained; x = retained + k (beta residual); o = q^T x
    float kr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (i >= K) continue;
      const float d = ds[i], k = ks[i];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        x[r][c] = x[r][c] * d;
        kr[c] += k * x[r][c];
      }
    }
    float vv[4] = {0.f, 0.f, 0.f, 0.f}, o[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) load4(S.v, S.qkv_dtype, (int64_t)b * S.v_stride + (int64_t)h * V + j0, vv);
    float br[4];
#pragma unroll
    for (int c = 0; c < 4; c++) br[c] = beta * (vv[c] - fast::rg8_sum(kr[c]));
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (i >= K) continue;
      const float k = ks[i], q = qs[i];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        x[r][c] = x[r][c] + k * br[c];
        o[c] += q * x[r][c];
      }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = fast::rg8_sum(o[c]);
    if (act && rg == 0) store4(S.out, S.out_dtype, bh * V + j0, o);
  }

  // ---- encode x into the page
  if (KIND == SQ_FMT_FP32) {
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (!act || i >= K) continue;
      float *fr = (float *)(page + F.offsets[(int64_t)h * K + i]) + j0;
#pragma unroll
      for (int c = 0; c < 4; c++) fr[c] = x[r][c];
    }
    return;
  }
  const float Lf = (float)L;
  float div[4];  // per column (DSQ) divisor; SYMMETRIC uses the per-row s
  if (KIND == SQ_FMT_SYMMETRIC) {
    // s_i = fp16(max_j |x_ij| / L) over the tile's 128 columns (one group)
    float *red = big;  // [TV/4][K]
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (!act || i >= K) continue;
      red[cg * K + i] = fmaxf(fmaxf(fabsf(x[r][0]), fabsf(x[r][1])), fmaxf(fabsf(x[r][2]), fabsf(x[r][3])));
    }
    __syncthreads();
    for (int i = tid; i < K; i += 256) {
      float m = 0.0f;
      for (int t = 0; t < TV / 4; t++) m = fmaxf(m, red[t * K + i]);
      uint32_t hb;
      rowv[i] = fp16_scale(m / Lf, &hb);
      const int64_t meta = F.rows[(int64_t)h * K + i] + 4 * (tile * TV / FMT_TV);
      put_page_half(page, meta, hb);
      put_page_half(page, meta + 2, f2h(Lf));
    }
    __syncthreads();
  } else {
    // r_i = fp16(sqrt(max(mean_j |x_ij|, 1e-20))), mean in PyTorch's order
    const int XS = TV + 1;  // row pitch of the staged |x| (odd: no bank conflicts)
    float *xs = big;
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (!act || i >= K) continue;
#pragma unroll
      for (int c = 0; c < 4; c++) xs[i * XS + 4 * cg + c] = fabsf(x[r][c]);
    }
    __syncthreads();
    auto put_r = [&](int i, float s) {
      float m = s / (float)V;
      m = m < 1e-20f ? 1e-20f : m;
      uint32_t hb;
      rowv[i] = fp16_scale(__builtin_sqrtf(m), &hb);
      put_page_half(page, F.rows[(int64_t)h * K + i], hb);
    };
    if (V == 128) {
      // 32 lanes per row: lane (l, k) = (lane / 4, lane % 4) adds columns
      // 8(4ii + k) + l for ii ascending (PyTorch's 8 vector lanes with 4
      // accumulators each), then the partial sums combine in PyTorch's order
      const int lane = tid & 31, l = lane >> 2, kq = lane & 3;
      for (int i = tid >> 5; i < K; i += 8) {
        const float *row = xs + i * XS;
        float acc = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 4; ii++) acc += row[8 * (4 * ii + kq) + l];
        float sl = acc;
        sl += row_shl<1>(acc);
        sl += row_shl<2>(acc);
        sl += row_shl<3>(acc);
        const float up = __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(sl), __float_as_uint(sl),
                                                                          false, false)[1]);  // lane + 16
        float total = 0.0f;
        total += sl;
        total += row_shl<4>(sl);
        total += row_shl<8>(sl);
        total += row_shl<12>(sl);
        total += up;
        total += row_shl<4>(up);
        total += row_shl<8>(up);
        total += row_shl<12>(up);
        if (lane == 0) put_r(i, total);
      }
    } else {
      for (int i = tid; i < K; i += 256) put_r(i, inner_sum_lanewise(xs + i * XS, V));
    }
    __syncthreads();
    // y = x / r; c_j = fp16(max_i |y_ij| / L).  The quotients by the fp16
    // scales come from their reciprocals with one correction where that is
    // exact for every value of the thread, else from IEEE division.
    float mx[4] = {0.f, 0.f, 0.f, 0.f};
    float rinv[FMT_RPT];
    bool fast = true;
    {
      float amin = INFINITY, amax = 0.0f, imax = 0.0f;
#pragma unroll
      for (int r = 0; r < FMT_RPT; r++) {
        const int i = rg + 8 * r;
        if (i >= K) continue;
        rinv[r] = 1.0f / rowv[i];
        imax = fmaxf(imax, rinv[r]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          amin = fminf(amin, fabsf(x[r][c]));
          amax = fmaxf(amax, fabsf(x[r][c]));
        }
      }
      fast = amin >= 0x1p-100f && amax * imax <= 0x1p+125f;
    }
    auto scale_rows = [&](auto ieee) {
#pragma unroll
      for (int r = 0; r < FMT_RPT; r++) {
        const int i = rg + 8 * r;
        if (i >= K) continue;
        const float rr = rowv[i];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          bool ok = true;
          x[r][c] = decltype(ieee)::value ? x[r][c] / rr : div_fp16_divisor(x[r][c], rr, rinv[r], ok);
          mx[c] = fmaxf(mx[c], fabsf(x[r][c]));
        }
      }
    };
    if (fast) scale_rows(BoolTag<false>());
    else scale_rows(BoolTag<true>());
#pragma unroll
    for (int c = 0; c < 4; c++) {
      uint32_t hb;
      div[c] = fp16_scale(fast::rg8_max_nonneg(mx[c]) / Lf, &hb);
      if (act && rg == 0) {
        put_page_half(page, F.columns[h] + 4 * (int64_t)(j0 + c), hb);
        put_page_half(page, F.columns[h] + 4 * (int64_t)(j0 + c) + 2, 0u);
      }
    }
  }
  // codes: the quotients as above (reciprocal where exact for the thread)
  float rinvq[FMT_RPT], cinvq[4];  // 1 / divisor: per row (SYMMETRIC) or per column (DSQ)
  bool fastq;
  {
    float amin = INFINITY, amax = 0.0f, imax = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      cinvq[c] = KIND == SQ_FMT_SYMMETRIC ? 0.0f : 1.0f / div[c];
      imax = fmaxf(imax, cinvq[c]);
    }
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      rinvq[r] = 0.0f;
      if (!act || i >= K) continue;
      if (KIND == SQ_FMT_SYMMETRIC) {
        rinvq[r] = 1.0f / rowv[i];
        imax = fmaxf(imax, rinvq[r]);
      }
#pragma unroll
      for (int c = 0; c < 4; c++) {
        amin = fminf(amin, fabsf(x[r][c]));
        amax = fmaxf(amax, fabsf(x[r][c]));
      }
    }
    fastq = amin >= 0x1p-100f && amax * imax <= 0x1p+125f;
  }
  auto codes = [&](auto ieee) {
#pragma unroll
    for (int r = 0; r < FMT_RPT; r++) {
      const int i = rg + 8 * r;
      if (!act || i >= K) continue;
      uint32_t word = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float d = KIND == SQ_FMT_SYMMETRIC ? rowv[i] : div[c];
        const float dinv = KIND == SQ_FMT_SYMMETRIC ? rinvq[r] : cinvq[c];
        bool ok = true;
        float q = __builtin_rintf(decltype(ieee)::value ? x[r][c] / d : div_fp16_divisor(x[r][c], d, dinv, ok));
        q = q > -Lf ? q : -Lf;
        q = q < Lf ? q : Lf;
        word |= (uint32_t)(int)(q + Lf) << (c * W);
      }
      if (staged) lds_put_bytes(stg, shift + (int)(((int64_t)i * V + j0) * W / 8), word, W / 2);
      else fmt_write_codes(page + F.offsets[(int64_t)h * K + i], j0, W, word);
    }
  };
  if (fastq) codes(BoolTag<false>());
  else codes(BoolTag<true>());
  if (staged) {
    __syncthreads();
    stage_out(page + code_start, code_bytes, stg, tid, 256);
  }
}

// ------------------------------------------------------------ host side

thread_local char g_err[512] = "";

int fail(int code, const char *msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

int validate_pool(const sq_pool *p) {
  if (!p || !p->data || !p->bits || !p->offsets || !p->rows || !p->columns || !p->impact || !p->head_meta)
    return fail(SQ_EINVAL, "pool: null pointer");
  if (p->heads < 1 || p->page_bytes <= 0 || p->num_slots < 1) return fail(SQ_EINVAL, "pool: bad sizes");
  if (!pow2(p->keys) || !pow2(p->values) || p->values < 4 || p->keys < 4)
    return fail(SQ_ESHAPE, "pool: K and V must be powers of two >= 4");
  if ((int64_t)p->keys * p->values > 16384 || p->keys > 256 || p->values > 256)
    return fail(SQ_ESHAPE, "pool: K*V above 16384 (K, V <= 256) is not supported");
  if (!p->kda && (p->group < 4 || p->values % p->group))
    return fail(SQ_ESHAPE, "pool: GDN value_group_size must divide V and be >= 4");
  if (p->storage != 0 && p->storage != 1) return fail(SQ_ESTORAGE, "pool: storage must be packed (0) or byte (1)");
  return 0;
}

PoolDev to_dev(const sq_pool *p) {
  PoolDev d;
  d.data = p->data;
  d.page_bytes = p->page_bytes;
  d.num_slots = p->num_slots;
  d.bits = p->bits;
  d.offsets = p->offsets;
  d.rows = p->rows;
  d.columns = p->columns;
  d.head_meta = p->head_meta;
  d.impact = p->impact;
  d.H = p->heads;
  d.K = p->keys;
  d.V = p->values;
  d.G = p->group > 0 ? p->group : p->values;
  d.ng = d.G >= 32 ? 128 / d.G : 1;
  d.ngsh = 31 - __builtin_clz((unsigned)d.ng);
  d.kda = p->kda;
  d.stage = (p->max_code_bytes + 47) & ~15;
  d.rstage = (p->max_row_bytes + 15) & ~15;
  d.fast = p->flags & (SQ_POOL_FAST_GDN128 | SQ_POOL_FAST_KDA128);
  d.storage = p->storage;
  d.hrot = (p->heads & (p->heads - 1)) == 0 ? p->heads - 1 : 0;
  return d;
}

int stage_bytes(const sq_pool *p) { return (p->max_code_bytes + 47) & ~15; }

template <int MODE>
int launch_step_mode(const sq_pool *pool, StepDev sd, int64_t batch, hipStream_t st) {
  PoolDev pd = to_dev(pool);
  // The K=V=128 kernels take a (heads, requests) grid and the key head of value
  // head h as (h * hk_mul) >> 20 (exact for h * (H / HK) < 2^20): larger shapes
  // run on the general kernels below.
  if (pool->heads > 1024 || batch > 65535) pd.fast = 0;
  if (pd.fast & (SQ_POOL_FAST_GDN128 | SQ_POOL_FAST_KDA128)) {
    const int ratio = sd.HK > 0 ? pool->heads / sd.HK : 1;
    sd.hk_mul = ((1 << 20) + ratio - 1) / ratio;
  }
  if (MODE == MODE_DECODE && (pd.fast & SQ_POOL_FAST_GDN128)) {
    size_t lds = (size_t)pd.stage + pd.rstage + 2 * 128;  // staging | rows | columns
    hipLaunchKernelGGL((gdn128_kernel<MODE_DECODE, true>), dim3((unsigned)pool->heads, (unsigned)batch), dim3(256),
                       lds, st, pd, sd);
    return check_launch("gdn128_kernel (decode)");
  }
  if (MODE == MODE_DECODE && (pd.fast & SQ_POOL_FAST_KDA128)) {
    // row-scale regions may start at any even byte: room for the alignment shift
    pd.rstage = (pool->max_row_bytes + 47) & ~15;
    // code blocks in padded windows (the largest head's stride)
    pd.stage = 32 * kfast::block_pitch(pool->max_code_bytes / 32);
    // the step's layout (staging | rows | columns | ... | rc, rl, rm, rk | pivot mask)
    size_t lds = (size_t)pd.stage + pd.rstage + fast::KDA_COL_STAGE + 4 * 128 * 4 + fast::MISC_FLOATS * 4 +
                 4 * 128 * 4 + 2 * 128 * 4 + 4 * 128 * 16 + 16;
    hipLaunchKernelGGL((kda128_kernel<MODE_DECODE, true>), dim3((unsigned)pool->heads, (unsigned)batch), dim3(256),
                       lds, st, pd, sd);
    return check_launch("kda128_kernel (decode)");
  }
  if constexpr (MODE != MODE_DECODE) {
    if (pd.fast & SQ_POOL_FAST_GDN128) {
      const int ng_max = pool->group >= 32 ? 128 / pool->group : 1;
      // staging | rows | columns | q,k raw + w | misc | red | ks, qs | rc (float4), iu (float2) per (row, group)
      size_t lds = (size_t)pd.stage + pd.rstage + 2 * 128 + 3 * 128 * 4 + 48 * 4 + 4 * 128 * 4 + 2 * 128 * 4 +
                   (size_t)6 * 128 * ng_max * 4;
      // q, k, v element width as a compile-time choice (the writer reads fp32 only)
      if (MODE == MODE_WRITE || sd.qkv_dtype == SQ_F32)
        hipLaunchKernelGGL((gdn128_kernel<MODE, true>), dim3((unsigned)pool->heads, (unsigned)batch), dim3(256), lds, st, pd,
                           sd);
      else
        hipLaunchKernelGGL((gdn128_kernel<MODE, MODE == MODE_WRITE>), dim3((unsigned)pool->heads, (unsigned)batch), dim3(256),
                           lds, st, pd, sd);
      return check_launch("gdn128_kernel");
    }
    if (pd.fast & SQ_POOL_FAST_KDA128) {
      // row-scale regions may start at any even byte: room for the alignment shift
      pd.rstage = (pool->max_row_bytes + 47) & ~15;
      // code blocks in padded windows (the largest head's stride)
      pd.stage = 32 * kfast::block_pitch(pool->max_code_bytes / 32);
      // staging | rows | columns | q,k raw, w, retention | misc | red | ks, qs | rc, rl, rm, rk | pivot mask
      size_t lds = (size_t)pd.stage + pd.rstage + fast::KDA_COL_STAGE + 4 * 128 * 4 + fast::MISC_FLOATS * 4 +
                   4 * 128 * 4 + 2 * 128 * 4 + 4 * 128 * 16 + 16;
      if (MODE == MODE_WRITE || sd.qkv_dtype == SQ_F32)
        hipLaunchKernelGGL((kda128_kernel<MODE, true>), dim3((unsigned)pool->heads, (unsigned)batch), dim3(256), lds, st, pd,
                           sd);
      else
        hipLaunchKernelGGL((kda128_kernel<MODE, MODE == MODE_WRITE>), dim3((unsigned)pool->heads, (unsigned)batch), dim3(256),
                           lds, st, pd, sd);
      return check_launch("kda128_kernel");
    }
  }
  const int K = pool->keys, V = pool->values;
  const int RG = K >= 8 ? 8 : 4;
  const int RPT = K / RG;
  int NT = RG * (V / 4);
  NT = (NT + 63) / 64 * 64;
  size_t lds = (size_t)stage_bytes(pool);
  if (MODE == MODE_FUSED || MODE == MODE_WRITE) lds += (size_t)(V / 4) * K * 4;
  lds += (size_t)3 * K * 4 + 64;
  dim3 grid((unsigned)(batch * pool->heads));
#define SQ_LAUNCH(R, G_)                                                                    \
  hipLaunchKernelGGL((step_kernel<R, G_, MODE>), grid, dim3(NT), lds, st, pd, sd);         \
  break;
  switch (RG * 1000 + RPT) {
    case 4001: SQ_LAUNCH(1, 4)
    case 8001: SQ_LAUNCH(1, 8)
    case 8002: SQ_LAUNCH(2, 8)
    case 8004: SQ_LAUNCH(4, 8)
    case 8008: SQ_LAUNCH(8, 8)
    case 8016: SQ_LAUNCH(16, 8)
    case 8032: SQ_LAUNCH(32, 8)
    default: return fail(SQ_ESHAPE, "unsupported key dimension");
  }
#undef SQ_LAUNCH
  return check_launch("step_kernel");
}

int fill_step(int heads, const sq_step_args *a, StepDev &sd) {
  if (!a || !a->q || !a->k || !a->v || !a->g || !a->beta || !a->out || !a->slots)
    return fail(SQ_EINVAL, "step: null input pointer");
  if (a->batch < 0) return fail(SQ_EINVAL, "step: negative batch");
  if (a->q_stride < 0 || a->k_stride < 0 || a->v_stride < 0)
    return fail(SQ_EINVAL, "step: negative q/k/v row stride");
  if (a->key_heads < 1 || heads % a->key_heads) return fail(SQ_EINVAL, "step: heads not divisible by key heads");
  if ((a->a_log == nullptr) != (a->dt_bias == nullptr)) return fail(SQ_EINVAL, "step: a_log and dt_bias go together");
  if (a->qkv_dtype < 0 || a->qkv_dtype > 2 || a->gate_dtype < 0 || a->gate_dtype > 2 || a->out_dtype < 0 ||
      a->out_dtype > 2 || (a->slots_dtype != SQ_I32 && a->slots_dtype != SQ_I64))
    return fail(SQ_EINVAL, "step: bad dtype code");
  memset(&sd, 0, sizeof(sd));
  sd.q = a->q;
  sd.k = a->k;
  sd.v = a->v;
  sd.g = a->g;
  sd.beta = a->beta;
  sd.a_log = a->a_log;
  sd.dt_bias = a->dt_bias;
  sd.out = a->out;
  sd.slots = a->slots;
  sd.q_stride = a->q_stride;
  sd.k_stride = a->k_stride;
  sd.v_stride = a->v_stride;
  sd.HK = a->key_heads;
  sd.qkv_dtype = a->qkv_dtype;
  sd.gate_dtype = a->gate_dtype;
  sd.out_dtype = a->out_dtype;
  sd.slots_dtype = a->slots_dtype;
  sd.normalize = a->normalize;
  sd.scale = a->scale;
  return 0;
}

int validate_format(const sq_format_pool *f) {
  if (!f || !f->data || !f->offsets || !f->rows || !f->columns) return fail(SQ_EINVAL, "format pool: null pointer");
  if (f->heads < 1 || f->page_bytes <= 0 || f->num_slots < 1) return fail(SQ_EINVAL, "format pool: bad sizes");
  if (!pow2(f->keys) || f->keys > 128 || !pow2(f->values) || f->values < 4)
    return fail(SQ_ESHAPE, "format pool: K must be a power of two <= 128, V a power of two >= 4");
  if (f->page_bytes % 4) return fail(SQ_EINVAL, "format pool: page_bytes must be a multiple of 4");
  switch (f->kind) {
    case SQ_FMT_FP32:
      if (f->bits != 32) return fail(SQ_ESHAPE, "format pool: fp32 pages hold 32-bit values");
      break;
    case SQ_FMT_SYMMETRIC:
      if (f->bits != 4 && f->bits != 6 && f->bits != 8) return fail(SQ_ESHAPE, "format pool: code width 4, 6 or 8");
      if (f->group != 128 || f->values % 128) return fail(SQ_ESHAPE, "format pool: symmetric groups are 128 values");
      break;
    case SQ_FMT_DSQ:
      if (f->bits != 4 && f->bits != 6 && f->bits != 8) return fail(SQ_ESHAPE, "format pool: code width 4, 6 or 8");
      if (f->values > 128) return fail(SQ_ESHAPE, "format pool: dual-axis pages need V <= 128");
      break;
    default:
      return fail(SQ_EINVAL, "format pool: unknown kind");
  }
  return 0;
}

FmtDev to_fmt(const sq_format_pool *f) {
  FmtDev d;
  memset(&d, 0, sizeof(d));
  if ((f->flags & SQ_FMT_ROWS_CONTIGUOUS) && f->kind != SQ_FMT_FP32 && f->values <= 128)
    d.stage = (int)(((int64_t)f->keys * f->values * f->bits / 8 + 47) & ~15);
  d.data = f->data;
  d.page_bytes = f->page_bytes;
  d.num_slots = f->num_slots;
  d.offsets = f->offsets;
  d.rows = f->rows;
  d.columns = f->columns;
  d.H = f->heads;
  d.K = f->keys;
  d.V = f->values;
  d.kind = f->kind;
  d.bits = f->bits;
  d.kda = f->kda;
  return d;
}

template <int MODE>
int launch_format(const sq_format_pool *f, const FmtDev &fd, const StepDev &sd, int64_t batch, hipStream_t st) {
  if (batch == 0) return 0;
  if (batch * f->heads > 0x7fffffffLL) return fail(SQ_EINVAL, "format: batch * heads too large");
  const int TV = f->values < FMT_TV ? f->values : FMT_TV;
  size_t lds = FMT_SMALL_LDS + (size_t)fd.stage;
  if (MODE != FMT_DECODE) {
    if (f->kind == SQ_FMT_SYMMETRIC) lds += (size_t)(TV / 4) * f->keys * 4;
    if (f->kind == SQ_FMT_DSQ) lds += (size_t)f->keys * (TV + 1) * 4;
  }
  const dim3 grid((unsigned)(batch * f->heads), (unsigned)(f->values / TV));
  auto go = [&](auto kernel) {
    if (lds > 65536) {
      hipError_t e = hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return fail((int)e, "format: LDS attribute");
    }
    hipLaunchKernelGGL(kernel, grid, dim3(256), lds, st, fd, sd);
    return check_launch("format_kernel");
  };
  if (f->kind == SQ_FMT_FP32) return go(format_kernel<MODE, SQ_FMT_FP32>);
  if (f->kind == SQ_FMT_SYMMETRIC) return go(format_kernel<MODE, SQ_FMT_SYMMETRIC>);
  return go(format_kernel<MODE, SQ_FMT_DSQ>);
}

// Staging of sq_copy_slots_static: a file-scope device array.  Every GPU the
// library runs on holds its own copy at its own address until the process
// ends.  In host code the name is only a stand-in: kernels receive the
// device address that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[SQ_COPY_STATIC_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per
// device (on the first call made with that device current).
int static_scratch(uint8_t **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "copy_static: hipGetDevice: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(SQ_EINVAL, "copy_static: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      snprintf(g_err, sizeof(g_err), "copy_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return e != hipSuccess ? (int)e : SQ_EINVAL;
    }
    g_scratch_ptr[dev] = (uint8_t *)ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int launch_copy(const sq_pool *pool, const void *src, const void *dst, int32_t slots_dtype, int64_t n,
                uint8_t *temp, hipStream_t stream) {
  unsigned gx = (unsigned)((pool->page_bytes + 255) / 256);
  if (gx > 1024) gx = 1024;
  hipLaunchKernelGGL(gather_kernel, dim3(gx, (unsigned)n), dim3(256), 0, stream, pool->data,
                     pool->page_bytes, pool->num_slots, src, dst, slots_dtype, temp, 0);
  int rc = check_launch("gather_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(gather_kernel, dim3(gx, (unsigned)n), dim3(256), 0, stream, pool->data,
                     pool->page_bytes, pool->num_slots, src, dst, slots_dtype, temp, 1);
  return check_launch("scatter_kernel");
}

}  // namespace

extern "C" {

int sq_abi_version(void) { return SQ_ABI_VERSION; }

const char *sq_last_error(void) { return g_err; }

int sq_encode(const sq_pool *pool, const float *state, const void *slots, int32_t slots_dtype, int64_t batch,
              void *stream) {
  int rc = validate_pool(pool);
  if (rc) return rc;
  if (batch == 0) return 0;
  if (!state || !slots || batch < 0) return fail(SQ_EINVAL, "encode: null pointer or negative batch");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "encode: slots dtype");
  PoolDev pd = to_dev(pool);
  const int NG = (!pool->kda) ? pool->values / pd.G : 1;
  const int K = pool->keys, V = pool->values;
  // rows of a column split over up to 4 threads (whole 16-row blocks each)
  int split = V >= 32 ? 512 / V : 1;
  split = split > 4 ? 4 : split;
  while (split > 1 && K % (16 * split)) split >>= 1;
  const int NT = split > 1 ? split * V : (V < 64 ? 64 : V);  // lanes per value column
  size_t lds = (size_t)stage_bytes(pool) + (size_t)((K * NG + 3) & ~3) * 4 + 16;
  if (split > 1) lds += (size_t)split * 4 * V * 4 + (size_t)(K / 16) * 2 * V * 4;
  if (pool->kda && pool->storage == 0 && K == 128 && V == 128) {
    // rows, 1 / rows, w, widths, row offsets [K] | column maxima [4][4][V] | block sums [K/16][2][V] |
    // per-row factors [K] float4 + int4
    const size_t fl = (size_t)stage_bytes(pool) + (size_t)(5 * K + 16 * V + (K / 16) * 2 * V + 8 * K) * 4;
    hipLaunchKernelGGL(encode_kda128_kernel, dim3((unsigned)(batch * pool->heads)), dim3(512), fl,
                       (hipStream_t)stream, pd, state, slots, slots_dtype);
    return check_launch("encode_kda128_kernel");
  }
  if (!pool->kda && pool->storage == 0 && K == 128 && V == 128 && pd.G == 32) {
    // rows [K][4] | w [K] | row offsets [K] | column maxima [NT/V][V] | block sums [K/16][2][V] | 1/rows [K][4]
    const size_t fl =
        (size_t)stage_bytes(pool) + (size_t)(K * 4 + 2 * K + (ENC128_NT / V) * V + (K / 16) * 2 * V + K * 4) * 4;
    hipLaunchKernelGGL(encode128_kernel, dim3((unsigned)(batch * pool->heads)), dim3(ENC128_NT), fl,
                       (hipStream_t)stream, pd, state, slots, slots_dtype);
    return check_launch("encode128_kernel");
  }
  hipLaunchKernelGGL(encode_kernel, dim3((unsigned)(batch * pool->heads)), dim3(NT), lds, (hipStream_t)stream, pd,
                     state, slots, slots_dtype, split);
  return check_launch("encode_kernel");
}

int sq_decode_dense(const sq_pool *pool, const void *slots, int32_t slots_dtype, int64_t batch, float *state,
                    void *stream) {
  int rc = validate_pool(pool);
  if (rc) return rc;
  if (batch == 0) return 0;
  if (!state || !slots || batch < 0) return fail(SQ_EINVAL, "decode: null pointer or negative batch");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "decode: slots dtype");
  StepDev sd;
  memset(&sd, 0, sizeof(sd));
  sd.slots = slots;
  sd.slots_dtype = slots_dtype;
  sd.dense = state;
  return launch_step_mode<MODE_DECODE>(pool, sd, batch, (hipStream_t)stream);
}

int sq_decode_step(const sq_pool *pool, const sq_step_args *args, void *stream) {
  int rc = validate_pool(pool);
  if (rc) return rc;
  StepDev sd;
  rc = fill_step(pool->heads, args, sd);
  if (rc) return rc;
  if (args->batch == 0) return 0;
  return launch_step_mode<MODE_FUSED>(pool, sd, args->batch, (hipStream_t)stream);
}

int sq_decode_readout(const sq_pool *pool, const sq_step_args *args, const sq_writeback_scratch *scratch,
                      void *stream) {
  int rc = validate_pool(pool);
  if (rc) return rc;
  StepDev sd;
  rc = fill_step(pool->heads, args, sd);
  if (rc) return rc;
  if (!scratch || !scratch->key || !scratch->decay || !scratch->delta || !scratch->stable_slots)
    return fail(SQ_EINVAL, "readout: null scratch");
  if (args->batch > scratch->capacity) return fail(SQ_EINVAL, "readout: batch exceeds scratch capacity");
  if (args->batch == 0) return 0;
  sd.s_key = scratch->key;
  sd.s_decay = scratch->decay;
  sd.s_delta = scratch->delta;
  sd.s_slots = scratch->stable_slots;
  return launch_step_mode<MODE_READ>(pool, sd, args->batch, (hipStream_t)stream);
}

int sq_writeback(const sq_pool *pool, const sq_writeback_scratch *scratch, int64_t batch, void *stream) {
  int rc = validate_pool(pool);
  if (rc) return rc;
  if (!scratch || !scratch->key || !scratch->decay || !scratch->delta || !scratch->stable_slots)
    return fail(SQ_EINVAL, "writeback: null scratch");
  if (batch < 0 || batch > scratch->capacity) return fail(SQ_EINVAL, "writeback: bad batch");
  if (batch == 0) return 0;
  StepDev sd;
  memset(&sd, 0, sizeof(sd));
  sd.s_key = scratch->key;
  sd.s_decay = scratch->decay;
  sd.s_delta = scratch->delta;
  sd.s_slots = scratch->stable_slots;
  return launch_step_mode<MODE_WRITE>(pool, sd, batch, (hipStream_t)stream);
}

int sq_pool_flags(const int32_t *bits, const int32_t *head_meta, const int32_t *columns, int32_t heads,
                  int32_t keys, int32_t values, int32_t group, int32_t kda, int32_t storage, int64_t page_bytes) {
  if (!bits || !head_meta || !columns || heads < 1) return fail(SQ_EINVAL, "pool flags: bad arguments");
  int flags = 0;
  bool fast = !kda && keys == 128 && values == 128 && storage == 0 && page_bytes % 16 == 0;
  for (int h = 0; fast && h < heads; h++) {
    const int w = bits[(int64_t)h * keys];
    for (int i = 1; i < keys; i++) fast = fast && bits[(int64_t)h * keys + i] == w;
    fast = fast && head_meta[4 * h] % 16 == 0 && head_meta[4 * h + 1] % 16 == 0;
    if (w != 16) fast = fast && head_meta[4 * h + 2] % 16 == 0 && head_meta[4 * h + 3] % 16 == 0 &&
                        columns[h] >= 0 && columns[h] % 16 == 0;
    if (w == 2) fast = fast && (group == 32 || group == 64 || group == 128);
  }
  if (fast) flags |= SQ_POOL_FAST_GDN128;
  if (kda && keys == 128 && values == 128 && storage == 0) flags |= SQ_POOL_FAST_KDA128;
  return flags;
}

int sq_stream_capture_id(void *stream, int32_t *capturing, uint64_t *id) {
  if (!capturing || !id) return fail(SQ_EINVAL, "capture id: null output");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long ident = 0;
  hipError_t e = hipStreamGetCaptureInfo((hipStream_t)stream, &status, &ident);
  if (e != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "hipStreamGetCaptureInfo: %s", hipGetErrorString(e));
    return (int)e;
  }
  *capturing = status == hipStreamCaptureStatusActive ? 1 : (status == hipStreamCaptureStatusNone ? 0 : 2);
  *id = (uint64_t)ident;
  return 0;
}

int sq_event_create(void **event) {
  if (!event) return fail(SQ_EINVAL, "event: null output");
  hipEvent_t e = nullptr;
  hipError_t rc = hipEventCreateWithFlags(&e, hipEventDisableTiming);
  if (rc != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "hipEventCreateWithFlags: %s", hipGetErrorString(rc));
    return (int)rc;
  }
  *event = (void *)e;
  return 0;
}

int sq_event_destroy(void *event) {
  if (!event) return 0;
  hipError_t rc = hipEventDestroy((hipEvent_t)event);
  if (rc != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "hipEventDestroy: %s", hipGetErrorString(rc));
    return (int)rc;
  }
  return 0;
}

// Event record (wait == 0) or wait (wait == 1) on `stream`.  On a stream that
// is capturing, the operation becomes an event node of the capture's graph,
// placed after the stream's current capture dependencies and made the only
// one: a record node records the event on every replay of the graph, a wait
// node makes later captured work wait for the event's latest record.  A
// graph can therefore order itself against eager work and other graphs
// (hipEventRecordWithFlags with hipEventRecordExternal is refused under
// capture on this platform; explicit nodes are not).
static int event_op(void *event, void *stream, int wait) {
  if (!event) return fail(SQ_EINVAL, "event: null event");
  hipStream_t s = (hipStream_t)stream;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long ident = 0;
  hipGraph_t graph = nullptr;
  const hipGraphNode_t *deps = nullptr;
  size_t ndeps = 0;
  hipError_t rc = hipStreamGetCaptureInfo_v2(s, &status, &ident, &graph, &deps, &ndeps);
  if (rc != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "hipStreamGetCaptureInfo_v2: %s", hipGetErrorString(rc));
    return (int)rc;
  }
  if (status == hipStreamCaptureStatusInvalidated) return fail(SQ_EINVAL, "event: capture was invalidated");
  if (status == hipStreamCaptureStatusNone) {
    rc = wait ? hipStreamWaitEvent(s, (hipEvent_t)event, 0) : hipEventRecord((hipEvent_t)event, s);
    if (rc != hipSuccess) {
      snprintf(g_err, sizeof(g_err), "%s: %s", wait ? "hipStreamWaitEvent" : "hipEventRecord",
               hipGetErrorString(rc));
      return (int)rc;
    }
    return 0;
  }
  hipGraphNode_t node = nullptr;
  rc = wait ? hipGraphAddEventWaitNode(&node, graph, deps, ndeps, (hipEvent_t)event)
            : hipGraphAddEventRecordNode(&node, graph, deps, ndeps, (hipEvent_t)event);
  if (rc != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "%s: %s", wait ? "hipGraphAddEventWaitNode" : "hipGraphAddEventRecordNode",
             hipGetErrorString(rc));
    return (int)rc;
  }
  rc = hipStreamUpdateCaptureDependencies(s, &node, 1, hipStreamSetCaptureDependencies);
  if (rc != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "hipStreamUpdateCaptureDependencies: %s", hipGetErrorString(rc));
    return (int)rc;
  }
  return 0;
}

int sq_event_record(void *event, void *stream) { return event_op(event, stream, 0); }

int sq_event_wait(void *stream, void *event) { return event_op(event, stream, 1); }

int sq_event_query(void *event) {
  if (!event) return fail(SQ_EINVAL, "event: null event");
  hipError_t rc = hipEventQuery((hipEvent_t)event);
  if (rc == hipSuccess) return 0;
  if (rc == hipErrorNotReady) return 1;
  snprintf(g_err, sizeof(g_err), "hipEventQuery: %s", hipGetErrorString(rc));
  return (int)rc;
}

int sq_event_synchronize(void *event) {
  if (!event) return fail(SQ_EINVAL, "event: null event");
  hipError_t rc = hipEventSynchronize((hipEvent_t)event);
  if (rc != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "hipEventSynchronize: %s", hipGetErrorString(rc));
    return (int)rc;
  }
  return 0;
}

int sq_create_cu_stream(int32_t device, int32_t cus, void **stream, int32_t *actual, int32_t *total) {
  if (!stream || !actual || !total) return fail(SQ_EINVAL, "cu stream: null output");
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return fail((int)e, "cu stream: hipSetDevice failed");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail((int)e, "cu stream: hipGetDeviceProperties failed");
  const int n = prop.multiProcessorCount;
  *total = n;
  if (cus < 0 || cus > n) return fail(SQ_EINVAL, "cu stream: budget outside [0, CU count]");
  hipStream_t s = nullptr;
  if (cus == 0 || cus == n) {
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *actual = n;
  } else {
    // Mask bit i selects a CU of XCD i mod 8, so the first `cus` bits give
    // every XCD the same share of the budget (a mask that leaves an XCD
    // without CUs is rejected by the runtime).
    uint32_t mask[32] = {0};
    const int words = (n + 31) / 32;
    int chosen = 0;
    for (int c = 0; c < cus; c++) {
      mask[c / 32] |= 1u << (c % 32);
      chosen++;
    }
    e = hipExtStreamCreateWithCUMask(&s, (uint32_t)words, mask);
    *actual = chosen;
  }
  if (e != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "cu stream creation: %s", hipGetErrorString(e));
    return (int)e;
  }
  *stream = (void *)s;
  return 0;
}

int sq_prefill(const sq_pool *pool, const sq_prefill_args *a, void *stream) {
  int rc = validate_pool(pool);
  if (rc) return rc;
  if (!a) return fail(SQ_EINVAL, "prefill: null arguments");
  if (pool->keys != 128 || pool->values != 128)
    return fail(SQ_ESHAPE, "prefill: the prefill kernels handle pools with K = V = 128");
  if (a->batch < 0 || a->n_checkpoints < 0) return fail(SQ_EINVAL, "prefill: negative batch or checkpoint count");
  if (a->batch == 0) return 0;
  // packed pools that the K = V = 128 decode kernels take: the recurrence
  // kernel reads the initial pages itself (no dense initial state in between)
  const bool page_init = a->init_slots && pool->storage == 0 &&
                         (pool->flags & (pool->kda ? SQ_POOL_FAST_KDA128 : SQ_POOL_FAST_GDN128));
  if (!a->q || !a->k || !a->v || !a->g || !a->beta || !a->out || !a->cu_seqlens || (!a->init_state && !page_init))
    return fail(SQ_EINVAL, "prefill: null input, output, sequence offsets or initial-state workspace");
  if (a->n_checkpoints > 0 && (!a->checkpoints || !a->slots || !a->checkpoint_state))
    return fail(SQ_EINVAL, "prefill: checkpoints need positions, slots and a state workspace");
  if (a->n_checkpoints > pf::MAX_CK) return fail(SQ_EINVAL, "prefill: at most 64 checkpoints per sequence");
  if (a->qkv_dtype != SQ_BF16) return fail(SQ_EINVAL, "prefill: q, k, v must be bf16 (the MFMA operand type)");
  if (a->gate_dtype != SQ_F32 && a->gate_dtype != SQ_BF16 && a->gate_dtype != SQ_F16)
    return fail(SQ_EINVAL, "prefill: gate dtype");
  if (a->out_dtype != SQ_F32 && a->out_dtype != SQ_BF16 && a->out_dtype != SQ_F16)
    return fail(SQ_EINVAL, "prefill: output dtype");
  if (a->slots_dtype != SQ_I32 && a->slots_dtype != SQ_I64) return fail(SQ_EINVAL, "prefill: slots dtype");
  if (a->key_heads < 1 || pool->heads % a->key_heads) return fail(SQ_EINVAL, "prefill: key heads must divide heads");
  if ((a->a_log == nullptr) != (a->dt_bias == nullptr)) return fail(SQ_EINVAL, "prefill: a_log needs dt_bias");
  if (a->q_stride % 8 || a->k_stride % 8 || a->v_stride % 8 || ((uintptr_t)a->q & 15) || ((uintptr_t)a->k & 15) ||
      ((uintptr_t)a->v & 15))
    return fail(SQ_EINVAL, "prefill: q, k, v rows must start on 16-byte boundaries (strides multiple of 8)");
  if (a->q_stride < 0 || a->k_stride < 0 || a->v_stride < 0 || a->q_stride >= (1 << 23) || a->k_stride >= (1 << 23) ||
      a->v_stride >= (1 << 23))
    return fail(SQ_EINVAL, "prefill: q, k, v row strides must be below 2^23 elements");
  hipStream_t st = (hipStream_t)stream;
  const int H = pool->heads;
  const int64_t dense = a->batch * (int64_t)H * 128 * 128;
  if (page_init) {
    // decoded inside the recurrence kernel
  } else if (a->init_slots) {
    StepDev sd;
    memset(&sd, 0, sizeof(sd));
    sd.slots = a->init_slots;
    sd.slots_dtype = a->slots_dtype;
    sd.dense = a->init_state;
    rc = launch_step_mode<MODE_DECODE>(pool, sd, a->batch, st);
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(fill_zero_kernel, dim3(1024), dim3(256), 0, st, a->init_state, dense);
    rc = check_launch("fill_zero_kernel");
    if (rc) return rc;
  }
  pf::PrefillDev D;
  D.q = a->q;
  D.k = a->k;
  D.v = a->v;
  D.g = a->g;
  D.beta = a->beta;
  D.a_log = a->a_log;
  D.dt_bias = a->dt_bias;
  D.out = a->out;
  D.cu = a->cu_seqlens;
  D.ckpt = a->checkpoints;
  D.init = a->init_state;
  D.ck_state = a->checkpoint_state;
  D.q_stride = a->q_stride;
  D.k_stride = a->k_stride;
  D.v_stride = a->v_stride;
  D.H = H;
  D.HK = a->key_heads;
  D.NC = a->n_checkpoints;
  D.gate_dtype = a->gate_dtype;
  D.out_dtype = a->out_dtype;
  D.normalize = a->normalize;
  D.beta_logits = a->beta_logits != 0;
  D.scale = a->scale;
  D.page_init = page_init ? 1 : 0;
  D.pi.data = pool->data;
  D.pi.page_bytes = pool->page_bytes;
  D.pi.num_slots = pool->num_slots;
  D.pi.bits = pool->bits;
  D.pi.head_meta = pool->head_meta;
  D.pi.columns = pool->columns;
  D.pi.offsets = pool->offsets;
  D.pi.rows = pool->rows;
  D.pi.slots = a->init_slots;
  D.pi.slots_dtype = a->slots_dtype;
  D.pi.ng = pool->group >= 32 ? 128 / pool->group : 1;
  if (pool->kda) {
    hipError_t e = hipFuncSetAttribute((const void *)kc::kda_chunk_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kc::LDS_BYTES);
    if (e != hipSuccess) return fail((int)e, "prefill: cannot raise the KDA kernel's LDS limit");
    if (a->events && (e = hipEventRecord((hipEvent_t)a->events[0], st)) != hipSuccess)
      return fail((int)e, "prefill: hipEventRecord failed");
    hipLaunchKernelGGL(kc::kda_chunk_kernel, dim3((unsigned)(a->batch * H)), dim3(kc::NT), kc::LDS_BYTES, st, D);
    rc = check_launch("kda_chunk_kernel");
  } else {
    hipError_t e = hipFuncSetAttribute((const void *)pf::prefill_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       pf::LDS_BYTES);
    if (e != hipSuccess) return fail((int)e, "prefill: cannot raise the kernel's LDS limit");
    if (a->events && (e = hipEventRecord((hipEvent_t)a->events[0], st)) != hipSuccess)
      return fail((int)e, "prefill: hipEventRecord failed");
    hipLaunchKernelGGL(pf::prefill_kernel, dim3((unsigned)(a->batch * H)), dim3(pf::NT), pf::LDS_BYTES, st, D);
    rc = check_launch("prefill_kernel");
  }
  if (rc) return rc;
  if (a->events) {
    const hipError_t e = hipEventRecord((hipEvent_t)a->events[1], st);
    if (e != hipSuccess) return fail((int)e, "prefill: hipEventRecord failed");
  }
  if (a->n_checkpoints > 0)
    return sq_encode(pool, a->checkpoint_state, a->slots, a->slots_dtype, a->batch * a->n_checkpoints, stream);
  return 0;
}

int sq_clear_slots(const sq_pool *pool, const void *slots, int32_t slots_dtype, int64_t n, void *stream) {
  if (!pool || !pool->data) return fail(SQ_EINVAL, "clear: null pool");
  if (n == 0) return 0;
  if (!slots || n < 0 || n > 65535) return fail(SQ_EINVAL, "clear: bad slot list");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "clear: slots dtype");
  unsigned gx = (unsigned)((pool->page_bytes + 255) / 256);
  if (gx > 1024) gx = 1024;
  hipLaunchKernelGGL(clear_kernel, dim3(gx, (unsigned)n), dim3(256), 0, (hipStream_t)stream, pool->data,
                     pool->page_bytes, pool->num_slots, slots, slots_dtype);
  return check_launch("clear_kernel");
}

int sq_copy_slots(const sq_pool *pool, const void *src, const void *dst, int32_t slots_dtype, int64_t n,
                  uint8_t *temp, void *stream) {
  if (!pool || !pool->data) return fail(SQ_EINVAL, "copy: null pool");
  if (n == 0) return 0;
  if (!src || !dst || !temp || n < 0 || n > 65535) return fail(SQ_EINVAL, "copy: bad arguments");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "copy: slots dtype");
  return launch_copy(pool, src, dst, slots_dtype, n, temp, (hipStream_t)stream);
}

int sq_copy_slots_static(const sq_pool *pool, const void *src, const void *dst, int32_t slots_dtype, int64_t n,
                         void *stream) {
  if (!pool || !pool->data) return fail(SQ_EINVAL, "copy_static: null pool");
  if (n == 0) return 0;
  if (!src || !dst || n < 0 || n > 65535 || pool->page_bytes <= 0)
    return fail(SQ_EINVAL, "copy_static: bad arguments");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "copy_static: slots dtype");
  if (n > (int64_t)SQ_COPY_STATIC_BYTES / pool->page_bytes) {
    snprintf(g_err, sizeof(g_err),
             "copy_static: %lld pages of %lld bytes exceed the static staging of %lld bytes",
             (long long)n, (long long)pool->page_bytes, (long long)SQ_COPY_STATIC_BYTES);
    return SQ_EINVAL;
  }
  uint8_t *temp = nullptr;
  int rc = static_scratch(&temp);
  if (rc) return rc;
  return launch_copy(pool, src, dst, slots_dtype, n, temp, (hipStream_t)stream);
}

int sq_format_encode(const sq_format_pool *pool, const float *state, const void *slots, int32_t slots_dtype,
                     int64_t batch, void *stream) {
  int rc = validate_format(pool);
  if (rc) return rc;
  if (batch < 0 || (batch && (!state || !slots))) return fail(SQ_EINVAL, "format encode: bad arguments");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "format encode: slots dtype");
  FmtDev fd = to_fmt(pool);
  fd.in = state;
  fd.slots = slots;
  fd.slots_dtype = slots_dtype;
  StepDev sd;
  memset(&sd, 0, sizeof(sd));
  return launch_format<FMT_ENCODE>(pool, fd, sd, batch, (hipStream_t)stream);
}

int sq_format_decode(const sq_format_pool *pool, const void *slots, int32_t slots_dtype, int64_t batch,
                     float *state, void *stream) {
  int rc = validate_format(pool);
  if (rc) return rc;
  if (batch < 0 || (batch && (!state || !slots))) return fail(SQ_EINVAL, "format decode: bad arguments");
  if (slots_dtype != SQ_I32 && slots_dtype != SQ_I64) return fail(SQ_EINVAL, "format decode: slots dtype");
  FmtDev fd = to_fmt(pool);
  fd.dense = state;
  fd.slots = slots;
  fd.slots_dtype = slots_dtype;
  StepDev sd;
  memset(&sd, 0, sizeof(sd));
  return launch_format<FMT_DECODE>(pool, fd, sd, batch, (hipStream_t)stream);
}

int sq_format_step(const sq_format_pool *pool, const sq_step_args *args, void *stream) {
  int rc = validate_format(pool);
  if (rc) return rc;
  StepDev sd;
  rc = fill_step(pool->heads, args, sd);
  if (rc) return rc;
  FmtDev fd = to_fmt(pool);
  fd.slots = args->slots;
  fd.slots_dtype = args->slots_dtype;
  return launch_format<FMT_STEP>(pool, fd, sd, args->batch, (hipStream_t)stream);
}

}  // extern "C"
