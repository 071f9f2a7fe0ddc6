// Shared helpers for the gfx950 kernels of the FSCTEP hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <string>

typedef float f4 __attribute__((ext_vector_type(4)));

namespace fsc {

// v_mfma_f32_16x16x4_f32, wave64.  Operand lanes: lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; the result register j of lane l is D[4*(l/16)+j][l%16].
__device__ __forceinline__ f4 mfma16x16x4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One 16-deep K step: lane (r=l%16, q=l/16) holds A[r][k0+4q+j] in a[j] and
// B[k0+4q+j][r] in b[j]; any fixed K order works as long as A and B agree.
__device__ __forceinline__ f4 mfma_k16(const f4& a, const f4& b, f4 acc) {
  acc = mfma16x16x4(a.x, b.x, acc);
  acc = mfma16x16x4(a.y, b.y, acc);
  acc = mfma16x16x4(a.z, b.z, acc);
  acc = mfma16x16x4(a.w, b.w, acc);
  return acc;
}

// ---- fp32 products from bf16 MFMA (v_mfma_f32_16x16x32_bf16, 16x the fp32 MFMA rate).
// A float is split into three bf16 parts, a = h + m + l (each part the round-to-nearest bf16 of the
// remainder so far; the remainders are exact in fp32), which keeps its 24 significant bits.  A product
// keeps the six terms hh' + hm' + mh' + mm' + hl' + lh'; the dropped ml' + lm' + ll' are below 2^-23 of
// |a b|, the size of one fp32 rounding, and the sums accumulate in fp32 inside the MFMA.  Lane (r, q)
// of the MFMA supplies A[r][8q..8q+7] and B[8q..8q+7][r]; the result layout is that of the fp32 MFMA.
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void split3(const float (&v)[8], bf8& h, bf8& m, bf8& l) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const __bf16 hb = (__bf16)v[j];
    const float r1 = v[j] - (float)hb;
    const __bf16 mb = (__bf16)r1;
    h[j] = hb;
    m[j] = mb;
    l[j] = (__bf16)(r1 - (float)mb);
  }
}

__device__ __forceinline__ f4 mfma_bf16(const bf8& a, const bf8& b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// c += (ah + am + al)(bh + bm + bl) without the three smallest terms; small terms first.
__device__ __forceinline__ f4 mfma_x6(const bf8& ah, const bf8& am, const bf8& al, const bf8& bh, const bf8& bm,
                                      const bf8& bl, f4 c) {
  c = mfma_bf16(al, bh, c);
  c = mfma_bf16(ah, bl, c);
  c = mfma_bf16(am, bm, c);
  c = mfma_bf16(am, bh, c);
  c = mfma_bf16(ah, bm, c);
  return mfma_bf16(ah, bh, c);
}

// ---- fp32 products from fp16 MFMA (v_mfma_f32_16x16x32_f16 / 32x32x16_f16, the bf16 rate), half the
// MFMAs of split-bf16.  An operand is first scaled by a power of two s with |a s| < 2^14 (one s per MFMA
// row or column, undone on the fp32 result), then split into two fp16 parts a s = h + l (h the
// round-to-nearest fp16 of a s, l that of the remainder, which is exact in fp32): 22 significant bits.
// A product keeps hh' + hl' + lh'; the dropped ll' is below 2^-22 of |a b|.  Parts under fp16's normal
// range (2^-14) keep an absolute accuracy of 2^-25, i.e. 2^-38 of the largest scaled value.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// 2^k with bound * 2^k in [2^13, 2^14) (k within +-100; 1 for a zero, negative or non-finite bound)
__device__ __forceinline__ float pow2_scale(float bound) {
  if (!(bound > 0.f) || !(bound <= 3.4e38f)) return 1.f;
  int e;
  frexpf(bound, &e);   // bound = f 2^e, f in [0.5, 1)
  return ldexpf(1.f, min(max(14 - e, -100), 100));
}

__device__ __forceinline__ void split2h(const float (&v)[8], float s, h8& h, h8& l) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = v[j] * s;
    const _Float16 hh = (_Float16)x;
    h[j] = hh;
    l[j] = (_Float16)(x - (float)hh);
  }
}

// split2h without a scale (the caller's values are already scaled) in 12 VALU operations for 8 values: the
// high parts two at a time by v_cvt_pk_f16_f32, each low part by one v_fma_mix reading its high part from
// the packed word (v - h, exact in fp32, rounded to fp16).  The compiler's own form converts each high part
// twice (28 operations).  Register hazards of asm-written VGPRs are not tracked by the compiler, so the block
// ends with the two wait states a VALU write needs before an MFMA reads it.
__device__ __forceinline__ void split2h_pk(const float (&v)[8], h8& h, h8& l) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  u4 hw, lw;
  asm volatile(
      "v_cvt_pk_f16_f32 %0, %8, %9\n\t"
      "v_cvt_pk_f16_f32 %1, %10, %11\n\t"
      "v_cvt_pk_f16_f32 %2, %12, %13\n\t"
      "v_cvt_pk_f16_f32 %3, %14, %15\n\t"
      "v_fma_mixlo_f16 %4, %8, 1.0, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %4, %9, 1.0, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixlo_f16 %5, %10, 1.0, -%1 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %5, %11, 1.0, -%1 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixlo_f16 %6, %12, 1.0, -%2 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %6, %13, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixlo_f16 %7, %14, 1.0, -%3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %7, %15, 1.0, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "s_nop 1"
      : "=&v"(hw.x), "=&v"(hw.y), "=&v"(hw.z), "=&v"(hw.w), "=&v"(lw.x), "=&v"(lw.y), "=&v"(lw.z), "=&v"(lw.w)
      : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]));
  h = __builtin_bit_cast(h8, hw);
  l = __builtin_bit_cast(h8, lw);
}

__device__ __forceinline__ f4 mfma_h16(const h8& a, const h8& b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// c += (ah + al)(bh + bl) without al bl; small terms first.
__device__ __forceinline__ f4 mfma_x3(const h8& ah, const h8& al, const h8& bh, const h8& bl, f4 c) {
  c = mfma_h16(al, bh, c);
  c = mfma_h16(ah, bl, c);
  return mfma_h16(ah, bh, c);
}

__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ void st4(float* p, const f4& v) { *reinterpret_cast<f4*>(p) = v; }

// Raw buffer descriptor over [base, base + bytes) (bytes < 2^32).  A vector buffer store whose
// byte offset lies outside the range is dropped by the hardware, which lets a kernel store
// unconditionally and send the lanes of out-of-range rows to kDropOffset instead of branching.
constexpr uint32_t kDropOffset = 0xF0000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buffer_st4(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off, const f4& v) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rsrc, (int)byte_off, 0, 0);
}
// One float at byte offset voff (per lane) + soff (wave-uniform, kept in a scalar register): a load
// loop whose offsets are compile-time multiples of a large stride needs one address VGPR, not one
// 64-bit address per load.
__device__ __forceinline__ float buffer_ld1(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)voff, (int)soff, 0));
}
// bf16 storage of fp32 values: four values (8 bytes) stored, one value loaded and widened exactly.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc_bytes(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buffer_st4_bf16(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off, const f4& v) {
  typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const bf4 b = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, b), rsrc, (int)byte_off, 0, 0);
}
__device__ __forceinline__ float buffer_ld1_bf16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff) {
  const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(rsrc, (int)voff, (int)soff, 0);
  return __uint_as_float((uint32_t)u << 16);
}
__device__ __forceinline__ f4 buffer_ld4(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ void buffer_st4(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff, const f4& v) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), rsrc, (int)voff, (int)soff, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over lanes that share lane%width groups of `width` (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One-block-per-node launches over xcd_grid(n) workgroups.  Workgroup w runs on XCD w % 8, so XCD x
// is given the contiguous run [x*per, (x+1)*per) of the node order; with a spatial order (nodes close
// in space close in the order) the neighbour gathers of the blocks an XCD runs together then share its
// L2.  `order` null: the identity.  Returns -1 for the padding workgroups (block-uniform).
inline unsigned xcd_grid(int64_t n) { return (unsigned)(((n + 7) / 8) * 8); }
__device__ __forceinline__ int xcd_node(int64_t n, const int32_t* __restrict__ order) {
  const int64_t per = (n + 7) / 8;
  const int64_t w = blockIdx.x;
  const int64_t li = (w & 7) * per + (w >> 3);
  if (li >= n) return -1;
  if (!order) return (int)li;
  const int v = order[li];
  return (v >= 0 && v < n) ? v : -1;   // a malformed order leaves nodes unprocessed, never out of bounds
}

// Persistent form: a grid of at most the resident capacity (persist_grid) whose block b walks the nodes
// j = b/8, b/8 + G/8, ... of its XCD's range, so the blocks an XCD runs together still take neighbouring
// nodes and per-block set-up is paid once per block, not once per node.  Returns the k-th node of the
// block, -1 for an order entry to skip (block-uniform) and -2 past the end.
__device__ __forceinline__ int xcd_node_k(int64_t n, const int32_t* __restrict__ order, int k) {
  const int64_t per = (n + 7) / 8;
  const int64_t j = (blockIdx.x >> 3) + (int64_t)k * (gridDim.x >> 3);
  if (j >= per) return -2;
  const int64_t li = (blockIdx.x & 7) * per + j;
  if (li >= n) return -2;
  if (!order) return (int)li;
  const int v = order[li];
  return (v >= 0 && v < n) ? v : -1;
}

// Grid of a persistent one-block-per-node launch of `kernel` (256 threads, lds bytes of dynamic LDS):
// min(xcd_grid(n), the blocks the device holds at once, at most max_per_cu per CU), a multiple of 8.
unsigned persist_grid(int64_t n, const void* kernel, size_t lds, int max_per_cu = 1 << 20);

void set_error(const std::string& msg);
int check_launch(const char* what);
int timing_mark_begin(const char* kernel, hipStream_t st);
void timing_mark_end(int slot, hipStream_t st);

// Brackets one launch with HIP events when fsc_timing_begin(name) is active.
struct LaunchTimer {
  int slot;
  hipStream_t st;
  LaunchTimer(const char* name, hipStream_t s) : slot(timing_mark_begin(name, s)), st(s) {}
  ~LaunchTimer() { timing_mark_end(slot, st); }
};

}  // namespace fsc

#define FSC_CHECK_ARG(cond, msg)            \
  do {                                      \
    if (!(cond)) {                          \
      fsc::set_error(std::string(msg));     \
      return 1;                             \
    }                                       \
  } while (0)
