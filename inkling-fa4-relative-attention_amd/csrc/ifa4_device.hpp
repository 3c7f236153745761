// Device-side helpers shared by the gfx950 kernels: operand types, MFMA
// wrappers, wave-level exchanges and element conversions.
//
// Wave64 MFMA layouts used throughout (CDNA3/CDNA4 "32x32" and "16x16" forms):
//   v_mfma_f32_32x32x16_{bf16,f16}:  lane l, g = l / 32
//     A (32 x 16):  row l % 32, eight k-slots 8g .. 8g+7
//     B (16 x 32):  col l % 32, eight k-slots 8g .. 8g+7
//     C (32 x 32):  acc[4*i + j] = C[8*i + 4*g + j][l % 32]   (i, j in 0..3)
//   v_mfma_f32_16x16x32_{bf16,f16}:  lane l, g = l / 16
//     A (16 x 32):  row l % 16, k-slots 8g .. 8g+7
//     B (32 x 16):  col l % 16, k-slots 8g .. 8g+7
//     C (16 x 16):  acc[j] = C[4*g + j][l % 16]
// A k-slot of A is multiplied with the same k-slot of B, so which physical
// index a slot stands for is a free choice as long as A and B agree.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ifa4 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Deferred-rescale threshold (log2 units): the running max used for the
// exponentials is only raised when a row's max grows by more than this, so
// p <= 2^8 stays exact in fp32 and representable in bf16/fp16.
constexpr float kRescaleThreshold = 8.0f;

struct Bf16Tag {};
struct F16Tag {};

template <typename Tag> struct Elem;
template <> struct Elem<Bf16Tag> {
  // Two fp32 -> packed 16-bit pair (round to nearest even).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  // acc + lo(w) + hi(w), one v_dot2 (sum of a packed pair)
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one, acc, false);
  }
  // OCP e4m3 bytes 2*HI, 2*HI+1 of w -> packed pair, one conversion, exact
  // (scale 1; every e4m3 value is a bf16 value).
  template <bool HI>
  static __device__ __forceinline__ uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Elem<F16Tag> {
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    f16x2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), one, acc, false);
  }
  // OCP e4m3 bytes 2*HI, 2*HI+1 of w -> packed pair, exact (e4m3 fits fp16).
  template <bool HI>
  static __device__ __forceinline__ uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  static __device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(x[lane], x[lane ^ 32]) in every lane.
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// x[lane] + x[lane ^ 32] in every lane.
__device__ __forceinline__ float add_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x[lane] + x[lane ^ 16] / max of the pair, in every lane.  permlane16_swap
// exchanges the odd 16-lane rows of its first operand with the even rows of
// its second; with x in both, the two results hold x and its xor-16 partner.
__device__ __forceinline__ float add_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Rows [start, start + len) of sequence `seq` from a cu_seqlens array, clamped
// to [0, total]: offsets that are out of range or decreasing give a shorter (or
// empty) sequence instead of reads and writes outside the tensors.
struct SeqBounds {
  int start, len;
};
__device__ __forceinline__ SeqBounds seq_bounds(const int32_t* cu, int seq, int total) {
  const int s = min(max(cu[seq], 0), total);
  const int e = min(max(cu[seq + 1], s), total);
  return SeqBounds{s, e - s};
}

// Value of x in lane `src` (wave-uniform index), broadcast.
__device__ __forceinline__ float readlane_f(float x, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}

// Orders LDS traffic inside one wave: a wave's LDS operations execute in
// order, so only the compiler has to be kept from reordering them.
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ bool wave_any(bool p) {
  return __builtin_amdgcn_ballot_w64(p) != 0;
}
__device__ __forceinline__ bool wave_all(bool p) { return !wave_any(!p); }

__device__ __forceinline__ u32x4_t ld_global_16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// ---- buffer addressing -------------------------------------------------------------
// A buffer resource covers [base, base + bytes); a load whose offset lies past
// the end returns zeros instead of touching memory.  The kernels use this for
// ragged tails (no branches around loads) and 32-bit per-sequence offsets.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOutOfRange = 0x80000000u;  // offset past any resource used here

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// Same, for a base and size the caller knows to be wave-uniform but the
// compiler may not (values carried through loops and lambdas): forces them
// into scalar registers, where a buffer resource must live.
__device__ __forceinline__ rsrc_t make_rsrc_uniform(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo),
                   __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ u32x4_t buf_load_16(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}
// Same, marked non-temporal (streamed once; not kept in the caches).
__device__ __forceinline__ u32x4_t buf_load_16_nt(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 2));
}
__device__ __forceinline__ uint32_t buf_load_4(rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load_2(rsrc_t r, uint32_t byte_off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)byte_off, 0, 0);
}

// Direct HBM -> LDS load of 16 bytes per lane: lane L's bytes land at
// lds_dst + 16 L (lds_dst wave-uniform), out-of-range lanes write zeros.
// Written as inline asm on purpose: the compiler's wait-count pass cannot tell
// which LDS bytes a DMA writes, so with the builtin it puts a full vmcnt wait
// in front of LDS reads of the *other* stage, draining the prefetch of the next
// tile every iteration.  Hidden from the compiler, the DMA is ordered only by
// the kernel's explicit s_waitcnt + s_barrier; the compiler's own waits for its
// loads stay correct because loads complete in issue order (they only wait
// longer when a DMA was issued after the load they wait for).
// The compiler does not resolve hazards into inline asm either: a VALU write
// of an SGPR (v_readfirstlane, or v_readlane restoring a spilled resource)
// needs 5 wait states before a VMEM instruction reads that SGPR, and an SALU
// write of M0 needs 1 before an LDS DMA reads it.  Without them the DMA reads
// a stale resource (seen as wrong rows when the decode kernel spilled its Q
// resource), so the asm starts with s_nop 4 (5 wait states).
__device__ __forceinline__ void dma_16(rsrc_t r, uint32_t byte_off, const void* lds_dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_dst);
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(byte_off), "s"(r),
               "{m0}"(m0)
               : "memory");
}

// Same DMA through a resource the caller builds per tile (its base at the
// tile's first row, its size ending where the sequence's rows end), with the
// per-lane offset kept in a register across tiles and the LDS byte address
// already in an SGPR value.  The buffer range check on gfx9 covers the per-lane
// and instruction offsets only, not the scalar offset, so the tile's start must
// be in the resource base for rows past the sequence end to read as zero.
// Each DMA carries its own hazard cover (s_nop 4: 5 wait states, enough for a
// VALU write of the resource or M0 and for the SALU write of M0), so no
// instruction the compiler schedules between two DMAs can expose one.
// IFA4_DMA_COVER_EACH=0 (a sweep knob) restores the earlier form, one s_nop 4
// per batch issued by the caller and s_nop 0 here, which is only safe while no
// VALU writes those SGPRs inside the batch.
#ifndef IFA4_DMA_COVER_EACH
#define IFA4_DMA_COVER_EACH 1
#endif
__device__ __forceinline__ void dma_16_tile(rsrc_t r, uint32_t lane_off, uint32_t lds_addr) {
#if IFA4_DMA_COVER_EACH
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(lane_off), "s"(r),
               "{m0}"(lds_addr)
               : "memory");
#else
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(lane_off), "s"(r),
               "{m0}"(lds_addr)
               : "memory");
#endif
}
__device__ __forceinline__ void hazard_nop5() { asm volatile("s_nop 4" ::: "memory"); }

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Bias element types: storage size and conversion of the loaded bits to fp32.
struct RelF32 {
  static constexpr int kBytes = 4;
  static __device__ __forceinline__ float load(rsrc_t r, uint32_t off) {
    return __uint_as_float(buf_load_4(r, off));
  }
};
struct RelBf16 {
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float load(rsrc_t r, uint32_t off) {
    return __uint_as_float(buf_load_2(r, off) << 16);
  }
  // x rounded to this type, as the low half of a packed pair (high half 0)
  static __device__ __forceinline__ uint32_t pack_lo(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
  }
  static __device__ __forceinline__ float unpack_lo(uint32_t w) { return __uint_as_float(w << 16); }
  // acc + lo(w) * lo(sel) + hi(w) * hi(sel): one v_dot2_f32_bf16
  static __device__ __forceinline__ float dot2(uint32_t w, uint32_t sel, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w),
                                           __builtin_bit_cast(bf16x2_t, sel), acc, false);
  }
  // element 0 / 1 of a packed pair
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};
struct RelF16 {
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float load(rsrc_t r, uint32_t off) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)buf_load_2(r, off));
  }
  static __device__ __forceinline__ uint32_t pack_lo(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
  }
  static __device__ __forceinline__ float unpack_lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  // acc + lo(w) * lo(sel) + hi(w) * hi(sel): one v_dot2_f32_f16
  static __device__ __forceinline__ float dot2(uint32_t w, uint32_t sel, float acc) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), __builtin_bit_cast(f16x2_t, sel),
                                  acc, false);
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
};

}  // namespace ifa4
