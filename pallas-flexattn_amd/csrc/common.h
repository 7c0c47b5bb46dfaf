// Device-side building blocks shared by the FlexAttention kernels (gfx950).
//
// MFMA conventions used throughout (v_mfma_f32_32x32x16_bf16, wave64):
//   A operand (32 x 16): lane l holds row (l % 32), k = 8*(l / 32) + [0..7]
//   B operand (16 x 32): lane l holds col (l % 32), k = 8*(l / 32) + [0..7]
//   C (32 x 32, 16 fp32 per lane): acc[4*j + i] is row 8*j + 4*(l / 32) + i, col l % 32
// The fp32 path issues eight v_mfma_f32_32x32x2f32 per 16-wide k step; in the
// t-th of them lane half h supplies its t-th element, so the per-lane operand
// layout (eight consecutive k per lane half) is the same as for bf16.
//
// Row permutation ("bit-2/3 swap"): when the 32 rows of an A operand are
// loaded as physical rows perm23(r), the C accumulator values a lane holds
// for output row 8*j + 4*h + i (j = 0,1) are physical rows 8*h + [0..7], and
// for j = 2,3 rows 16 + 8*h + [0..7].  The fp32 accumulators of such a tile
// therefore feed the next MFMA directly as a B (or A) operand with eight
// consecutive k per lane half — no LDS round trip for P or dS.
#pragma once
// hipRTC (the run-time compiler that builds kernels with user score / mask
// mods from these same headers) provides the HIP runtime and the integer
// types itself and has no system headers.
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#else
using __hip_internal::int16_t;
using __hip_internal::int32_t;
using __hip_internal::int64_t;
using __hip_internal::uint16_t;
using __hip_internal::uint32_t;
using __hip_internal::uint64_t;
using __hip_internal::uint8_t;
typedef __hip_internal::uint64_t uintptr_t;
typedef __SIZE_TYPE__ size_t;
#endif
#ifndef INFINITY
#define INFINITY __builtin_inff()
#endif
#include "index.h"

namespace fa {

// compile-time booleans used as tag arguments (std::integral_constant without
// <type_traits>, which hipRTC lacks)
template <bool B>
struct Bool {
  static constexpr bool value = B;
};
using False = Bool<false>;
using True = Bool<true>;
template <int N>
struct Int {
  static constexpr int value = N;
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32, 64); }

// v_permlane32_swap(x, x) yields {x[l % 32], x[l % 32 + 32]} in every lane l,
// so reductions over the lane pair (l, l ^ 32) need no LDS traffic.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Waves per SIMD a kernel can reach when its workgroup of NW waves holds
// lds_bytes of LDS (160 KiB per CU, four SIMDs), capped at `want`: the
// occupancy target given to the register allocator.
constexpr int occupancy_for(int lds_bytes, int nw, int want) {
  const int wg_per_cu = (160 * 1024) / lds_bytes;
  const int per_simd = wg_per_cu * nw / 4;
  return per_simd < 1 ? 1 : (per_simd > want ? want : per_simd);
}

// Load through the scalar data cache (the address must be wave-uniform).
__device__ __forceinline__ int scalar_load(const int* p, int i) {
  typedef const __attribute__((address_space(4))) int* cptr;
  return ((cptr)(p))[i];
}

// Scheduling hints (llvm.amdgcn.sched.group.barrier masks).
constexpr int kSchedMfma = 0x008;
constexpr int kSchedVmemRead = 0x020;
constexpr int kSchedDsRead = 0x100;
constexpr int kSchedDsWrite = 0x200;
constexpr int kSchedValu = 0x002;

// ---- accumulate-in-place MFMA ---------------------------------------------
// acc += A * B (v_mfma_f32_32x32x16_bf16) with acc tied in place, in AGPRs
// (kReg = 'a') or VGPRs ('v').  Used for accumulators that only MFMAs touch
// inside a loop (dQ, dK, dV): the builtin's VGPR form picks a fresh
// destination and copies it back every iteration.  Inline asm is opaque to
// the compiler's hazard recognizer, so the wait states the ISA requires are
// explicit:
//   * a VALU write of A or B needs 2 wait states before an MFMA reads it:
//     every call starts with s_nop 1, unless kNop is false (for schedules
//     whose operands are written at least a step before);
//   * an MFMA result (8-pass XDL) needs up to 12 wait states before another
//     unit reads it: mfma_drain() after the last accumulation;
//   * back-to-back accumulation into the same registers needs none.
template <char kReg, bool kNop = true>
__device__ __forceinline__ void mfma_acc(f32x16& acc, u32x4 a, u32x4 b) {
  if constexpr (kReg == 'a' && kNop)
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else if constexpr (kReg == 'a')
    asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else if constexpr (kNop)
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
  else
    asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
// Orders later reads of acc after 20 wait states (and earlier writes of acc,
// e.g. zero-initialisation, before later MFMAs by at least as much).
template <char kReg>
__device__ __forceinline__ void mfma_drain(f32x16& acc) {
  if constexpr (kReg == 'a')
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+a"(acc));
  else
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(acc));
}

// Store of a wave's 32-row accumulator block as bf16 rows of a row-major
// (rows, D) tensor.  In the MFMA 32x32 layout lane l holds row (l & 31) and
// element e of tile i holds column 32 i + 8 (e / 4) + 4 (l / 32) + e % 4 (the
// A operand's rows in natural order, as transposing reads give them): stored directly,
// every instruction would write 8 bytes into each of 32 rows.  The block is
// staged instead through `stage` (the wave's own 32 * 2D bytes of LDS, 16-byte
// chunks swizzled by the row) and written back 16 bytes per lane with
// consecutive lanes along a row, so each instruction writes whole row
// segments.  `scale` multiplies lane l's row (per-row factors: the lane's
// own value); rows at or past `rows_left` are not written.  The caller makes
// sure no other wave uses `stage` meanwhile.
template <int D>
__device__ __forceinline__ void store_rows_bf16(const f32x16* acc, float scale, char* stage, uint16_t* rows,
                                                int rows_left, int lane) {
  constexpr int RB = 2 * D, NCH = D / 8, DT = D / 32;
  constexpr int RPI = 64 / NCH;  // rows per store instruction
  const int r = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 4 * i + j;  // 16-byte chunk of columns 32 i + 8 j .. + 7
      *reinterpret_cast<u32x2*>(stage + r * RB + ((c ^ (r % NCH)) * 16) + hh * 8) =
          u32x2{pack_bf16x2(acc[i][4 * j] * scale, acc[i][4 * j + 1] * scale),
                pack_bf16x2(acc[i][4 * j + 2] * scale, acc[i][4 * j + 3] * scale)};
    }
  const int c = lane % NCH;
#pragma unroll
  for (int k = 0; k < 32 / RPI; ++k) {
    const int rr = k * RPI + lane / NCH;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + rr * RB + ((c ^ (rr % NCH)) * 16));
    if (rr < rows_left) *reinterpret_cast<u32x4*>(rows + (size_t)rr * D + c * 8) = v;
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// tanh from the identity tanh(x) = 1 - 2 / (exp(2x) + 1), with exp2 / rcp.
__device__ __forceinline__ float tanh_fast(float x) {
  const float e = fast_exp2(x * (2.0f * kLog2e));
  return 1.0f - 2.0f * fast_rcp(e + 1.0f);
}

// ---- element-type traits --------------------------------------------------
// A "fragment" is what one lane contributes to one 16-deep MFMA k step: eight
// consecutive elements along k.
template <typename T> struct Elt;

template <> struct Elt<uint16_t> {  // bfloat16 storage
  using frag = u32x4;
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // eight fp32 values -> fragment (RNE to bf16)
  __device__ static __forceinline__ frag pack(const float* x) {
    frag f;
    f[0] = pack_bf16x2(x[0], x[1]);
    f[1] = pack_bf16x2(x[2], x[3]);
    f[2] = pack_bf16x2(x[4], x[5]);
    f[3] = pack_bf16x2(x[6], x[7]);
    return f;
  }
  __device__ static __forceinline__ frag zero() { return frag{0u, 0u, 0u, 0u}; }
};

template <> struct Elt<float> {
  using frag = f32x8;
  static constexpr int kBytes = 4;
  __device__ static __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
#pragma unroll
    for (int t = 0; t < 8; ++t) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], b[t], c, 0, 0, 0);
    return c;
  }
  __device__ static __forceinline__ frag pack(const float* x) {
    frag f;
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] = x[t];
    return f;
  }
  __device__ static __forceinline__ frag zero() { return frag{0, 0, 0, 0, 0, 0, 0, 0}; }
};

// 16-byte global load (zero when !ok) ---------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p, bool ok) {
  return ok ? *reinterpret_cast<const u32x4*>(p) : u32x4{0u, 0u, 0u, 0u};
}

// load one fragment (8 consecutive elements) from global memory
template <typename T>
__device__ __forceinline__ typename Elt<T>::frag ld_frag(const T* p, bool ok) {
  if constexpr (sizeof(T) == 2) {
    return ld16(p, ok);
  } else {
    u32x4 a = ld16(p, ok), b = ld16(p + 4, ok);
    return f32x8{__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]),
                 __uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[2]), __uint_as_float(b[3])};
  }
}

// ---- swizzled LDS tiles ---------------------------------------------------
// A tile of R rows x C elements, stored as 16-byte chunks; the chunk index of
// row r is XOR-ed with a 3-bit function of r so that the access patterns used
// by the kernels (32 different rows, same chunk) hit distinct banks.
template <typename T, int R, int C, int SW>
struct LdsTile {
  static constexpr int kChunks = C * (int)sizeof(T) / 16;  // chunks per row
  static constexpr int kMask = (kChunks >= 8 ? 8 : kChunks) - 1;
  static constexpr int kBytes = R * C * (int)sizeof(T);
  __device__ static __forceinline__ int swz(int r) {
    if constexpr (SW == 0) return ((r + 4 * (r >> 3)) & kMask);  // rows read via perm23
    else return ((r + (r >> 3)) & kMask);                         // rows read in order
  }
  __device__ static __forceinline__ int off(int r, int chunk) {  // byte offset
    return (r * kChunks + (chunk ^ swz(r))) * 16;
  }
  // fragment of 8 elements of row r starting at element col (multiple of 8)
  __device__ static __forceinline__ typename Elt<T>::frag read(const char* base, int r, int col) {
    if constexpr (sizeof(T) == 2) {
      return *reinterpret_cast<const u32x4*>(base + off(r, col >> 3));
    } else {
      const int c = col >> 2;
      f32x4 a = *reinterpret_cast<const f32x4*>(base + off(r, c));
      f32x4 b = *reinterpret_cast<const f32x4*>(base + off(r, c + 1));
      return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
  }
};

// Write a transposed block into an LdsTile: `rows4` holds four consecutive
// source rows (r0..r0+3) x one 16-byte chunk (E = 16/sizeof(T) columns
// c0..c0+E-1); they land as E destination rows c0.. each receiving the four
// elements r0..r0+3.
template <typename Tile, typename T>
__device__ __forceinline__ void write_transposed4(char* base, const u32x4* rows4, int r0, int c0) {
  if constexpr (sizeof(T) == 2) {
    // chunk = 8 bf16 = 4 words; word j holds columns (2j, 2j+1)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w0 = rows4[0][j], w1 = rows4[1][j], w2 = rows4[2][j], w3 = rows4[3][j];
      const u32x2 lo{(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
      const u32x2 hi{(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
      const int byte_in_row = r0 * 2;  // 4 elements = 8 bytes, r0 multiple of 4
      const int d0 = c0 + 2 * j, d1 = d0 + 1;
      *reinterpret_cast<u32x2*>(base + Tile::off(d0, byte_in_row >> 4) + (byte_in_row & 15)) = lo;
      *reinterpret_cast<u32x2*>(base + Tile::off(d1, byte_in_row >> 4) + (byte_in_row & 15)) = hi;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 col{rows4[0][j], rows4[1][j], rows4[2][j], rows4[3][j]};
      *reinterpret_cast<u32x4*>(base + Tile::off(c0 + j, r0 >> 2)) = col;
    }
  }
}

}  // namespace fa
