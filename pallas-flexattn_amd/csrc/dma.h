// Buffer-resource loads for gfx950: branch-free bounds handling (reads past
// the resource's byte range return zero) and direct HBM -> LDS copies.
#pragma once
#include "common.h"

namespace fa {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
#define FA_LDS __attribute__((address_space(3)))

__device__ i32x4 raw_buffer_load_b128(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");
__device__ void raw_buffer_load_lds(i32x4 rsrc, FA_LDS uint32_t* lds, int size, int voffset, int soffset,
                                    int offset, int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

// 128-bit buffer descriptor: base address, byte range, gfx9 data-format word.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

__device__ int raw_buffer_load_b32(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");

// Element i of an int array of n elements through the vector memory path
// (zero past the end).  Used for block-table entries inside tile loops: the
// load completes by the loop's end-of-tile vmcnt wait, whereas a scalar load
// shares lgkmcnt with the LDS reads and stalls the first LDS wait after it.
__device__ __forceinline__ int vload_i32(const int* base, int i, int n) {
  return raw_buffer_load_b32(make_rsrc(base, (uint32_t)n * 4u), i * 4, 0, 0);
}

// Table reads of the walks (index.h) on the device: counts through the
// scalar cache, entries through the vector memory path (vload_i32), tile
// starts made wave-uniform.
struct DeviceLoad {
  __device__ static __forceinline__ int scalar(const int* p, int i) { return scalar_load(p, i); }
  __device__ static __forceinline__ int vector(const int* p, int i, int n) { return vload_i32(p, i, n); }
  __device__ static __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
};

__device__ __forceinline__ u32x4 buf_load16(i32x4 rsrc, int byte_off) {
  return __builtin_bit_cast(u32x4, raw_buffer_load_b128(rsrc, byte_off, 0, 0));
}

// Copy 16 bytes per lane from the buffer at byte_off into LDS at
// lds_wave_base + 16 * lane (lds_wave_base must be wave-uniform).
//
// Issued as inline asm on purpose: for the intrinsic form the compiler tracks
// the asynchronous LDS write and, unable to tell the next tile's buffer from
// the current one, puts an s_waitcnt vmcnt(0) before LDS reads it cannot
// disambiguate (the transposing reads), so every tile would wait for the
// next tile's copy.  Callers make the data visible themselves: wait_vmem()
// and a workgroup barrier before any wave reads the tile.  The compiler's own
// vmcnt waits stay correct: loads counted in order only complete later when
// unknown copies are queued behind them.
//
// The copy's LDS base goes in M0, a register the compiler reserves: it is an
// input operand bound to M0, so the compiler writes M0 itself right before the
// asm (and knows its value afterwards); the asm only reads it.
//
// Wait states: a VMEM instruction that reads an SGPR written by a VALU
// instruction (here the descriptor's v_readfirstlane) needs 5 wait states
// after that write, and an LDS DMA needs 1 after an SALU write of M0.  The
// compiler's hazard recognizer does not look inside inline asm, and it often
// places the descriptor's readfirstlane a few instructions before the copy,
// so the first copy through a new descriptor (`fresh`) provides all 5 itself
// (s_nop 4), whatever precedes it.  Later copies through the same descriptor
// come after that one (its SGPRs were written before it) and wait 1; the
// static scan of the compiled kernels checks every copy on every path.
__device__ __forceinline__ void dma16(i32x4 rsrc, int byte_off, char* lds_wave_base, bool fresh = true) {
  // the low 32 bits of a flat pointer into the shared aperture are the LDS
  // byte address
  const uint32_t m0v = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)lds_wave_base);
  if (fresh)
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(byte_off), "s"(rsrc), "{m0}"(m0v)
                 : "memory");
  else
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(byte_off), "s"(rsrc), "{m0}"(m0v)
                 : "memory");
}

// s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima) through the
// builtin, so the compiler's own wait insertion knows that every earlier
// vector-memory load has completed; the empty asm keeps memory accesses from
// moving across it.
__device__ __forceinline__ void wait_vmem() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(N): every vector-memory load but the N most recent has
// completed (loads complete in order).  With N the count of copies issued
// for a later tile, the earlier tile's copies are done.
template <int N>
__device__ __forceinline__ void wait_vmem_but() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

// ds_read_b64_tr_b16: within each group of 16 lanes, source lane s supplies the
// address of 4 consecutive 16-bit elements (row s/4 of a 4x16 block at column
// 4*(s%4)); lane j receives column j of that block, i.e. the 4 elements
// (row t, column j) for t = 0..3.
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS s16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

}  // namespace fa
