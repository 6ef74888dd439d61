// Device helpers shared by the gfx950 kernels: buffer-resource loads,
// wave reductions and scalar conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "eff_formats.h"
#include "eff_kernels.h"

namespace eff {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Loads go through buffer resources: a base address in SGPRs, 32-bit byte
// offsets per lane with immediate displacements, and a byte count past which
// reads return 0 (so no read can leave the buffer). Blocks start at even byte
// offsets; 4-byte words are read aligned and re-assembled with v_alignbyte.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcFlags = 0x00020000;  // dword 3 of the buffer descriptor (gfx9 family)

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)n, kRsrcFlags);
}

__device__ __forceinline__ uint32_t ld32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

__device__ __forceinline__ uint32_t ld_u16_a2(rsrc_t r, uint32_t off) {
  const uint32_t w = ld32(r, off & ~3u);
  return (off & 2u) ? (w >> 16) : (w & 0xFFFFu);
}

template <int N>
__device__ __forceinline__ void ld_words_a2(rsrc_t r, uint32_t off, uint32_t *out) {
  const uint32_t base = off & ~3u, sh = off & 3u;
  uint32_t v[N + 1];
#pragma unroll
  for (int i = 0; i <= N; ++i) v[i] = ld32(r, base + 4u * i);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
}

// Sum over each 16-lane row with DPP; every lane of the row gets the sum.
__device__ __forceinline__ float dpp_row_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

// Sum over the 64 lanes of the wave (wave-uniform result).
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_row_sum(v);
  const int iv = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48)));
}

__device__ __forceinline__ float h2f(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}


// ---------------------------------------------------------------------------
// Direct-to-LDS loads: 4 or 16 bytes per lane from the buffer (voffset +
// soffset) into LDS at lds + 4 * lane or lds + 16 * lane. Written as inline
// assembly so that the compiler, which cannot tell a stage being filled from
// one being read, adds no vmcnt(0) before LDS reads; callers wait explicitly
// (wait_vm) before reading what they loaded. The LDS address goes in through
// an m0 operand constraint, so the compiler itself sets m0 for the load.
__device__ __forceinline__ void dma16(rsrc_t r, const uint8_t *lds, uint32_t voff, uint32_t soff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(so), "{m0}"(m0)
               : "memory");
}

__device__ __forceinline__ void dma4(rsrc_t r, const uint8_t *lds, uint32_t voff, uint32_t soff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("buffer_load_dword %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(so), "{m0}"(m0)
               : "memory");
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((int)((N & 15u) | ((N >> 4) << 14) | 0x0F70u));
}


// Where the blocks of a weight tile live: `q` covers the GGUF blocks (or the
// Q8_0R quants) from the tile's first block on, `s` the Q8_0R scales.
struct BufSrc {
  rsrc_t q, s;
};

__device__ __forceinline__ BufSrc make_src(const WeightView &wv, uint64_t first_block) {
  BufSrc src;
  if (wv.type == Q8_0R) {
    const uint64_t qo = 32ull * first_block, so = wv.scales_off + 2ull * first_block;
    src.q = make_rsrc(wv.w + qo, wv.w_bytes > qo ? wv.w_bytes - qo : 0);
    src.s = make_rsrc(wv.w + so, wv.w_bytes > so ? wv.w_bytes - so : 0);
  } else {
    const uint64_t bo = first_block * geometry(wv.type).bytes;
    src.q = make_rsrc(wv.w + bo, wv.w_bytes > bo ? wv.w_bytes - bo : 0);
    src.s = src.q;
  }
  return src;
}

}  // namespace eff
