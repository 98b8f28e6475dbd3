// Wave-level helpers for gfx950 kernels: global -> LDS copies through buffer
// resources, and exchanges between the two 32-lane halves of a wave.
#pragma once
#include "common.h"

namespace va {

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Buffer resource of a raw buffer (stride 0, 32-bit data format) of `bytes`
// bytes at `base`: loads at offsets >= bytes return 0.
// Every field is made wave-uniform explicitly so that the resource lives in
// SGPRs, as buffer instructions require.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))));
  const uint64_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(lo | (hi << 32)), (short)0,
                                           __builtin_amdgcn_readfirstlane(int(bytes)),
                                           0x00020000);
}

// Buffer resource over `rows` records of `stride` bytes (stride < 2^14, the
// field's width): an access with index >= rows reads zeros, so any key id
// outside [0, rows) is safe to use as an index.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc_rows(const void* base, uint32_t stride,
                                                        uint32_t rows) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))));
  const uint64_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(lo | (hi << 32)),
                                           (short)__builtin_amdgcn_readfirstlane(int(stride)),
                                           __builtin_amdgcn_readfirstlane(int(rows)), 0x00020000);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ inline uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((lds_void_ptr)(const_cast<void*>(p))));
}

// Global -> LDS copies (buffer_load ... lds): lane i writes `size` bytes at LDS
// address lds + size*i, read from buffer offset voffset.  Issued from inline
// assembly so that the compiler's memory-counter bookkeeping does not make
// LDS reads of the other stage wait for these copies; completion is awaited
// explicitly with vm_lds_barrier().  M0 (the LDS base) is set in the same
// statement.  M0 is a reserved register to the compiler, which ignores it in
// a clobber list; these kernels issue no instruction of their own that reads
// M0 (no LDS-DMA builtins, no indirect register indexing), which
// tests/test_native_cpu.py checks on the generated assembly.  A statement that
// sets M0 with a scalar add lists SCC as clobbered.
__device__ inline void copy16_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(int(lds))), "v"(voffset), "s"(r)
               : "memory");
}
// The same through a row resource (make_rsrc_rows): the lane's address is
// row index * stride + byte offset, the pair packed as index | offset << 32.
// Device scope (sc1): the rows are gathered once per work-group and not
// reused by the CU, so the load is not kept in the CU's vector L1 (measured
// faster on gfx950 than the default; non-temporal is much slower, since other
// work-groups re-read the same rows from L2).
__device__ inline void copy16_row_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t lds,
                                         uint64_t index_offset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 idxen offen sc1 lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(int(lds))), "v"(index_offset), "s"(r)
               : "memory");
}
// The same with the LDS address given as a wave-uniform base plus a
// compile-time offset, so that setting M0 costs one scalar add.
template <uint32_t kOffset>
__device__ inline void copy16_row_to_lds_at(__amdgpu_buffer_rsrc_t r, uint32_t lds_base,
                                            uint64_t index_offset) {
  asm volatile("s_add_u32 m0, %0, %3\n\tbuffer_load_dwordx4 %1, %2, 0 idxen offen sc1 lds"
               :
               : "s"(lds_base), "v"(index_offset), "s"(r), "n"(kOffset)
               : "memory", "scc");
}
// One dword per lane, device scope (read once, as copy16_row_to_lds).
__device__ inline void copy4_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen sc1 lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(int(lds))), "v"(voffset), "s"(r)
               : "memory");
}

// Max of x over lanes l and l ^ 32.  x must not be a signaling NaN (it is an
// arithmetic result or an infinity here), so the plain v_max_f32 is used
// without the quieting that fmaxf adds in front of it.
__device__ inline float max_halves(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"((uint32_t)p[0]), "v"((uint32_t)p[1]));
  return r;
}
// max(a, b) for values that are not signaling NaNs (as max_halves): the
// plain v_max_f32, without the quieting fmaxf adds in front of it.
__device__ inline float max_plain(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// max(a, b, c) for values that are not signaling NaNs (as max_halves).
__device__ inline float max3_plain(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ inline float sum_halves(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
}

// Cross-lane helpers read other lanes' registers: call them where the whole
// wave is active (never under a divergent branch or short-circuit operand).

// Value of x held by lane l ^ 32.  The two results of v_permlane32_swap(x, x)
// hold x[l] and x[l ^ 32] in every lane; XOR-ing both with x leaves the
// partner's value whichever result carries which.
__device__ inline uint32_t other_half(uint32_t x) {
  const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return uint32_t(p[0]) ^ uint32_t(p[1]) ^ x;
}
__device__ inline float other_half(float x) {
  return __builtin_bit_cast(float, other_half(__builtin_bit_cast(uint32_t, x)));
}

// Inclusive prefix sum over the 64 lanes, in registers (DPP): shifts by 1,
// 2, 4, 8 inside each row of 16 lanes, then the total of row 0 (lane 15)
// added to row 1 and that of row 2 to row 3 (row_bcast:15), then the total
// of rows 0-1 (lane 31) added to rows 2-3 (row_bcast:31).  A lane whose DPP
// source is outside its row, or whose row is masked off, adds the `old`
// operand, 0.
__device__ inline int wave_inclusive_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return x;
}

}  // namespace va
