// Row-gather probe: va_probe_gather (measurement helper, built into
// tests/numerics/libgatherprobe.so by __graft_entry__.build(); not part of
// libvecattn.so).
//
// The sparse attention kernel moves every selected key's K and V rows from L2
// (or, on an L2 miss, from the data fabric) into LDS with buffer_load_dwordx4
// ... idxen offen sc1 lds, 1 KB per instruction, and on MI355X that data path,
// not the matrix cores, is what limits it.  This probe runs the same copy
// instruction on its own: every wave of 4-wave work-groups copies `steps`
// tiles of four 256-byte rows into a 16 KB LDS ring, keeping up to 8 copies
// in flight, with row ids spread by an integer hash (or consecutive).  Its
// rate for a table that fits one XCD's L2 (2 MiB) and for one that does not
// (tens of MiB, served by the Infinity Cache) bounds what any kernel built on
// these gathers can reach; bench.py reports the attention's gather rate
// against it.
#include <cstdio>

#include "../../include/vecattn.h"
#include "../../vecattention_amd/csrc/common.h"
#include "../../vecattention_amd/csrc/lanes.h"

namespace va {
namespace {

constexpr int kProbeWaves = 4;
constexpr int kProbeRing = 16;  // 1 KB slots per wave
constexpr int kProbeKeep = 8;   // copies in flight per wave

__global__ __launch_bounds__(64 * kProbeWaves) void gather_probe_kernel(
    const void* table, uint32_t rows, int sequential, int steps, uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) unsigned char ring[kProbeWaves * kProbeRing * 1024];
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x / 64)), lane = threadIdx.x % 64;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc_rows(table, 256, rows);
  const uint32_t first = (blockIdx.x * kProbeWaves + uint32_t(wave)) * uint32_t(steps) * 4u;
  const uint32_t base = uint32_t(
      __builtin_amdgcn_readfirstlane(int(lds_addr(ring) + uint32_t(wave * kProbeRing * 1024))));
  for (int s0 = 0; s0 < steps; s0 += kProbeRing) {
#pragma unroll
    for (int j = 0; j < kProbeRing; ++j) {
      // lane l copies 16-byte chunk l % 16 of row l / 16 of the tile
      uint32_t x = first + uint32_t((s0 + j) * 4 + lane / 16);
      if (!sequential) {  // integer hash (Wellons' lowbias32)
        x ^= x >> 16;
        x *= 0x7feb352du;
        x ^= x >> 15;
        x *= 0x846ca68bu;
        x ^= x >> 16;
      }
      const uint64_t pair = uint64_t(x % rows) | (uint64_t(16u * uint32_t(lane % 16)) << 32);
      copy16_row_to_lds(rs, base + uint32_t(j * 1024), pair);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kProbeKeep) : "memory");
    }
  }
  vm_lds_barrier();
  if (threadIdx.x == 0) sink[blockIdx.x] = ring[lane];  // keeps the copies observable
}

}  // namespace
}  // namespace va

extern "C" int va_probe_gather(const void* table, int64_t rows, int64_t work_groups,
                               int64_t steps, int sequential, uint32_t* sink, void* stream) {
  if (table == nullptr || sink == nullptr || rows <= 0 || rows > (int64_t(1) << 31) / 256 ||
      work_groups <= 0 || work_groups > (int64_t(1) << 20) || steps <= 0 || steps % 16 != 0 ||
      work_groups * va::kProbeWaves * steps * 4 > (int64_t(1) << 32))
    return VA_ERR_ARG;  // rows in (0, 2^23], work_groups in (0, 2^20], steps % 16 == 0,
                        // ids below 2^32
  hipLaunchKernelGGL(va::gather_probe_kernel, dim3(unsigned(work_groups)),
                     dim3(64 * va::kProbeWaves), 0, static_cast<hipStream_t>(stream), table,
                     uint32_t(rows), sequential, int(steps), sink);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    std::fprintf(stderr, "va_probe_gather: launch failed: %s\n", hipGetErrorString(e));
    return VA_ERR_HIP;
  }
  return VA_OK;
}
