// mxq_ring.hpp — pieces shared by the MFMA kernels: buffer descriptors,
// LDS-direct loads, explicit vmcnt waits, the ring barrier, the LDS swizzle
// and the XCD-aware tile order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxq {
namespace ring {

// Raw (untyped) buffer descriptor over [base, base + bytes): loads past the end
// return zeros. Word 3 = 0x00020000 selects dword access on gfx9-family parts.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}

// SIZE bytes per lane from the buffer straight into LDS at dst + SIZE*lane
// (buffer_load_dword{,x4} ... lds; dst must be wave-uniform). These loads count
// in vmcnt but have no VGPR destination, so the compiler never waits for them:
// the kernels do, with wait_vmcnt / ring_barrier.
template <int SIZE>
__device__ __forceinline__ void lds_load(__amdgpu_buffer_rsrc_t r, const void* dst, int voff,
                                         int soff) {
  static_assert(SIZE == 4 || SIZE == 16, "LDS-direct load size");
  if constexpr (SIZE == 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)dst, 4, voff, soff, 0, 0);
}

// vmcnt-only wait (expcnt and lgkmcnt left at their maxima), gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier of a load ring: this wave's requests older than its last
// N have landed (vmcnt(N)), its LDS reads are done (lgkmcnt(0)), then
// s_barrier. __syncthreads() would also wait for every outstanding load
// (vmcnt(0)) and empty the ring.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  wait_vmcnt<N>();
  __builtin_amdgcn_s_waitcnt((15 & 15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 128-byte LDS rows of 16-byte chunks, chunk c of row r stored at c ^ swz(r):
// 32 rows read at one logical chunk, and 8 rows written whole, both touch
// every bank once.
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Tile order: consecutive workgroup ids go to different XCDs (dispatch is
// round-robin over the 8 XCDs), so ids are first regrouped into 8 contiguous
// ranges, one per XCD; inside a range, groups of GROUP_M token tiles sweep the
// feature tiles together so an XCD's concurrent tiles share operands in its L2.
// Returns false for the padding ids of the last round.
template <int GROUP_M>
__device__ __forceinline__ bool tile_coords(int m_tiles, int n_tiles, int& m_tile,
                                            int& n_tile) {
  const int tiles = m_tiles * n_tiles;
  const int nblk = gridDim.x;  // a multiple of 8 (see grid_blocks)
  const int bid = (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3);
  if (bid >= tiles) return false;
  const int per_group = GROUP_M * n_tiles;
  const int first_m = (bid / per_group) * GROUP_M;
  const int gsize = min(m_tiles - first_m, GROUP_M);
  const int in_group = bid % per_group;
  m_tile = first_m + in_group % gsize;
  n_tile = in_group / gsize;
  return true;
}

inline int grid_blocks(int tiles) { return (tiles + 7) / 8 * 8; }

}  // namespace ring
}  // namespace mxq
