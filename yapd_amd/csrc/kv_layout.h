// Paged KV pool layout shared by the attention, KV-write and gather kernels.
//
// One layer's pool is [pages][2][heads][page_size * head_dim] bf16 with
// page_size = 16 and head_dim = 64 (64 KiB per page at 16 heads):
//   plane 0 (K): head-major, then token-major: element t*64 + d;
//   plane 1 (V): head-major, then transposed: element d*16 + t,
// so the PV MFMA operand (8 consecutive tokens of one V column) is a single
// 16-byte load.  A position `pos` of row r lives on page table[r][pos / 16],
// slot pos % 16 (engines/flashinfer.py:318-344 with an arbitrary table).
#pragma once

#include <cstdint>

namespace yapd {

constexpr int kPageSize = 16;
constexpr int kHeadDim = 64;
constexpr int kHeadTile = kPageSize * kHeadDim;  // elements of one head on one page (per plane)

__host__ __device__ __forceinline__ int64_t kv_plane_offset(int64_t page, int plane, int head, int n_heads) {
  return ((page * 2 + plane) * n_heads + head) * static_cast<int64_t>(kHeadTile);
}

__host__ __device__ __forceinline__ int64_t k_offset(int64_t page, int head, int n_heads, int slot, int d) {
  return kv_plane_offset(page, 0, head, n_heads) + slot * kHeadDim + d;
}

__host__ __device__ __forceinline__ int64_t v_offset(int64_t page, int head, int n_heads, int slot, int d) {
  return kv_plane_offset(page, 1, head, n_heads) + d * kPageSize + slot;
}

}  // namespace yapd
