// Streaming-read probes for bench.py's secondary rooflines: how many bytes a second this MI355X reads from HBM with a
// plain kernel, to set beside the decode kernel's rate.  Not part of the attention library (they are built into their
// own libread_probe.so and loaded only by the bench).
//
// read_probe_lds: the load method of the decode kernels.  Each single-wave workgroup streams one contiguous span of
// `tiles` 16 KiB tiles into a private LDS ring of DEPTH tiles with direct buffer->LDS loads (16 per tile, 1 KiB each,
// non-temporal), waits for the oldest tile, reads one word of it and issues the next tile into that slot.
// read_probe_vec: plain 16-byte non-temporal vector loads to registers over a grid-stride loop.
// Both write one word per lane, so their writes are negligible next to the reads.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kTile = 16384;
constexpr int kNT = 2;  // the non-temporal cache-policy bit of a buffer load

// vmcnt(n) with expcnt and lgkmcnt left open (gfx9 encoding: vmcnt bits 3:0 and 15:14)
constexpr int wait_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

template <int DEPTH>
__global__ __launch_bounds__(64) void read_probe_lds(const uint8_t* __restrict__ p, int tiles,
                                                     unsigned* __restrict__ out) {
  static_assert(DEPTH >= 2 && (DEPTH - 1) * 16 <= 63, "vmcnt holds at most 63 loads");
  __shared__ __attribute__((aligned(16))) uint8_t ring[DEPTH][kTile];
  const int lane = threadIdx.x;
  const size_t span = (size_t)tiles * kTile;
  // the descriptor covers exactly this wave's span (the host keeps span below 2^32 bytes)
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p + blockIdx.x * span), (short)0, (int)span, 0x00020000);
  unsigned acc = 0;
  for (int t = 0; t < tiles; ++t) {
    uint8_t* slot = ring[t % DEPTH];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(slot + 1024 * u), 16,
                                               (uint32_t)(t * kTile + 1024 * u + 16 * lane), 0, 0, kNT);
    if (t >= DEPTH - 1) {
      __builtin_amdgcn_s_waitcnt(wait_vm((DEPTH - 1) * 16));
      acc ^= *reinterpret_cast<const unsigned*>(ring[(t - DEPTH + 1) % DEPTH] + 16 * lane);
    }
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0));
  for (int t = tiles - DEPTH + 1 > 0 ? tiles - DEPTH + 1 : 0; t < tiles; ++t)
    acc ^= *reinterpret_cast<const unsigned*>(ring[t % DEPTH] + 16 * lane);
  out[blockIdx.x * 64 + lane] = acc;
}

__global__ __launch_bounds__(256) void read_probe_vec(const u32x4* __restrict__ p, size_t n16,
                                                      unsigned* __restrict__ out) {
  constexpr int kUnroll = 4;
  const size_t tid = blockIdx.x * (size_t)256 + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * 256;
  unsigned acc = 0;
  size_t i = tid;
  // the furthest load of a step is i + (kUnroll - 1) * stride, checked before the step
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  out[tid] = acc;
}

}  // namespace

extern "C" {

// Words `out` must hold for a launch of `blocks` workgroups of either probe.
size_t lcl_probe_out_words(int blocks) { return (size_t)blocks * 256; }

// read_probe_lds over `bytes` at `src`: `waves` single-wave workgroups, each streaming bytes / waves (a whole
// number of 16 KiB tiles, below 2^31) with `depth` tiles in its ring (2, 3 or 4).  `src` 16-byte aligned.
// Returns 0, -1 for bad arguments, or the launch's hipError_t.
int lcl_probe_read_lds(const void* src, size_t bytes, unsigned* out, int waves, int depth, hipStream_t stream) {
  if (!src || !out || waves < 1 || waves > 65536 || (uintptr_t)src % 16) return -1;
  if (bytes % ((size_t)waves * kTile)) return -1;
  const size_t tiles = bytes / waves / kTile;
  if (tiles < 1 || tiles * kTile >= ((size_t)1 << 31)) return -1;
  const uint8_t* p = static_cast<const uint8_t*>(src);
  switch (depth) {
    case 2: read_probe_lds<2><<<waves, 64, 0, stream>>>(p, (int)tiles, out); break;
    case 3: read_probe_lds<3><<<waves, 64, 0, stream>>>(p, (int)tiles, out); break;
    case 4: read_probe_lds<4><<<waves, 64, 0, stream>>>(p, (int)tiles, out); break;
    default: return -1;
  }
  return (int)hipGetLastError();
}

// read_probe_vec over `bytes` (a multiple of 16) at `src` (16-byte aligned) with `blocks` workgroups of 256.
int lcl_probe_read_vec(const void* src, size_t bytes, unsigned* out, int blocks, hipStream_t stream) {
  if (!src || !out || blocks < 1 || blocks > 65536 || bytes % 16 || (uintptr_t)src % 16) return -1;
  read_probe_vec<<<blocks, 256, 0, stream>>>(static_cast<const u32x4*>(src), bytes / 16, out);
  return (int)hipGetLastError();
}

}  // extern "C"
