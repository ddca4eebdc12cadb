// Row moves of the 8-bit cache triples: the data movement of BatchQuantizedKVCache's merge / extend / filter /
// extract / finalize (locals/qkv.py:340-440) in one launch per triple.
//
// Every one of those operations builds a new (rows, KVH, cap, .) buffer whose row b is one source row shifted
// along the position axis: merge right-aligns each request's keys (qkv.py:419-430), extend pads rows on the left
// and trims or pads on the right (qkv.py:384-406), filter picks rows and drops their common left padding
// (qkv.py:370-380), extract takes one row's live positions (qkv.py:408-415), finalize rolls each row right by its
// right padding (mlx-lm's dynamic_roll, qkv.py:340-346).  So one gather covers them all:
//     dst[b, h, t] = src_b[h, t - shift_b]   if 0 <= t - shift_b < len_b, else 0          (linear)
//     dst[b, h, t] = src_b[h, (t - shift_b) mod len_b]                                     (cyclic: the roll)
// for the three arrays of a triple at once: D / 4 words, D / 64 scales and D / 64 biases (16-bit) a position.
// The copy is exact (bytes).  HBM-bound: 2 x 136 B a position and kv head for D = 128.
//
// Mapping: D / 16 lanes a position (16 bytes of words each; the first D / 64 lanes also move a scale, the next
// D / 64 a bias), consecutive positions on consecutive lane groups, so a wave reads and writes whole runs of
// 128-byte rows.  Rows' descriptors travel in the kernel arguments, kGatherRows a launch.

#include <hip/hip_runtime.h>

#include "lcl_common.h"
#include "locals_amd.h"

namespace lcl {

constexpr int kGatherRows = 32;

struct GatherRow {
  const uint32_t* w;   // source words of the row at (kv head 0, position 0)
  const uint16_t* s;   // source scales, same origin
  const uint16_t* b;   // source biases
  long long src_cap;   // positions a kv head in the source (the stride between its kv heads)
  int shift, len, wrap;
};

struct GatherParams {
  uint32_t* dw;
  uint16_t* ds;
  uint16_t* db;
  int row0, nrows, KVH, cap, D;  // destination rows [row0, row0 + nrows)
  GatherRow row[kGatherRows];
};

__global__ __launch_bounds__(256) void kv_gather(GatherParams p) {
  const int lpp = p.D / 16;           // lanes a position
  const int G = p.D / 64;             // scales (and biases) a position
  const long long per_row = (long long)p.KVH * p.cap * lpp;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= per_row * p.nrows) return;
  const int r = int(gid / per_row);
  const long long rem = gid - (long long)r * per_row;
  const int j = int(rem % lpp);
  const long long ht = rem / lpp;  // kv head * cap + position
  const int h = int(ht / p.cap), t = int(ht % p.cap);
  const GatherRow& src = p.row[r];
  int s = t - src.shift;
  bool ok;
  if (src.wrap) {
    ok = src.len > 0;
    if (ok) {
      s %= src.len;
      if (s < 0) s += src.len;
    }
  } else {
    ok = s >= 0 && s < src.len;
  }
  const long long dpos = ((long long)(p.row0 + r) * p.KVH + h) * p.cap + t;
  const long long spos = (long long)h * src.src_cap + s;
  uint4 w = make_uint4(0u, 0u, 0u, 0u);
  if (ok) w = *reinterpret_cast<const uint4*>(src.w + spos * (p.D / 4) + 4 * j);
  *reinterpret_cast<uint4*>(p.dw + dpos * (p.D / 4) + 4 * j) = w;
  if (j < G) {
    p.ds[dpos * G + j] = ok ? src.s[spos * G + j] : uint16_t(0);
  } else if (j < 2 * G) {
    p.db[dpos * G + j - G] = ok ? src.b[spos * G + j - G] : uint16_t(0);
  }
}

}  // namespace lcl

using namespace lcl;

extern "C" {

int lcl_kv_gather(uint32_t* dw, void* ds, void* db, int rows, int KVH, int cap, int D, const uint32_t* const* src_w,
                  const void* const* src_s, const void* const* src_b, const long long* src_cap, const int* shift,
                  const int* len, const int* wrap, void* stream_) {
  if (rows < 0 || KVH <= 0 || cap < 0 || D <= 0 || D % 64) return -1;
  if (rows == 0 || cap == 0) return 0;
  if (!dw || !ds || !db || !src_w || !src_s || !src_b || !src_cap || !shift || !len || !wrap) return -1;
  for (int r = 0; r < rows; r++) {
    if (len[r] < 0 || src_cap[r] < 0 || (len[r] > 0 && (!src_w[r] || !src_s[r] || !src_b[r]))) return -1;
    // linear rows read source positions [0, len); a cyclic row reads them all as well
    if (len[r] > src_cap[r]) return -1;
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  for (int r0 = 0; r0 < rows; r0 += kGatherRows) {
    GatherParams p{};
    p.dw = dw;
    p.ds = static_cast<uint16_t*>(ds);
    p.db = static_cast<uint16_t*>(db);
    p.row0 = r0;
    p.nrows = rows - r0 < kGatherRows ? rows - r0 : kGatherRows;
    p.KVH = KVH;
    p.cap = cap;
    p.D = D;
    for (int i = 0; i < p.nrows; i++) {
      GatherRow& g = p.row[i];
      g.w = src_w[r0 + i];
      g.s = static_cast<const uint16_t*>(src_s[r0 + i]);
      g.b = static_cast<const uint16_t*>(src_b[r0 + i]);
      g.src_cap = src_cap[r0 + i];
      g.shift = shift[r0 + i];
      g.len = len[r0 + i];
      g.wrap = wrap[r0 + i];
    }
    const long long threads = (long long)p.nrows * KVH * cap * (D / 16);
    hipLaunchKernelGGL(kv_gather, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, stream, p);
  }
  return int(hipGetLastError());
}

}  // extern "C"
