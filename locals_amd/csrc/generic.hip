// Attention for head sizes the tiled MFMA kernels are not built for (head_dim != 128): the reference's ragged
// decode kernels are templated on D (locals/attention.py:14-20, 100-106) and its prompt path sends any head size
// to MLX's attention over dequantized K/V (locals/qkv.py:264-272), so these shapes need an implementation too.
//
// One wave per (query row, head, query position), four a workgroup (four heads of one row and position):
//  * scores: lane t takes key t of a 64-key tile -- its D values (16-bit, or 8-bit codes dequantized as
//    scale * code + bias in fp32 and, as the reference's dequantized() does, rounded to the scales' dtype) against
//    q (fp32, scaled by scale * log2 e, in LDS, read by broadcast);
//  * online softmax in base 2 over the tiles (tile max by a wave reduction), fp32 weights;
//  * P V: lane (key group kg, dim group dg) accumulates 8 consecutive dims of the keys kg, kg + nkg, ... of the
//    tile (16-byte loads of V), the key groups are summed at the end;
//  * the sink joins the denominator; a query with no visible key and no sink gives 0.
// Masks as in lcl_sdpa (causal aligned to the last key, tree bits over the last L keys, dense, sliding window)
// and the key range [start, end) of left padding or of a ragged row's nkeys.  fp32 throughout.

#include <hip/hip_runtime.h>

#include "lcl_common.h"
#include "locals_amd.h"

namespace lcl {

constexpr int kGenMaxD = 512;

__device__ __forceinline__ float kv_val16(const void* p, size_t i, int dt) {
  const uint16_t b = static_cast<const uint16_t*>(p)[i];
  return dt == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// 8-bit value: scale * code + bias in fp32, rounded to the scales' dtype
__device__ __forceinline__ float dq8(uint32_t code, float s, float b, int dt) {
  const float x = __builtin_fmaf(s, float(code), b);
  return dt == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x)) : float(_Float16(x));
}

__global__ __launch_bounds__(256) void attn_generic(GenParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hg = (p.H + 3) / 4;
  const int blk = blockIdx.x;
  const int i = blk % p.L, hgi = (blk / p.L) % hg, r = blk / (p.L * hg);
  const int h = 4 * hgi + wave;
  __shared__ float qs[4][kGenMaxD];
  __shared__ float red[4][kGenMaxD];
  const int D = p.D;
  const float C = (p.scale_dev ? p.scale_dev[0] : p.scale) * kLog2e;
  const bool active = h < p.H;  // every wave stays to the barriers
  if (active) {
    const size_t qo = ((size_t(r) * p.H + h) * p.L + i) * D;
    for (int d = lane; d < D; d += 64)
      qs[wave][d] = C * (p.qdt == DT_F32 ? static_cast<const float*>(p.q)[qo + d] : kv_val16(p.q, qo + d, p.qdt));
  }
  __syncthreads();
  const int G = p.H / p.KVH, kvh = (active ? h : 0) / G;
  const int slot = p.slots ? min(max(p.slots[r], 0), p.kv_rows - 1) : r;
  const size_t tok0 = (size_t(slot) * p.KVH + kvh) * p.cap;
  const int lo = p.start ? max(p.start[r], 0) : 0;
  const int hi = p.nkeys ? min(max(p.nkeys[r], 0), p.cap) : p.N;
  const int off = p.N - p.L;
  unsigned long long tb = 0ull;
  if (p.mask == 2) tb = p.tree[r * p.tree_bs + i];
  const uint8_t* drow = p.mask == 3 ? p.dense + r * p.msb + h * p.msh + i * p.msq : nullptr;
  // P V roles: D / 8 dim groups of 8 dims and floor(64 / (D / 8)) key groups; lanes past the last whole key group
  // take no keys
  const int ndg = D / 8, nkg = 64 / ndg, dg = lane % ndg, kg = lane / ndg;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  for (int t0 = lo & ~63; active && t0 < hi; t0 += 64) {
    const int j = t0 + lane;
    bool vis = j >= lo && j < hi;
    if (p.mask == 1) vis = vis && j <= off + i;
    else if (p.mask == 2) vis = vis && (j < off || ((tb >> ((j - off) & 63)) & 1ull));
    else if (p.mask == 3) vis = vis && drow[min(max(j, 0), p.N - 1) * p.msk] != 0;
    else if (p.mask == 4) vis = vis && j <= off + i && j > off + i - p.window;
    float s = -INFINITY;
    if (vis) {
      float acc = 0.0f;
      const size_t kr = tok0 + j;
      if (p.kvfmt == 1) {
        const uint4* kp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.kf) + kr * D);
        for (int c = 0; c < D / 8; c++) {
          const uint4 w = kp[c];
          const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            acc = __builtin_fmaf(qs[wave][8 * c + 2 * e], half_of(ww[e], 0, p.kvdt), acc);
            acc = __builtin_fmaf(qs[wave][8 * c + 2 * e + 1], half_of(ww[e], 1, p.kvdt), acc);
          }
        }
      } else {
        const uint32_t* kp = p.kw + kr * (D / 4);
        for (int g = 0; g < D / 64; g++) {
          const float sc = kv_val16(p.ks, kr * (D / 64) + g, p.kvdt), bi = kv_val16(p.kb, kr * (D / 64) + g, p.kvdt);
          for (int c = 0; c < 16; c++) {
            const uint32_t w = kp[16 * g + c];
#pragma unroll
            for (int e = 0; e < 4; e++) acc = __builtin_fmaf(qs[wave][64 * g + 4 * c + e], dq8((w >> (8 * e)) & 0xffu, sc, bi, p.kvdt), acc);
          }
        }
      }
      s = acc;
    }
    float tmax = s;
#pragma unroll
    for (int x = 1; x < 64; x <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, x));
    if (tmax == -INFINITY) continue;  // no visible key in this tile
    const float mn = fmaxf(m, tmax);
    const float corr = m == -INFINITY ? 0.0f : fast_exp2(m - mn);
    m = mn;
    l *= corr;
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] *= corr;
    const float pj = vis ? fast_exp2(s - m) : 0.0f;
    l += pj;
    // P V: this lane's keys t = kg, kg + nkg, ... of the tile, dims 8 dg .. 8 dg + 7
    for (int t = kg; kg < nkg && t < 64; t += nkg) {
      const float w = __shfl(pj, t);
      const int jt = t0 + t;
      if (w == 0.0f) continue;
      const size_t vr = tok0 + jt;
      if (p.kvfmt == 1) {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.vf) + vr * D + 8 * dg);
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          o[2 * e] = __builtin_fmaf(w, half_of(vv[e], 0, p.kvdt), o[2 * e]);
          o[2 * e + 1] = __builtin_fmaf(w, half_of(vv[e], 1, p.kvdt), o[2 * e + 1]);
        }
      } else {
        const int g = (8 * dg) / 64;
        const float sc = kv_val16(p.vs, vr * (D / 64) + g, p.kvdt), bi = kv_val16(p.vb, vr * (D / 64) + g, p.kvdt);
        const uint2 c = *reinterpret_cast<const uint2*>(p.vw + vr * (D / 4) + 2 * dg);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          o[e] = __builtin_fmaf(w, dq8((c.x >> (8 * e)) & 0xffu, sc, bi, p.kvdt), o[e]);
          o[4 + e] = __builtin_fmaf(w, dq8((c.y >> (8 * e)) & 0xffu, sc, bi, p.kvdt), o[4 + e]);
        }
      }
    }
  }
  // l over all lanes; o summed over the key groups through LDS (nkg * D <= 512 floats a wave)
#pragma unroll
  for (int x = 1; x < 64; x <<= 1) l += __shfl_xor(l, x);
  if (kg < nkg) {
#pragma unroll
    for (int e = 0; e < 8; e++) red[wave][kg * D + 8 * dg + e] = o[e];
  }
  __syncthreads();
  if (!active) return;
  if (kg == 0) {
    for (int k = 1; k < nkg; k++) {
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] += red[wave][k * D + 8 * dg + e];
    }
  }
  const float sink = p.sinks ? p.sinks[h] * kLog2e : -INFINITY;
  const float M = fmaxf(m, sink);
  float f = 0.0f, Lt = 0.0f;
  if (M != -INFINITY) {
    f = m == -INFINITY ? 0.0f : fast_exp2(m - M);
    Lt = f * l + (sink == -INFINITY ? 0.0f : fast_exp2(sink - M));
  }
  const float w = Lt > 0.0f ? f / Lt : 0.0f;
  if (kg == 0) {
    const size_t ob = ((size_t(r) * p.H + h) * p.L + i) * D + 8 * dg;
    store4_from_f32(p.out, ob, o[0] * w, o[1] * w, o[2] * w, o[3] * w, p.odt);
    store4_from_f32(p.out, ob + 4, o[4] * w, o[5] * w, o[6] * w, o[7] * w, p.odt);
  }
}

// launch: every argument already checked by the entry point that calls it
int attn_generic_launch(const GenParams& p, hipStream_t stream) {
  const long long blocks = (long long)p.R * ((p.H + 3) / 4) * p.L;
  if (blocks <= 0) return 0;
  if (blocks > (1LL << 31) - 1) return -2;
  hipLaunchKernelGGL(attn_generic, dim3(unsigned(blocks)), dim3(256), 0, stream, p);
  return int(hipGetLastError());
}

}  // namespace lcl
