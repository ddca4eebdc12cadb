// Per-head RMS norm of q and k, RoPE over halves, v split out -- and the same with k and v
// quantized straight into the 8-bit cache.
//
// Reference behaviour: qk_kernel.qk_norm_rope (locals/qk_kernel.py:24-109).  For each
// (row b, position l, head) of qkv (B, L, (H + 2 KV) * HD), 16-bit dtype T:
//     q/k heads: r = 1 / sqrt(mean(x^2) + eps); a_i = T(w_i * T(x_i * r))   (qk_kernel.py:50,56-57)
//       RoPE (non-traditional, halves): theta_i = pos * exp2(-(2i / HD) * log2(base)) in fp32,
//       pos = offsets[b or 0] + l; out_i = T(a_i cos - a_{i+HD/2} sin),
//       out_{i+HD/2} = T(a_i sin + a_{i+HD/2} cos)                           (qk_kernel.py:51,59-62)
//     v heads: copied exactly                                               (qk_kernel.py:33-37)
// Outputs q (B, H, L, HD), k and v (B, KV, L, HD).
//
// Rounding: the angle follows the reference's fp32 steps (an fp32 exp2 result, an fp32 product
// with the position); the sum of squares, r, x * r, cos, sin and the rotation are evaluated in
// fp64 and rounded once to fp32 and then to T, so every value is the correctly rounded form of
// the reference's formula at its rounding points.
//
// The fused form (qk_norm_rope_append) writes q as above and quantizes the normed/rotated k and
// the raw v with MLX's affine 8 bits (group 64, bit-exact, as quantize_append in quant.hip) into
// positions [prev, prev + L) of the cache triples (B, KV, cap, .): what
// BatchQuantizedKVCache.update_and_fetch (locals/qkv.py:309-326) does with qk_norm_rope's k, v
// (locals/fuse.py:80-83), without the 16-bit k and v ever reaching HBM.
//
// MI355X mapping: one workgroup (256 lanes) a token, or a token's heads over several workgroups
// when there are few tokens.  The HD/2 (cos, sin) pairs depend only on the token's position, so
// a workgroup computes them once (fp64, in LDS) for all its heads.
// A head is a 32-lane half-wave: lane j holds elements 2j, 2j + 1 (+ 64 p) of each half, one
// 32-bit load each, and its RoPE partners in the other half, so a rotation never leaves the
// lane.  Sums and group min/max reduce over the half-wave with xor shuffles.  HBM-bound:
// 2 B read + 2 B (or 1.06 B for cached k, v) written a value.

#include "lcl_common.h"
#include "locals_amd.h"

namespace lcl {

struct QkParams {
  const uint16_t* qkv;  // (B, L, (H + 2 KV) * HD)
  const uint16_t* qw;   // (HD,)
  const uint16_t* kw;   // (HD,)
  const int* offsets;   // (B,) or (1,)
  uint16_t* q;          // (B, H, L, HD)
  uint16_t* k;          // (B, KV, L, HD) (unfused)
  uint16_t* v;          // (B, KV, L, HD) (unfused)
  uint32_t* cw[2];      // fused: K, V words (B, KV, cap, HD / 4)
  uint16_t* cs[2];      // fused: scales (B, KV, cap, HD / 64)
  uint16_t* cb[2];      // fused: biases
  int B, L, H, KV, per_row, cap, prev, round_even;
  float eps, log2_base;
};

template <int DT>
__device__ __forceinline__ float tval(uint16_t b) {
  return DT == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}
template <int DT>
__device__ __forceinline__ uint16_t tbits(float x) {
  return DT == DT_BF16 ? f32_to_bf16_bits(x) : __builtin_bit_cast(uint16_t, _Float16(x));
}
template <int DT>
__device__ __forceinline__ float tround(float x) {
  return tval<DT>(tbits<DT>(x));
}

// fp64 -> fp32, kept as an fp32 value: without the barrier the compiler merges this rounding and a following
// fp32 -> fp16 conversion into one rounding from fp64, which differs from the reference's two roundings (an fp32
// result, then T) wherever the fp32 value is an fp16 midpoint
__device__ __forceinline__ float f32_of(double d) {
  float f = float(d);
  asm volatile("" : "+v"(f));
  return f;
}

__device__ __forceinline__ double half_sum(double x) {
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

__device__ __forceinline__ float qround(float x, int even) { return even ? __builtin_rintf(x) : __builtin_roundf(x); }

// MLX affine 8-bit quantization of the 64 values the half-wave holds two a lane (v0, v1): returns this lane's
// two codes as bytes 0, 1 of a 16-bit value and the group's fp32 scale and bias (the arithmetic of
// quantize_append in quant.hip).
__device__ __forceinline__ uint32_t quant_pair(float v0, float v1, int even, float& scale, float& bias) {
  float mx = fmaxf(v0, v1), mn = fminf(v0, v1);
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, m));
    mn = fminf(mn, __shfl_xor(mn, m));
  }
  const float n_bins = 255.0f;
  scale = fmaxf((mx - mn) / n_bins, 1e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float q0 = qround(edge / scale, even);
  bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  const float c0 = fminf(fmaxf(qround((v0 - bias) / scale, even), 0.0f), n_bins);
  const float c1 = fminf(fmaxf(qround((v1 - bias) / scale, even), 0.0f), n_bins);
  return uint32_t(c0) | (uint32_t(c1) << 8);
}

// Quantize a head held as lo[p][u], hi[p][u] (elements (32 p + j) 2 + u and HD/2 + that) into cache row `row`.
// Group of lo[p] is p, of hi[p] is PER + p; lane j's pair is half of word 16 g + j / 2: even lanes write the lo
// group's word, odd lanes the hi group's, after one xor-1 exchange.
template <int DT, int PER>
__device__ __forceinline__ void quant_head(const float (&lo)[PER][2], const float (&hi)[PER][2], int j, int even,
                                           uint32_t* words, uint16_t* scales, uint16_t* biases, size_t row) {
  constexpr int HD = 128 * PER;
#pragma unroll
  for (int p = 0; p < PER; p++) {
    float sl, bl, sh, bh;
    const uint32_t cl = quant_pair(lo[p][0], lo[p][1], even, sl, bl);
    const uint32_t ch = quant_pair(hi[p][0], hi[p][1], even, sh, bh);
    const uint32_t send = (j & 1) ? cl : ch;
    const uint32_t recv = uint32_t(__shfl_xor(int(send), 1));
    const uint32_t word = (j & 1) ? (recv | (ch << 16)) : (cl | (recv << 16));
    const int g = (j & 1) ? PER + p : p;
    words[row * (HD / 4) + 16 * g + (j >> 1)] = word;
    if (j < 2) {
      scales[row * (HD / 64) + g] = tbits<DT>(j ? sh : sl);
      biases[row * (HD / 64) + g] = tbits<DT>(j ? bh : bl);
    }
  }
}

template <int DT, int PER, bool ROPE, bool FUSED>
__global__ __launch_bounds__(256) void qk_norm_rope_k(QkParams p) {
  constexpr int HD = 128 * PER, HALF = HD / 2;
  __shared__ double s_cos[HALF], s_sin[HALF];
  const int bl = blockIdx.x;
  const int b = bl / p.L, l = bl % p.L;
  const int hw = threadIdx.x >> 5, j = threadIdx.x & 31;
  const int NH = p.H + 2 * p.KV;
  const uint16_t* src_tok = p.qkv + size_t(bl) * NH * HD;
  // a head's values, loaded one head ahead (the first before the (cos, sin) table, whose fp64 sincos is slow)
  uint32_t nlo[PER], nhi[PER];
  auto load_head = [&](int head) {
    const uint16_t* src = src_tok + size_t(head) * HD;
#pragma unroll
    for (int q = 0; q < PER; q++) {
      nlo[q] = *reinterpret_cast<const uint32_t*>(src + 2 * (32 * q + j));
      nhi[q] = *reinterpret_cast<const uint32_t*>(src + HALF + 2 * (32 * q + j));
    }
  };
  const int head0 = hw + 8 * int(blockIdx.y), hstep = 8 * int(gridDim.y);
  if (head0 < NH) load_head(head0);
  if (ROPE) {
    const float pos = float(p.offsets[p.per_row ? b : 0] + l);
    for (int i = threadIdx.x; i < HALF; i += 256) {
      // the reference's fp32 steps: -float(2 i) / float(HD) * log2(base), exp2, times the position
      const float e = (-float(2 * i) / float(HD)) * p.log2_base;
      const float inv = float(exp2(double(e)));
      const float theta = pos * inv;
      double sn, cs;
      sincos(double(theta), &sn, &cs);
      s_cos[i] = cs;
      s_sin[i] = sn;
    }
    __syncthreads();
  }
  for (int head = head0; head < NH; head += hstep) {
    uint32_t rlo[PER], rhi[PER];
#pragma unroll
    for (int q = 0; q < PER; q++) {
      rlo[q] = nlo[q];
      rhi[q] = nhi[q];
    }
    if (head + hstep < NH) load_head(head + hstep);
    if (head >= p.H + p.KV) {  // v
      const int kvh = head - p.H - p.KV;
      const size_t row = (size_t(b) * p.KV + kvh) * (FUSED ? p.cap : p.L) + (FUSED ? p.prev + l : l);
      if (FUSED) {
        float lo[PER][2], hi[PER][2];
#pragma unroll
        for (int q = 0; q < PER; q++) {
          lo[q][0] = tval<DT>(uint16_t(rlo[q])), lo[q][1] = tval<DT>(uint16_t(rlo[q] >> 16));
          hi[q][0] = tval<DT>(uint16_t(rhi[q])), hi[q][1] = tval<DT>(uint16_t(rhi[q] >> 16));
        }
        quant_head<DT, PER>(lo, hi, j, p.round_even, p.cw[1], p.cs[1], p.cb[1], row);
      } else {
        uint16_t* dst = p.v + row * HD;
#pragma unroll
        for (int q = 0; q < PER; q++) {
          *reinterpret_cast<uint32_t*>(dst + 2 * (32 * q + j)) = rlo[q];
          *reinterpret_cast<uint32_t*>(dst + HALF + 2 * (32 * q + j)) = rhi[q];
        }
      }
      continue;
    }
    const bool is_q = head < p.H;
    const uint16_t* w = is_q ? p.qw : p.kw;
    float x[PER][2][2];  // [q][half][u]
    double ss = 0.0;
#pragma unroll
    for (int q = 0; q < PER; q++) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        x[q][0][u] = tval<DT>(uint16_t(rlo[q] >> (16 * u)));
        x[q][1][u] = tval<DT>(uint16_t(rhi[q] >> (16 * u)));
        ss += double(x[q][0][u]) * double(x[q][0][u]) + double(x[q][1][u]) * double(x[q][1][u]);
      }
    }
    ss = half_sum(ss);
    const double r = 1.0 / sqrt(ss / double(HD) + double(p.eps));
    float lo[PER][2], hi[PER][2];
#pragma unroll
    for (int q = 0; q < PER; q++) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int i = 2 * (32 * q + j) + u;
        // T(w * T(x r)): the product of two T values is exact in fp32
        const float a = tround<DT>(tval<DT>(w[i]) * tround<DT>(f32_of(double(x[q][0][u]) * r)));
        const float c = tround<DT>(tval<DT>(w[HALF + i]) * tround<DT>(f32_of(double(x[q][1][u]) * r)));
        if (ROPE) {
          const double cs = s_cos[i], sn = s_sin[i];
          lo[q][u] = tround<DT>(f32_of(double(a) * cs - double(c) * sn));
          hi[q][u] = tround<DT>(f32_of(double(a) * sn + double(c) * cs));
        } else {
          lo[q][u] = a;
          hi[q][u] = c;
        }
      }
    }
    if (is_q || !FUSED) {
      uint16_t* dst = is_q ? p.q + ((size_t(b) * p.H + head) * p.L + l) * HD
                           : p.k + ((size_t(b) * p.KV + (head - p.H)) * p.L + l) * HD;
#pragma unroll
      for (int q = 0; q < PER; q++) {
        *reinterpret_cast<uint32_t*>(dst + 2 * (32 * q + j)) =
            uint32_t(tbits<DT>(lo[q][0])) | (uint32_t(tbits<DT>(lo[q][1])) << 16);
        *reinterpret_cast<uint32_t*>(dst + HALF + 2 * (32 * q + j)) =
            uint32_t(tbits<DT>(hi[q][0])) | (uint32_t(tbits<DT>(hi[q][1])) << 16);
      }
    } else {
      const size_t row = (size_t(b) * p.KV + (head - p.H)) * p.cap + p.prev + l;
      quant_head<DT, PER>(lo, hi, j, p.round_even, p.cw[0], p.cs[0], p.cb[0], row);
    }
  }
}

// Grid (token, head split): a token's heads go 8 at a time to gridDim.y workgroups until the grid has ~2048 of
// them (8 a CU), so a decode step or a prompt chunk spreads over the CUs with few heads a workgroup in turn; each
// workgroup computes its token's (cos, sin).
template <int DT, int PER, bool FUSED>
static void launch_rope(bool rope, const QkParams& p, hipStream_t s) {
  const int tokens = p.B * p.L, groups = (p.H + 2 * p.KV + 7) / 8;
  const int split = min(groups, max(1, (2048 + tokens - 1) / tokens));
  const dim3 grid(tokens, split);
  if (rope) hipLaunchKernelGGL((qk_norm_rope_k<DT, PER, true, FUSED>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((qk_norm_rope_k<DT, PER, false, FUSED>), grid, dim3(256), 0, s, p);
}

template <int DT, bool FUSED>
static void launch_per(int per, bool rope, const QkParams& p, hipStream_t s) {
  switch (per) {
    case 1: launch_rope<DT, 1, FUSED>(rope, p, s); break;
    case 2: launch_rope<DT, 2, FUSED>(rope, p, s); break;
    case 3: launch_rope<DT, 3, FUSED>(rope, p, s); break;
    case 4: launch_rope<DT, 4, FUSED>(rope, p, s); break;
    case 5: launch_rope<DT, 5, FUSED>(rope, p, s); break;
    case 6: launch_rope<DT, 6, FUSED>(rope, p, s); break;
    case 7: launch_rope<DT, 7, FUSED>(rope, p, s); break;
    default: launch_rope<DT, 8, FUSED>(rope, p, s); break;
  }
}

template <bool FUSED>
static int launch_qk(int dt, int head_dim, bool rope, const QkParams& p, hipStream_t s) {
  const int per = head_dim / 128;
  if (dt == DT_F16) launch_per<DT_F16, FUSED>(per, rope, p, s);
  else launch_per<DT_BF16, FUSED>(per, rope, p, s);
  return int(hipGetLastError());
}

// shapes first (an empty call may pass null data pointers), then the pointers of a non-empty call
static int check_dims(int dt, int B, int L, int H, int KV, int head_dim) {
  if (dt != DT_F16 && dt != DT_BF16) return LCL_EUNSUPPORTED;
  if (B < 0 || L < 0 || H <= 0 || KV <= 0 || H % KV) return LCL_EINVAL;
  if (head_dim <= 0 || head_dim % 128 || head_dim > 1024) return LCL_EUNSUPPORTED;  // 128 x (1 .. 8)
  if ((long long)B * L > 0x7fffffffLL) return LCL_EINVAL;
  return 0;
}

}  // namespace lcl

using namespace lcl;

extern "C" int lcl_qk_norm_rope(const void* qkv, int dt, const void* q_w, const void* k_w, const int32_t* offsets,
                                int offsets_per_row, float eps, float log2_base, int rope, int B, int L, int H, int KV,
                                int head_dim, void* q, void* k, void* v, void* stream) {
  const int rc = check_dims(dt, B, L, H, KV, head_dim);
  if (rc || B * L == 0) return rc;
  if (!qkv || !q_w || !k_w || !offsets || !q || !k || !v) return LCL_EINVAL;
  QkParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qw = static_cast<const uint16_t*>(q_w);
  p.kw = static_cast<const uint16_t*>(k_w);
  p.offsets = offsets;
  p.q = static_cast<uint16_t*>(q);
  p.k = static_cast<uint16_t*>(k);
  p.v = static_cast<uint16_t*>(v);
  p.B = B, p.L = L, p.H = H, p.KV = KV, p.per_row = offsets_per_row != 0;
  p.eps = eps, p.log2_base = log2_base;
  return launch_qk<false>(dt, head_dim, rope != 0, p, static_cast<hipStream_t>(stream));
}

extern "C" int lcl_qk_norm_rope_append(const void* qkv, int dt, const void* q_w, const void* k_w, const int32_t* offsets,
                                       int offsets_per_row, float eps, float log2_base, int rope, int B, int L, int H,
                                       int KV, int head_dim, void* q, void* kw, void* ks, void* kb, void* vw, void* vs,
                                       void* vb, int cap, int prev, int round_mode, void* stream) {
  const int rc = check_dims(dt, B, L, H, KV, head_dim);
  if (rc) return rc;
  if (round_mode != 0 && round_mode != 1) return LCL_EINVAL;
  if (prev < 0 || cap < 0 || L > cap - prev) return LCL_EINVAL;
  if (B * L == 0) return 0;
  if (!qkv || !q_w || !k_w || !offsets || !q || !kw || !ks || !kb || !vw || !vs || !vb) return LCL_EINVAL;
  QkParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qw = static_cast<const uint16_t*>(q_w);
  p.kw = static_cast<const uint16_t*>(k_w);
  p.offsets = offsets;
  p.q = static_cast<uint16_t*>(q);
  p.cw[0] = static_cast<uint32_t*>(kw), p.cw[1] = static_cast<uint32_t*>(vw);
  p.cs[0] = static_cast<uint16_t*>(ks), p.cs[1] = static_cast<uint16_t*>(vs);
  p.cb[0] = static_cast<uint16_t*>(kb), p.cb[1] = static_cast<uint16_t*>(vb);
  p.B = B, p.L = L, p.H = H, p.KV = KV, p.per_row = offsets_per_row != 0;
  p.cap = cap, p.prev = prev, p.round_even = round_mode;
  p.eps = eps, p.log2_base = log2_base;
  return launch_qk<true>(dt, head_dim, rope != 0, p, static_cast<hipStream_t>(stream));
}
