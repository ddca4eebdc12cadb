// MLX affine 8-bit quantization (group 64) and its cache append, bit-exact.
//
// Reference behaviour: BatchQuantizedKVCache.update_and_fetch (locals/qkv.py:309-326)
// quantizes the step's new keys and values with mx.quantize(x, group_size=64, bits=8)
// and writes the (words, scales, biases) triples at positions [prev, prev + L) of the
// cache buffers (B, KVH, cap, .); dequantized (locals/qkv.py:252-253) is
// mx.dequantize.  Per group of 64 values (fp32 arithmetic, correctly rounded division):
//     scale = max((max - min) / 255, 1e-7); side = |min| > |max|; scale = side ? scale : -scale
//     edge = side ? min : max; q0 = round(edge / scale)
//     q0 != 0: scale = edge / q0, bias = edge;  else bias = 0
//     code = clamp(round((w - bias) / scale), 0, 255); scale, bias stored in the input dtype (RNE)
// round() ties away from zero (MLX's Metal path) or to even (MLX's CPU path), by argument.
//
// MI355X mapping: one wave quantizes four 64-value groups; a lane owns 4 values
// (one output word, 8-byte load), group min/max by a 4-step xor reduction over its
// 16 lanes, one 32-bit store per lane and one scale/bias store per group.  K and V
// of a step share one launch (blockIdx.y).  HBM-bound: 2 B read + 1.06 B written a
// value.  Dequantization is the mirror image (one word in, 4 values out a lane).

#include "lcl_common.h"
#include "locals_amd.h"

namespace lcl {

struct QuantParams {
  const void* src[2];  // (B, KVH, L, D) rows, dtype dt; src[1] may be null
  uint32_t* words[2];  // (B, KVH, cap, D/4)
  void* scales[2];     // (B, KVH, cap, D/64), dtype dt
  void* biases[2];
  long long rows;      // B * KVH * L
  int L, D, cap, prev, dt, round_even;
};

__device__ __forceinline__ float round_mode(float x, int even) { return even ? __builtin_rintf(x) : __builtin_roundf(x); }

__global__ __launch_bounds__(256) void quantize_append(QuantParams p) {
  const int which = blockIdx.y;
  if (!p.src[which]) return;
  const int lane = threadIdx.x & 63;
  const int groups_per_row = p.D / 64;
  const long long gid = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) / 16;  // global group index
  const long long ngroups = p.rows * groups_per_row;
  if (gid >= ngroups) return;  // whole 16-lane groups exit together
  const long long row = gid / groups_per_row;
  const int g = int(gid % groups_per_row);
  const int sub = lane & 15;  // lane within the group: values 4 sub .. 4 sub + 3
  const uint16_t* src = static_cast<const uint16_t*>(p.src[which]);
  const uint2 raw = *reinterpret_cast<const uint2*>(src + row * p.D + g * 64 + 4 * sub);
  float w[4];
  w[0] = half_of(raw.x, 0, p.dt);
  w[1] = half_of(raw.x, 1, p.dt);
  w[2] = half_of(raw.y, 0, p.dt);
  w[3] = half_of(raw.y, 1, p.dt);
  float mx = fmaxf(fmaxf(w[0], w[1]), fmaxf(w[2], w[3]));
  float mn = fminf(fminf(w[0], w[1]), fminf(w[2], w[3]));
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, m));
    mn = fminf(mn, __shfl_xor(mn, m));
  }
  const float n_bins = 255.0f, eps = 1e-7f;
  float scale = fmaxf((mx - mn) / n_bins, eps);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float q0 = round_mode(edge / scale, p.round_even);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float c = round_mode((w[i] - bias) / scale, p.round_even);
    c = fminf(fmaxf(c, 0.0f), n_bins);
    word |= uint32_t(c) << (8 * i);
  }
  // destination row: (b, h, prev + l) of the (B, KVH, cap, .) buffers
  const long long bh = row / p.L;
  const int l = int(row % p.L);
  const long long drow = bh * p.cap + p.prev + l;
  p.words[which][drow * (p.D / 4) + g * 16 + sub] = word;
  if (sub == 0) {
    store_from_f32(p.scales[which], drow * groups_per_row + g, scale, p.dt);
    store_from_f32(p.biases[which], drow * groups_per_row + g, bias, p.dt);
  }
}

struct DequantParams {
  const uint32_t* words;
  const void* scales;
  const void* biases;
  void* out;
  long long rows;  // rows of D values (words rows)
  int D, sdt, odt;
};

__global__ __launch_bounds__(256) void dequantize_rows(DequantParams p) {
  const long long wid = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;  // word index
  const int wpr = p.D / 4;
  if (wid >= p.rows * wpr) return;
  const long long row = wid / wpr;
  const int w = int(wid % wpr);
  const int g = w / 16;
  const uint32_t x = p.words[wid];
  const float s = load_as_f32(p.scales, row * (p.D / 64) + g, p.sdt);
  const float b = load_as_f32(p.biases, row * (p.D / 64) + g, p.sdt);
  store4_from_f32(p.out, row * p.D + 4 * w, s * float(x & 0xffu) + b, s * float((x >> 8) & 0xffu) + b,
                  s * float((x >> 16) & 0xffu) + b, s * float(x >> 24) + b, p.odt);
}

// Four words a thread, 256 words apart, so that every load (4 bytes a lane) and every store (4 values a lane) of a
// wave is contiguous; a block covers 1024 consecutive words.  Rows of D = 4 << WSH values, so the row and group of a
// word come from shifts.  The same arithmetic as dequantize_rows.
template <int WSH>
__device__ __forceinline__ void dequantize_p2_block(const DequantParams& p) {
  const long long nw = p.rows << WSH;
  const long long w0 = static_cast<long long>(blockIdx.x) * 1024 + threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const long long wid = w0 + 256 * k;
    if (wid >= nw) return;
    const uint32_t x = p.words[wid];
    const long long gi = wid >> 4;  // group of 64 values = 16 words
    const float s = load_as_f32(p.scales, gi, p.sdt);
    const float b = load_as_f32(p.biases, gi, p.sdt);
    store4_from_f32(p.out, wid * 4, s * float(x & 0xffu) + b, s * float((x >> 8) & 0xffu) + b,
                    s * float((x >> 16) & 0xffu) + b, s * float(x >> 24) + b, p.odt);
  }
}
template <int WSH>
__global__ __launch_bounds__(256) void dequantize_rows_p2(DequantParams p) {
  dequantize_p2_block<WSH>(p);
}
// K and V of a cache in one launch: blockIdx.y picks the buffer
struct DequantPair {
  DequantParams d[2];
};
template <int WSH>
__global__ __launch_bounds__(256) void dequantize_pair_p2(DequantPair pp) {
  dequantize_p2_block<WSH>(blockIdx.y ? pp.d[1] : pp.d[0]);
}

// The same pass with 16-byte accesses for 16-bit output and 16-byte aligned buffers: 8 words (32 codes) a thread,
// two 16-byte loads 1 KB apart in its wave's 2 KB run, both issued before either is used (codes streamed from
// HBM keep two requests a lane in flight instead of one), then four 16-byte stores.  The same arithmetic as
// dequantize_rows: one fp32 fused multiply-add a value, rounded once to the output type.
template <int ODT>
__global__ __launch_bounds__(256) void dequantize_pair_x16(DequantPair pp) {
  const DequantParams& p = blockIdx.y ? pp.d[1] : pp.d[0];
  const long long nw = p.rows * 32;  // rows of 128 values: 32 words each
  const long long w0 = static_cast<long long>(blockIdx.x) * 2048 + (threadIdx.x >> 6) * 512 + 4 * (threadIdx.x & 63);
  u4 x[2];
  float s[2], b[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const long long wid = w0 + 256 * h;
    const bool in = wid < nw;  // nw and wid are multiples of 4: a lane's 4 words are all in or all out
    x[h] = in ? __builtin_nontemporal_load(reinterpret_cast<const u4*>(p.words + wid)) : u4{0u, 0u, 0u, 0u};
    s[h] = in ? load_as_f32(p.scales, size_t(wid >> 4), p.sdt) : 0.0f;
    b[h] = in ? load_as_f32(p.biases, size_t(wid >> 4), p.sdt) : 0.0f;
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const long long wid = w0 + 256 * h;
    if (wid >= nw) continue;
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t w = x[h][j];
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = s[h] * float((w >> (8 * i)) & 0xffu) + b[h];
      if constexpr (ODT == DT_BF16) {
        o[2 * j] = f32_to_bf16_bits(v[0]) | (uint32_t(f32_to_bf16_bits(v[1])) << 16);
        o[2 * j + 1] = f32_to_bf16_bits(v[2]) | (uint32_t(f32_to_bf16_bits(v[3])) << 16);
      } else {
        o[2 * j] = __builtin_bit_cast(uint16_t, _Float16(v[0])) |
                   (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[1]))) << 16);
        o[2 * j + 1] = __builtin_bit_cast(uint16_t, _Float16(v[2])) |
                       (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[3]))) << 16);
      }
    }
    u4* dst = reinterpret_cast<u4*>(static_cast<uint16_t*>(p.out) + wid * 4);
    dst[0] = u4{o[0], o[1], o[2], o[3]};
    dst[1] = u4{o[4], o[5], o[6], o[7]};
  }
}

// K and V (rows of 128 values each) of an 8-bit cache dequantized to 16 bits in one launch.  Declared in
// lcl_common.h for the masked-attention entry point; 0 or a hipError_t.
int dequantize_kv128(const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw, const void* vs,
                     const void* vb, int sdt, long long rows, void* kout, void* vout, hipStream_t stream) {
  DequantPair pp{{{kw, ks, kb, kout, rows, 128, sdt, sdt}, {vw, vs, vb, vout, rows, 128, sdt, sdt}}};
  const auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  if (a16(kw) && a16(vw) && a16(kout) && a16(vout) && (sdt == DT_F16 || sdt == DT_BF16)) {
    const long long blocks = (rows * 32 + 2047) / 2048;
    if (blocks > 0x7fffffffLL) return int(hipErrorInvalidValue);
    if (sdt == DT_BF16)
      hipLaunchKernelGGL(dequantize_pair_x16<DT_BF16>, dim3(static_cast<unsigned>(blocks), 2), dim3(256), 0, stream,
                         pp);
    else
      hipLaunchKernelGGL(dequantize_pair_x16<DT_F16>, dim3(static_cast<unsigned>(blocks), 2), dim3(256), 0, stream,
                         pp);
    return int(hipGetLastError());
  }
  const long long blocks = (rows * 32 + 1023) / 1024;
  if (blocks > 0x7fffffffLL) return int(hipErrorInvalidValue);
  hipLaunchKernelGGL(dequantize_pair_p2<5>, dim3(static_cast<unsigned>(blocks), 2), dim3(256), 0, stream, pp);
  return int(hipGetLastError());
}

}  // namespace lcl

using namespace lcl;

extern "C" {

int lcl_quantize_append(const void* k, const void* v, int dt, uint32_t* kw, void* ks, void* kb, uint32_t* vw,
                        void* vs, void* vb, int B, int KVH, int L, int D, int cap, int prev, int round_mode,
                        void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!k || !kw || !ks || !kb) return -1;
  if (v && (!vw || !vs || !vb)) return -1;
  if (dt != DT_F16 && dt != DT_BF16) return -1;
  if (B < 0 || KVH <= 0 || L < 0 || D <= 0 || D % 64 || cap <= 0 || prev < 0 || prev + L > cap) return -1;
  if (round_mode != 0 && round_mode != 1) return -1;
  if (B == 0 || L == 0) return 0;
  QuantParams p{};
  p.src[0] = k; p.src[1] = v;
  p.words[0] = kw; p.words[1] = vw;
  p.scales[0] = ks; p.scales[1] = vs;
  p.biases[0] = kb; p.biases[1] = vb;
  p.rows = static_cast<long long>(B) * KVH * L;
  p.L = L; p.D = D; p.cap = cap; p.prev = prev; p.dt = dt; p.round_even = round_mode;
  const long long groups = p.rows * (D / 64);
  const long long blocks = (groups * 16 + 255) / 256;
  if (blocks > 0x7fffffffLL) return -2;
  hipLaunchKernelGGL(quantize_append, dim3(unsigned(blocks), 2), dim3(256), 0, stream, p);
  return int(hipGetLastError());
}

int lcl_dequantize(const uint32_t* words, const void* scales, const void* biases, int sdt, long long rows, int D,
                   void* out, int odt, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!words || !scales || !biases || !out) return -1;
  if (rows < 0 || D <= 0 || D % 64) return -1;
  if ((sdt != DT_F16 && sdt != DT_BF16) || (odt != DT_F16 && odt != DT_BF16 && odt != DT_F32)) return -1;
  if (rows == 0) return 0;
  DequantParams p{words, scales, biases, out, rows, D, sdt, odt};
  if (D == 64 || D == 128 || D == 256 || D == 512) {
    const long long blocks = (rows * (D / 4) + 1023) / 1024;
    if (blocks > 0x7fffffffLL) return -2;
    const dim3 grid = dim3(static_cast<unsigned>(blocks));
    if (D == 64) hipLaunchKernelGGL(dequantize_rows_p2<4>, grid, dim3(256), 0, stream, p);
    else if (D == 128) hipLaunchKernelGGL(dequantize_rows_p2<5>, grid, dim3(256), 0, stream, p);
    else if (D == 256) hipLaunchKernelGGL(dequantize_rows_p2<6>, grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(dequantize_rows_p2<7>, grid, dim3(256), 0, stream, p);
    return int(hipGetLastError());
  }
  const long long blocks = (rows * (D / 4) + 255) / 256;
  if (blocks > 0x7fffffffLL) return -2;
  hipLaunchKernelGGL(dequantize_rows, dim3(unsigned(blocks)), dim3(256), 0, stream, p);
  return int(hipGetLastError());
}

}  // extern "C"
