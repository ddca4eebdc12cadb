// Multi-query masked attention over 8-bit affine or 16-bit KV, split-K, on MFMA.
//
// Reference behaviour: the chunked-prefill, span and tree-verification variants, all
// MLX scaled_dot_product_attention(q, k, v, scale, mask, sinks) in the reference:
//  * qkv.attention's L > 1 branch: attend_few(q, dequantized(K), dequantized(V), ...)
//    (locals/qkv.py:270-272, locals/fuse.py:131-144), "causal" aligning the last query
//    with the last key (query i of L sees key j of N iff j <= N - L + i);
//  * tree verification: prefix visible to every new token, ancestor-only within the
//    new tokens (locals/treedec.py:56-79, locals/packed.py:107-116,161-182);
//  * any boolean array mask (locals/fuse.py:139, tests/test_flint.py:534-552);
//  * the sink is a logit in the denominator only.
//
// MI355X design.  Grid (key chunk, row block, row x kv head); a workgroup = 4 waves =
// 64 rows, a row being one (query, head) of the kv head's G heads (row r: query r / G,
// head r % G, so any G works).  Per 64-key tile the workgroup dequantizes K and V once
// into LDS as MFMA operands (fp32 scale * code + bias, rounded once to the MFMA type,
// as the reference's dequantized() feeds its attention in T) -- K row-major and V
// transposed, rows padded so the operand reads are bank-conflict free -- and every wave
// reuses the tile for its 16 rows:
//  * S^T = K Q^T on v_mfma_f32_16x16x16 (A = 16 keys x 16 dims from LDS, B = Q^T from
//    registers): lane l gets S[row l % 16][keys 4 (l / 16) + i] -- the softmax state of
//    a row lives in one lane column, its max needs two cross-lane steps;
//  * O^T = V^T P^T (A = V^T 16 dims x 16 keys from LDS, B = P^T in the S^T registers):
//    lane l holds O[row l % 16][dims 4 (l / 16) + i], so rescaling O is lane-local.
//  P is rounded to the MFMA type, as MLX's attention does; accumulation is fp32.
//  A partial (m, l, o[128]) per (row, chunk) goes to the workspace; sdpa_combine joins
//  the chunks with the sink.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "lcl_common.h"
#include "locals_amd.h"

namespace lcl {

constexpr int kD = 128;
constexpr int kKT = 64;                 // keys a tile
constexpr int kKsStride = 136;          // halves a K row in LDS (272 B: 16 B aligned, 4-bank skew a row)
constexpr int kVtStride = 72;           // halves a V^T row in LDS (144 B: 36-bank skew a row)
constexpr float kThr = 6.0f;

enum MaskKind { MK_NONE = 0, MK_CAUSAL = 1, MK_TREE = 2, MK_DENSE = 3 };
enum KvFmt { KV_Q8 = 0, KV_16 = 1 };

struct SdpaParams {
  const void* q;  // (B, H, L, 128), dtype qdt
  const uint32_t* kw;
  const void* ks;
  const void* kb;
  const uint32_t* vw;
  const void* vs;
  const void* vb;
  const void* kf;  // 16-bit K/V (B, KVH, cap, 128)
  const void* vf;
  const int32_t* start;  // (B,) first key of each row, or null
  const unsigned long long* tree;  // (B or 1, L) bit j: the query sees key N - L + j
  const uint8_t* dense;            // dense mask, element (b, h, i, j) at b*msb + h*msh + i*msq + j*msk
  long long msb, msh, msq, msk;
  long long tree_bs;               // L (one mask a row) or 0 (shared)
  const float* sinks;              // (H,), natural log units, or null
  float* pm;
  float* pl;
  float* po;
  float scale_log2;
  int B, H, KVH, G, L, N, cap, nchunks, chunk, nrowblocks, mask;
};

template <int MT>
__device__ __forceinline__ uint16_t to_mt(float x) {
  if constexpr (MT == DT_BF16) return f32_to_bf16_bits(x);
  else return __builtin_bit_cast(uint16_t, _Float16(x));
}

template <int MT>
__device__ __forceinline__ f4 mma(uint2 a, uint2 b, f4 c) {
  if constexpr (MT == DT_BF16) return mfma16bf(pack_s4(a.x, a.y), pack_s4(b.x, b.y), c);
  else return mfma16(pack_h4(a.x, a.y), pack_h4(b.x, b.y), c);
}

template <int DT>
__device__ __forceinline__ float ldv(const void* p, size_t i) {
  if constexpr (DT == DT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == DT_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// key j visible to query i of batch row b and head h (inside the chunk's key range)
__device__ __forceinline__ bool visible(const SdpaParams& p, int b, int h, int i, int j) {
  if (p.mask == MK_CAUSAL) return j <= p.N - p.L + i;
  if (p.mask == MK_TREE) {
    const int d = j - (p.N - p.L);
    if (d < 0) return true;
    return (p.tree[b * p.tree_bs + i] >> d) & 1ull;
  }
  if (p.mask == MK_DENSE) return p.dense[b * p.msb + h * p.msh + i * p.msq + j * p.msk] != 0;
  return true;
}

// One workgroup: rows [64 rb, 64 rb + 64) of (batch row b, kv head kvh), keys of chunk c.
// QDT: dtype of q; SDT: dtype of the scales/biases (8-bit) or of K/V (16-bit); MT: MFMA type.
template <int QDT, int SDT, int FMT, int MT>
__global__ __launch_bounds__(256) void sdpa_pass1(SdpaParams p) {
  const int c = blockIdx.x, rb = blockIdx.y;
  const int b = blockIdx.z / p.KVH, kvh = blockIdx.z % p.KVH;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int R = p.L * p.G;
  const int row0 = 64 * rb;
  const int wrow = row0 + 16 * wave + c16;  // this lane's row in the S^T / O^T layouts
  const bool real = wrow < R;
  const int qi = real ? wrow / p.G : 0, g = real ? wrow % p.G : 0;
  const int head = kvh * p.G + g;
  // keys of this chunk any row of the workgroup may see
  const int last_q = min(R - 1, row0 + 63) / p.G;
  int klo = max(p.start ? max(p.start[b], 0) : 0, c * p.chunk);
  int khi = min(p.N, (c + 1) * p.chunk);
  if (p.mask == MK_CAUSAL) khi = min(khi, p.N - p.L + last_q + 1);
  const size_t part_base = (size_t(b) * p.H + head) * p.L + qi;  // (b, h, i) row of the partials
  if (klo >= khi) {  // uniform: nothing here; rows record an empty part
    if (real && q4 == 0) {
      p.pm[part_base * p.nchunks + c] = -INFINITY;
      p.pl[part_base * p.nchunks + c] = 0.0f;
    }
    return;
  }

  __shared__ __attribute__((aligned(16))) uint16_t Ks[kKT * kKsStride];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * kVtStride];

  // Q^T as B operands: qb[kk] = q[row c16][16 kk + 4 q4 + i]
  uint2 qb[8];
  {
    const size_t qrow = ((size_t(b) * p.H + head) * p.L + qi) * kD;
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
      uint16_t t[4];
#pragma unroll
      for (int i = 0; i < 4; i++) t[i] = to_mt<MT>(real ? ldv<QDT>(p.q, qrow + 16 * kk + 4 * q4 + i) : 0.0f);
      qb[kk] = make_uint2(t[0] | (uint32_t(t[1]) << 16), t[2] | (uint32_t(t[3]) << 16));
    }
  }

  const size_t tok0 = (size_t(b) * p.KVH + kvh) * p.cap;
  const int qlim = p.N - p.L + qi;  // causal bound of this lane's row
  const int slo = p.start ? max(p.start[b], 0) : 0;

  float m_run = -INFINITY, l_acc = 0.0f;
  f4 O[8];
#pragma unroll
  for (int dd = 0; dd < 8; dd++) O[dd] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int t0 = klo & ~(kKT - 1); t0 < khi; t0 += kKT) {
    // ---- dequantize / stage the tile: K row-major, V transposed; keys outside [klo, khi) are 0
    {
      const int key = tid >> 2, part = tid & 3;  // K: one key, 32 dims
      const int kg = t0 + key;
      const bool kin = kg >= klo && kg < khi;
      const size_t row = tok0 + min(kg, p.cap - 1);
      uint32_t outw[16];
      if constexpr (FMT == KV_Q8) {
        const uint4 c0 = *reinterpret_cast<const uint4*>(p.kw + row * 32 + part * 8);
        const uint4 c1 = *reinterpret_cast<const uint4*>(p.kw + row * 32 + part * 8 + 4);
        const float sc = ldv<SDT>(p.ks, row * 2 + (part >> 1)), bi = ldv<SDT>(p.kb, row * 2 + (part >> 1));
        const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
        for (int w = 0; w < 8; w++) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; i++) v[i] = kin ? sc * float((cw[w] >> (8 * i)) & 0xffu) + bi : 0.0f;
          outw[2 * w] = to_mt<MT>(v[0]) | (uint32_t(to_mt<MT>(v[1])) << 16);
          outw[2 * w + 1] = to_mt<MT>(v[2]) | (uint32_t(to_mt<MT>(v[3])) << 16);
        }
      } else {
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.kf) + row * kD + part * 32);
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const uint4 x = src[u];
          outw[4 * u] = kin ? x.x : 0u;
          outw[4 * u + 1] = kin ? x.y : 0u;
          outw[4 * u + 2] = kin ? x.z : 0u;
          outw[4 * u + 3] = kin ? x.w : 0u;
        }
      }
      uint4* dst = reinterpret_cast<uint4*>(Ks + key * kKsStride + part * 32);
#pragma unroll
      for (int u = 0; u < 4; u++) dst[u] = make_uint4(outw[4 * u], outw[4 * u + 1], outw[4 * u + 2], outw[4 * u + 3]);
    }
    {
      const int kq = tid >> 4, dq = tid & 15;  // V: keys 4 kq .. 4 kq + 3, dims 8 dq .. 8 dq + 7
      uint16_t v16[4][8];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int kg = t0 + 4 * kq + k;
        const bool kin = kg >= klo && kg < khi;
        const size_t row = tok0 + min(kg, p.cap - 1);
        if constexpr (FMT == KV_Q8) {
          const uint2 cw = *reinterpret_cast<const uint2*>(p.vw + row * 32 + dq * 2);
          const float sc = ldv<SDT>(p.vs, row * 2 + (dq >> 3)), bi = ldv<SDT>(p.vb, row * 2 + (dq >> 3));
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const uint32_t w = e < 4 ? cw.x : cw.y;
            v16[k][e] = to_mt<MT>(kin ? sc * float((w >> (8 * (e & 3))) & 0xffu) + bi : 0.0f);
          }
        } else {
          const uint4 x = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.vf) + row * kD + dq * 8);
          const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
          for (int e = 0; e < 8; e++) v16[k][e] = kin ? uint16_t((xw[e >> 1] >> (16 * (e & 1))) & 0xffffu) : 0;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        uint2* dst = reinterpret_cast<uint2*>(Vt + (8 * dq + e) * kVtStride + 4 * kq);
        *dst = make_uint2(v16[0][e] | (uint32_t(v16[1][e]) << 16), v16[2][e] | (uint32_t(v16[3][e]) << 16));
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for this wave's 16 rows: st[t][i] = S[row c16][key t0 + 16 t + 4 q4 + i]
    f4 st[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      f4 a = f4{0.0f, 0.0f, 0.0f, 0.0f};
      const uint16_t* krow = Ks + (16 * t + c16) * kKsStride + 4 * q4;
#pragma unroll
      for (int kk = 0; kk < 8; kk++) a = mma<MT>(*reinterpret_cast<const uint2*>(krow + 16 * kk), qb[kk], a);
      st[t] = a;
    }
    // ---- mask, base-2 logits, running max
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int j = t0 + 16 * t + 4 * q4 + i;
        bool ok = real && j >= klo && j < khi && j >= slo;
        if (p.mask == MK_CAUSAL) ok = ok && j <= qlim;
        else if (p.mask != MK_NONE) ok = ok && visible(p, b, head, qi, j);
        const float s = ok ? st[t][i] * p.scale_log2 : -INFINITY;
        st[t][i] = s;
        tmax = fmaxf(tmax, s);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    if (tmax > m_run + kThr) {  // per-lane (row) rescale: O^T rows are lane-local
      const float corr = m_run == -INFINITY ? 0.0f : fast_exp2(m_run - tmax);
      m_run = tmax;
      l_acc *= corr;
#pragma unroll
      for (int dd = 0; dd < 8; dd++) O[dd] *= corr;
    }
    // ---- P (rounded to the MFMA type) and O^T += V^T P^T
    uint2 pb[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pv[i] = st[t][i] == -INFINITY ? 0.0f : fast_exp2(st[t][i] - m_run);
        l_acc += pv[i];
      }
      pb[t] = make_uint2(to_mt<MT>(pv[0]) | (uint32_t(to_mt<MT>(pv[1])) << 16),
                         to_mt<MT>(pv[2]) | (uint32_t(to_mt<MT>(pv[3])) << 16));
    }
#pragma unroll
    for (int dd = 0; dd < 8; dd++) {
      const uint16_t* vrow = Vt + (16 * dd + c16) * kVtStride + 4 * q4;
#pragma unroll
      for (int t = 0; t < 4; t++) O[dd] = mma<MT>(*reinterpret_cast<const uint2*>(vrow + 16 * t), pb[t], O[dd]);
    }
    __syncthreads();
  }

  // ---- the row's part: m, l (summed over the 4 lanes of the row), o[dims]
  l_acc += __shfl_xor(l_acc, 16);
  l_acc += __shfl_xor(l_acc, 32);
  if (!real) return;
  const size_t part = part_base * p.nchunks + c;
  if (q4 == 0) {
    p.pm[part] = m_run;
    p.pl[part] = l_acc;
  }
  if (m_run == -INFINITY) return;
  float4* po4 = reinterpret_cast<float4*>(p.po + part * kD);
#pragma unroll
  for (int dd = 0; dd < 8; dd++) po4[4 * dd + q4] = make_float4(O[dd][0], O[dd][1], O[dd][2], O[dd][3]);
}

// Join the chunks of each (b, h, i) row with the head's sink; no key and no sink gives 0.
struct SdpaCombineParams {
  const float* pm;
  const float* pl;
  const float* po;
  const float* sinks;
  void* out;  // (B, H, L, 128), dtype odt
  int rows, H, L, nchunks, odt;
};

__global__ __launch_bounds__(256) void sdpa_combine(SdpaCombineParams p) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= p.rows) return;
  const int head = (row / p.L) % p.H;
  const size_t base = size_t(row) * p.nchunks;
  const float sink = p.sinks ? p.sinks[head] * kLog2e : -INFINITY;
  float M = sink;
  for (int c = 0; c < p.nchunks; c++) M = fmaxf(M, p.pm[base + c]);
  float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
  if (M != -INFINITY) {
    L = sink == -INFINITY ? 0.0f : fast_exp2(sink - M);
    for (int c = 0; c < p.nchunks; c++) {
      const float mc = p.pm[base + c];
      if (!(mc > -INFINITY)) continue;
      const float w = fast_exp2(mc - M);
      L += w * p.pl[base + c];
      const float2 o = reinterpret_cast<const float2*>(p.po + (base + c) * kD)[lane];
      o0 += w * o.x;
      o1 += w * o.y;
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  store_from_f32(p.out, size_t(row) * kD + 2 * lane, o0 * inv, p.odt);
  store_from_f32(p.out, size_t(row) * kD + 2 * lane + 1, o1 * inv, p.odt);
}

template <int QDT, int SDT, int FMT, int MT>
static void launch_t(dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const SdpaParams& p) {
  hipExtLaunchKernelGGL((sdpa_pass1<QDT, SDT, FMT, MT>), grid, dim3(256), 0, s, e0, e1, 0, p);
}

template <int FMT>
static void launch_fmt(int qdt, int sdt, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const SdpaParams& p) {
  // MFMA type: bf16 when the keys/values (or their scales) are bf16, fp16 otherwise
  if (sdt == DT_BF16) {
    if (qdt == DT_F16) launch_t<DT_F16, DT_BF16, FMT, DT_BF16>(grid, s, e0, e1, p);
    else if (qdt == DT_BF16) launch_t<DT_BF16, DT_BF16, FMT, DT_BF16>(grid, s, e0, e1, p);
    else launch_t<DT_F32, DT_BF16, FMT, DT_BF16>(grid, s, e0, e1, p);
  } else {
    if (qdt == DT_F16) launch_t<DT_F16, DT_F16, FMT, DT_F16>(grid, s, e0, e1, p);
    else if (qdt == DT_BF16) launch_t<DT_BF16, DT_F16, FMT, DT_F16>(grid, s, e0, e1, p);
    else launch_t<DT_F32, DT_F16, FMT, DT_F16>(grid, s, e0, e1, p);
  }
}

}  // namespace lcl

using namespace lcl;

static int sdpa_chunk(int block) { return block > 0 ? block : 512; }

extern "C" {

size_t lcl_sdpa_workspace_bytes(int B, int H, int L, int N, int block) {
  const int chunk = sdpa_chunk(block);
  const int nchunks = N > 0 ? (N + chunk - 1) / chunk : 1;
  return size_t(B) * H * L * nchunks * (2 + kD) * sizeof(float);
}

int lcl_sdpa_ex(const void* q, int qdt, int kvfmt, const uint32_t* kw, const void* ks, const void* kb,
                const uint32_t* vw, const void* vs, const void* vb, const void* kf, const void* vf, int kvdt,
                const int32_t* start, int mask_kind, const unsigned long long* tree, long long tree_bs,
                const uint8_t* dense, long long msb, long long msh, long long msq, long long msk, const float* sinks,
                float scale, int B, int H, int KVH, int L, int N, int head_dim, int cap, int block, void* out,
                void* workspace, size_t workspace_bytes, void* stream_, void* ev_start, void* ev_stop) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!q || !out) return -1;
  if (head_dim != kD) return -2;
  if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH || L <= 0 || N < 0 || N > cap || cap <= 0 || L > N + 1000000) return -1;
  if (block < 0 || block % kKT) return -1;
  if (qdt != DT_F16 && qdt != DT_BF16 && qdt != DT_F32) return -1;
  if (kvdt != DT_F16 && kvdt != DT_BF16) return -1;
  if (kvfmt == KV_Q8) {
    if (!kw || !ks || !kb || !vw || !vs || !vb) return -1;
  } else if (kvfmt == KV_16) {
    if (!kf || !vf) return -1;
  } else {
    return -1;
  }
  if (mask_kind < MK_NONE || mask_kind > MK_DENSE) return -1;
  if (mask_kind == MK_CAUSAL && L > N) return -1;
  if (mask_kind == MK_TREE && (!tree || L > 64 || L > N)) return -2;
  if (mask_kind == MK_DENSE && !dense) return -1;
  const int chunk = sdpa_chunk(block);
  const int nchunks = N > 0 ? (N + chunk - 1) / chunk : 1;
  if (!workspace || workspace_bytes < lcl_sdpa_workspace_bytes(B, H, L, N, block)) return -3;
  SdpaParams p{};
  p.q = q;
  p.kw = kw; p.ks = ks; p.kb = kb; p.vw = vw; p.vs = vs; p.vb = vb; p.kf = kf; p.vf = vf;
  p.start = start;
  p.tree = tree; p.tree_bs = tree_bs;
  p.dense = dense; p.msb = msb; p.msh = msh; p.msq = msq; p.msk = msk;
  p.sinks = sinks;
  float* ws = static_cast<float*>(workspace);
  const size_t np = size_t(B) * H * L * nchunks;
  p.pm = ws; p.pl = ws + np; p.po = ws + 2 * np;
  p.scale_log2 = scale * kLog2e;
  p.B = B; p.H = H; p.KVH = KVH; p.G = H / KVH; p.L = L; p.N = N; p.cap = cap;
  p.nchunks = nchunks; p.chunk = chunk; p.mask = mask_kind;
  p.nrowblocks = (L * p.G + 63) / 64;
  hipEvent_t e0 = static_cast<hipEvent_t>(ev_start), e1 = static_cast<hipEvent_t>(ev_stop);
  {  // with no key in reach every workgroup records empty parts, so the combine needs no cleared workspace
    const dim3 grid(nchunks, p.nrowblocks, B * KVH);
    if (kvfmt == KV_Q8) launch_fmt<KV_Q8>(qdt, kvdt, grid, stream, e0, e1, p);
    else launch_fmt<KV_16>(qdt, kvdt, grid, stream, e0, e1, p);
  }
  SdpaCombineParams c{p.pm, p.pl, p.po, sinks, out, B * H * L, H, L, nchunks, qdt};
  hipLaunchKernelGGL(sdpa_combine, dim3((B * H * L + 3) / 4), dim3(256), 0, stream, c);
  return int(hipGetLastError());
}

int lcl_sdpa(const void* q, int qdt, int kvfmt, const uint32_t* kw, const void* ks, const void* kb,
             const uint32_t* vw, const void* vs, const void* vb, const void* kf, const void* vf, int kvdt,
             const int32_t* start, int mask_kind, const unsigned long long* tree, long long tree_bs,
             const uint8_t* dense, long long msb, long long msh, long long msq, long long msk, const float* sinks,
             float scale, int B, int H, int KVH, int L, int N, int head_dim, int cap, int block, void* out,
             void* workspace, size_t workspace_bytes, void* stream) {
  return lcl_sdpa_ex(q, qdt, kvfmt, kw, ks, kb, vw, vs, vb, kf, vf, kvdt, start, mask_kind, tree, tree_bs, dense, msb,
                     msh, msq, msk, sinks, scale, B, H, KVH, L, N, head_dim, cap, block, out, workspace,
                     workspace_bytes, stream, nullptr, nullptr);
}

}  // extern "C"
