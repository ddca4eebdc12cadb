// GQA flash-decode over 8-bit affine KV (MLX layout) and over fp16/bf16 KV, split-K.
//
// Reference behaviour: locals/qkv.py:213-249 (attend: one query a row, keys
// [start[b], n) of whole-buffer (words, scales, biases) triples read in place,
// softmax with a per-head sink, split into key blocks joined by a log-sum-exp
// pass, qkv.py:30-87 and 179-208) and locals/attention.py:200-224
// (ragged_attention: row r reads KV slot slots[r], keys [0, nkeys[r]), no sink,
// 0 for an empty row).
//
// Pass-1 kernels (the host picks one; pass 2, decode_combine, joins their parts):
//  * qkv_pass1_q8_quad (8-bit, G <= 8: BASELINE configs 2-4 and Flint's G = 8): stream-K
//    over all (row, kv head, 64-key tile) work, one wave a workgroup, tiles by direct
//    buffer->LDS loads, Q K^T on the 4x4x4 MFMA so no lane computes a padding head (one
//    or two groups of 4 heads); described where it is defined.
//  * qkv_pass1_q8 (8-bit, G > 8), below.
//  * ragged_pass1_16 (16-bit K/V, ragged rows).
//
// qkv_pass1_q8 (one workgroup = 4 waves = one (row, kv head, head slice, key
// chunk); each wave streams a quarter of the chunk in tiles of 16 keys):
//  * Q K^T on MFMA 16x16x16 f16: A = 16 keys x 16 dims of codes turned into exact
//    fp16 (1024 + code) by one v_perm per two codes, B = Q^T with the G query
//    heads of the kv head in the 16 columns (one key tile is read once for all of
//    them).  Two accumulators, one per 64-dim group, so the per-(key, group)
//    scale and bias apply after the product:
//        s = sum_g sc_g * (acc_g - 1024 Qs_g) + b_g * Qs_g,   Qs_g = sum of q over g.
//  * The score tile comes out of the MFMA as D[key][head]; that is exactly the A
//    layout of the P V product (lane = head, 4 consecutive keys), so P never
//    moves between lanes.  P V on MFMA: A = w = p * vscale (per key and group)
//    split into fp16 hi + lo, both rounded to nearest, B = V codes as 1024 + code,
//    transposed from 4 keys' words by v_perm.  The bias and the 1024 offset go into
//    one fp32 accumulator per (head, group):
//        o_d = sum_t w_t (1024 + c_td) + sum_t (p_t b_t - 1024 w_t).
//  * Online softmax in base 2, lazily rescaled: the running max only moves when
//    a tile's max exceeds it by more than 2^6, so p <= 64; the rescale is a
//    wave-uniform branch taken a handful of times.  p is taken against the max
//    minus a wave-uniform exponent E (lcl_common.h, "prescale"), chosen from the
//    largest V scale seen so that w < 2^15: the weights that matter then have a
//    normal fp16 hi and lo (relative error 2^-22), where at E = 0 small weights
//    would lose their lo half to fp16 subnormals, a loss the (1024 + code) factor
//    multiplies.  l, o and the side sums carry the same 2^E.
//  * The 4 waves' partials are joined in LDS into one (m, l, o[128]) per (row,
//    head, chunk); pass 2 joins the chunks with the sink.
// Loads: per 16-key tile a lane issues 2 x 128-bit loads of K codes, 8 x 32-bit
// loads of V codes (4 keys x 2 groups) and 4 x 128-bit loads of the four keys'
// scale/bias pairs; the next tile's loads are in flight while a tile computes.

#include <hip/hip_ext.h>

#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <type_traits>

#include "lcl_common.h"
#include "locals_amd.h"

namespace lcl {

constexpr int kHD = 128;
constexpr int kWaves = 4;
constexpr float kRescaleThr = 6.0f;

struct DecodeParams {
  const void* q;       // (R, H, HD), dtype qdt
  const uint32_t* kw;  // 8-bit: (rows, KVH, cap, 32) words
  const void* ks;
  const void* kb;      // 8-bit: (rows, KVH, cap, 2) scales / biases, dtype sdt
  const uint32_t* vw;
  const void* vs;
  const void* vb;
  const void* kf;      // 16-bit KV: (rows, KVH, cap, HD), dtype sdt
  const void* vf;
  const int32_t* start;  // (R,) first key of each row, or null
  const int32_t* slots;  // (R,) KV row of each query row, or null (row r -> r)
  const int32_t* nkeys;  // (R,) end of each row, or null (n)
  float* pm;
  float* pl;
  float* po;
  int32_t* qparts;  // quad pass 1: parts of each (row, kv head) stream, written by the wave holding its first tile
  int n, cap, H, KVH, G, nslices, nchunks, chunk;
  int kv_rows;  // rows of the KV buffers (B, or n_slots); a slot outside is clamped
  int R;        // query rows
  int qwaves, qmint;  // quad pass 1: waves launched, least tiles a wave
  int qwa, qwb, qya, qyb, qold;  // quad pass 1: split weights (see quad_prefix)
  float scale_log2;
  const float* scale_dev;  // if set, the scale is read from device memory (times log2 e in the kernel)
  int qdt, sdt;
};

struct CombineParams {
  const float* pm;
  const float* pl;
  const float* po;
  const float* sinks;  // (H,) natural-log units, or null
  void* out;           // (R, H, HD), dtype odt
  const int32_t* start;
  const int32_t* nkeys;
  int n, cap, H, nchunks, chunk, odt;
  int quad, R, KVH, G;  // quad: parts are the stream-K slots of the quad pass 1, counted in qparts
  const int32_t* qparts;
};

__device__ __forceinline__ void row_range(const int32_t* start, const int32_t* nkeys, int n, int cap, int r, int& lo,
                                          int& hi) {
  lo = start ? max(start[r], 0) : 0;
  hi = nkeys ? min(max(nkeys[r], 0), cap) : n;
}

// Join the 4 waves' (m, l, o[128]) of each head of the slice into one part per
// (row, head, chunk) of the split-K workspace.
__device__ __forceinline__ void join_waves(const DecodeParams& p, const float (&s_m)[kWaves][16],
                                           const float (&s_l)[kWaves][16], const float (&s_o)[kWaves][16][kHD],
                                           int Gs, int r, int head0, int c) {
  for (int e = threadIdx.x; e < Gs * kHD; e += 256) {
    const int h = e >> 7, d = e & (kHD - 1);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, s_m[w][h]);
    float L = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float f = s_m[w][h] == -INFINITY ? 0.0f : fast_exp2(s_m[w][h] - M);
      L += f * s_l[w][h];
      o += f * s_o[w][h][d];
    }
    const size_t part = (size_t(r) * p.H + head0 + h) * p.nchunks + c;
    p.po[part * kHD + d] = o;
    if (d == 0) {
      p.pm[part] = M;
      p.pl[part] = L;
    }
  }
}

template <int DT>
__device__ __forceinline__ float ld16(const void* p, size_t i) {
  if constexpr (DT == DT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == DT_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// elements i .. i + N - 1 (N a multiple of 8) of dtype DT as fp32, loaded unconditionally (the compiler turns the
// runs into 16-byte loads; gfx950 takes unaligned ones)
template <int DT, int N>
__device__ __forceinline__ void ldn(const void* p, size_t i, float (&v)[N]) {
#pragma unroll
  for (int j = 0; j < N; j++) v[j] = ld16<DT>(p, i + j);
}

template <int DT>
__device__ __forceinline__ float hpart(uint32_t w, int k) {
  const uint16_t b = uint16_t(k ? (w >> 16) : (w & 0xffffu));
  return DT == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// One 16-key tile of 8-bit K/V as a lane holds it:
//  ka, kc  K codes of key (tb + c16), dims [16 q4, +16) and [64 + 16 q4, +16)
//  sc[j][k] for keys tb + 4 q4 + k: j = 0 K scales, 1 K biases, 2 V scales, 3 V biases (a 16-bit pair a key)
//  vd[2k + g] V codes of key tb + 4 q4 + k, dims [64 g + 4 c16, +4)
struct TileQ8 {
  u4 ka, kc;
  u4 sc[4];
  uint32_t vd[8];
};

// ---------------------------------------------------------------- 8-bit pass 1
// Loads are raw buffer loads: one descriptor per array of this (row, kv head), a per-lane
// offset fixed for the whole loop plus the tile's, so a tile's addressing is 3 VALU adds,
// and keys past the capacity read 0 (they are masked).  Tiles wholly inside the wave's
// key range take a path without masking.
// 3 waves a SIMD (<= 168 VGPRs): with one tile in flight per wave that keeps ~50 KB of
// loads in flight per CU.
template <int QDT, int SDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void qkv_pass1_q8(DecodeParams p) {
  const int c = blockIdx.x;
  const int kvh = blockIdx.y / p.nslices, sl = blockIdx.y % p.nslices;
  const int r = blockIdx.z;
  int lo, hi;
  row_range(p.start, p.nkeys, p.n, p.cap, r, lo, hi);
  const int c0 = c * p.chunk;
  if (max(lo, c0) >= min(hi, c0 + p.chunk)) return;  // uniform: no key of this row in this chunk

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int sub = p.chunk / kWaves;
  const int wlo = c0 + wave * sub, whi = c0 + (wave + 1) * sub;
  const int tlo = max(lo, wlo), thi = min(hi, whi);
  const int Gs = min(16, p.G - sl * 16);
  const int head0 = kvh * p.G + sl * 16;
  const int slot = p.slots ? min(max(p.slots[r], 0), p.kv_rows - 1) : r;
  const size_t tok0 = (size_t(slot) * p.KVH + kvh) * p.cap;
  const int cap = p.cap;
  const BufRsrc rk = make_rsrc(p.kw + tok0 * 32, uint32_t(cap) * 128u);
  const BufRsrc rv = make_rsrc(p.vw + tok0 * 32, uint32_t(cap) * 128u);
  const BufRsrc rks = make_rsrc(static_cast<const uint32_t*>(p.ks) + tok0, uint32_t(cap) * 4u);
  const BufRsrc rkb = make_rsrc(static_cast<const uint32_t*>(p.kb) + tok0, uint32_t(cap) * 4u);
  const BufRsrc rvs = make_rsrc(static_cast<const uint32_t*>(p.vs) + tok0, uint32_t(cap) * 4u);
  const BufRsrc rvb = make_rsrc(static_cast<const uint32_t*>(p.vb) + tok0, uint32_t(cap) * 4u);
  const uint32_t offK = uint32_t(c16) * 128u + 16u * q4;  // + tb * 128
  const uint32_t offS = 16u * q4;                          // + tb * 4
  const uint32_t offV = uint32_t(q4) * 512u + 4u * c16;    // + tb * 128

  auto load = [&](int tb, TileQ8& T) {
    const uint32_t k = uint32_t(tb) * 128u, s4 = uint32_t(tb) * 4u;
    T.ka = buf_load_b128(rk, offK + k, 0);
    T.kc = buf_load_b128(rk, offK + k, 64);
    T.sc[0] = buf_load_b128(rks, offS + s4, 0);
    T.sc[1] = buf_load_b128(rkb, offS + s4, 0);
    T.sc[2] = buf_load_b128(rvs, offS + s4, 0);
    T.sc[3] = buf_load_b128(rvb, offS + s4, 0);
    const uint32_t v = offV + k;
    T.vd[0] = buf_load_b32(rv, v, 0);
    T.vd[1] = buf_load_b32(rv, v, 64);
    T.vd[2] = buf_load_b32(rv, v, 128);
    T.vd[3] = buf_load_b32(rv, v, 192);
    T.vd[4] = buf_load_b32(rv, v, 256);
    T.vd[5] = buf_load_b32(rv, v, 320);
    T.vd[6] = buf_load_b32(rv, v, 384);
    T.vd[7] = buf_load_b32(rv, v, 448);
  };

  // the first tile's loads go out before the query is read, so their latency overlaps the prologue
  TileQ8 A, B;  // ping-pong: the tile in flight is never copied, so no wait is forced on it
  const int tb0 = tlo & ~15, tbl = (thi - 1) & ~15;
  if (tlo < thi) load(tb0, A);

  // B operands of Q K^T: qb[4g + jj] = q[head c16][64g + 16q4 + 4jj + i]
  h4 qb[8];
  float qs0 = 0.0f, qs1 = 0.0f;
  {
    const bool real = c16 < Gs;
    const size_t qrow = (size_t(r) * p.H + head0 + (real ? c16 : 0)) * kHD;
    float qv0[16], qv1[16];  // dims 16 q4 .. + 15 and 64 + 16 q4 .. + 15 of the lane's head
    ldn<QDT, 16>(p.q, qrow + 16 * q4, qv0);
    ldn<QDT, 16>(p.q, qrow + 64 + 16 * q4, qv1);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      _Float16 t[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        t[i] = _Float16(real ? (j < 4 ? qv0[4 * j + i] : qv1[4 * (j - 4) + i]) : 0.0f);
        (j < 4 ? qs0 : qs1) += float(t[i]);
      }
      qb[j] = h4{t[0], t[1], t[2], t[3]};
    }
  }
  qs0 += __shfl_xor(qs0, 16);
  qs0 += __shfl_xor(qs0, 32);
  qs1 += __shfl_xor(qs1, 16);
  qs1 += __shfl_xor(qs1, 32);
  // base-2 logits: s = C (sc0 (a0 - 1024 Qs0) + sc1 (a1 - 1024 Qs1) + b0 Qs0 + b1 Qs1), C = scale log2 e
  const float C = p.scale_log2;
  const float zc0 = 1024.0f * qs0 * C, zc1 = 1024.0f * qs1 * C, qc0 = qs0 * C, qc1 = qs1 * C;

  // lazy running max, the reference the weights are taken against (m_run - pE), sums; pE is the wave-uniform
  // prescale exponent of the V weights (lcl_common.h) and pthr the least V-scale magnitude that needs it lowered
  float m_run = -INFINITY, mref = -INFINITY, l_acc = 0.0f, wb0 = 0.0f, wb1 = 0.0f;
  int pE = kPreInit, pthr = pre_thr<SDT>(kPreInit);
  f4 O[8];
#pragma unroll
  for (int ii = 0; ii < 8; ii++) O[ii] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int tb, const TileQ8& T, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    // ---- S^T = K Q^T, one accumulator per 64-dim group
    f4 a0 = f4{0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
    a0 = mfma16(codes4_to_h4(T.ka.x), qb[0], a0);
    a1 = mfma16(codes4_to_h4(T.kc.x), qb[4], a1);
    a0 = mfma16(codes4_to_h4(T.ka.y), qb[1], a0);
    a1 = mfma16(codes4_to_h4(T.kc.y), qb[5], a1);
    a0 = mfma16(codes4_to_h4(T.ka.z), qb[2], a0);
    a1 = mfma16(codes4_to_h4(T.kc.z), qb[6], a1);
    a0 = mfma16(codes4_to_h4(T.ka.w), qb[3], a0);
    a1 = mfma16(codes4_to_h4(T.kc.w), qb[7], a1);

    // ---- V codes as the B operands of P V (keys tb + 4q4 + k, dims 64g + 4c16 + jj)
    h4 bv[8];
#pragma unroll
    for (int g = 0; g < 2; g++) {
      const uint32_t x01 = __builtin_amdgcn_perm(T.vd[2 + g], T.vd[g], 0x05010400u);
      const uint32_t y01 = __builtin_amdgcn_perm(T.vd[2 + g], T.vd[g], 0x07030602u);
      const uint32_t x23 = __builtin_amdgcn_perm(T.vd[6 + g], T.vd[4 + g], 0x05010400u);
      const uint32_t y23 = __builtin_amdgcn_perm(T.vd[6 + g], T.vd[4 + g], 0x07030602u);
      bv[4 * g + 0] = pack_h4(codes_to_h2(x01, 0x00050004u), codes_to_h2(x23, 0x00050004u));
      bv[4 * g + 1] = pack_h4(codes_to_h2(x01, 0x00070006u), codes_to_h2(x23, 0x00070006u));
      bv[4 * g + 2] = pack_h4(codes_to_h2(y01, 0x00050004u), codes_to_h2(y23, 0x00050004u));
      bv[4 * g + 3] = pack_h4(codes_to_h2(y01, 0x00070006u), codes_to_h2(y23, 0x00070006u));
    }

    // ---- scores of keys tb + 4q4 + i for head c16 (base-2 logits)
    const uint32_t ksc[4] = {T.sc[0].x, T.sc[0].y, T.sc[0].z, T.sc[0].w};
    const uint32_t kbi[4] = {T.sc[1].x, T.sc[1].y, T.sc[1].z, T.sc[1].w};
    const uint32_t vsc[4] = {T.sc[2].x, T.sc[2].y, T.sc[2].z, T.sc[2].w};
    const uint32_t vbi[4] = {T.sc[3].x, T.sc[3].y, T.sc[3].z, T.sc[3].w};
    float s[4];
    bool valid[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float u0 = __builtin_fmaf(a0[i], C, -zc0), u1 = __builtin_fmaf(a1[i], C, -zc1);
      float v = hpart<SDT>(ksc[i], 0) * u0;
      v = __builtin_fmaf(hpart<SDT>(ksc[i], 1), u1, v);
      v = __builtin_fmaf(hpart<SDT>(kbi[i], 0), qc0, v);
      v = __builtin_fmaf(hpart<SDT>(kbi[i], 1), qc1, v);
      if constexpr (MASKED) {
        const int t = tb + 4 * q4 + i;
        valid[i] = t >= tlo && t < thi;
        s[i] = valid[i] ? v : -INFINITY;
      } else {
        valid[i] = true;
        s[i] = v;
      }
    }
    float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const bool need = tmax > m_run + kRescaleThr;
    // largest |V scale| of this lane's valid keys (both groups): a scale at or above pthr needs pE lowered
    uint32_t vmag = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) vmag = mag_max2(vmag, valid[i] ? vsc[i] : 0u);
    vmag = mag_fold(vmag);
    const bool needE = int(vmag) >= pthr;
    if (__any(need || needE)) {
      if (__any(needE)) {  // the tile's largest scale (the lanes of a 16-lane row hold the same keys)
        uint32_t x = vmag;
        x = max(x, uint32_t(__shfl_xor(int(x), 16)));
        x = max(x, uint32_t(__shfl_xor(int(x), 32)));
        pE = min(pE, 9 - scale_exp<SDT>(uint32_t(__builtin_amdgcn_readfirstlane(int(x)))));
        pthr = pre_thr<SDT>(pE);
      }
      if (need) m_run = tmax;
      const float nref = m_run - float(pE);
      const float corr = mref == -INFINITY ? 0.0f : fast_exp2(mref - nref);
      mref = nref;
      l_acc *= corr;
      wb0 *= corr;
      wb1 *= corr;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ci = __shfl(corr, 4 * q4 + i);
#pragma unroll
        for (int ii = 0; ii < 8; ii++) O[ii][i] *= ci;
      }
    }
    float w0[4], w1[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float pr = fast_exp2(s[i] - mref);
      float x0 = pr * hpart<SDT>(vsc[i], 0), x1 = pr * hpart<SDT>(vsc[i], 1);
      float y0 = pr * hpart<SDT>(vbi[i], 0), y1 = pr * hpart<SDT>(vbi[i], 1);
      if constexpr (MASKED) {  // garbage scales of masked keys must not reach the sums (0 * inf)
        pr = valid[i] ? pr : 0.0f;
        x0 = valid[i] ? x0 : 0.0f;
        x1 = valid[i] ? x1 : 0.0f;
        y0 = valid[i] ? y0 : 0.0f;
        y1 = valid[i] ? y1 : 0.0f;
      }
      l_acc += pr;
      w0[i] = x0;
      w1[i] = x1;
      wb0 += __builtin_fmaf(-1024.0f, x0, y0);
      wb1 += __builtin_fmaf(-1024.0f, x1, y1);
    }
    uint32_t h0a, l0a, h0b, l0b, h1a, l1a, h1b, l1b;
    split_h2(w0[0], w0[1], h0a, l0a);
    split_h2(w0[2], w0[3], h0b, l0b);
    split_h2(w1[0], w1[1], h1a, l1a);
    split_h2(w1[2], w1[3], h1b, l1b);
    const h4 A0h = pack_h4(h0a, h0b), A0l = pack_h4(l0a, l0b);
    const h4 A1h = pack_h4(h1a, h1b), A1l = pack_h4(l1a, l1b);

    // ---- O[head][64g + 4c16 + jj] += sum_k w[head][k] (1024 + V[tb + 4q4 + k][...])
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      O[jj] = mfma16(A0h, bv[jj], O[jj]);
      O[4 + jj] = mfma16(A1h, bv[4 + jj], O[4 + jj]);
    }
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      O[jj] = mfma16(A0l, bv[jj], O[jj]);
      O[4 + jj] = mfma16(A1l, bv[4 + jj], O[4 + jj]);
    }
  };

  if (tlo < thi) {
    for (int tb = tb0;;) {
      load(min(tb + 16, tbl), B);
      if (tb >= tlo && tb + 16 <= thi) compute(tb, A, std::false_type{});
      else compute(tb, A, std::true_type{});
      tb += 16;
      if (tb > tbl) break;
      load(min(tb + 16, tbl), A);
      if (tb >= tlo && tb + 16 <= thi) compute(tb, B, std::false_type{});
      else compute(tb, B, std::true_type{});
      tb += 16;
      if (tb > tbl) break;
    }
  }

  // ---- join the 4 waves in LDS, one part per (row, head, chunk)
  l_acc += __shfl_xor(l_acc, 16);
  l_acc += __shfl_xor(l_acc, 32);
  wb0 += __shfl_xor(wb0, 16);
  wb0 += __shfl_xor(wb0, 32);
  wb1 += __shfl_xor(wb1, 16);
  wb1 += __shfl_xor(wb1, 32);
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ float s_o[kWaves][16][kHD];
  if (q4 == 0) {
    s_m[wave][c16] = mref;
    s_l[wave][c16] = l_acc;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float b0 = __shfl(wb0, 4 * q4 + i), b1 = __shfl(wb1, 4 * q4 + i);
#pragma unroll
    for (int ii = 0; ii < 8; ii++) s_o[wave][4 * q4 + i][64 * (ii >> 2) + 4 * c16 + (ii & 3)] = O[ii][i] + (ii < 4 ? b0 : b1);
  }
  __syncthreads();
  join_waves(p, s_m, s_l, s_o, Gs, r, head0, c);
}

// ------------------------------------------- 8-bit pass 1 for G <= 8 (quad)
// With 4 or fewer query heads a kv head, 16 head columns of a 16x16 MFMA are mostly
// padding, and so is the softmax work done on them.  This pass 1 computes Q K^T on
// v_mfma_f32_4x4x4_16b_f16 instead: 16 blocks of 4 keys x 4 heads, so a 64-key tile
// fills every lane with real (key, head) scores:
//   lane 4b + m holds A_b[m][0..3] (key row m of block b, 4 dims),
//   lane 4b + n holds B_b[0..3][n] (4 dims of head n) and D_b[0..3][n] (4 keys, head n).
// Block b = 4 q4 + sigma holds tile keys 16 sigma + 4 q4 + m, chosen so that for the
// 16-key sub-tile sigma the P V A operand of lane (head n, q4) -- w of keys
// 16 sigma + 4 q4 + 0..3 -- is exactly what lane 16 q4 + 4 sigma + n computed: one DPP
// row shift by 4 sigma.  P V stays on 16x16x16 MFMA with the V transposition of the
// register kernel (rows of heads >= 4 are discarded).
// Work: a workgroup is one wave owning an equal share of all tiles (the stream-K split
// below) and writing one partial per (row, kv head) it touches.  Each 64-key
// tile (K codes 8 KB, V codes 8 KB, four 256 B scale/bias arrays) arrives by direct
// buffer->LDS loads of whole 128-byte lines (20 instructions) into the wave's LDS
// slot, K half (codes + ks / kb) and V half (codes + vs / vb) in two named arrays; the wave
// copies the K half into registers and sends the next tile's K loads, then does the same
// for the V half, so the next tile is in flight while this one's V half is read and the
// tile computes.  No barrier is needed: a wave only reads what it loaded (vmcnt).  C2
// pass 1 went 102.6 -> 102.3 us and C3 90 -> 89.5 us with the split.  K rows are stored with 16-byte chunk c at slot
// c ^ hk(key) and V rows at c ^ hv(key), so the 128-bit K reads and the 32-bit V reads
// are free of bank conflicts.
// Two head groups (HG = 2, 5 <= G <= 8): the K fragments of a tile feed a second set of
// 4x4x4 products against heads 4..7 (the fp16 form of the codes is shared), each group
// keeps its own softmax state, and the P V A operand carries group 0 in rows 0..3 and
// group 1 in rows 4..7 (row_take2), so P V costs no more MFMA than with one group.  The
// 8 heads' q staging raises LDS to 21.5 KB a wave (16-bit q): 7 waves a CU instead of 8.
// Flint's G = 8 over C2's rows: pass 1 74.7 us (16x16 register-fed kernel) -> 62.9 us.
constexpr int kQT = 64;                     // keys a tile
constexpr int kQSlot = 8192 + 8192 + 1024;  // K codes, V codes, ks / kb / vs / vb words

// tile key of QK lane l = 4 b + m (b = 4 q4 + sigma): 16 sigma + 4 q4 + m
__device__ __forceinline__ int quad_key(int l) { return 16 * ((l >> 2) & 3) + 4 * (l >> 4) + (l & 3); }
// 16-byte slot swizzles of tile key t's K and V rows
__device__ __forceinline__ int quad_hk(int t) { return (t & 3) | (((t >> 4) & 1) << 2); }
__device__ __forceinline__ int quad_hv(int t) { return 4 * ((t >> 2) & 1); }

__device__ __forceinline__ f4 mfma4(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0); }

// lane i of each 16-lane row takes lane i + SH of the same row (0 past the row's end)
template <int SH>
__device__ __forceinline__ uint32_t row_take(uint32_t x) {
  if constexpr (SH == 0) return x;
  else return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x100 + SH, 0xf, 0xf, true));
}

// Two head groups in one P V A operand: lanes 0..3 of each 16-lane row take x0 of lane i + 4 SG, lanes 4..7 take
// x1 of lane i + 4 SG - 4 (lanes 8..15 are don't-care).  DPP bank_mask (4-lane banks) writes only one bank over
// an `old` that already holds the other.
template <int SG>
__device__ __forceinline__ uint32_t row_take2(uint32_t x0, uint32_t x1) {
  if constexpr (SG == 0)  // bank 1 <- x1 of lane i - 4 (row_shr:4) over x0
    return uint32_t(__builtin_amdgcn_update_dpp(int(x0), int(x1), 0x114, 0xf, 0x2, false));
  else if constexpr (SG == 1)  // bank 0 <- x0 of lane i + 4 (row_shl:4) over x1
    return uint32_t(__builtin_amdgcn_update_dpp(int(x1), int(x0), 0x104, 0xf, 0x1, false));
  else  // bank 0 <- x0 of lane i + 4 SG over x1 of lane i + 4 SG - 4
    return uint32_t(__builtin_amdgcn_update_dpp(int(row_take<4 * SG - 4>(x1)), int(x0), 0x100 + 4 * SG, 0xf, 0x1,
                                                false));
}

// Stream-K split of the quad pass 1: the (row, kv head, 64-key tile) list in row-major order
// (a row's tiles are the 64-aligned ones overlapping its keys [lo, hi)) is cut into W ranges,
// W <= min(waves launched, total / mint), so every wave gets >= mint tiles and one resident
// round of waves finishes together whatever the row lengths.  The ranges are weighted by how
// fast a wave runs, measured per wave on the MI355X (`s_memrealtime` at entry and exit):
//  * by XCD: one-wave workgroups go to XCD w mod 8 in turn, so even w run on even XCDs and odd w
//    on odd ones, and the odd XCDs' waves took ~10% longer a tile;
//  * by age: the first `old` waves (one a SIMD) are each SIMD's older wave, which the SIMD's
//    issue favours; the younger ones took ~22% longer a tile.
// Weights: even old a, odd old b, even young c, odd young d (SplitW).  A wave writes one partial
// for each (row, kv head) stream its range touches, at slot j = wave - (wave holding the
// stream's first tile); that first wave also records the stream's part count for pass 2.
struct SplitW {
  int a, b, c, d, old;  // old: even
};
__device__ __forceinline__ long long quad_prefix(int w, const SplitW& s) {
  if (w <= s.old) return (long long)((w + 1) / 2) * s.a + (long long)(w / 2) * s.b;
  const int y = w - s.old;
  return (long long)(s.old / 2) * (s.a + s.b) + (long long)((y + 1) / 2) * s.c + (long long)(y / 2) * s.d;
}
// first global tile of wave w
__device__ __forceinline__ long long quad_start(int w, long long T, int W, const SplitW& s) {
  return T * quad_prefix(w, s) / quad_prefix(W, s);
}
// whether every share of W waves under weights s keeps >= mint tiles (floor(T min weight / Q) <= any range's length)
__device__ __forceinline__ bool quad_split_ok(long long T, int W, int mint, const SplitW& s) {
  const int m = W <= s.old ? min(s.a, s.b) : min(min(s.a, s.b), min(s.c, s.d));  // the weights in use
  return T * m >= (long long)mint * quad_prefix(W, s);
}
// wave count W = min(waves launched, T / mint).  The weights stand where the lightest share still gets >= mint tiles;
// else the default 24 : 22 : 20 : 18 (for stronger weights set through LOCALS_AMD_DECODE_XW), if that fits; else every
// wave weighs the same (few tiles a wave: fewer waves would cost more than uneven ones save).  Pass 1 and pass 2 take
// the same decision.
__device__ __forceinline__ int quad_wave_count(long long T, int wlaunch, int mint, SplitW& s) {
  const int W = int(min((long long)wlaunch, max(1LL, T / mint)));
  if (!quad_split_ok(T, W, mint, s)) {
    const SplitW mild{24, 22, 20, 18, s.old};
    s = quad_split_ok(T, W, mint, mild) ? mild : SplitW{1, 1, 1, 1, s.old};
  }
  return W;
}
__device__ __forceinline__ int quad_row_tiles(const int32_t* start, const int32_t* nkeys, int n, int cap, int r,
                                              int& t0, int& lo, int& hi) {
  row_range(start, nkeys, n, cap, r, lo, hi);
  if (hi <= lo) {
    t0 = 0;
    return 0;
  }
  t0 = lo / kQT;
  return (hi + kQT - 1) / kQT - t0;
}

// Lane-parallel scans over the rows (64 a step): the tile counts of rows base + lane.
__device__ __forceinline__ int quad_lane_count(const int32_t* start, const int32_t* nkeys, int n, int cap, int R,
                                               int row) {
  int t0, lo, hi;
  return row < R ? quad_row_tiles(start, nkeys, n, cap, row, t0, lo, hi) : 0;
}

__device__ __forceinline__ int wave_incl_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// total tiles T (all rows x KVH) and the wave count W of the split; with `row` >= 0 also the tiles of the rows
// before it (`before`, in row units)
__device__ __forceinline__ void quad_split(const int32_t* start, const int32_t* nkeys, int n, int cap, int R, int KVH,
                                           int wlaunch, int mint, SplitW& sw, long long& T, int& W, int row,
                                           long long& before) {
  const int lane = threadIdx.x & 63;
  long long t = 0;
  before = 0;
  for (int base = 0; base < R; base += 64) {
    const int c = quad_lane_count(start, nkeys, n, cap, R, base + lane);
    const int incl = wave_incl_scan(c);
    if (row >= base && row < base + 64) before = t + __shfl(incl - c, row - base);
    t += __shfl(incl, 63);
  }
  T = t * KVH;
  W = quad_wave_count(T, wlaunch, mint, sw);
}

// the row holding global tile g (0 <= g < T) and the global index of its first tile
__device__ __forceinline__ int quad_locate(const int32_t* start, const int32_t* nkeys, int n, int cap, int R, int KVH,
                                           long long g, long long& row_first) {
  const int lane = threadIdx.x & 63;
  long long acc = 0;
  for (int base = 0; base < R; base += 64) {
    const int c = quad_lane_count(start, nkeys, n, cap, R, base + lane);
    const int incl = wave_incl_scan(c);
    const long long lo = acc + (long long)(incl - c) * KVH, hi = acc + (long long)incl * KVH;
    const unsigned long long m = __ballot(c > 0 && g >= lo && g < hi);
    if (m) {
      const int l = __ffsll((long long)m) - 1;
      row_first = acc + (long long)__shfl(incl - c, l) * KVH;
      return base + l;
    }
    acc += (long long)__shfl(incl, 63) * KVH;
  }
  row_first = acc;
  return R;  // not reached for g < T
}

// the first row after `row` with tiles (R if none)
__device__ __forceinline__ int quad_next_row(const int32_t* start, const int32_t* nkeys, int n, int cap, int R,
                                             int row) {
  const int lane = threadIdx.x & 63;
  for (int base = row + 1; base < R; base += 64) {
    const unsigned long long m = __ballot(quad_lane_count(start, nkeys, n, cap, R, base + lane) > 0);
    if (m) return base + __ffsll((long long)m) - 1;
  }
  return R;
}

// wave holding global tile g (0 <= g < T): the largest w with quad_start(w) <= g, i.e. with
// quad_prefix(w) <= X = floor(((g + 1) Q - 1) / T); the prefix grows by a, b, a, b, ... up to
// the old waves, then by c, d, c, d, ...
__device__ __forceinline__ int quad_wave_of(long long g, long long T, int W, const SplitW& s) {
  const long long X = ((g + 1) * quad_prefix(W, s) - 1) / T;
  const long long Po = (long long)(s.old / 2) * (s.a + s.b);
  if (X < Po || W <= s.old) {
    const long long k = X / (s.a + s.b);
    return int(2 * k + (X - k * (s.a + s.b) >= s.a ? 1 : 0));
  }
  const long long Y = X - Po, k = Y / (s.c + s.d);
  return int(s.old + 2 * k + (Y - k * (s.c + s.d) >= s.c ? 1 : 0));
}

// a (row, kv head) stream of the quad pass 1
struct QStream {
  int r, kvh, t0, lo, hi, cnt;
  long long Gs;  // global index of its first tile
};

// Values equal in every lane, marked so for the compiler: what comes through a shuffle counts as divergent, and
// buffer descriptors built from divergent values get a loop over their distinct values around every load.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ long long uni(long long x) {
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(x))));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(x) >> 32))));
  return (long long)((uint64_t(hi) << 32) | lo);
}
__device__ __forceinline__ QStream uni(const QStream& S) {
  QStream u;
  u.r = uni(S.r);
  u.kvh = uni(S.kvh);
  u.t0 = uni(S.t0);
  u.lo = uni(S.lo);
  u.hi = uni(S.hi);
  u.cnt = uni(S.cnt);
  u.Gs = uni(S.Gs);
  return u;
}
// its buffer descriptors (built where used, so only one stream's are live at a time)
struct QRsrc {
  BufRsrc rk, rv, rks, rkb, rvs, rvb;
};
__device__ __forceinline__ QRsrc quad_rsrc(const DecodeParams& p, const QStream& S) {
  const int slot = p.slots ? min(max(p.slots[S.r], 0), p.kv_rows - 1) : S.r;
  // the slot comes through a vector load, so the offset is marked uniform here: a descriptor base the compiler
  // takes for divergent puts a readfirstlane loop around every load through it
  const size_t tok0 = size_t(uni((long long)((size_t(slot) * p.KVH + S.kvh) * p.cap)));
  const uint32_t cap = uint32_t(p.cap);
  QRsrc d;
  d.rk = make_rsrc(p.kw + tok0 * 32, cap * 128u);
  d.rv = make_rsrc(p.vw + tok0 * 32, cap * 128u);
  d.rks = make_rsrc(static_cast<const uint32_t*>(p.ks) + tok0, cap * 4u);
  d.rkb = make_rsrc(static_cast<const uint32_t*>(p.kb) + tok0, cap * 4u);
  d.rvs = make_rsrc(static_cast<const uint32_t*>(p.vs) + tok0, cap * 4u);
  d.rvb = make_rsrc(static_cast<const uint32_t*>(p.vb) + tok0, cap * 4u);
  return d;
}
// the G query rows of a stream (rows past G read as 0)
template <int QB>
__device__ __forceinline__ BufRsrc quad_qrsrc(const DecodeParams& p, const QStream& S) {
  const size_t off = size_t(uni((long long)((size_t(S.r) * p.H + size_t(S.kvh) * p.G) * kHD * QB)));
  return make_rsrc(static_cast<const uint8_t*>(p.q) + off, uint32_t(p.G * kHD * QB));
}

template <int QDT, int SDT, int HG>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void qkv_pass1_q8_quad(DecodeParams p) {
  const int wv = blockIdx.x;
  const int lane = threadIdx.x;
  constexpr int QB = QDT == DT_F32 ? 4 : 2;

  // ---- the split and this wave's first stream (one lane-parallel pass over the rows when R <= 64)
  SplitW sw{p.qwa, p.qwb, p.qya, p.qyb, p.qold};
  long long T, g, gend, row_first;
  int W, r0;
  if (p.R <= 64) {
    const int c = quad_lane_count(p.start, p.nkeys, p.n, p.cap, p.R, lane);
    const int incl = wave_incl_scan(c);
    T = uni((long long)__shfl(incl, 63) * p.KVH);
    W = quad_wave_count(T, p.qwaves, p.qmint, sw);
    if (wv >= W) return;
    g = uni(quad_start(wv, T, W, sw));
    gend = uni(quad_start(wv + 1, T, W, sw));
    if (g >= gend) return;
    const long long lo_t = (long long)(incl - c) * p.KVH, hi_t = (long long)incl * p.KVH;
    const unsigned long long m = __ballot(c > 0 && g >= lo_t && g < hi_t);
    r0 = uni(__ffsll((long long)m) - 1);
    row_first = uni((long long)__shfl(incl - c, r0) * p.KVH);
  } else {
    long long unused;
    quad_split(p.start, p.nkeys, p.n, p.cap, p.R, p.KVH, p.qwaves, p.qmint, sw, T, W, -1, unused);
    T = uni(T);
    W = uni(W);
    if (wv >= W) return;
    g = uni(quad_start(wv, T, W, sw));
    gend = uni(quad_start(wv + 1, T, W, sw));
    if (g >= gend) return;
    r0 = uni(quad_locate(p.start, p.nkeys, p.n, p.cap, p.R, p.KVH, g, row_first));
    row_first = uni(row_first);
  }

  const int n = lane & 3;  // QK: head column of this lane
  const int c16 = lane & 15, q4 = lane >> 4;
  const int G = p.G;       // <= 4 * HG

  // the tile slot in two named halves, so that the next tile's K loads can be in flight while V is read here:
  // K codes (8 KB) + ks / kb words, V codes (8 KB) + vs / vb words
  __shared__ __attribute__((aligned(16))) uint8_t qK[kQSlot / 2];
  __shared__ __attribute__((aligned(16))) uint8_t qV[kQSlot / 2];
  __shared__ __attribute__((aligned(16))) uint8_t qraw[4 * HG * kHD * QB];  // the next stream's q as loaded
  __shared__ __attribute__((aligned(16))) _Float16 qh[4 * HG * kHD];          // this stream's q in fp16
  constexpr int kWaitAll = (0xF << 8) | (0x7 << 4);        // s_waitcnt vmcnt(0)
  constexpr int kWaitTen = (0xF << 8) | (0x7 << 4) | 10;    // s_waitcnt vmcnt(10)
  constexpr int kWaitLds = (0x3 << 14) | (0x7 << 4) | 0xF;  // s_waitcnt lgkmcnt(0)

  // DMA lane roles: instruction u moves tile keys 8u + (lane >> 3), lane slot (lane & 7)
  const uint32_t dk_lo = 128u * uint32_t(lane >> 3);
  const uint32_t dk_c0 = 16u * uint32_t((lane & 7) ^ ((lane >> 3) & 3));        // hk for u with bit 1 clear
  const uint32_t dk_c1 = 16u * uint32_t((lane & 7) ^ (((lane >> 3) & 3) | 4));  // hk for u with bit 1 set
  const uint32_t dv_c = 16u * uint32_t((lane & 7) ^ (4 * ((lane >> 5) & 1)));
  const int tk = quad_key(lane);               // QK row key of this lane
  const uint32_t krow = 128u * uint32_t(tk);
  const int hk = quad_hk(tk);
  const int ts0 = quad_key(lane & ~3);         // first of the 4 keys whose scores this lane holds
  // P V B operands: lane (c16, q4) reads V words of keys 16 sigma + 4 q4 + k, dims 64 g + 4 c16 .. + 3
  const uint32_t vcol = 64u * uint32_t(q4 & 1) + 4u * uint32_t(c16);

  // a tile's loads: the K half (10 instructions), then the V half (10)
  auto issue_k = [&](const QRsrc& D, const QStream& S, int k) {
    const uint32_t kt = uint32_t((S.t0 + k) * kQT);
#pragma unroll
    for (int u = 0; u < 8; u++)
      lds_load16(D.rk, qK + 1024 * u, (kt + 8u * u) * 128u + dk_lo + ((u & 2) ? dk_c1 : dk_c0));
    const uint32_t so = (kt + uint32_t(lane)) * 4u;
    lds_load4(D.rks, qK + 8192, so);
    lds_load4(D.rkb, qK + 8192 + 256, so);
  };
  auto issue_v = [&](const QRsrc& D, const QStream& S, int k) {
    const uint32_t kt = uint32_t((S.t0 + k) * kQT);
#pragma unroll
    for (int u = 0; u < 8; u++) lds_load16(D.rv, qV + 1024 * u, (kt + 8u * u) * 128u + dk_lo + dv_c);
    const uint32_t so = (kt + uint32_t(lane)) * 4u;
    lds_load4(D.rvs, qV + 8192, so);
    lds_load4(D.rvb, qV + 8192 + 256, so);
  };
  auto issue = [&](const QRsrc& D, const QStream& S, int k) {
    issue_k(D, S, k);
    issue_v(D, S, k);
  };
  auto issue_q = [&](const QStream& S) {
    const BufRsrc rq = quad_qrsrc<QB>(p, S);
#pragma unroll
    for (int j = 0; j < 2 * QB * HG; j++) lds_load4(rq, qraw + 256 * j, uint32_t(256 * j + 4 * lane));
  };

  // the stream (row r0, kv head) holding tile g
  QStream cur;
  cur.r = r0;
  cur.cnt = quad_row_tiles(p.start, p.nkeys, p.n, p.cap, r0, cur.t0, cur.lo, cur.hi);
  cur.kvh = int((g - row_first) / cur.cnt);
  cur.Gs = row_first + (long long)cur.kvh * cur.cnt;
  cur = uni(cur);
  int k0 = uni(int(g - cur.Gs));
  issue(quad_rsrc(p, cur), cur, k0);
  issue_q(cur);

  for (;;) {
    // the segment: tiles [k0, k1) of stream cur; its first tile and q are in flight
    const long long seg_end = min(gend, cur.Gs + cur.cnt);
    const int k1 = uni(int(seg_end - cur.Gs));
    const bool more = seg_end < gend;
    QStream nxt = cur;  // the next stream (the next kv head, or the next row with keys), when there is one
    if (more) {
      nxt.Gs = cur.Gs + cur.cnt;
      if (++nxt.kvh == p.KVH) {
        nxt.kvh = 0;
        nxt.r = quad_next_row(p.start, p.nkeys, p.n, p.cap, p.R, cur.r);
        nxt.cnt = quad_row_tiles(p.start, p.nkeys, p.n, p.cap, nxt.r, nxt.t0, nxt.lo, nxt.hi);
      }
      nxt = uni(nxt);
    }
    const QRsrc D = quad_rsrc(p, cur);
    const int lo = cur.lo, hi = cur.hi;
    const int head0 = cur.kvh * G;

    __builtin_amdgcn_s_waitcnt(kWaitAll);
    const float C = p.scale_log2;
    // per head group e (heads 4 e .. 4 e + 3): sums of head 4 e + n's fp16 q over dims [0, 64) and [64, 128),
    // scaled
    float zc0[HG], zc1[HG], qc0[HG], qc1[HG];
#pragma unroll
    for (int e = 0; e < HG; e++) {
      // lane l converts elements 8 l .. 8 l + 7 of the group (head 4 e + l / 16, dim group (l / 8) & 1) into qh
      _Float16 t[8];
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        t[i] = _Float16(ld16<QDT>(qraw, size_t(4 * kHD * e + 8 * lane + i)));
        part += float(t[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) qh[4 * kHD * e + 8 * lane + i] = t[i];
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      part += __shfl_xor(part, 4);
      // lane 16 h + 8 g holds the sum of head 4 e + h, dim group g
      float qs0 = 0.0f, qs1 = 0.0f;
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const float g0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 16 * h));
        const float g1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 16 * h + 8));
        qs0 = n == h ? g0 : qs0;
        qs1 = n == h ? g1 : qs1;
      }
      zc0[e] = 1024.0f * qs0 * C;
      zc1[e] = 1024.0f * qs1 * C;
      qc0[e] = qs0 * C;
      qc1[e] = qs1 * C;
    }

    // softmax state of head 4 e + n: lazy running max, the reference the weights are taken against (m - pE), sums;
    // pE is the wave-uniform prescale exponent of the V weights (lcl_common.h) and pthr the least V-scale magnitude
    // that needs it lowered
    float m_run[HG], mref[HG], l_acc[HG], wb0[HG], wb1[HG];
#pragma unroll
    for (int e = 0; e < HG; e++) {
      m_run[e] = mref[e] = -INFINITY;
      l_acc[e] = wb0[e] = wb1[e] = 0.0f;
    }
    int pE = kPreInit, pthr = pre_thr<SDT>(kPreInit);
    f4 O[8];
#pragma unroll
    for (int ii = 0; ii < 8; ii++) O[ii] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // the tile as a lane holds it: K chunks of its QK key, the scale words of its 4 score keys, and for each
    // 16-key sub-tile the V words of keys 16 sigma + 4 q4 + k (dims 64 g + 4 c16 .. + 3) at [sigma][2 k + g]
    struct QuadTile {
      u4 k[8];
      u4 ksc, kbi, vsc, vbi;
      uint32_t v[4][8];
    };
    auto fetch_k = [&](QuadTile& T) {
  #pragma unroll
      for (int cc = 0; cc < 8; cc++) T.k[cc] = *reinterpret_cast<const u4*>(qK + krow + 16 * (cc ^ hk));
      T.ksc = *reinterpret_cast<const u4*>(qK + 8192 + 4 * ts0);
      T.kbi = *reinterpret_cast<const u4*>(qK + 8192 + 256 + 4 * ts0);
    };
    auto fetch_v = [&](QuadTile& T) {
      T.vsc = *reinterpret_cast<const u4*>(qV + 8192 + 4 * ts0);
      T.vbi = *reinterpret_cast<const u4*>(qV + 8192 + 256 + 4 * ts0);
  #pragma unroll
      for (int sg = 0; sg < 4; sg++) {
  #pragma unroll
        for (int k = 0; k < 4; k++) {
          const uint32_t row = 128u * uint32_t(16 * sg + 4 * q4 + k);
          T.v[sg][2 * k + 0] = *reinterpret_cast<const uint32_t*>(qV + row + vcol);
          T.v[sg][2 * k + 1] = *reinterpret_cast<const uint32_t*>(qV + row + (vcol ^ 64u));
        }
      }
    };

    auto compute = [&](int kt, const QuadTile& T) {
      // ---- S^T = K Q^T for each head group, four chains each (dim group = chunk >> 2, chunk parity); the
      // K codes' fp16 form is shared by the groups
      f4 acc[HG][4];
  #pragma unroll
      for (int e = 0; e < HG; e++)
  #pragma unroll
        for (int i = 0; i < 4; i++) acc[e][i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  #pragma unroll
      for (int cc = 0; cc < 8; cc++) {
        const u4 kv = T.k[cc];
        const h4 kx = codes4_to_h4(kv.x), ky = codes4_to_h4(kv.y), kz = codes4_to_h4(kv.z), kw = codes4_to_h4(kv.w);
  #pragma unroll
        for (int e = 0; e < HG; e++) {
          const u4 qa = *reinterpret_cast<const u4*>(qh + kHD * (4 * e + n) + 16 * cc);
          const u4 qc = *reinterpret_cast<const u4*>(qh + kHD * (4 * e + n) + 16 * cc + 8);
          f4& a = acc[e][2 * (cc >> 2) + (cc & 1)];
          a = mfma4(kx, pack_h4(qa.x, qa.y), a);
          a = mfma4(ky, pack_h4(qa.z, qa.w), a);
          a = mfma4(kz, pack_h4(qc.x, qc.y), a);
          a = mfma4(kw, pack_h4(qc.z, qc.w), a);
        }
      }
      const uint32_t kscw[4] = {T.ksc.x, T.ksc.y, T.ksc.z, T.ksc.w}, kbiw[4] = {T.kbi.x, T.kbi.y, T.kbi.z, T.kbi.w};
      const uint32_t vscw[4] = {T.vsc.x, T.vsc.y, T.vsc.z, T.vsc.w}, vbiw[4] = {T.vbi.x, T.vbi.y, T.vbi.z, T.vbi.w};
      // ---- scores of keys ts0 + m for head 4 e + n (base-2 logits)
      const bool full = kt >= lo && kt + kQT <= hi;
      float s[HG][4];
      bool valid[4];
  #pragma unroll
      for (int m = 0; m < 4; m++) {
        const int t = kt + ts0 + m;
        valid[m] = full || (t >= lo && t < hi);
  #pragma unroll
        for (int e = 0; e < HG; e++) {
          const float a0 = acc[e][0][m] + acc[e][1][m], a1 = acc[e][2][m] + acc[e][3][m];
          const float u0 = __builtin_fmaf(a0, C, -zc0[e]), u1 = __builtin_fmaf(a1, C, -zc1[e]);
          float v = hpart<SDT>(kscw[m], 0) * u0;
          v = __builtin_fmaf(hpart<SDT>(kscw[m], 1), u1, v);
          v = __builtin_fmaf(hpart<SDT>(kbiw[m], 0), qc0[e], v);
          v = __builtin_fmaf(hpart<SDT>(kbiw[m], 1), qc1[e], v);
          s[e][m] = valid[m] ? v : -INFINITY;
        }
      }
      // ---- tile max of head 4 e + n over the 16 lanes holding it
      float tmax[HG];
      bool need[HG], any_need = false;
  #pragma unroll
      for (int e = 0; e < HG; e++) {
        float x = fmaxf(fmaxf(s[e][0], s[e][1]), fmaxf(s[e][2], s[e][3]));
        x = fmaxf(x, __shfl_xor(x, 4));
        x = fmaxf(x, __shfl_xor(x, 8));
        x = fmaxf(x, __shfl_xor(x, 16));
        x = fmaxf(x, __shfl_xor(x, 32));
        tmax[e] = x;
        need[e] = x > m_run[e] + kRescaleThr;
        any_need = any_need || need[e];
      }
      // largest |V scale| of this lane's valid keys (both groups): a scale at or above pthr needs pE lowered
      uint32_t vmag = 0;
  #pragma unroll
      for (int m = 0; m < 4; m++) vmag = mag_max2(vmag, valid[m] ? vscw[m] : 0u);
      vmag = mag_fold(vmag);
      const bool needE = int(vmag) >= pthr;
      if (__any(any_need || needE)) {
        if (__any(needE)) {  // the tile's largest scale (lanes 4 b .. 4 b + 3 hold the same keys)
          uint32_t x = vmag;
          x = max(x, uint32_t(__shfl_xor(int(x), 4)));
          x = max(x, uint32_t(__shfl_xor(int(x), 8)));
          x = max(x, uint32_t(__shfl_xor(int(x), 16)));
          x = max(x, uint32_t(__shfl_xor(int(x), 32)));
          pE = min(pE, 9 - scale_exp<SDT>(uint32_t(uni(int(x)))));
          pthr = pre_thr<SDT>(pE);
        }
        float corr[HG];
  #pragma unroll
        for (int e = 0; e < HG; e++) {
          if (need[e]) m_run[e] = tmax[e];
          const float nref = m_run[e] - float(pE);
          corr[e] = mref[e] == -INFINITY ? 0.0f : fast_exp2(mref[e] - nref);
          mref[e] = nref;
          l_acc[e] *= corr[e];
          wb0[e] *= corr[e];
          wb1[e] *= corr[e];
        }
        // P V rows: lane (c16, q4) register i is head 4 q4 + i; head group e lives in lanes 16 e .. 16 e + 15
  #pragma unroll
        for (int i = 0; i < 4; i++) {
          float ci = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr[0]), i));
          if constexpr (HG == 2) {
            const float c1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr[HG - 1]), i));
            ci = q4 == 1 ? c1 : ci;
          }
  #pragma unroll
          for (int ii = 0; ii < 8; ii++) O[ii][i] *= ci;
        }
      }
      // [e][g][pair]: fp16 hi / lo of w_g of head group e for keys m = 0, 1 and 2, 3
      uint32_t wh[HG][4], wl[HG][4];
  #pragma unroll
      for (int e = 0; e < HG; e++) {
        float w0[4], w1[4];
  #pragma unroll
        for (int m = 0; m < 4; m++) {
          float pr = fast_exp2(s[e][m] - mref[e]);
          float x0 = pr * hpart<SDT>(vscw[m], 0), x1 = pr * hpart<SDT>(vscw[m], 1);
          float y0 = pr * hpart<SDT>(vbiw[m], 0), y1 = pr * hpart<SDT>(vbiw[m], 1);
          // garbage scales of keys outside the range must not reach the sums (0 * inf)
          pr = valid[m] ? pr : 0.0f;
          x0 = valid[m] ? x0 : 0.0f;
          x1 = valid[m] ? x1 : 0.0f;
          y0 = valid[m] ? y0 : 0.0f;
          y1 = valid[m] ? y1 : 0.0f;
          l_acc[e] += pr;
          w0[m] = x0;
          w1[m] = x1;
          wb0[e] += __builtin_fmaf(-1024.0f, x0, y0);
          wb1[e] += __builtin_fmaf(-1024.0f, x1, y1);
        }
        split_h2(w0[0], w0[1], wh[e][0], wl[e][0]);
        split_h2(w0[2], w0[3], wh[e][1], wl[e][1]);
        split_h2(w1[0], w1[1], wh[e][2], wl[e][2]);
        split_h2(w1[2], w1[3], wh[e][3], wl[e][3]);
      }

      // ---- P V on 16x16x16, one 16-key sub-tile at a time.  A row c16 < 4 (head c16) takes group 0's w of
      // lane c16 + 4 sigma; with two groups, row 4 + j (head 4 + j) takes group 1's w of lane j + 4 sigma
      auto take = [&](auto sig, uint32_t x0, uint32_t x1) -> uint32_t {
        constexpr int SG = decltype(sig)::value;
        if constexpr (HG == 1) {
          (void)x1;
          return row_take<4 * SG>(x0);
        } else {
          return row_take2<SG>(x0, x1);
        }
      };
      auto pv = [&](auto sig) {
        constexpr int SG = decltype(sig)::value;
        const h4 A0h = pack_h4(take(sig, wh[0][0], wh[HG - 1][0]), take(sig, wh[0][1], wh[HG - 1][1]));
        const h4 A0l = pack_h4(take(sig, wl[0][0], wl[HG - 1][0]), take(sig, wl[0][1], wl[HG - 1][1]));
        const h4 A1h = pack_h4(take(sig, wh[0][2], wh[HG - 1][2]), take(sig, wh[0][3], wh[HG - 1][3]));
        const h4 A1l = pack_h4(take(sig, wl[0][2], wl[HG - 1][2]), take(sig, wl[0][3], wl[HG - 1][3]));
        const uint32_t (&vd)[8] = T.v[SG];
        h4 bv[8];
  #pragma unroll
        for (int g = 0; g < 2; g++) {
          const uint32_t x01 = __builtin_amdgcn_perm(vd[2 + g], vd[g], 0x05010400u);
          const uint32_t y01 = __builtin_amdgcn_perm(vd[2 + g], vd[g], 0x07030602u);
          const uint32_t x23 = __builtin_amdgcn_perm(vd[6 + g], vd[4 + g], 0x05010400u);
          const uint32_t y23 = __builtin_amdgcn_perm(vd[6 + g], vd[4 + g], 0x07030602u);
          bv[4 * g + 0] = pack_h4(codes_to_h2(x01, 0x00050004u), codes_to_h2(x23, 0x00050004u));
          bv[4 * g + 1] = pack_h4(codes_to_h2(x01, 0x00070006u), codes_to_h2(x23, 0x00070006u));
          bv[4 * g + 2] = pack_h4(codes_to_h2(y01, 0x00050004u), codes_to_h2(y23, 0x00050004u));
          bv[4 * g + 3] = pack_h4(codes_to_h2(y01, 0x00070006u), codes_to_h2(y23, 0x00070006u));
        }
  #pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          O[jj] = mfma16(A0h, bv[jj], O[jj]);
          O[4 + jj] = mfma16(A1h, bv[4 + jj], O[4 + jj]);
        }
  #pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          O[jj] = mfma16(A0l, bv[jj], O[jj]);
          O[4 + jj] = mfma16(A1l, bv[4 + jj], O[4 + jj]);
        }
      };
      pv(std::integral_constant<int, 0>{});
      pv(std::integral_constant<int, 1>{});
      pv(std::integral_constant<int, 2>{});
      pv(std::integral_constant<int, 3>{});
    };

    for (int k = k0; k < k1; k++) {
      // outstanding here (k > k0): this tile's K half, then its V half, 10 loads each; the segment's first
      // tile and q were awaited above
      const bool nextk = k + 1 < k1;
      QuadTile T;
      if (k > k0) __builtin_amdgcn_s_waitcnt(kWaitTen);  // the K half is in (the V half may not be)
      fetch_k(T);
      __builtin_amdgcn_s_waitcnt(kWaitLds);  // the K half is read: the next tile's may overwrite it
      if (nextk) issue_k(D, cur, k + 1);
      if (k > k0) {  // the V half is in (the next tile's K half may not be)
        if (nextk) __builtin_amdgcn_s_waitcnt(kWaitTen);
        else __builtin_amdgcn_s_waitcnt(kWaitAll);
      }
      fetch_v(T);
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      if (nextk) {
        issue_v(D, cur, k + 1);
      } else if (more) {  // the next stream's first tile and q, in flight while this tile computes
        issue(quad_rsrc(p, nxt), nxt, 0);
        issue_q(nxt);
      }
      compute((cur.t0 + k) * kQT, T);
    }

    // ---- this segment's partial: heads 0..G-1 of the kv head, slot j of the stream
#pragma unroll
    for (int e = 0; e < HG; e++) {
      l_acc[e] += __shfl_xor(l_acc[e], 4);
      l_acc[e] += __shfl_xor(l_acc[e], 8);
      l_acc[e] += __shfl_xor(l_acc[e], 16);
      l_acc[e] += __shfl_xor(l_acc[e], 32);
      wb0[e] += __shfl_xor(wb0[e], 4);
      wb0[e] += __shfl_xor(wb0[e], 8);
      wb0[e] += __shfl_xor(wb0[e], 16);
      wb0[e] += __shfl_xor(wb0[e], 32);
      wb1[e] += __shfl_xor(wb1[e], 4);
      wb1[e] += __shfl_xor(wb1[e], 8);
      wb1[e] += __shfl_xor(wb1[e], 16);
      wb1[e] += __shfl_xor(wb1[e], 32);
    }
    const int jslot = wv - quad_wave_of(cur.Gs, T, W, sw);
    if (jslot == 0 && lane == 0)  // the stream's parts run from this wave to the one holding its last tile
      p.qparts[cur.r * p.KVH + cur.kvh] = quad_wave_of(cur.Gs + cur.cnt - 1, T, W, sw) - wv + 1;
    // lanes of quad q4 < HG write head group q4: row i of O is head 4 q4 + i
    if (q4 < HG) {
      const int e = HG == 1 ? 0 : q4;
      const float mr = HG == 1 ? mref[0] : (e ? mref[HG - 1] : mref[0]);
      const float la = HG == 1 ? l_acc[0] : (e ? l_acc[HG - 1] : l_acc[0]);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float b0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wb0[0]), i));
        float b1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wb1[0]), i));
        if constexpr (HG == 2) {
          const float c0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wb0[HG - 1]), i));
          const float c1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wb1[HG - 1]), i));
          b0 = e ? c0 : b0;
          b1 = e ? c1 : b1;
        }
        const int h = 4 * e + i;
        if (h < G) {
          const size_t part = (size_t(cur.r) * p.H + head0 + h) * p.nchunks + jslot;
          float4* po = reinterpret_cast<float4*>(p.po + part * kHD);
          po[c16] = make_float4(O[0][i] + b0, O[1][i] + b0, O[2][i] + b0, O[3][i] + b0);
          po[16 + c16] = make_float4(O[4][i] + b1, O[5][i] + b1, O[6][i] + b1, O[7][i] + b1);
          if (c16 == i) {
            p.pm[part] = mr;
            p.pl[part] = la;
          }
        }
      }
    }

    if (!more) break;
    cur = nxt;
    k0 = 0;
  }
}

// ------------------------------------------------------------ 16-bit pass 1
// K/V of dtype KDT (fp16 or bf16) in (rows, KVH, cap, 128).  Q K^T: lane (key
// c16, quad q4) supplies dims 32q4 + 4j + i of its key for MFMA j; P V: N-tile ii
// column n is dim 8n + ii, so a lane reads 16 contiguous bytes of each of its 4 keys.
template <int QDT, int KDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void ragged_pass1_16(DecodeParams p) {
  const int c = blockIdx.x;
  const int kvh = blockIdx.y / p.nslices, sl = blockIdx.y % p.nslices;
  const int r = blockIdx.z;
  int lo, hi;
  row_range(p.start, p.nkeys, p.n, p.cap, r, lo, hi);
  const int c0 = c * p.chunk;
  if (max(lo, c0) >= min(hi, c0 + p.chunk)) return;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int sub = p.chunk / kWaves;
  const int tlo = max(lo, c0 + wave * sub), thi = min(hi, c0 + (wave + 1) * sub);
  const int Gs = min(16, p.G - sl * 16);
  const int head0 = kvh * p.G + sl * 16;
  const int slot = p.slots ? min(max(p.slots[r], 0), p.kv_rows - 1) : r;
  const size_t tok0 = (size_t(slot) * p.KVH + kvh) * p.cap;
  const int cap = p.cap;
  const uint16_t* __restrict__ K = static_cast<const uint16_t*>(p.kf) + tok0 * kHD;
  const uint16_t* __restrict__ V = static_cast<const uint16_t*>(p.vf) + tok0 * kHD;
  const float scale_log2 = p.scale_dev ? p.scale_dev[0] * kLog2e : p.scale_log2;

  uint32_t qb[8][2];
  {
    const bool real = c16 < Gs;
    const size_t qrow = (size_t(r) * p.H + head0 + (real ? c16 : 0)) * kHD;
    float qv[32];  // dims 32 q4 .. 32 q4 + 31 of the lane's head
    ldn<QDT, 32>(p.q, qrow + 32 * q4, qv);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t bits[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float v = real ? qv[4 * j + i] : 0.0f;
        bits[i] = KDT == DT_BF16 ? f32_to_bf16_bits(v) : __builtin_bit_cast(uint16_t, _Float16(v));
      }
      qb[j][0] = bits[0] | (bits[1] << 16);
      qb[j][1] = bits[2] | (bits[3] << 16);
    }
  }

  // lazy running max and the reference p is taken against: for fp16 V, m_ref = m_run - 8, so p' = 2^8 p <= 2^14
  // and the fp16 hi + lo split of p' keeps a normal lo down to p = 2^-11 (l and O carry the same 2^8; the partial
  // is (m_ref, l', o')); bf16's split has no subnormal range to avoid
  constexpr float kPPre = 8.0f;
  float m_run = -INFINITY, mref = -INFINITY, l_acc = 0.0f;
  f4 O[8];
#pragma unroll
  for (int ii = 0; ii < 8; ii++) O[ii] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  struct Tile16 {
    uint4 kd[4], vd[4];
  };
  auto load = [&](int tb, Tile16& T) {
    const uint32_t tk = uint32_t(min(tb + c16, cap - 1));
#pragma unroll
    for (uint32_t u = 0; u < 4; u++) T.kd[u] = *reinterpret_cast<const uint4*>(K + (tk * kHD + 32u * q4 + 8u * u));
#pragma unroll
    for (int k = 0; k < 4; k++)
      T.vd[k] = *reinterpret_cast<const uint4*>(V + (uint32_t(min(tb + 4 * q4 + k, cap - 1)) * kHD + 8u * c16));
  };

  auto compute = [&](int tb, const Tile16& T) {
    f4 a = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint4 u = T.kd[j >> 1];
      const uint32_t w0 = (j & 1) ? u.z : u.x, w1 = (j & 1) ? u.w : u.y;
      if constexpr (KDT == DT_BF16) a = mfma16bf(pack_s4(w0, w1), pack_s4(qb[j][0], qb[j][1]), a);
      else a = mfma16(pack_h4(w0, w1), pack_h4(qb[j][0], qb[j][1]), a);
    }
    float s[4];
    bool valid[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int t = tb + 4 * q4 + i;
      valid[i] = t >= tlo && t < thi;
      s[i] = valid[i] ? a[i] * scale_log2 : -INFINITY;
    }
    float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const bool need = tmax > m_run + kRescaleThr;
    if (__any(need)) {
      if (need) m_run = tmax;
      const float nref = KDT == DT_BF16 ? m_run : m_run - kPPre;
      const float corr = mref == -INFINITY ? 0.0f : fast_exp2(mref - nref);
      mref = nref;
      l_acc *= corr;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ci = __shfl(corr, 4 * q4 + i);
#pragma unroll
        for (int ii = 0; ii < 8; ii++) O[ii][i] *= ci;
      }
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pr[i] = valid[i] ? fast_exp2(s[i] - mref) : 0.0f;
      l_acc += pr[i];
    }
    uint32_t ha, la, hb, lb;
    if constexpr (KDT == DT_BF16) {
      split_bf2(pr[0], pr[1], ha, la);
      split_bf2(pr[2], pr[3], hb, lb);
    } else {
      split_h2(pr[0], pr[1], ha, la);
      split_h2(pr[2], pr[3], hb, lb);
    }
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
      const uint32_t sel = (ii & 1) ? 0x07060302u : 0x05040100u;
      const int u = ii >> 1;
      const uint32_t w0 = u == 0 ? T.vd[0].x : u == 1 ? T.vd[0].y : u == 2 ? T.vd[0].z : T.vd[0].w;
      const uint32_t w1 = u == 0 ? T.vd[1].x : u == 1 ? T.vd[1].y : u == 2 ? T.vd[1].z : T.vd[1].w;
      const uint32_t w2 = u == 0 ? T.vd[2].x : u == 1 ? T.vd[2].y : u == 2 ? T.vd[2].z : T.vd[2].w;
      const uint32_t w3 = u == 0 ? T.vd[3].x : u == 1 ? T.vd[3].y : u == 2 ? T.vd[3].z : T.vd[3].w;
      const uint32_t b01 = __builtin_amdgcn_perm(w1, w0, sel);
      const uint32_t b23 = __builtin_amdgcn_perm(w3, w2, sel);
      if constexpr (KDT == DT_BF16) {
        O[ii] = mfma16bf(pack_s4(ha, hb), pack_s4(b01, b23), O[ii]);
        O[ii] = mfma16bf(pack_s4(la, lb), pack_s4(b01, b23), O[ii]);
      } else {
        O[ii] = mfma16(pack_h4(ha, hb), pack_h4(b01, b23), O[ii]);
        O[ii] = mfma16(pack_h4(la, lb), pack_h4(b01, b23), O[ii]);
      }
    }
  };

  if (tlo < thi) {
    const int tb0 = tlo & ~15, tbl = (thi - 1) & ~15;
    Tile16 A, B;
    load(tb0, A);
    for (int tb = tb0;;) {
      load(min(tb + 16, tbl), B);
      compute(tb, A);
      tb += 16;
      if (tb > tbl) break;
      load(min(tb + 16, tbl), A);
      compute(tb, B);
      tb += 16;
      if (tb > tbl) break;
    }
  }

  l_acc += __shfl_xor(l_acc, 16);
  l_acc += __shfl_xor(l_acc, 32);
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ float s_o[kWaves][16][kHD];
  if (q4 == 0) {
    s_m[wave][c16] = mref;
    s_l[wave][c16] = l_acc;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int ii = 0; ii < 8; ii++) s_o[wave][4 * q4 + i][8 * c16 + ii] = O[ii][i];
  }
  __syncthreads();
  join_waves(p, s_m, s_l, s_o, Gs, r, head0, c);
}

// ------------------------------------------------------------------- pass 2
// Grid (row x head, S slices of 128 / S dims), S = 1..32 chosen so the grid is ~1024
// workgroups; a workgroup is 8 S part lanes x 32 / S dim lanes (4 dims each).  Part lane c
// merges parts c, c + 8 S, ... online (running max, rescaled sums).  The
// first part's loads do not wait for the part count: they go out with the row-length reads
// and are discarded past the count (the slots exist in the workspace either way).  Lanes are
// merged by xor shuffles inside each wave, the four waves and the sink in LDS:
// out = sum_c 2^(m_c - M) o_c / (2^(sink - M) + sum_c 2^(m_c - M) l_c)  (locals/qkv.py:179-208).
// Parts with m = -inf (no key) weigh 0; no key and no sink: 0.
constexpr int kCombMaxSlices = 32;

// merge (m2, l2, o2) into (m, l, o)
__device__ __forceinline__ void lse_merge(float& m, float& l, float4& o, float m2, float l2, const float4& o2) {
  if (m2 == -INFINITY) return;
  const float mn = fmaxf(m, m2);
  const float a = m == -INFINITY ? 0.0f : fast_exp2(m - mn), b = fast_exp2(m2 - mn);
  o.x = o.x * a + o2.x * b;
  o.y = o.y * a + o2.y * b;
  o.z = o.z * a + o2.z * b;
  o.w = o.w * a + o2.w * b;
  l = l * a + l2 * b;
  m = mn;
}

__global__ __launch_bounds__(256) void decode_combine(CombineParams p) {
  const int rh = blockIdx.x, r = rh / p.H, head = rh % p.H;
  const int ds = blockIdx.y, S = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nd = 32 / S, np = 8 * S;        // dim lanes (4 dims each), part lanes
  const int dl = tid % nd, cs = tid / nd;
  const size_t base = size_t(rh) * p.nchunks;
  const float4* po4 = reinterpret_cast<const float4*>(p.po) + ds * nd + dl;
  // the first part of this lane, loaded before the count is known (slot cs < nchunks always exists)
  const bool pre = cs < p.nchunks;
  float m0 = -INFINITY, l0 = 0.0f;
  float4 o0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (pre) {
    m0 = p.pm[base + cs];
    l0 = p.pl[base + cs];
    o0 = po4[(base + cs) * (kHD / 4)];
  }
  // quad: the stream's part count as pass 1 recorded it, loaded beside the first part (read only for a row with
  // keys: no wave writes the count of an empty stream)
  const int qp = p.quad ? p.qparts[r * p.KVH + head / p.G] : 0;
  int lo, hi;
  row_range(p.start, p.nkeys, p.n, p.cap, r, lo, hi);
  int cl = 0, ch = 0;
  if (p.quad) {
    if (hi > lo) ch = qp;
  } else if (hi > lo) {
    cl = lo / p.chunk;
    ch = (hi + p.chunk - 1) / p.chunk;
  }
  float m = -INFINITY, L = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  int c = cl + cs;
  if (cl == 0 && pre) {  // the preloaded part is part cs
    if (cs < ch) lse_merge(m, L, acc, m0, l0, o0);
    c += np;
  }
#pragma unroll 2
  for (; c < ch; c += np) lse_merge(m, L, acc, p.pm[base + c], p.pl[base + c], po4[(base + c) * (kHD / 4)]);
  // part lanes of the wave: lanes differing in the bits above the dim lane
  for (int x = nd; x < 64; x <<= 1) {
    const float m2 = __shfl_xor(m, x), l2 = __shfl_xor(L, x);
    float4 o2;
    o2.x = __shfl_xor(acc.x, x);
    o2.y = __shfl_xor(acc.y, x);
    o2.z = __shfl_xor(acc.z, x);
    o2.w = __shfl_xor(acc.w, x);
    lse_merge(m, L, acc, m2, l2, o2);
  }
  __shared__ float4 s_o[4][32];  // a wave's merged dim lanes (nd = 32 / S of them)
  __shared__ float s_m[4], s_l[4];
  if (lane < nd) {
    s_o[wave][lane] = acc;
    if (lane == 0) {
      s_m[wave] = m;
      s_l[wave] = L;
    }
  }
  __syncthreads();
  if (tid >= nd) return;
  const float sink = p.sinks ? p.sinks[head] * kLog2e : -INFINITY;
  float M = sink;
  float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float Lt = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; w++) M = fmaxf(M, s_m[w]);
  if (M != -INFINITY) {
    if (sink != -INFINITY) Lt = fast_exp2(sink - M);
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float f = s_m[w] == -INFINITY ? 0.0f : fast_exp2(s_m[w] - M);
      t.x += f * s_o[w][tid].x;
      t.y += f * s_o[w][tid].y;
      t.z += f * s_o[w][tid].z;
      t.w += f * s_o[w][tid].w;
      Lt += f * s_l[w];
    }
  }
  const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
  const size_t ob = size_t(rh) * kHD + 4 * nd * ds + 4 * tid;
  store4_from_f32(p.out, ob, t.x * inv, t.y * inv, t.z * inv, t.w * inv, p.odt);
}

}  // namespace lcl

using namespace lcl;

// 8-bit pass 1 variant: the quad kernel for G <= 8 (one head group for G <= 4, two above), the register-fed one
// otherwise.  LOCALS_AMD_DECODE=reg forces the register-fed 16x16 kernel (for comparisons).
enum { kVarAuto = 0, kVarReg = 1 };
static int decode_variant() {
  static int v = -1;
  if (v < 0) {
    const char* e = getenv("LOCALS_AMD_DECODE");
    v = e && e[0] == 'r' ? kVarReg : kVarAuto;
  }
  return v;
}

static bool use_quad(const DecodeParams& p) { return p.G <= 8 && decode_variant() == kVarAuto; }

template <int QDT, int SDT>
static void launch_q8_t(dim3 grid, hipStream_t stream, hipEvent_t e0, hipEvent_t e1, const DecodeParams& p) {
  if (use_quad(p) && p.G <= 4)
    hipExtLaunchKernelGGL((qkv_pass1_q8_quad<QDT, SDT, 1>), grid, dim3(64), 0, stream, e0, e1, 0, p);
  else if (use_quad(p))
    hipExtLaunchKernelGGL((qkv_pass1_q8_quad<QDT, SDT, 2>), grid, dim3(64), 0, stream, e0, e1, 0, p);
  else hipExtLaunchKernelGGL((qkv_pass1_q8<QDT, SDT>), grid, dim3(256), 0, stream, e0, e1, 0, p);
}

static void launch_q8(int qdt, int sdt, dim3 grid, hipStream_t stream, hipEvent_t e0, hipEvent_t e1,
                      const DecodeParams& p) {
  if (sdt == DT_BF16) {
    if (qdt == DT_F16) launch_q8_t<DT_F16, DT_BF16>(grid, stream, e0, e1, p);
    else if (qdt == DT_BF16) launch_q8_t<DT_BF16, DT_BF16>(grid, stream, e0, e1, p);
    else launch_q8_t<DT_F32, DT_BF16>(grid, stream, e0, e1, p);
  } else {
    if (qdt == DT_F16) launch_q8_t<DT_F16, DT_F16>(grid, stream, e0, e1, p);
    else if (qdt == DT_BF16) launch_q8_t<DT_BF16, DT_F16>(grid, stream, e0, e1, p);
    else launch_q8_t<DT_F32, DT_F16>(grid, stream, e0, e1, p);
  }
}

template <int QDT, int KVDT>
static void launch_16_t(dim3 grid, hipStream_t stream, hipEvent_t e0, hipEvent_t e1, const DecodeParams& p) {
  hipExtLaunchKernelGGL((ragged_pass1_16<QDT, KVDT>), grid, dim3(256), 0, stream, e0, e1, 0, p);
}

static void launch_16(int qdt, int kvdt, dim3 grid, hipStream_t stream, hipEvent_t e0, hipEvent_t e1,
                      const DecodeParams& p) {
  if (kvdt == DT_BF16) {
    if (qdt == DT_F16) launch_16_t<DT_F16, DT_BF16>(grid, stream, e0, e1, p);
    else if (qdt == DT_BF16) launch_16_t<DT_BF16, DT_BF16>(grid, stream, e0, e1, p);
    else launch_16_t<DT_F32, DT_BF16>(grid, stream, e0, e1, p);
  } else {
    if (qdt == DT_F16) launch_16_t<DT_F16, DT_F16>(grid, stream, e0, e1, p);
    else if (qdt == DT_BF16) launch_16_t<DT_BF16, DT_F16>(grid, stream, e0, e1, p);
    else launch_16_t<DT_F32, DT_F16>(grid, stream, e0, e1, p);
  }
}

// pass 2 dim slices: the largest power of two in [1, 32] keeping the grid within ~1024 workgroups (C2's 512
// row-heads take 2, C3's 16 take 32)
static int comb_slices(int rows_heads) {
  static int forced = -1;
  if (forced < 0) {  // LOCALS_AMD_COMB_SLICES forces the slice count (a power of two in [1, 32]; tuning)
    const char* e = getenv("LOCALS_AMD_COMB_SLICES");
    const int v = e ? atoi(e) : 0;
    forced = (v >= 1 && v <= kCombMaxSlices && (v & (v - 1)) == 0) ? v : 0;
  }
  if (forced) return forced;
  int S = 1;
  while (S < kCombMaxSlices && (long long)rows_heads * S * 2 <= 1024) S <<= 1;
  return S;
}

static int pick_chunk(int block, int extent) {
  if (block > 0) return block;
  (void)extent;
  return 512;
}

static size_t ws_bytes_for(int R, int H, int nchunks) {
  // m, l and o of every part, then one part count a (row, head) (the quad pass 1's streams)
  return size_t(R) * H * nchunks * (2 + kHD) * sizeof(float) + size_t(R) * H * sizeof(int32_t);
}

// quad pass 1: least keys a wave = the block (a multiple of 64); slots a (row, head) for `extent` keys
static int quad_mint(int chunk) { return max(1, chunk / kQT); }
static int quad_slots(int extent, int chunk) {
  const int tiles = (max(extent, 1) + kQT - 1) / kQT;
  return (tiles + quad_mint(chunk) - 1) / quad_mint(chunk) + 1;
}
// resident waves a CU of the two-head-group quad pass 1 (its 8 heads' q staging leaves room for 7 a CU with
// 16-bit q, 6 with fp32 q); 6 if the runtime cannot tell
template <int QDT, int SDT>
static int quad_hg2_per_cu() {
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, qkv_pass1_q8_quad<QDT, SDT, 2>, 64, 0) != hipSuccess ||
      nb <= 0)
    nb = 6;
  return min(nb, 8);
}
static int quad_hg2_per_cu(int qdt, int sdt) {
  if (sdt == DT_BF16)
    return qdt == DT_F16 ? quad_hg2_per_cu<DT_F16, DT_BF16>() : qdt == DT_BF16 ? quad_hg2_per_cu<DT_BF16, DT_BF16>()
                                                                              : quad_hg2_per_cu<DT_F32, DT_BF16>();
  return qdt == DT_F16 ? quad_hg2_per_cu<DT_F16, DT_F16>() : qdt == DT_BF16 ? quad_hg2_per_cu<DT_BF16, DT_F16>()
                                                                           : quad_hg2_per_cu<DT_F32, DT_F16>();
}

// waves of the quad pass 1, one resident round: one a SIMD for G <= 4 (the kernel's occupancy allows two, but at one
// a SIMD each wave issues alone and pass 2 joins half the parts: C2 105.3-105.5 us a step against 107.5-107.8 at
// two, C3 91.8-92.6 against 95.3-95.6, C4's decode rows 60.7-61.0 against 63.8-64.1; counts between the two, such
// as 1152 or 1408 waves on 256 CUs, ran slower than either), the occupancy calculator's count for 5 <= G <= 8
// (Flint's G = 8: 68 us at 1792 waves, 72.5 at 1024)
static int quad_waves(int G, int qdt, int sdt) {
  static int cache[64][7] = {{0}};  // [device][0: G <= 4, 1 + 2 qdt + sdt: the two-group kernel]
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  const int v = G <= 4 ? 0 : 1 + 2 * qdt + sdt;
  if (!cache[dev][v]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev][v] = (v == 0 ? 4 : quad_hg2_per_cu(qdt, sdt)) * cus;
    // LOCALS_AMD_DECODE_WAVES overrides the count (a tuning knob: fewer waves than resident slots)
    const char* e = getenv("LOCALS_AMD_DECODE_WAVES");
    if (e && atoi(e) > 0) cache[dev][v] = atoi(e);
  }
  return cache[dev][v];
}

// Split weights of the quad pass 1 (see quad_prefix): even-XCD and odd-XCD waves among each SIMD's older waves,
// then among its younger ones.  The tile rates measured per wave at C2 on one MI355X (4.12 / 4.55 / 5.06 / 5.52 us
// a tile with equal weights, two waves a SIMD) give 24 : 22 : 20 : 18.  With one wave a SIMD (G <= 4) only the
// first pair applies; 24 : 22 ran C2, C3 and C4's decode rows fastest there (against 22 : 22 up to 30 : 22).  The
// older waves are the first one a SIMD: 4 x the CU count.
// LOCALS_AMD_DECODE_XW="a,b,c,d" overrides the weights (1..1000 each; "a,b" sets c = a, d = b).
static void quad_weights(DecodeParams& p) {
  static const long long packed = [] {  // thread-safe one-time initialisation
    int w[4] = {24, 22, 20, 18};
    const char* e = getenv("LOCALS_AMD_DECODE_XW");
    if (e) {
      int x[4];
      const int k = sscanf(e, "%d,%d,%d,%d", &x[0], &x[1], &x[2], &x[3]);
      if (k == 2) x[2] = x[0], x[3] = x[1];
      bool ok = k == 2 || k == 4;
      for (int i = 0; ok && i < 4; i++) ok = x[i] >= 1 && x[i] <= 1000;
      if (ok)
        for (int i = 0; i < 4; i++) w[i] = x[i];
    }
    return ((long long)w[0] << 48) | ((long long)w[1] << 32) | ((long long)w[2] << 16) | (long long)w[3];
  }();
  p.qwa = int((packed >> 48) & 0xffff);
  p.qwb = int((packed >> 32) & 0xffff);
  p.qya = int((packed >> 16) & 0xffff);
  p.qyb = int(packed & 0xffff);
  static int cus_of[64];  // CU count a device (0: not looked up yet; a racing lookup writes the same value)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cus_of[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cus_of[dev] = cus;
  }
  p.qold = 4 * cus_of[dev];  // even (4 SIMDs a CU)
}

// the argument checks of lcl_qkv_attend (before anything touches the GPU)
static int attend_args(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw,
                       const void* vs, const void* vb, int sdt, int B, int H, int KVH, int hd, int cap, int n,
                       int block, const void* out) {
  if (!q || !kw || !ks || !kb || !vw || !vs || !vb || !out) return -1;
  if (hd != kHD) return -2;
  if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH || cap <= 0 || n < 0 || n > cap) return -1;
  if (block < 0 || block % 64) return -1;
  if ((qdt != DT_F16 && qdt != DT_BF16 && qdt != DT_F32) || (sdt != DT_F16 && sdt != DT_BF16)) return -1;
  return 0;
}

// ---- scratch of the allocation-free decode (lcl_qkv_attend_noalloc)
// A file-scope device array takes the place of the caller's split-K workspace.  Each GPU the library runs on holds
// its own copy at its own address until the process ends.  On the host, `scratch` names a host-side stand-in, not
// device memory: host code only ever uses the per-device address hipGetSymbolAddress returns (looked up once per
// device, with that device current).  Every call on a GPU shares that GPU's array; pass 1 writes every part pass 2
// reads (empty ones included), so nothing in it needs clearing, and calls that overlap on one GPU race.
constexpr size_t kScratchBytes = size_t(LCL_NOALLOC_SCRATCH_BYTES);
static_assert(kScratchBytes % 256 == 0, "scratch size");
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// the scratch address on device dev (0 = ok, else a hipError_t)
static int scratch_on(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return int(hipErrorInvalidDevice);
  void* p = __atomic_load_n(&g_scratch[dev], __ATOMIC_ACQUIRE);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev];
    if (!p) {
      int cur = -1;
      hipError_t e = hipGetDevice(&cur);
      if (e != hipSuccess) return int(e);
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return int(e);
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess) return int(e);
      if (!p) return int(hipErrorInvalidSymbol);
      __atomic_store_n(&g_scratch[dev], p, __ATOMIC_RELEASE);
    }
  }
  *out = p;
  return 0;
}

extern "C" {

size_t lcl_decode_workspace_bytes(int R, int H, int extent, int block) {
  const int chunk = pick_chunk(block, extent);
  const int nchunks = extent > 0 ? (extent + chunk - 1) / chunk : 1;
  return ws_bytes_for(R, H, max(nchunks, quad_slots(extent, chunk)));
}

int lcl_qkv_attend(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw,
                   const void* vs, const void* vb, int sdt, const int32_t* start, const float* sinks, float scale,
                   int B, int H, int KVH, int hd, int cap, int n, int block, void* out, void* workspace,
                   size_t workspace_bytes, void* stream_) {
  return lcl_qkv_attend_ex(q, qdt, kw, ks, kb, vw, vs, vb, sdt, start, sinks, scale, B, H, KVH, hd, cap, n, block,
                           out, workspace, workspace_bytes, stream_, nullptr, nullptr);
}

int lcl_qkv_attend_ex(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw,
                      const void* vs, const void* vb, int sdt, const int32_t* start, const float* sinks, float scale,
                      int B, int H, int KVH, int hd, int cap, int n, int block, void* out, void* workspace,
                      size_t workspace_bytes, void* stream_, void* ev_start, void* ev_stop) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (const int rc = attend_args(q, qdt, kw, ks, kb, vw, vs, vb, sdt, B, H, KVH, hd, cap, n, block, out)) return rc;
  const int chunk = pick_chunk(block, n);
  DecodeParams p{};
  p.G = H / KVH;
  const bool quad = use_quad(p);
  // parts a (row, head): the chunks of the grid, or the stream-K slots of the quad pass 1
  const int nparts = quad ? quad_slots(n, chunk) : (n > 0 ? (n + chunk - 1) / chunk : 1);
  if (!workspace || workspace_bytes < ws_bytes_for(B, H, nparts)) return -3;
  p.q = q;
  p.kw = kw; p.ks = ks; p.kb = kb;
  p.vw = vw; p.vs = vs; p.vb = vb;
  p.start = start;
  float* ws = static_cast<float*>(workspace);
  const size_t np = size_t(B) * H * nparts;
  p.pm = ws;
  p.pl = ws + np;
  p.po = ws + 2 * np;
  p.qparts = reinterpret_cast<int32_t*>(ws + (2 + kHD) * np);
  p.n = n; p.cap = cap; p.H = H; p.KVH = KVH; p.kv_rows = B; p.R = B;
  p.nslices = (p.G + 15) / 16;
  p.nchunks = nparts; p.chunk = chunk;
  p.scale_log2 = scale * kLog2e;
  p.qdt = qdt; p.sdt = sdt;
  if (quad) {
    p.qmint = quad_mint(chunk);
    const long long tmax = (long long)B * KVH * ((n + kQT - 1) / kQT);
    p.qwaves = int(min((long long)quad_waves(p.G, qdt, sdt), max(1LL, tmax / p.qmint)));
    quad_weights(p);
  }
  if (n > 0) {
    const dim3 grid = quad ? dim3(p.qwaves) : dim3(nparts, KVH * p.nslices, B);
    hipEvent_t e0 = static_cast<hipEvent_t>(ev_start), e1 = static_cast<hipEvent_t>(ev_stop);
    launch_q8(qdt, sdt, grid, stream, e0, e1, p);
  }
  CombineParams c{};
  c.pm = p.pm; c.pl = p.pl; c.po = p.po; c.sinks = sinks; c.out = out;
  c.start = start; c.nkeys = nullptr; c.n = n; c.cap = cap; c.H = H; c.nchunks = nparts; c.chunk = chunk; c.odt = qdt;
  c.quad = quad; c.R = B; c.KVH = KVH; c.G = p.G; c.qparts = p.qparts;
  hipLaunchKernelGGL(decode_combine, dim3(B * H, comb_slices(B * H)), dim3(256), 0, stream, c);
  return int(hipGetLastError());
}

int lcl_qkv_attend_noalloc(const void* q, int qdt, const uint32_t* kw, const void* ks, const void* kb,
                           const uint32_t* vw, const void* vs, const void* vb, int sdt, const int32_t* start,
                           const float* sinks, float scale, int B, int H, int KVH, int hd, int cap, int n, int block,
                           void* out, void* stream_) {
  if (const int rc = attend_args(q, qdt, kw, ks, kb, vw, vs, vb, sdt, B, H, KVH, hd, cap, n, block, out)) return rc;
  if (lcl_decode_workspace_bytes(B, H, n, block) > kScratchBytes) return LCL_ESCRATCH;
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int dev = 0;
  const hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  void* ws = nullptr;
  if (const int rc = scratch_on(dev, &ws)) return rc;
  return lcl_qkv_attend_ex(q, qdt, kw, ks, kb, vw, vs, vb, sdt, start, sinks, scale, B, H, KVH, hd, cap, n, block,
                           out, ws, kScratchBytes, stream_, nullptr, nullptr);
}

int lcl_ragged_attention(const void* q, int qdt, const void* keys, const void* values, int kvdt, const int32_t* slots,
                         const int32_t* nkeys, float scale, const float* scale_dev, int R, int H, int n_slots, int Hkv, int hd, int cap,
                         int block, void* out, void* workspace, size_t workspace_bytes, void* stream_) {
  return lcl_ragged_attention_ex(q, qdt, keys, values, kvdt, slots, nkeys, scale, scale_dev, R, H, n_slots, Hkv, hd,
                                 cap, block, out, workspace, workspace_bytes, stream_, nullptr, nullptr);
}

int lcl_ragged_attention_ex(const void* q, int qdt, const void* keys, const void* values, int kvdt,
                            const int32_t* slots, const int32_t* nkeys, float scale, const float* scale_dev, int R,
                            int H, int n_slots, int Hkv, int hd, int cap, int block, void* out, void* workspace,
                            size_t workspace_bytes, void* stream_, void* ev_start, void* ev_stop) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!q || !keys || !values || !slots || !nkeys || !out) return -1;
  if (hd != kHD && !generic_head_dim_ok(hd, false)) return -2;
  if (R < 0 || H <= 0 || Hkv <= 0 || H % Hkv || n_slots <= 0 || cap <= 0) return -1;
  if (block < 0 || block % 64) return -1;
  if ((qdt != DT_F16 && qdt != DT_BF16 && qdt != DT_F32) || (kvdt != DT_F16 && kvdt != DT_BF16)) return -1;
  if (R == 0) return 0;
  if (hd != kHD) {  // other head sizes: the generic kernel (no split, no workspace)
    GenParams g{};
    g.q = q; g.qdt = qdt; g.kvfmt = 1; g.kf = keys; g.vf = values; g.kvdt = kvdt;
    g.slots = slots; g.nkeys = nkeys; g.mask = 0;
    g.scale = scale; g.scale_dev = scale_dev;
    g.R = R; g.H = H; g.KVH = Hkv; g.L = 1; g.N = cap; g.D = hd; g.cap = cap; g.kv_rows = n_slots;
    g.out = out; g.odt = qdt;
    return attn_generic_launch(g, stream);
  }
  const int chunk = pick_chunk(block, cap);
  const int nchunks = (cap + chunk - 1) / chunk;
  if (!workspace || workspace_bytes < ws_bytes_for(R, H, nchunks)) return -3;
  DecodeParams p{};
  p.q = q;
  p.kf = keys; p.vf = values;
  p.slots = slots; p.nkeys = nkeys;
  float* ws = static_cast<float*>(workspace);
  const size_t np = size_t(R) * H * nchunks;
  p.pm = ws; p.pl = ws + np; p.po = ws + 2 * np;
  p.n = cap; p.cap = cap; p.H = H; p.KVH = Hkv; p.G = H / Hkv; p.kv_rows = n_slots;
  p.nslices = (p.G + 15) / 16;
  p.nchunks = nchunks; p.chunk = chunk;
  p.scale_log2 = scale * kLog2e;
  p.scale_dev = scale_dev;
  p.qdt = qdt; p.sdt = kvdt;
  const dim3 grid(nchunks, Hkv * p.nslices, R);
  launch_16(qdt, kvdt, grid, stream, static_cast<hipEvent_t>(ev_start), static_cast<hipEvent_t>(ev_stop), p);
  CombineParams c{};
  c.pm = p.pm; c.pl = p.pl; c.po = p.po; c.sinks = nullptr; c.out = out;
  c.start = nullptr; c.nkeys = nkeys; c.n = cap; c.cap = cap; c.H = H; c.nchunks = nchunks; c.chunk = chunk;
  c.odt = qdt;
  hipLaunchKernelGGL(decode_combine, dim3(R * H, comb_slices(R * H)), dim3(256), 0, stream, c);
  return int(hipGetLastError());
}

}  // extern "C"
