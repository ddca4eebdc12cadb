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
//  * the sliding-window layers' prompt chunks (locals/fuse.py:113-125, locals/models/flint_streamed.py:114-128):
//    causal within a window of W keys, query i (position N - L + i) seeing keys (N - L + i - W, N - L + i];
//    the reference slices the keys a band of queries reaches, here each workgroup reads only its rows' band;
//  * the sink is a logit in the denominator only.
//
// MI355X design.  Work units (key chunk, row block, batch row x kv head), dealt to the
// XCDs in contiguous runs; a workgroup = 4 waves = 64 or 128 rows (one or two 16-row
// tiles a wave), or 8 waves = 256 rows with two row tiles under a causal or no mask (and a
// window, 16-bit K/V): one workgroup a CU, each tile loaded and staged in LDS serving twice
// the rows; a row being one (query, head) of the kv head's G heads (row r: query r / G,
// head r % G, so any G works).  Per 64-key tile: 8-bit K and V are dequantized
// once into LDS as MFMA operands (fp32 scale * code + bias, rounded once to the MFMA
// type, as the reference's dequantized() feeds its attention in T); 16-bit tiles are the
// operands as loaded.  Every wave reuses the tile for its rows:
//  * S^T = K Q^T on v_mfma_f32_16x16x32 (A = 16 keys x 32 dims from LDS, B = Q^T from
//    registers): lane l gets S[row l % 16][keys 4 (l / 16) + i] -- the softmax state of
//    a row lives in one lane column, its max needs two cross-lane steps;
//  * O^T = V^T P^T (A = V^T 16 dims x 32 keys from LDS, B = P^T in the S^T registers):
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
// halves a K row in LDS: 288 B, 16 B aligned with an 8-bank skew a row (measured on C4 / C5 against strides of 128,
// 136, 152 and 160 halves and a 256 B row with the 16-bit path's XOR chunk swizzle: 136 -> 144 took C4 pass 1
// 220.6 -> 216.5 us and C5 55.5 -> 53.0 us; no padding costs 30%)
constexpr int kKsStride = 144;
constexpr int kRawSlot = 8192 + 8192 + 1024;  // an 8-bit raw tile: K codes, V codes, ks / kb / vs / vb
constexpr float kThr = 6.0f;
// A 16-bit K + V tile (64 key rows of 256 B each).  K row r keeps its 16-byte chunk c at slot c ^ swk(r), V row
// r at slot c ^ swv(r).  Chosen by measuring each operand read pattern alone on an MI355X (8 waves a CU; B/clk
// a workgroup): the K reads (lane c16 + 16 q4 takes chunk 4 kk + q4 of row c16) reach the 128 of a contiguous
// read with swk, 85 with the swizzle that maps rows 0..3 to even chunks only; the transposing V reads (chunks
// 2 d, 2 d + 1 of 16 consecutive rows, four lanes a row) 112 with swv against 85 with that one or with swk.
constexpr int kRaw16 = 2 * kKT * kD * 2;
__device__ __forceinline__ int swk(int r) { return r & 15; }
__device__ __forceinline__ int swv(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

enum MaskKind { MK_NONE = 0, MK_CAUSAL = 1, MK_TREE = 2, MK_DENSE = 3, MK_WINDOW = 4 };
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
  int window;  // MK_WINDOW: keys a query sees, itself included
  void* out;  // direct: one chunk covers every key, so pass 1 writes the normalized output (B, H, L, 128), dtype odt
  int direct, odt;
  int nw;  // waves a workgroup: 8 for 16-bit K/V with two row tiles (causal or no mask), else 4
};

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));

template <int MT>
__device__ __forceinline__ uint16_t to_mt(float x) {
  if constexpr (MT == DT_BF16) return f32_to_bf16_bits(x);
  else return __builtin_bit_cast(uint16_t, _Float16(x));
}

// two floats -> a packed pair of the MFMA type, round to nearest even (bf16: one v_cvt_pk_bf16_f32)
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <int MT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (MT == DT_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  else return __builtin_bit_cast(uint32_t, h2{_Float16(a), _Float16(b)});
}

// v_mfma_f32_16x16x32: lane l holds A[l % 16][8 (l / 16) + j], B[8 (l / 16) + j][l % 16], j = 0..7
template <int MT>
__device__ __forceinline__ f4 mma32(uint4 a, uint4 b, f4 c) {
  if constexpr (MT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

// code pair (1024 + a, 1024 + b) -> scale * code + bias for fp16 scale/bias pairs: exact code, one fp16 rounding
__device__ __forceinline__ uint32_t dq_h2(uint32_t codes1024, uint32_t sc2, uint32_t bi2) {
  const h2 c = __builtin_bit_cast(h2, codes1024) - h2{_Float16(1024.0f), _Float16(1024.0f)};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, sc2) * c + __builtin_bit_cast(h2, bi2));
}

// The raw bytes of one 64-key tile a thread stages (8-bit: codes + its keys' scale/bias; 16-bit: values)
struct RawTile {
  u4 k[2], v[2];   // 32 K codes and 32 V codes of the thread's key (dims 32 kpart ..)
  uint32_t ks, kb, vs, vb;  // the key's scale / bias pairs (one 16-bit entry a 64-dim group)
};

// Direct buffer -> LDS loads issued as asm, outside the compiler's LDS-DMA wait tracking (merged at a loop head it
// cannot tell two slots apart and makes every read of one wait for the loads into the other).  Their completion
// is awaited with explicit s_waitcnt vmcnt by the caller, before a barrier.  Lane l's 16 bytes at voff land at
// lds + 16 l; the descriptor covers `bytes` bytes (loads past it read 0), raw, default cache policy (every row
// block of a kv head reads the same K/V, so the lines are worth keeping in L2).
typedef uint32_t sg4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ sg4 rsrc_words(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return sg4{uint32_t(a), uint32_t(a >> 32) & 0xffffu, bytes, 0x00020000u};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(uintptr_t((const __attribute__((address_space(3))) uint8_t*)(p)));
}
__device__ __forceinline__ void dma16(sg4 r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(lds), "v"(voff), "s"(r)
               : "memory", "m0");
}

// ds_read_b64_tr_b16: in each 16-lane group, lane i's element e is element i % 4 of the 8 bytes that lane
// 4 e + i / 4 of the group addresses (checked in bounds on the MI355X).
typedef short s4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const uint8_t* p) {
  const s4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4v*)(p));
  return __builtin_bit_cast(uint2, v);
}

// One workgroup: RT x 64 rows of (batch row b, kv head kvh) -- a row is one (query, head) -- and the keys of
// chunk c.  8-bit, two row tiles: per 64-key tile the raw bytes arrive in one of two LDS slots while the other's
// tile is dequantized into the operand buffer and multiplied; one row tile: the codes arrive in registers two tiles
// ahead and are dequantized into one of two operand buffers while the other's tile is multiplied.  16-bit: the K and V tiles arrive in one of two slots and
// are multiplied in place while the next tile's loads are in flight.
template <int QDT, int SDT, int FMT, int MT, int MASK, int RT, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void sdpa_pass1(SdpaParams p) {
  static_assert(NW == 4 || (NW == 8 && RT == 2), "eight-wave workgroups: two row tiles");
  // XCD-aware order: the hardware deals workgroups to the 8 XCDs round-robin, so physical workgroup P runs on
  // XCD P % 8; logical workgroup (P % 8) * ceil(total / 8) + P / 8 gives each XCD a contiguous run of (chunk,
  // row block, batch row x kv head) -- the same kv head's K/V for all of it, which its own L2 then holds
  const int total = p.nchunks * p.nrowblocks * p.B * p.KVH;
  const int lg = int(blockIdx.x % 8u) * ((total + 7) / 8) + int(blockIdx.x / 8u);
  if (lg >= total) return;  // padding of the grid to a multiple of 8
  const int c = lg % p.nchunks, rb = (lg / p.nchunks) % p.nrowblocks;
  const int bz = lg / (p.nchunks * p.nrowblocks);
  const int b = bz / p.KVH, kvh = bz % p.KVH;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, tid = threadIdx.x;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int R = p.L * p.G;
  const int row0 = 16 * NW * RT * rb;
  // this lane's rows (one a row tile): r-th tile rows row0 + 16 NW r + 16 wave + [0, 16)
  int rowi[RT], qi[RT], head[RT];
  bool real[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    rowi[r] = row0 + 16 * NW * r + 16 * wave + c16;
    real[r] = rowi[r] < R;
    qi[r] = real[r] ? rowi[r] / p.G : 0;
    head[r] = kvh * p.G + (real[r] ? rowi[r] % p.G : 0);
  }
  const int last_q = min(R - 1, row0 + 16 * NW * RT - 1) / p.G;
  const int wave_q0 = (row0 + 16 * wave) / p.G;  // the smallest query index among this wave's rows
  const int slo = p.start ? max(p.start[b], 0) : 0;
  // keys the workgroup's rows can see: [blo, bhi); chunks are counted from base (the band's first tile for a
  // window, key 0 otherwise)
  int blo = slo, bhi = p.N, base = 0;
  if constexpr (MASK == MK_CAUSAL || MASK == MK_WINDOW) bhi = min(bhi, p.N - p.L + last_q + 1);
  if constexpr (MASK == MK_WINDOW) {
    blo = max(blo, p.N - p.L + row0 / p.G - p.window + 1);
    base = max(blo, 0) & ~(kKT - 1);
  }
  const int klo = __builtin_amdgcn_readfirstlane(max(blo, base + c * p.chunk));
  const int khi = __builtin_amdgcn_readfirstlane(min(bhi, base + (c + 1) * p.chunk));
  if (klo >= khi) {  // uniform: nothing here; rows record an empty part (or, direct, a zero output)
#pragma unroll
    for (int r = 0; r < RT; r++) {
      if (!real[r]) continue;
      const size_t row = (size_t(b) * p.H + head[r]) * p.L + qi[r];
      if (p.direct) {
#pragma unroll
        for (int dd = 0; dd < 8; dd++)
          store4_from_f32(p.out, row * kD + 16 * dd + 4 * q4, 0.0f, 0.0f, 0.0f, 0.0f, p.odt);
      } else if (q4 == 0) {
        p.pm[row * p.nchunks + c] = -INFINITY;
        p.pl[row * p.nchunks + c] = 0.0f;
      }
    }
    return;
  }

  // 8-bit: raw tiles arrive by direct buffer->LDS loads into two named slots (one in flight while the other is
  // staged) and are dequantized into one operand buffer (Ks; Vk key-major as the 16-bit V region, read through the
  // transposing read).  16-bit: the K and V tiles arrive the same way
  // (chunks swizzled by swk / swv) and are the MFMA operands themselves -- K rows read as they are, V^T through the
  // transposing read -- so nothing is staged.
  // 8-bit with one row tile, or in eight-wave workgroups: the codes come into registers two tiles ahead (32 or 16
  // dims of a key's K and V a thread) and there are two operand buffers
  // (tile i multiplied from buffer i % 2 while tile i + 1 is staged into the other: one barrier a tile); the raw
  // slots are then unused
  constexpr bool kRegPipe = FMT == KV_Q8 && (RT == 1 || NW == 8);
  constexpr int kOpBufs = kRegPipe ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[FMT == KV_Q8 ? kOpBufs * kKT * kKsStride : 8];
  __shared__ __attribute__((aligned(16))) uint8_t Vk[FMT == KV_Q8 ? kOpBufs * kKT * 256 : 16];
  __shared__ __attribute__((aligned(16))) uint8_t raw0[kRegPipe ? 16 : FMT == KV_Q8 ? kRawSlot : kRaw16];
  __shared__ __attribute__((aligned(16))) uint8_t raw1[kRegPipe ? 16 : FMT == KV_Q8 ? kRawSlot : kRaw16];

  // Q^T as B operands: qb[r][kk] = scale log2(e) q[row][32 kk + 8 q4 + j], scaled in fp32 before its one rounding
  // to the MFMA type, so the products come out as base-2 logits.  Loaded (16 bytes a lane a step) after the first
  // tiles' loads are issued, so the two latencies overlap.
  uint4 qb[RT][4];
  auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < RT; r++) {
      const size_t qrow = ((size_t(b) * p.H + head[r]) * p.L + qi[r]) * kD;
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const size_t qo = qrow + 32 * kk + 8 * q4;
        float x[8];
        if constexpr (QDT == DT_F32) {
          const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + qo);
          const float4 c = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + qo + 4);
          x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
        } else {
          const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + qo);
          const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            x[2 * i] = QDT == DT_BF16 ? bf16_bits_to_f32(uint16_t(wv[i])) : f16_bits_to_f32(uint16_t(wv[i]));
            x[2 * i + 1] =
                QDT == DT_BF16 ? bf16_bits_to_f32(uint16_t(wv[i] >> 16)) : f16_bits_to_f32(uint16_t(wv[i] >> 16));
          }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = real[r] ? x[j] * p.scale_log2 : 0.0f;
        qb[r][kk] =
            make_uint4(pack2<MT>(x[0], x[1]), pack2<MT>(x[2], x[3]), pack2<MT>(x[4], x[5]), pack2<MT>(x[6], x[7]));
      }
    }
  };

  // buffers of this (row, kv head); loads past the capacity read 0
  const size_t tok0 = (size_t(b) * p.KVH + kvh) * p.cap;
  const uint32_t cap = uint32_t(p.cap);
  BufRsrc rk, rv, rks, rkb, rvs, rvb;
  if constexpr (FMT == KV_Q8) {
    rk = make_rsrc(p.kw + tok0 * 32, cap * 128u);
    rv = make_rsrc(p.vw + tok0 * 32, cap * 128u);
    rks = make_rsrc(static_cast<const uint16_t*>(p.ks) + tok0 * 2, cap * 4u);
    rkb = make_rsrc(static_cast<const uint16_t*>(p.kb) + tok0 * 2, cap * 4u);
    rvs = make_rsrc(static_cast<const uint16_t*>(p.vs) + tok0 * 2, cap * 4u);
    rvb = make_rsrc(static_cast<const uint16_t*>(p.vb) + tok0 * 2, cap * 4u);
  }
  const sg4 dk16 = rsrc_words(static_cast<const uint16_t*>(FMT == KV_16 ? p.kf : p.kw) + tok0 * kD, cap * 256u);
  const sg4 dv16 = rsrc_words(static_cast<const uint16_t*>(FMT == KV_16 ? p.vf : p.vw) + tok0 * kD, cap * 256u);
  // 8-bit DMA: the scale / bias array this wave sends (wave 0 K scales, 1 K biases, 2 V scales, 3 V biases)
  const int warr = wave & 3;  // eight waves: waves w and w + 4 send the two halves of array w
  const void* sarr = FMT != KV_Q8 ? p.kf : warr == 0 ? p.ks : warr == 1 ? p.kb : warr == 2 ? p.vs : p.vb;
  const BufRsrc rsw = make_rsrc(static_cast<const uint16_t*>(sarr) + tok0 * 2, cap * 4u);
  const int kkey = tid / NW, kpart = tid % NW;   // staging: one key, 128 / NW dims of its K and V

  // 8-bit raw tile in LDS: K codes (key-major 128 B rows, 8 KB), V codes (8 KB), ks / kb / vs / vb words (256 B
  // each).  Wave w sends K and V rows 16 w .. 16 w + 15 (two 1 KB pieces each) and the w-th scale array.  Row r
  // keeps its 16-byte chunk c at slot c ^ ((r >> 1) & 1), so the staging reads (32 bytes of each of 16 rows a
  // wave) cover every bank group.
  auto dma = [&](int t0, uint8_t* S) __attribute__((always_inline)) {
    constexpr int kRowsW = 64 / NW;  // key rows a wave sends, 8 a 1 KB piece
#pragma unroll
    for (int i = 0; i < kRowsW / 8; i++) {
      const int r = kRowsW * wave + 8 * i + (lane >> 3);
      const uint32_t voff = uint32_t(t0 + r) * 128u + 16u * uint32_t((lane & 7) ^ ((r >> 1) & 1));
      lds_load16<0>(rk, S + 128 * kRowsW * wave + 1024 * i, voff);
      lds_load16<0>(rv, S + 8192 + 128 * kRowsW * wave + 1024 * i, voff);
    }
    if constexpr (NW == 4) {
      lds_load4<0>(rsw, S + 16384 + 256 * wave, (uint32_t(t0) + uint32_t(lane)) * 4u);
    } else if (lane < 32) {
      const int h = wave >> 2;
      lds_load4<0>(rsw, S + 16384 + 256 * warr + 128 * h, (uint32_t(t0 + 32 * h) + uint32_t(lane)) * 4u);
    }
  };
  // the thread's share of a raw tile in LDS, as the register-prefetch path would hold it
  auto load_lds = [&](const uint8_t* S, RawTile& T) __attribute__((always_inline)) {
    const int f = (kkey >> 1) & 1;  // the row's chunk swizzle: chunk c at slot c ^ f
    if constexpr (NW == 4) {  // chunks 2 kpart, 2 kpart + 1
      const uint8_t* kr = S + kkey * 128 + 32 * kpart;
      T.k[0] = *reinterpret_cast<const u4*>(kr + 16 * f);
      T.k[1] = *reinterpret_cast<const u4*>(kr + 16 * (f ^ 1));
      T.v[0] = *reinterpret_cast<const u4*>(kr + 8192 + 16 * f);
      T.v[1] = *reinterpret_cast<const u4*>(kr + 8192 + 16 * (f ^ 1));
    } else {  // chunk kpart
      const uint8_t* kr = S + kkey * 128 + 16 * (kpart ^ f);
      T.k[0] = *reinterpret_cast<const u4*>(kr);
      T.v[0] = *reinterpret_cast<const u4*>(kr + 8192);
      T.k[1] = T.v[1] = u4{0u, 0u, 0u, 0u};  // not read: a thread stages one 16-byte chunk
    }
    T.ks = *reinterpret_cast<const uint32_t*>(S + 16384 + 4 * kkey);
    T.kb = *reinterpret_cast<const uint32_t*>(S + 16640 + 4 * kkey);
    T.vs = *reinterpret_cast<const uint32_t*>(S + 16896 + 4 * kkey);
    T.vb = *reinterpret_cast<const uint32_t*>(S + 17152 + 4 * kkey);
  };
  // the same share loaded from the buffers into registers (register pipeline)
  auto load_glb = [&](int t0, RawTile& T) __attribute__((always_inline)) {
    const uint32_t key = uint32_t(t0 + kkey), co = key * 128u + uint32_t(128 / NW) * uint32_t(kpart);
    T.k[0] = buf_load_b128(rk, co, 0);
    T.v[0] = buf_load_b128(rv, co, 0);
    if constexpr (NW == 4) {
      T.k[1] = buf_load_b128(rk, co, 16);
      T.v[1] = buf_load_b128(rv, co, 16);
    } else {
      T.k[1] = T.v[1] = u4{0u, 0u, 0u, 0u};
    }
    T.ks = buf_load_b32(rks, key * 4u, 0);
    T.kb = buf_load_b32(rkb, key * 4u, 0);
    T.vs = buf_load_b32(rvs, key * 4u, 0);
    T.vb = buf_load_b32(rvb, key * 4u, 0);
  };

  // dequantize 32 codes (dims 32 kpart ..) with the key's scale / bias pair: 16 packed pairs of the MFMA type
  constexpr int kW = 32 / NW;  // code words a thread stages of a key's K (and of its V)
  auto dequant = [&](const u4 (&c)[2], uint32_t sc, uint32_t bi, uint32_t (&o)[16]) __attribute__((always_inline)) {
    const uint32_t cw[8] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w};
    const int gsel = kpart / (NW / 2);  // group of the thread's dims (128 / NW kpart ..)
    if constexpr (MT == DT_F16) {
      const uint32_t s1 = (sc >> (16 * gsel)) & 0xffffu, b1 = (bi >> (16 * gsel)) & 0xffffu;
      const uint32_t s2 = s1 | (s1 << 16), b2 = b1 | (b1 << 16);
#pragma unroll
      for (int w = 0; w < kW; w++) {
        o[2 * w] = dq_h2(codes_to_h2(cw[w], 0x00050004u), s2, b2);
        o[2 * w + 1] = dq_h2(codes_to_h2(cw[w], 0x00070006u), s2, b2);
      }
    } else {
      const float sf = half_of(sc, gsel, SDT), bf = half_of(bi, gsel, SDT);
#pragma unroll
      for (int w = 0; w < kW; w++) {
        o[2 * w] = pack2<MT>(sf * float(cw[w] & 0xffu) + bf, sf * float((cw[w] >> 8) & 0xffu) + bf);
        o[2 * w + 1] = pack2<MT>(sf * float((cw[w] >> 16) & 0xffu) + bf, sf * float(cw[w] >> 24) + bf);
      }
    }
  };
  // dequantize an 8-bit tile into the operand buffers: K rows into Ks, V rows into Vk (16-byte chunk c of key r at
  // slot c ^ swv(r)); keys outside [klo, khi) become 0 (MASKED: the tile straddles an end of the range;
  // otherwise every key is inside and no test is made)
  auto stage = [&](int t0, const RawTile& T, auto masked, int ob) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked)::value;
    const int kg = t0 + kkey;
    const bool kin = !MASKED || (kg >= klo && kg < khi);
    uint32_t o[16];
    dequant(T.k, T.ks, T.kb, o);
    uint4* kdst = reinterpret_cast<uint4*>(&Ks[ob * (kKT * kKsStride) + kkey * kKsStride + kpart * (128 / NW)]);
#pragma unroll
    for (int u = 0; u < kW / 2; u++)
      kdst[u] = kin ? make_uint4(o[4 * u], o[4 * u + 1], o[4 * u + 2], o[4 * u + 3]) : make_uint4(0u, 0u, 0u, 0u);
    dequant(T.v, T.vs, T.vb, o);
    const int sw = swv(kkey);
#pragma unroll
    for (int u = 0; u < kW / 2; u++)
      *reinterpret_cast<uint4*>(&Vk[ob * (kKT * 256) + kkey * 256 + 16 * (((kW / 2) * kpart + u) ^ sw)]) =
          kin ? make_uint4(o[4 * u], o[4 * u + 1], o[4 * u + 2], o[4 * u + 3]) : make_uint4(0u, 0u, 0u, 0u);
  };

  // Softmax state of this lane's row in each row tile: the lazy running max m_run (moved only when a tile's max
  // passes it by kThr, so p <= 2^kThr), negm = -m_run broadcast (0 before the first key), the C operand the
  // Q K^T chain starts from, so the scores come out as s - m_run and need no subtraction before exp2, and the
  // threshold a tile's max is checked against (kThr, or -inf before the first key).  The denominator is summed on
  // MFMA as P^T times a ones operand (Lacc: every lane gets its row's sum of exactly the rounded P that multiplies
  // V, so the weights of the output are consistent), rescaled with O.
  float m_run[RT], thr[RT];
  f4 negm[RT], Lacc[RT];
  f4 O[RT][8];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    m_run[r] = -INFINITY;
    thr[r] = -INFINITY;
    negm[r] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    Lacc[r] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int dd = 0; dd < 8; dd++) O[r][dd] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const uint32_t one2 = MT == DT_BF16 ? 0x3f803f80u : 0x3c003c00u;  // two 1.0 of the MFMA type
  const uint4 ones = make_uint4(one2, one2, one2, one2);
  // per-row mask state
  unsigned long long tbits[RT];
  const uint8_t* drow[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) {
    tbits[r] = 0ull;
    drow[r] = nullptr;
    if constexpr (MASK == MK_TREE) tbits[r] = real[r] ? p.tree[b * p.tree_bs + qi[r]] : 0ull;
    if constexpr (MASK == MK_DENSE) drow[r] = p.dense + b * p.msb + head[r] * p.msh + qi[r] * p.msq;
  }

  // The MFMA operand fragments of a tile.  8-bit: from the dequantized buffers.  16-bit: from the tile slot S --
  // K: key 16 t + c16, dims 32 kk + 8 q4 .. +7 (one 16-byte chunk); V^T: lane (g = q4, m = c16) points the
  // transposing read at key 32 u + 4 g + m / 4 (and + 16 for the second half), dims 16 dd + 4 (m % 4) .. +3, so
  // its 8 values are dim 16 dd + m of the keys whose P^T the B operand holds at k = 8 q4 + j.
  const int sk16 = swk(c16);
  const int vkey16 = 4 * q4 + (c16 >> 2), vsw16 = swv(vkey16);
  const int vch16 = (c16 & 3) >> 1, voff16 = vkey16 * 256 + 8 * (c16 & 1);
  auto kfrag = [&](const uint8_t* S, int ob, int t, int kk) __attribute__((always_inline)) -> uint4 {
    if constexpr (FMT == KV_Q8)
      return *reinterpret_cast<const uint4*>(&Ks[ob * (kKT * kKsStride) + (16 * t + c16) * kKsStride + 8 * q4 + 32 * kk]);
    else
      return *reinterpret_cast<const uint4*>(S + (16 * t + c16) * 256 + 16 * ((4 * kk + q4) ^ sk16));
  };
  auto vfrag = [&](const uint8_t* S, int ob, int u, int dd) __attribute__((always_inline)) -> uint4 {
    // the V region: the slot's second half (16-bit), the dequantized buffer Vk (8-bit), the same layout
    const uint8_t* a =
        (FMT == KV_Q8 ? Vk + ob * (kKT * 256) : S + 16384) + voff16 + 32 * u * 256 + 16 * ((2 * dd + vch16) ^ vsw16);
    const uint2 lo = lds_read_tr16(a), hi = lds_read_tr16(a + 16 * 256);
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
  };

  // Each K / V^T operand fragment is read from LDS once and applied to every row tile of the wave, so a
  // fragment is live for RT MFMAs only (the row tiles' scores, P and O are what stays in registers).
  // whether row tile r's row (this lane's) sees key j
  auto key_visible = [&](int r, int j) __attribute__((always_inline)) -> bool {
    bool ok = real[r] & (j >= klo) & (j < khi);
    if constexpr (MASK == MK_CAUSAL) ok = ok & (j <= p.N - p.L + qi[r]);
    if constexpr (MASK == MK_WINDOW) {
      const int pos = p.N - p.L + qi[r];
      ok = ok & (j <= pos) & (j > pos - p.window);
    }
    if constexpr (MASK == MK_TREE) {
      const int d = j - (p.N - p.L);
      ok = ok & ((d < 0) | (((tbits[r] >> (d & 63)) & 1ull) != 0ull));
    }
    if constexpr (MASK == MK_DENSE) ok = ok & (drow[r][min(max(j, 0), p.N - 1) * p.msk] != 0);
    return ok;
  };
  auto compute = [&](int t0, const uint8_t* S, int ob) __attribute__((always_inline)) {
    // S^T = K Q^T: st[r][t][i] = S[row][t0 + 16 t + 4 q4 + i].  Where registers allow (causal and window masks,
    // one row tile), the 32-dim step kk is the outer loop, so the 4 RT accumulators are independent chains and a
    // step's four K fragments are read together; otherwise a key block t at a time.
    constexpr bool kStepOuter = MASK == MK_CAUSAL || MASK == MK_WINDOW || RT == 1;
    f4 st[RT][4];  // relative to m_run: every chain starts from negm
    // a tile every key of which every row of the wave sees needs no mask (for causal prefill, all but the
    // diagonal tiles); rows past the row count are not written, so they need none either
    bool full = t0 >= klo && t0 + kKT <= khi;
    if constexpr (MASK == MK_CAUSAL) full = full && t0 + kKT - 1 <= p.N - p.L + wave_q0;
    if constexpr (MASK == MK_TREE) full = full && t0 + kKT <= p.N - p.L;
    if constexpr (MASK == MK_WINDOW)  // causal for the wave's first query, in the window of its last
      full = full && t0 + kKT - 1 <= p.N - p.L + wave_q0 &&
             t0 > p.N - p.L + (row0 + 16 * NW * (RT - 1) + 16 * wave + 15) / p.G - p.window;
    if constexpr (MASK == MK_DENSE) full = false;
    if constexpr (kStepOuter) {
      // The mask enters as the accumulators' initial value (-m_run or -inf), so the scores need no pass after the
      // products and a full tile's first step takes negm as it is.  Every key row of the tile is finite: rows
      // outside [klo, khi) were cleared in the slot (16-bit) or dequantized as 0 (8-bit).
      uint4 kf[4];
#pragma unroll
      for (int t = 0; t < 4; t++) kf[t] = kfrag(S, ob, t, 0);
      if (full) {
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < RT; r++) st[r][t] = mma32<MT>(kf[t], qb[r][0], negm[r]);
      } else {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
          for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
              st[r][t][i] = key_visible(r, t0 + 16 * t + 4 * q4 + i) ? negm[r][0] : -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < RT; r++) st[r][t] = mma32<MT>(kf[t], qb[r][0], st[r][t]);
      }
#pragma unroll
      for (int kk = 1; kk < 4; kk++) {
#pragma unroll
        for (int t = 0; t < 4; t++) kf[t] = kfrag(S, ob, t, kk);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < RT; r++) st[r][t] = mma32<MT>(kf[t], qb[r][kk], st[r][t]);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          const uint4 kf = kfrag(S, ob, t, kk);
#pragma unroll
          for (int r = 0; r < RT; r++) st[r][t] = mma32<MT>(kf, qb[r][kk], kk ? st[r][t] : negm[r]);
        }
    }
    uint4 pb[RT][2];  // P^T as B operands: k index 8 q4 + j <-> key 32 u + (j < 4 ? 4 q4 + j : 16 + 4 q4 + j - 4)
#pragma unroll
    for (int r = 0; r < RT; r++) {
      float tmax = -INFINITY;
      if (kStepOuter || full) {  // 16 scores in eight 3-input maxima
        const f4 *a = st[r];
        const float x0 = vmax3(a[0][0], a[0][1], a[0][2]), x1 = vmax3(a[0][3], a[1][0], a[1][1]);
        const float x2 = vmax3(a[1][2], a[1][3], a[2][0]), x3 = vmax3(a[2][1], a[2][2], a[2][3]);
        const float x4 = vmax3(a[3][0], a[3][1], a[3][2]);
        tmax = vmax(vmax3(x0, x1, x2), vmax3(x3, x4, a[3][3]));
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float sc = key_visible(r, t0 + 16 * t + 4 * q4 + i) ? st[r][t][i] : -INFINITY;
            st[r][t][i] = sc;
            tmax = vmax(tmax, sc);
          }
        }
      }
      tmax = max_x32(max_x16(tmax));  // relative to m_run (absolute before the first key)
      if (tmax > thr[r]) {  // lane-local rescale (O^T rows live in this lane column)
        const float corr = m_run[r] == -INFINITY ? 0.0f : fast_exp2(-tmax);
        m_run[r] = m_run[r] == -INFINITY ? tmax : m_run[r] + tmax;
        negm[r] = f4{-m_run[r], -m_run[r], -m_run[r], -m_run[r]};
        thr[r] = kThr;
        Lacc[r] *= corr;
#pragma unroll
        for (int dd = 0; dd < 8; dd++) O[r][dd] *= corr;
#pragma unroll
        for (int t = 0; t < 4; t++) st[r][t] -= f4{tmax, tmax, tmax, tmax};
      }
      // scores are relative to m_run; a row that has seen no key yet has only -inf here: exp2(-inf) = 0
      uint32_t pw[4][2];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pv[i] = fast_exp2(st[r][t][i]);  // -inf -> 0
        pw[t][0] = pack2<MT>(pv[0], pv[1]);
        pw[t][1] = pack2<MT>(pv[2], pv[3]);
      }
      pb[r][0] = make_uint4(pw[0][0], pw[0][1], pw[1][0], pw[1][1]);
      pb[r][1] = make_uint4(pw[2][0], pw[2][1], pw[3][0], pw[3][1]);
    }
    // O^T += V^T P^T, 32 keys a step; the denominator as ones times P^T
#pragma unroll
    for (int u = 0; u < 2; u++) {
#pragma unroll
      for (int dd = 0; dd < 8; dd++) {
        const uint4 vf = vfrag(S, ob, u, dd);
#pragma unroll
        for (int r = 0; r < RT; r++) O[r][dd] = mma32<MT>(vf, pb[r][u], O[r][dd]);
      }
#pragma unroll
      for (int r = 0; r < RT; r++) Lacc[r] = mma32<MT>(ones, pb[r][u], Lacc[r]);
    }
  };

  const int tfirst = klo & ~(kKT - 1);
  if constexpr (kRegPipe) {
    constexpr int kWaitLds = (0x3 << 14) | (0x7 << 4) | 0xF;
    auto barrier = [&]() __attribute__((always_inline)) {
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    auto stage_any = [&](int t0, const RawTile& T, int ob) __attribute__((always_inline)) {
      if (t0 >= klo && t0 + kKT <= khi) stage(t0, T, std::false_type{}, ob);
      else stage(t0, T, std::true_type{}, ob);
    };
    // tile i's codes sit in TA (i even) or TB (i odd) from two steps before it is staged.  Every step issues its
    // loads, past the last tile as a reload of it (an L2 hit): with a load skipped on some path, the in-order
    // counter could no longer wait for one tile's loads while the next tile's stay in flight.
    const int tlast = (khi - 1) & ~(kKT - 1);
    RawTile TA, TB;
    load_glb(tfirst, TA);
    load_glb(min(tfirst + kKT, tlast), TB);
    load_q();
    stage_any(tfirst, TA, 0);
    load_glb(min(tfirst + 2 * kKT, tlast), TA);
    // At the barrier every wave has staged tile t0 into buffer ob and is done multiplying the previous tile from
    // buffer ob ^ 1, which then takes tile t0 + 64 (codes in Tn, which then takes the codes of tile t0 + 192).
    auto step = [&](int t0, int ob, RawTile& Tn) __attribute__((always_inline)) {
      barrier();
      compute(t0, nullptr, ob);
      if (t0 + kKT < khi) stage_any(t0 + kKT, Tn, ob ^ 1);
      load_glb(min(t0 + 3 * kKT, tlast), Tn);
    };
    for (int t0 = tfirst;;) {
      step(t0, 0, TB);
      t0 += kKT;
      if (t0 >= khi) break;
      step(t0, 1, TA);
      t0 += kKT;
      if (t0 >= khi) break;
    }
  } else if constexpr (FMT == KV_Q8) {
    // s_waitcnt vmcnt(5) (the other slot's five loads of this wave may stay in flight), vmcnt(0), lgkmcnt(0)
    constexpr int kWaitOne = (0xF << 8) | (0x7 << 4) | (NW == 4 ? 5 : 3);
    constexpr int kWaitAll = (0xF << 8) | (0x7 << 4);
    constexpr int kWaitLds = (0x3 << 14) | (0x7 << 4) | 0xF;
    // a workgroup barrier for LDS that leaves the other slot's loads in flight (__syncthreads would wait for them)
    auto barrier = [&]() __attribute__((always_inline)) {
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    auto step = [&](int t0, uint8_t* S) __attribute__((always_inline)) {
      if (t0 + kKT < khi) __builtin_amdgcn_s_waitcnt(kWaitOne);
      else __builtin_amdgcn_s_waitcnt(kWaitAll);
      barrier();  // the slot's tile is in LDS; every wave is done with the previous tile's operands
      RawTile T;
      load_lds(S, T);
      if (t0 >= klo && t0 + kKT <= khi) stage(t0, T, std::false_type{}, 0);
      else stage(t0, T, std::true_type{}, 0);
      barrier();  // operands ready; the slot is free
      if (t0 + 2 * kKT < khi) dma(t0 + 2 * kKT, S);
      compute(t0, S, 0);
    };
    dma(tfirst, raw0);
    if (tfirst + kKT < khi) dma(tfirst + kKT, raw1);
    load_q();
    for (int t0 = tfirst;;) {
      step(t0, raw0);
      t0 += kKT;
      if (t0 >= khi) break;
      step(t0, raw1);
      t0 += kKT;
      if (t0 >= khi) break;
    }
  } else {
    // 16-bit: wave w loads key rows 64 / NW w .. of K and of V (16 / NW instructions of 1 KB each), chunk c of
    // row r to slot c ^ swk(r) (K) or c ^ swv(r) (V)
    constexpr int kWaitAll = (0xF << 8) | (0x7 << 4);
    constexpr int kWaitLds = (0x3 << 14) | (0x7 << 4) | 0xF;
    auto barrier = [&]() __attribute__((always_inline)) {
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    auto dma16t = [&](int t0, uint8_t* S) __attribute__((always_inline)) {
      const uint32_t ls = lds_addr(S);
      constexpr int kPieces = 16 / NW;  // 1 KB pieces (4 key rows) of K and of V a wave sends
#pragma unroll
      for (int u = 0; u < kPieces; u++) {
        const int r = 4 * kPieces * wave + 4 * u + (lane >> 4);
        const uint32_t voff = uint32_t(t0 + r) * 256u + 16u * uint32_t(lane & 15);
        dma16(dk16, ls + 1024u * uint32_t(kPieces * wave + u), voff ^ (16u * uint32_t(swk(r))));
        dma16(dv16, ls + 16384u + 1024u * uint32_t(kPieces * wave + u), voff ^ (16u * uint32_t(swv(r))));
      }
    };
    // a tile reaching past [klo, khi): the K and V rows of keys outside it are cleared (rows past n or before
    // start may hold anything, 0 * inf is not 0, and a masked score starts at -inf, which a NaN product would undo)
    auto clear_v = [&](int t0, uint8_t* S) __attribute__((always_inline)) {
      const int key = tid / NW, kg = t0 + key;  // NW threads a key row, 256 / NW bytes each
      if (kg < klo || kg >= khi) {
        uint4* row = reinterpret_cast<uint4*>(S + 16384 + key * 256 + (256 / NW) * (tid % NW));
        uint4* krow = reinterpret_cast<uint4*>(S + key * 256 + (256 / NW) * (tid % NW));
#pragma unroll
        for (int i = 0; i < 16 / NW; i++) row[i] = krow[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    };
    // One barrier a tile: at its top every wave's loads of this tile are in slot S and every wave is done with
    // the previous tile, whose slot (Snext) then takes the next tile's loads, in flight while this tile is
    // multiplied.
    auto step = [&](int t0, uint8_t* S, uint8_t* Snext) __attribute__((always_inline)) {
      __builtin_amdgcn_s_waitcnt(kWaitAll);  // this wave's loads of the tile: the only ones in flight
      barrier();
      if (t0 + kKT < khi) dma16t(t0 + kKT, Snext);
      if (t0 < klo || t0 + kKT > khi) {
        clear_v(t0, S);
        barrier();
      }
      compute(t0, S, 0);
    };
    dma16t(tfirst, raw0);
    load_q();
    for (int t0 = tfirst;;) {
      step(t0, raw0, raw1);
      t0 += kKT;
      if (t0 >= khi) break;
      step(t0, raw1, raw0);
      t0 += kKT;
      if (t0 >= khi) break;
    }
  }

  // ---- each row's part: m, l, o[dims]
#pragma unroll
  for (int r = 0; r < RT; r++) {
    const float l = Lacc[r][0];  // every lane of the row holds the whole sum
    if (!real[r]) continue;
    if (p.direct) {  // the only chunk: join with the sink here, as sdpa_combine would
      const size_t row = (size_t(b) * p.H + head[r]) * p.L + qi[r];
      const float sink = p.sinks ? p.sinks[head[r]] * kLog2e : -INFINITY;
      const float M = fmaxf(m_run[r], sink);
      float f = 0.0f, Lt = 0.0f;
      if (M != -INFINITY) {
        f = m_run[r] == -INFINITY ? 0.0f : fast_exp2(m_run[r] - M);
        Lt = f * l + (sink == -INFINITY ? 0.0f : fast_exp2(sink - M));
      }
      const float w = Lt > 0.0f ? f / Lt : 0.0f;
#pragma unroll
      for (int dd = 0; dd < 8; dd++)
        store4_from_f32(p.out, row * kD + 16 * dd + 4 * q4, O[r][dd][0] * w, O[r][dd][1] * w, O[r][dd][2] * w,
                        O[r][dd][3] * w, p.odt);
      continue;
    }
    const size_t part = ((size_t(b) * p.H + head[r]) * p.L + qi[r]) * p.nchunks + c;
    if (q4 == 0) {
      p.pm[part] = m_run[r];
      p.pl[part] = l;
    }
    if (m_run[r] == -INFINITY) continue;
    float4* po4 = reinterpret_cast<float4*>(p.po + part * kD);
#pragma unroll
    for (int dd = 0; dd < 8; dd++) po4[4 * dd + q4] = make_float4(O[r][dd][0], O[r][dd][1], O[r][dd][2], O[r][dd][3]);
  }
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

// One online pass over the chunks (running max, rescaled sums), their loads issued ahead of the merges; a half
// wave a row, 4 dims a lane.  Chunks with m = -inf (no key; their o was not written) weigh 0.
__global__ __launch_bounds__(256) void sdpa_combine(SdpaCombineParams p) {
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int lane = threadIdx.x & 31;
  if (row >= p.rows) return;
  const int head = (row / p.L) % p.H;
  const size_t base = size_t(row) * p.nchunks;
  const float4* po4 = reinterpret_cast<const float4*>(p.po) + base * (kD / 4) + lane;
  float m = -INFINITY, L = 0.0f;
  float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  // eight chunks at a time, all their loads issued before any merge: the index is clamped rather than tested, so
  // the loads sit in one block (a test around each made every chunk a load-wait-load-wait round trip), and a chunk
  // with no key (m = -inf, its o left unwritten) is merged by selects as weight 0 -- the same result as skipping it
  for (int c0 = 0; c0 < p.nchunks; c0 += 8) {
    float mc[8], lc[8];
    float4 oc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int c = min(c0 + i, p.nchunks - 1);
      mc[i] = p.pm[base + c];
      lc[i] = p.pl[base + c];
      oc[i] = po4[size_t(c) * (kD / 4)];
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const bool ok = c0 + i < p.nchunks && mc[i] > -INFINITY;
      const float mn = ok ? fmaxf(m, mc[i]) : m;
      const float a = !ok ? 1.0f : m == -INFINITY ? 0.0f : fast_exp2(m - mn), w = ok ? fast_exp2(mc[i] - mn) : 0.0f;
      const float4 x = ok ? oc[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      const float lx = ok ? lc[i] : 0.0f;
      o.x = o.x * a + x.x * w;
      o.y = o.y * a + x.y * w;
      o.z = o.z * a + x.z * w;
      o.w = o.w * a + x.w * w;
      L = L * a + lx * w;
      m = mn;
    }
  }
  const float sink = p.sinks ? p.sinks[head] * kLog2e : -INFINITY;
  const float M = fmaxf(m, sink);
  float f = 0.0f, Lt = 0.0f;
  if (M != -INFINITY) {
    f = m == -INFINITY ? 0.0f : fast_exp2(m - M);
    Lt = f * L + (sink == -INFINITY ? 0.0f : fast_exp2(sink - M));
  }
  const float w = Lt > 0.0f ? f / Lt : 0.0f;
  const size_t ob = size_t(row) * kD + 4 * lane;
  store4_from_f32(p.out, ob, o.x * w, o.y * w, o.z * w, o.w * w, p.odt);
}

template <int QDT, int SDT, int FMT, int MT, int MASK>
static void launch_rt(int rt, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const SdpaParams& p) {
  // two row tiles: 16-bit keys and values without a dense mask, 8-bit without a dense or window mask (their
  // per-key tests for two tiles would not fit beside the staging registers)
  if constexpr ((FMT == KV_16 && (MASK == MK_CAUSAL || MASK == MK_NONE || MASK == MK_WINDOW)) ||
                (FMT == KV_Q8 && (MASK == MK_CAUSAL || MASK == MK_NONE))) {
    if (rt == 2 && p.nw == 8) {
      hipExtLaunchKernelGGL((sdpa_pass1<QDT, SDT, FMT, MT, MASK, 2, 8>), grid, dim3(512), 0, s, e0, e1, 0, p);
      return;
    }
  }
  if constexpr (MASK != MK_DENSE && (FMT == KV_16 || MASK != MK_WINDOW)) {
    if (rt == 2) {
      hipExtLaunchKernelGGL((sdpa_pass1<QDT, SDT, FMT, MT, MASK, 2>), grid, dim3(256), 0, s, e0, e1, 0, p);
      return;
    }
  }
  hipExtLaunchKernelGGL((sdpa_pass1<QDT, SDT, FMT, MT, MASK, 1>), grid, dim3(256), 0, s, e0, e1, 0, p);
}

template <int QDT, int SDT, int FMT, int MT>
static void launch_mask(int rt, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const SdpaParams& p) {
  switch (p.mask) {
    case MK_CAUSAL: launch_rt<QDT, SDT, FMT, MT, MK_CAUSAL>(rt, grid, s, e0, e1, p); break;
    case MK_TREE: launch_rt<QDT, SDT, FMT, MT, MK_TREE>(rt, grid, s, e0, e1, p); break;
    case MK_DENSE: launch_rt<QDT, SDT, FMT, MT, MK_DENSE>(rt, grid, s, e0, e1, p); break;
    case MK_WINDOW: launch_rt<QDT, SDT, FMT, MT, MK_WINDOW>(rt, grid, s, e0, e1, p); break;
    default: launch_rt<QDT, SDT, FMT, MT, MK_NONE>(rt, grid, s, e0, e1, p); break;
  }
}

template <int FMT>
static void launch_fmt(int qdt, int sdt, int rt, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1,
                       const SdpaParams& p) {
  // MFMA type: bf16 when the keys/values (or their scales) are bf16, fp16 otherwise
  if (sdt == DT_BF16) {
    if (qdt == DT_F16) launch_mask<DT_F16, DT_BF16, FMT, DT_BF16>(rt, grid, s, e0, e1, p);
    else if (qdt == DT_BF16) launch_mask<DT_BF16, DT_BF16, FMT, DT_BF16>(rt, grid, s, e0, e1, p);
    else launch_mask<DT_F32, DT_BF16, FMT, DT_BF16>(rt, grid, s, e0, e1, p);
  } else {
    if (qdt == DT_F16) launch_mask<DT_F16, DT_F16, FMT, DT_F16>(rt, grid, s, e0, e1, p);
    else if (qdt == DT_BF16) launch_mask<DT_BF16, DT_F16, FMT, DT_F16>(rt, grid, s, e0, e1, p);
    else launch_mask<DT_F32, DT_F16, FMT, DT_F16>(rt, grid, s, e0, e1, p);
  }
}

}  // namespace lcl

using namespace lcl;

// Keys a pass-1 workgroup reads: the caller's block, or enough chunks that the grid (about B H L / wg_rows row
// blocks times the chunks) fills one resident round of `round` workgroups (~512 four-wave ones, two a CU; 256
// eight-wave ones) -- no more: every extra chunk adds a 520-byte part per row to write and read back.  One chunk
// (most prefill) writes the output directly.  For the same rows the eight-wave count never exceeds the four-wave
// one: ceil(R / 128) <= 2 ceil(R / 256).
static int sdpa_chunk(int block, int B, int H, int L, int N, int wg_rows, int round = 512) {
  if (block > 0) return block;
  const int tiles = max(1, (N + kKT - 1) / kKT);
  const long long rowblocks = max(1LL, ((long long)B * H * L + wg_rows - 1) / wg_rows);
  const int want = int(min((long long)tiles, max(1LL, (round + rowblocks - 1) / rowblocks)));
  return ((tiles + want - 1) / want) * kKT;
}

// Row tiles a wave: two (128 rows a workgroup) when there are more than 64 rows, halving the operand reads (and,
// 8-bit, the dequantization) per row; one under a dense mask, and for 8-bit under a window (their per-key tests
// would not fit beside two tiles' registers).
static int sdpa_row_tiles(int rows, int mask_kind, int kvfmt) {
  return (rows > 64 && mask_kind != MK_DENSE && (kvfmt == KV_16 || mask_kind != MK_WINDOW)) ? 2 : 1;
}

// Eight-wave workgroups (256 rows, one a CU): two row tiles under a causal or no mask (and a window, 16-bit K/V),
// and only where they add no padding rows over 128-row blocks -- the rows of a (row, KV head) a multiple of 256 or
// more than 128 in the last block -- since every row of a block costs its products (a 32-query chunk at G = 4 would
// otherwise compute 256 rows for 128).
static bool sdpa_eight_waves(int rows, int mask_kind, int kvfmt) {
  if (sdpa_row_tiles(rows, mask_kind, kvfmt) != 2) return false;
  if (!(mask_kind == MK_CAUSAL || mask_kind == MK_NONE || (kvfmt == KV_16 && mask_kind == MK_WINDOW))) return false;
  return rows % 256 == 0 || rows % 256 > 128;
}

// Whether an 8-bit call dequantizes K and V once into the workspace and runs the 16-bit kernel over them.  The
// fused kernel dequantizes every tile in each workgroup that reads it, i.e. once per row block of a (row, KV head),
// so past some number of row blocks one pass over the cache costs less.  With eight-wave workgroups (256-row
// blocks, sdpa_eight_waves) that is from 12 blocks: at C4 (8 blocks of 256 rows, 16k keys) the fused kernel's
// staging cost ~16.4 us over the 16-bit kernel's pass 1 (143.3 against 126.9 us) against ~25 us for the
// dequantization and its launch, and the staging grows with the row blocks while the dequantization does not.
// Otherwise (64- or 128-row blocks) from 16 blocks (199 us fused against 26.5 + 161 us at C4 with four-wave
// workgroups).  Not under a window (a workgroup reads only its band of keys), nor when the buffers hold many
// positions past N (the pass covers every position up to cap).
static bool sdpa_dequantize_first(int kvfmt, int mask_kind, int H, int KVH, int L, int N, int cap) {
  if (kvfmt != KV_Q8 || mask_kind == MK_WINDOW || N <= 0 || cap - N > 512) return false;
  const int rows = L * (H / KVH);
  if (sdpa_eight_waves(rows, mask_kind, KV_Q8)) return (rows + 255) / 256 >= 12;
  const int rt = sdpa_row_tiles(rows, mask_kind, KV_Q8);
  return (rows + 64 * rt - 1) / (64 * rt) >= 16;
}

// the dequantized K and V of that route: two (B, KVH, cap, 128) buffers of 16-bit values
static size_t sdpa_dq_bytes(int B, int KVH, int cap) { return 2 * size_t(B) * KVH * cap * kD * 2; }
static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

extern "C" {

size_t lcl_sdpa_workspace_bytes(int B, int H, int L, int N, int block) {
  const int chunk = sdpa_chunk(block, B, H, L, N, 128);  // 128-row workgroups take the most chunks
  const int nchunks = N > 0 ? (N + chunk - 1) / chunk : 1;
  return nchunks > 1 ? size_t(B) * H * L * nchunks * (2 + kD) * sizeof(float) : 0;
}

size_t lcl_sdpa_workspace_bytes_kv(int B, int H, int KVH, int L, int N, int cap, int block, int kvfmt,
                                   int mask_kind) {
  const size_t split = lcl_sdpa_workspace_bytes(B, H, L, N, block);
  if (B <= 0 || KVH <= 0 || H % KVH || cap <= 0 || !sdpa_dequantize_first(kvfmt, mask_kind, H, KVH, L, N, cap))
    return split;
  return align256(split) + sdpa_dq_bytes(B, KVH, cap);
}

int lcl_sdpa_ex(const void* q, int qdt, int kvfmt, const uint32_t* kw, const void* ks, const void* kb,
                const uint32_t* vw, const void* vs, const void* vb, const void* kf, const void* vf, int kvdt,
                const int32_t* start, int mask_kind, int window, const unsigned long long* tree, long long tree_bs,
                const uint8_t* dense, long long msb, long long msh, long long msq, long long msk, const float* sinks,
                float scale, int B, int H, int KVH, int L, int N, int head_dim, int cap, int block, void* out,
                void* workspace, size_t workspace_bytes, void* stream_, void* ev_start, void* ev_stop) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!q || !out) return -1;
  if (head_dim != kD && !generic_head_dim_ok(head_dim, kvfmt == KV_Q8)) return -2;
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
  if (mask_kind < MK_NONE || mask_kind > MK_WINDOW) return -1;
  if ((mask_kind == MK_CAUSAL || mask_kind == MK_WINDOW) && L > N) return -1;
  if (mask_kind == MK_WINDOW && window <= 0) return -1;
  if (mask_kind == MK_TREE && (!tree || L > 64 || L > N)) return -2;
  if (mask_kind == MK_DENSE && !dense) return -1;
  if (head_dim != kD) {  // other head sizes: the generic kernel (no split, no workspace)
    GenParams g{};
    g.q = q; g.qdt = qdt; g.kvfmt = kvfmt; g.kf = kf; g.vf = vf;
    g.kw = kw; g.ks = ks; g.kb = kb; g.vw = vw; g.vs = vs; g.vb = vb; g.kvdt = kvdt;
    g.start = start; g.mask = mask_kind; g.window = window; g.tree = tree; g.tree_bs = tree_bs;
    g.dense = dense; g.msb = msb; g.msh = msh; g.msq = msq; g.msk = msk;
    g.sinks = sinks; g.scale = scale;
    g.R = B; g.H = H; g.KVH = KVH; g.L = L; g.N = N; g.D = head_dim; g.cap = cap; g.kv_rows = B;
    g.out = out; g.odt = qdt;
    hipEvent_t e0 = static_cast<hipEvent_t>(ev_start), e1 = static_cast<hipEvent_t>(ev_stop);
    if (e0) (void)hipEventRecord(e0, stream);
    const int rc = attn_generic_launch(g, stream);
    if (e1) (void)hipEventRecord(e1, stream);
    return rc;
  }
  const int rows = L * (H / KVH);
  const int rt = sdpa_row_tiles(rows, mask_kind, kvfmt);
  int chunk = sdpa_chunk(block, B, H, L, N, 64 * rt);
  int nchunks = N > 0 ? (N + chunk - 1) / chunk : 1;
  if (mask_kind == MK_WINDOW && N > 0) {
    // a workgroup's band spans at most the window, its rows' queries and the alignment of its first tile; a
    // chunk no shorter than the unwindowed one keeps the chunk count within lcl_sdpa_workspace_bytes
    const long long ext = min((long long)N, (long long)window + (64 * rt - 1) / (H / KVH) + kKT);
    chunk = max(chunk, sdpa_chunk(block, B, H, L, int(ext), 64 * rt));
    nchunks = int((ext + chunk - 1) / chunk);
  }
  const size_t need = nchunks > 1 ? size_t(B) * H * L * nchunks * (2 + kD) * sizeof(float) : 0;
  if (need && (!workspace || workspace_bytes < need)) return -3;
  hipEvent_t e0 = static_cast<hipEvent_t>(ev_start), e1 = static_cast<hipEvent_t>(ev_stop);
  // the dequantize-first route, when the caller's workspace has room for it (lcl_sdpa_workspace_bytes_kv); the
  // 16-bit kernel takes the same row tiles and chunks, so the split-K part of the workspace is unchanged
  const bool dq = sdpa_dequantize_first(kvfmt, mask_kind, H, KVH, L, N, cap) && workspace &&
                  workspace_bytes >= align256(need) + sdpa_dq_bytes(B, KVH, cap);
  if (dq) {
    _Float16* kd = reinterpret_cast<_Float16*>(static_cast<uint8_t*>(workspace) + align256(need));
    _Float16* vd = kd + size_t(B) * KVH * cap * kD;
    const int rc = dequantize_kv128(kw, ks, kb, vw, vs, vb, kvdt, (long long)B * KVH * cap, kd, vd, stream);
    if (rc) return rc;
    kvfmt = KV_16;
    kf = kd;
    vf = vd;
  }
  // Eight-wave workgroups of 256 rows where sdpa_eight_waves allows them, one a CU, so each K/V tile the workgroup
  // loads (and, 8-bit, dequantizes) into LDS serves twice the rows (C4's 16-bit pass 1: 131.7 -> 123.7 us; its
  // fused 8-bit pass 1: 167.1 -> 143.3 us, its codes fed through registers).  They are taken only where their chunk count is at most the four-wave
  // one the workspace was checked for.
  int nw = sdpa_eight_waves(rows, mask_kind, kvfmt) ? 8 : 4;
  if (nw == 8 && N > 0) {
    int c8 = sdpa_chunk(block, B, H, L, N, 256, 256);
    int n8 = (N + c8 - 1) / c8;
    if (mask_kind == MK_WINDOW) {  // as above, for a 256-row workgroup's band
      const long long ext = min((long long)N, (long long)window + 255 / (H / KVH) + kKT);
      c8 = max(c8, sdpa_chunk(block, B, H, L, int(ext), 256, 256));
      n8 = int((ext + c8 - 1) / c8);
    }
    // and only where their grid still fills the CUs (a short context leaves few chunks to split)
    const long long grid8 = (long long)n8 * ((rows + 255) / 256) * B * KVH;
    if (n8 <= nchunks && grid8 >= 256) {
      chunk = c8;
      nchunks = n8;
    } else {
      nw = 4;
    }
  }
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
  p.nchunks = nchunks; p.chunk = chunk; p.mask = mask_kind; p.window = window;
  p.direct = nchunks == 1; p.out = out; p.odt = qdt;
  p.nw = nw;
  p.nrowblocks = (rows + 16 * nw * rt - 1) / (16 * nw * rt);
  {  // with no key in reach every workgroup records empty parts, so the combine needs no cleared workspace
    const long long total = (long long)nchunks * p.nrowblocks * B * KVH;  // one-dimensional, mapped per XCD
    if (total > (1LL << 30)) return -2;
    const dim3 grid(unsigned((total + 7) / 8 * 8));
    if (kvfmt == KV_Q8) launch_fmt<KV_Q8>(qdt, kvdt, rt, grid, stream, e0, e1, p);
    else launch_fmt<KV_16>(qdt, kvdt, rt, grid, stream, e0, e1, p);
  }
  if (!p.direct) {
    SdpaCombineParams c{p.pm, p.pl, p.po, sinks, out, B * H * L, H, L, nchunks, qdt};
    hipLaunchKernelGGL(sdpa_combine, dim3((B * H * L + 7) / 8), dim3(256), 0, stream, c);
  }
  return int(hipGetLastError());
}

int lcl_sdpa(const void* q, int qdt, int kvfmt, const uint32_t* kw, const void* ks, const void* kb,
             const uint32_t* vw, const void* vs, const void* vb, const void* kf, const void* vf, int kvdt,
             const int32_t* start, int mask_kind, int window, const unsigned long long* tree, long long tree_bs,
             const uint8_t* dense, long long msb, long long msh, long long msq, long long msk, const float* sinks,
             float scale, int B, int H, int KVH, int L, int N, int head_dim, int cap, int block, void* out,
             void* workspace, size_t workspace_bytes, void* stream) {
  return lcl_sdpa_ex(q, qdt, kvfmt, kw, ks, kb, vw, vs, vb, kf, vf, kvdt, start, mask_kind, window, tree, tree_bs, dense, msb,
                     msh, msq, msk, sinks, scale, B, H, KVH, L, N, head_dim, cap, block, out, workspace,
                     workspace_bytes, stream, nullptr, nullptr);
}

}  // extern "C"
