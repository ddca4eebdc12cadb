// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Conventions used by every kernel in this directory:
//  * wave64; MFMA v_mfma_f32_16x16x16{f16,bf16_1k} operand layout:
//      A (16 x 16, M x K): lane l holds A[l % 16][4 * (l / 16) + i], i = 0..3
//      B (16 x 16, K x N): lane l holds B[4 * (l / 16) + i][l % 16]
//      D (16 x 16, M x N): lane l holds D[4 * (l / 16) + i][l % 16]
//    (checked on an MI355X by an in-bounds probe of the builtin).
//  * An 8-bit code c becomes the exact fp16 value 1024 + c by byte-permuting it
//    under the exponent byte 0x64 (fp16 0x64cc == 1024 + cc); the constant 1024
//    is folded back out in fp32 by each kernel.
//  * Status codes: 0 ok, negative = argument error (see include/locals_amd.h),
//    positive = hipError_t passed through.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lcl {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum Dtype { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }

// round-to-nearest-even float -> bf16 bits (inputs here are finite)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) return uint16_t((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// value of a 16-bit (or fp32) element of dtype dt
__device__ __forceinline__ float load_as_f32(const void* p, size_t i, int dt) {
  if (dt == DT_F16) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == DT_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_from_f32(void* p, size_t i, float v, int dt) {
  if (dt == DT_F16) static_cast<_Float16*>(p)[i] = _Float16(v);
  else if (dt == DT_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else static_cast<float*>(p)[i] = v;
}

// elements i .. i + 3 of dtype dt: one 8-byte store (16-bit) or 16-byte store (fp32) where the address is aligned
// for it, else four element stores; the same rounding as store_from_f32
__device__ __forceinline__ void store4_from_f32(void* p, size_t i, float a, float b, float c, float d, int dt) {
  if (dt == DT_F32) {
    float* q = static_cast<float*>(p) + i;
    if ((reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
      *reinterpret_cast<float4*>(q) = make_float4(a, b, c, d);
      return;
    }
  } else {
    uint16_t* q = static_cast<uint16_t*>(p) + i;
    if ((reinterpret_cast<uintptr_t>(q) & 7u) == 0) {
      uint16_t h[4];
      if (dt == DT_BF16) {
        h[0] = f32_to_bf16_bits(a); h[1] = f32_to_bf16_bits(b); h[2] = f32_to_bf16_bits(c); h[3] = f32_to_bf16_bits(d);
      } else {
        h[0] = __builtin_bit_cast(uint16_t, _Float16(a)); h[1] = __builtin_bit_cast(uint16_t, _Float16(b));
        h[2] = __builtin_bit_cast(uint16_t, _Float16(c)); h[3] = __builtin_bit_cast(uint16_t, _Float16(d));
      }
      *reinterpret_cast<uint2*>(q) = make_uint2(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16));
      return;
    }
  }
  store_from_f32(p, i + 0, a, dt);
  store_from_f32(p, i + 1, b, dt);
  store_from_f32(p, i + 2, c, dt);
  store_from_f32(p, i + 3, d, dt);
}

// element k (0/1) of a packed pair of 16-bit values of dtype dt
__device__ __forceinline__ float half_of(uint32_t w, int k, int dt) {
  const uint16_t b = uint16_t(k ? (w >> 16) : (w & 0xffffu));
  return dt == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// bytes 0,1 (sel 0x00050004) or 2,3 (sel 0x00070006) of x as two fp16 values 1024 + byte
__device__ __forceinline__ uint32_t codes_to_h2(uint32_t x, uint32_t sel) {
  return __builtin_amdgcn_perm(x, 0x64646464u, sel);
}

__device__ __forceinline__ h4 codes4_to_h4(uint32_t x) {
  const uint32_t lo = codes_to_h2(x, 0x00050004u), hi = codes_to_h2(x, 0x00070006u);
  return __builtin_bit_cast(h4, (uint64_t(hi) << 32) | lo);
}

__device__ __forceinline__ h4 pack_h4(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(h4, (uint64_t(hi) << 32) | lo);
}

__device__ __forceinline__ s4 pack_s4(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(s4, (uint64_t(hi) << 32) | lo);
}

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16bf(s4 a, s4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// two floats -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t pkrn(float a, float b) {
  return __builtin_bit_cast(uint32_t, h2{_Float16(a), _Float16(b)});
}

// w ~= hi + lo with hi, lo fp16, both rounded to nearest: hi = fp16(w), lo = fp16(w - hi) (w - hi is exact in
// fp32).  While lo is a normal fp16 (|w| >= 2^-3) |w - hi - lo| <= 2^-22 |w|; below that lo is subnormal and the
// error is at most 2^-25 absolute, so callers scale w up to the top of fp16's range first.
__device__ __forceinline__ void split_h2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pkrn(a, b);
  asm("" : "+v"(hi));  // convert the pair back from the packed word (otherwise each half is converted twice)
  const h2 h = __builtin_bit_cast(h2, hi);
  lo = pkrn(a - float(h.x), b - float(h.y));
}

// ---- prescale of the V weights in the 8-bit decode kernels
// P V multiplies A = w = p * v_scale (as split_h2's hi + lo) by B = 1024 + code.  The softmax keeps a lazy running
// max m (a tile's scores are at most m + 6, so p = 2^(s - m) <= 2^6) and exponentiates against m_ref = m - E for a
// wave-uniform integer E, so p' = 2^E p and w' = p' v_scale < 2^15 whenever every |v_scale| seen is below 2^e with
// E <= 9 - e.  E starts at kPreInit and is lowered (never raised) to 9 - e of the largest |v_scale| of a tile that
// would break the bound; l, o and the side sums all carry the same 2^E, so the partial (m_ref, l', o') has the
// value of (m, l, o).  With E near 9 - e the weights that matter sit in fp16's normal range.
constexpr int kPreInit = 40;

// e with |x| < 2^e for the 15-bit magnitude (bits & 0x7fff) of a 16-bit scale of dtype SDT
template <int SDT>
__device__ __forceinline__ int scale_exp(uint32_t mag) {
  return SDT == DT_BF16 ? int(mag >> 7) - 126 : int(mag >> 10) - 14;
}
// the least magnitude whose scale_exp exceeds 9 - E (a scale that needs E lowered)
template <int SDT>
__device__ __forceinline__ int pre_thr(int E) {
  const int k = (SDT == DT_BF16 ? 136 : 24) - E;
  return k <= 0 ? 0 : (k << (SDT == DT_BF16 ? 7 : 10));
}
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
// running max of the magnitudes of a packed pair of 16-bit scales (magnitude order = integer order of bits & 0x7fff)
__device__ __forceinline__ uint32_t mag_max2(uint32_t acc, uint32_t w) {
  const us2 a = __builtin_bit_cast(us2, acc), b = __builtin_bit_cast(us2, w & 0x7fff7fffu);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}
__device__ __forceinline__ uint32_t mag_fold(uint32_t acc) { return max(acc & 0xffffu, acc >> 16); }

// bf16 pair by truncation: hi = top 16 bits, lo = top 16 bits of the remainder
__device__ __forceinline__ void split_bf2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const uint32_t ua = __float_as_uint(a) & 0xffff0000u, ub = __float_as_uint(b) & 0xffff0000u;
  hi = (ua >> 16) | ub;
  const uint32_t ra = __float_as_uint(a - __uint_as_float(ua)), rb = __float_as_uint(b - __uint_as_float(ub));
  lo = (ra >> 16) | (rb & 0xffff0000u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Maximum of floats as v_maximum3_f32 (NaN-propagating).  fmaxf's IEEE maxNum needs quieted inputs, so the
// compiler puts a v_max_f32 x, x, x before each operand it cannot prove canonical (every MFMA result): one extra
// VALU per score.  The scores compared here hold no NaN, so the two agree on them.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmax3(float a, float b, float c) { return vmax(vmax(a, b), c); }

// Max / sum of a value with lane l ^ 16 (or l ^ 32) of the wave on gfx950's v_permlane16_swap / v_permlane32_swap:
// VALU lane exchanges instead of an LDS-routed shuffle.  With both operands x, lane l gets x of lanes l and l ^ 16
// (l ^ 32) in some order (checked in bounds on an MI355X), so a commutative op gives the xor shuffle's result.
__device__ __forceinline__ float max_x16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_x16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_x32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t BufRsrc;

// Raw buffer descriptor over `bytes` bytes at p (gfx9 word 3: 32-bit data format, as CK uses
// for gfx90a/gfx94x/gfx950).  Loads at offsets >= bytes return 0; the range check covers the
// VGPR offset and the instruction offset, so callers keep every variable part there.
__device__ __forceinline__ BufRsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, int(bytes), 0x00020000);
}

// Cache policy of a load (gfx950): 0 = default, kNT = non-temporal (aux bit 1, `nt`).  Measured
// on an MI355X, a stream of whole 128-byte lines per instruction reaches ~7.0 TB/s with `nt`
// against ~6.0 TB/s without; but where two instructions each take half of the same lines (the
// register-fed decode tiles) `nt` costs ~12%, so those loads keep the default policy.
constexpr int kNT = 2;

__device__ __forceinline__ u4 buf_load_b128(BufRsrc r, uint32_t voff, const int imm) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, int(voff + uint32_t(imm)), 0, 0);
}

__device__ __forceinline__ uint32_t buf_load_b32(BufRsrc r, uint32_t voff, const int imm) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, int(voff + uint32_t(imm)), 0, 0);
}

// Direct buffer -> LDS loads: lane l's 16 (or 4) bytes at voff land at lds + 16 l (or 4 l).  The compiler tracks
// these per __shared__ object: an LDS read waits only for loads into the object it reads.  AUX is the cache
// policy: non-temporal (the default) for data read once, as the decode kernels stream K/V; 0 where other
// workgroups of the same XCD read the same lines soon after (the masked-attention kernel's K/V, which every row
// block of a kv head reads: C5 56.3 -> 52-53 us, W1 43.7 -> 42.4 us, C4 209 -> 207 us without the hint).
template <int AUX = kNT>
__device__ __forceinline__ void lds_load16(BufRsrc r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16, voff, 0, 0, AUX);
}
template <int AUX = kNT>
__device__ __forceinline__ void lds_load4(BufRsrc r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 4, voff, 0, 0, AUX);
}

// generic.hip: attention for head sizes other than 128 (every mask kind, 16-bit or 8-bit K/V, ragged rows)
struct GenParams {
  const void* q;  // (R, H, L, D), dtype qdt
  int qdt;
  int kvfmt;  // 0: 8-bit triples, 1: 16-bit
  const void* kf;
  const void* vf;  // 16-bit (kv_rows, KVH, cap, D), dtype kvdt
  const uint32_t* kw;
  const void* ks;
  const void* kb;
  const uint32_t* vw;
  const void* vs;
  const void* vb;  // 8-bit: words (kv_rows, KVH, cap, D / 4), scales / biases (.., D / 64) of dtype kvdt
  int kvdt;
  const int32_t* slots;  // KV row of each query row, or null (row r)
  const int32_t* start;  // first key of each row, or null
  const int32_t* nkeys;  // end of each row's keys, or null (N)
  int mask, window;
  const unsigned long long* tree;
  long long tree_bs;
  const uint8_t* dense;
  long long msb, msh, msq, msk;
  const float* sinks;  // (H,) natural log units, or null
  float scale;
  const float* scale_dev;
  int R, H, KVH, L, N, D, cap, kv_rows;
  void* out;
  int odt;
};

int attn_generic_launch(const GenParams& p, hipStream_t stream);
// head sizes it takes: a multiple of 16 up to 512 (16-bit K/V), of 64 (8-bit)
inline bool generic_head_dim_ok(int D, bool q8) { return D > 0 && D <= 512 && D % (q8 ? 64 : 16) == 0; }

// quant.hip: K and V (rows of 128 values) of an 8-bit cache dequantized to the scales' 16-bit dtype in one launch
int dequantize_kv128(const uint32_t* kw, const void* ks, const void* kb, const uint32_t* vw, const void* vs,
                     const void* vb, int sdt, long long rows, void* kout, void* vout, hipStream_t stream);

}  // namespace lcl
