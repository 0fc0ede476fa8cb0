// Paged-KV grouped-query decode attention for MI355X (gfx950, CDNA4).
//
// Replaces the two Triton kernels of the reference
// (ParamThakkar123/paged-decode-attention, pagedattn/triton_decode.py):
//   _paged_decode_kernel  (:33-195)  -> paged_decode_kernel<...> (unsplit and
//                                       the reference's per-sequence split)
//                                       and paged_decode_flat_kernel<...> (a
//                                       work-balanced split, no counterpart)
//   _split_reduce_kernel  (:198-240) -> split_reduce_kernel
// and the launch section of `paged_decode_triton` (:331-376) -> pa_decode.
//
// Work decomposition (paged_decode_kernel). One workgroup of kWaves wave64s
// per (batch, kv_head, head_tile, split). The workgroup's token range
// [lo, hi) is cut into 32-token tiles; wave w takes tiles w, w + kWaves, ...
// Every wave keeps its own online-softmax state in VGPRs and the waves are
// merged once through LDS at the end, so a workgroup is a split of kWaves
// sub-splits that costs a single partial write. The flat kernel's
// decomposition is described at its definition.
//
// Each wave double-buffers its tiles in registers: the K/V loads of its next
// tile are issued before the current tile is computed, so HBM requests stay in
// flight while the MFMAs and the softmax run.
//
// Per 32-token tile (two 16-token sub-tiles, each inside one page because the
// page size is a multiple of 16):
//   S^T[tok, h] = K[tok, :] . Q[h, :]   v_mfma_f32_16x16x32_f16, A = K rows
//                                        (lane row = token), B = Q^T (lane
//                                        column = query head of the group)
//   O^T[d, h] += V^T[d, tok] P^T[tok, h] v_mfma_f32_16x16x32_f16, A = V^T,
//                                        B = P^T taken straight from the QK
//                                        accumulator layout (no shuffles)
// K rows are loaded whole (consecutive lanes, consecutive 16-byte pieces) into
// a per-wave LDS slot and read back in the MFMA A-operand layout. V rows are
// loaded in the natural [tok][d] layout, 16 lanes covering one row
// contiguously, and transposed to [d][tok] pairs in registers with v_perm.
// All `group` query heads of a kv head share the tile (padded to the 16 MFMA
// columns), so each K/V byte is read from HBM once.
//
// Online softmax in the log2 domain as the reference (triton_decode.py:155-166)
// with one change: the running maximum is only moved when a tile's maximum
// exceeds it by more than kRescaleLog2, so the accumulator rescale is skipped
// on most tiles. This is exact algebra (the normaliser uses the same stale
// maximum); probabilities stay <= 2^kRescaleLog2, far from fp16 overflow.
//
// Quantised KV is dequantised in registers to the fp16 values the reference's
// dequantised cache holds (pagedattn/cache.py:51-62), with one v_perm per
// fp16 pair:
//   fp8_e5m2 -> fp16: the e5m2 byte is the high byte of the fp16 pattern.
//   int8 K and V: with the byte's sign bit flipped (one xor per 4 bytes),
//        b ^ 0x80 = x + 128 is the mantissa of an fp16 denormal,
//        (x + 128) * 2^-24, exact (v_fma_mix keeps fp16 denormals); one
//        v_fma_mix per element forms fp16((x + 128) * 2^-24 * s * 2^24
//        - 128 * s) = fp16(x * s), the product rounded once to fp32 and then
//        to fp16 as the reference's kernel rounds it
//        (triton_decode.py:145-149). K then enters the fp16 QK MFMA and V
//        the fp16 PV MFMA exactly as an fp16 cache's rows would. (Skipping
//        the fp16 rounding of K, i.e. attending over the exact x * s, moves
//        the output by up to ~2e-3 from the reference's on peaked heads;
//        folding s into P instead would round s to fp16.)

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "pagedattn.h"
#include "pa_errors.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;          // waves per workgroup (unsplit / classic split)
constexpr int kFlatWaves = 4;      // flat kernel: one wave per SIMD of a CU (2-byte, fp8)
// Waves per flat-kernel workgroup. int8 caches launch two flat waves per SIMD
// (their dequantisation keeps one wave busy issuing VALU work), so their
// workgroup is the CU's eight waves: eight neighbouring kv heads of one range,
// a whole 1 KB token row of a Llama-shape page read together instead of two
// 512-byte halves by two workgroups (C4's decode 175.6 -> 172.7 us).
constexpr int kFlatWavesInt8 = 8;
template <int KV> constexpr int flat_waves() { return KV == PA_KV_INT8 ? kFlatWavesInt8 : kFlatWaves; }
inline int flat_waves_of(int kv) { return kv == PA_KV_INT8 ? kFlatWavesInt8 : kFlatWaves; }
constexpr int kSplitAlign = 32;    // split ranges are multiples of this many tokens
constexpr float kRescaleLog2 = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr uint32_t kInt8Sign = 0x80808080u;      // int8 x -> x + 128 in every byte
constexpr float kInt8Unit = 16777216.0f;      // 2^24: int8 V operands are (x + 128) * 2^-24
// s_waitcnt immediate (gfx9 encoding): vmcnt(0), expcnt and lgkmcnt at their maxima
constexpr int kWaitVmcnt0 = 0x0F70;
// Buffer resource word 3 for raw (stride 0) byte buffers on gfx9, and the
// non-temporal cache policy of a buffer load (bit 1 = nt).
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kLoadNT = 2;
// A flat-split wave with at most this many tiles keeps two tiles in flight:
// short ranges are latency-bound; longer ones stream faster with one.
constexpr int kDeepTiles = 16;
// Entries of the launch tables the host builds from host-side lengths (the
// flat split's ranges, the merge's sequences); larger launches scan seq_lens
// on the GPU instead.
constexpr int kHostTab = PA_HOST_TABLE_MAX;

struct KParams {
  const uint8_t *q;
  const uint8_t *k;
  const uint8_t *v;
  const uint8_t *ks;
  const uint8_t *vs;
  uint8_t *out;
  float *part_out;
  float *part_lse;
  const int32_t *bt;
  const int32_t *seq_lens;
  int32_t hkv, group, head_tiles, num_splits, num_blocks, max_blocks, log2_page, max_seq_len;
  int32_t batch, max_tokens;  // max_tokens = max_blocks << log2_page
  int32_t flat_splits;        // > 0: the flat (work-balanced) split
  int32_t flat_cost;          // flat split: tiles charged per non-empty sequence
  // Strides are 32-bit (checked on the host; kernels widen them before they
  // multiply an index): with 64-bit ones the int8 instances ran out of scalar
  // registers, and three of them carried a scratch segment for the spills.
  int32_t sqb, sqh;          // elements
  uint32_t skn;              // bytes (< 2^32)
  int32_t skt, skh;          // bytes
  uint32_t ssn;              // bytes (< 2^32)
  int32_t sst;               // bytes
  int32_t sob, soh;          // elements
  int32_t spb, sph, sps;     // elements
  int32_t slb, slh;          // elements
  int32_t sbtb;              // elements
  float qk_scale;            // sm_scale * log2(e)
  int32_t io_bf16;           // q and out are bf16 (else fp16)
};

struct RParams {
  const float *part_out;
  const float *part_lse;
  uint8_t *out;
  int32_t io_bf16;  // out is bf16 (else fp16)
  const int32_t *seq_lens;  // AUTO and FLAT merges only
  int32_t max_tokens, max_seq_len;  // AUTO and FLAT merges only
  int32_t num_heads, num_splits;    // FLAT: num_splits = flat splits
  int32_t batch;                    // FLAT only
  int32_t flat_cost;                // FLAT only: tiles charged per non-empty sequence
  int64_t spb, sph, sps, slb, slh, sob, soh;  // elements
};

// Reductions over the four lanes l, l^16, l^32, l^48 that hold one MFMA
// column (one query head). permlane16/32_swap hand each lane the values of
// lane pairs (l, l^16) and (l, l^32); every lane of the column computes the
// same expression, so the result is identical in all four.
__device__ __forceinline__ float col_max(float x) {
  const uint32_t xu = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(xu, xu, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t yu = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(yu, yu, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float col_sum(float x) {
  const uint32_t xu = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(xu, xu, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t yu = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(yu, yu, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// v_perm_b32: byte k of the result is byte sel[k] of the 8 bytes {hi, lo}
// (codes 0-3 pick `lo`, 4-7 pick `hi`, 0x0c gives 0x00).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ f16x8 as_f16x8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  u32x4 u = {w0, w1, w2, w3};
  return __builtin_bit_cast(f16x8, u);
}

// Two bf16 values (one dword) -> two fp16, each rounded to nearest even.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  const f16x2 h = {(_Float16)__uint_as_float(w << 16), (_Float16)__uint_as_float(w & 0xffff0000u)};
  return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ f16x8 bf16x8_to_f16x8(u32x4 w) {
  return as_f16x8(bf16x2_to_f16x2(w.x), bf16x2_to_f16x2(w.y), bf16x2_to_f16x2(w.z),
                  bf16x2_to_f16x2(w.w));
}

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Store n (a multiple of 4, or 2) fp32 values to an fp16 or bf16 row.
__device__ __forceinline__ void store_row(uint8_t *dst, const float *y, int n, bool bf16) {
  for (int e = 0; e + 1 < n; e += 2) {
    uint32_t w;
    if (bf16) {
      w = f32_to_bf16_bits(y[e]) | (f32_to_bf16_bits(y[e + 1]) << 16);
    } else {
      const f16x2 h = {(_Float16)y[e], (_Float16)y[e + 1]};
      w = __builtin_bit_cast(uint32_t, h);
    }
    reinterpret_cast<uint32_t *>(dst)[e / 2] = w;
  }
}

// Selector placing byte i of `lo` and byte j of `hi` into the two halves of a
// dword: as the high byte (fp8 e5m2 -> fp16) or the low byte (int8 with its
// sign bit flipped -> the fp16 denormal (x + 128) * 2^-24).
template <int KV>
__device__ __forceinline__ constexpr uint32_t pair_sel(uint32_t i, uint32_t j) {
  if constexpr (KV == PA_KV_INT8) {
    return i | (0x0cu << 8) | ((4u + j) << 16) | (0x0cu << 24);
  } else {
    return 0x0cu | (i << 8) | (0x0cu << 16) | ((4u + j) << 24);
  }
}

// Two stored bytes -> two fp16 bit patterns: one v_perm (int8 sign bits are
// flipped on the words before it).
template <int KV>
__device__ __forceinline__ uint32_t bytes_to_halves(uint32_t hi, uint32_t lo, uint32_t sel) {
  return perm(hi, lo, sel);
}

// Two fp32 values -> an fp16 pair, each rounded to nearest even
// (v_cvt_pk_f16_f32). The empty asm statements hide where a and b come from,
// so the compiler converts the fp32 values as they are instead of folding
// the conversion into the fma that produced them (v_fma_mixlo/hi_f16, which
// runs at a third of the rate of ordinary VALU ops when waves share a SIMD).
// They emit no instruction: an instruction written in asm escapes the
// compiler's hazard checks, and an MFMA reading its result one instruction
// later read a stale register.
__device__ __forceinline__ uint32_t cvt_pk_f16(float a, float b) {
  asm("" : "+v"(a));
  asm("" : "+v"(b));
  const f16x2 h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, h);
}

// int8 -> fp16(x * s), the reference's dequantised value (cache.py:51-62;
// triton_decode.py:145-149: the fp32 product rounded to fp16), for a pair of
// stored bytes whose sign bits are already flipped (b ^ 0x80 = x + 128).
//   fp16 scales: the byte under the exponent byte 0x64 is the fp16 value
//     1024 + (x + 128); minus 1152 it is x, exactly, and one fp16 multiply
//     by s rounds the exact product x * s once (an 8-bit x times an 11-bit s
//     is exact in fp32, so this equals the reference's two roundings).
//     `lo` holds both bytes (positions i, j); 3 packed ops per pair.
//   fp32 scales: the byte as the fp16 denormal (x + 128) * 2^-24 (exact), one
//     fma per element in fp32 with s * 2^24 and -128 * s gives fp32(x * s),
//     then a round to fp16: the reference's fp32 product and fp16 cast.
constexpr uint32_t kF16Exp1024 = 0x64646464u;  // exponent byte of 1024 in every byte

__device__ __forceinline__ uint32_t i8pair_fp16_scale(uint32_t lo, uint32_t i, uint32_t j, uint32_t s2) {
  const uint32_t h = perm(kF16Exp1024, lo, i | (4u << 8) | (j << 16) | (4u << 24));
  const f16x2 x = __builtin_bit_cast(f16x2, h) - f16x2{(_Float16)1152.0f, (_Float16)1152.0f};
  return __builtin_bit_cast(uint32_t, x * __builtin_bit_cast(f16x2, s2));
}

__device__ __forceinline__ uint32_t i8pair_fp32_scale(uint32_t den, float s0_24, float c0, float s1_24,
                                                      float c1) {
  const f16x2 u2 = __builtin_bit_cast(f16x2, den);
  return cvt_pk_f16(__builtin_fmaf((float)u2[0], s0_24, c0), __builtin_fmaf((float)u2[1], s1_24, c1));
}

// A raw buffer over the `bytes` bytes from `base` on: a load at a per-lane
// offset at or past `bytes` returns zeros (the range check of raw buffers).
// bytes = -1 (2^32 - 1) leaves every offset used here in range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint8_t *base, int bytes = -1) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short)0, bytes, kRsrcWord3);
}

// BYTES from the buffer at voff (per lane) + soff (uniform), non-temporal.
template <int BYTES>
__device__ __forceinline__ void buf_load_bytes(uint32_t *w, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                               uint32_t soff) {
  if constexpr (BYTES == 32) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kLoadNT);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, kLoadNT);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (BYTES == 16) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kLoadNT);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (BYTES == 8) {
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kLoadNT);
    w[0] = a.x; w[1] = a.y;
  } else if constexpr (BYTES == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kLoadNT);
  } else {
    static_assert(BYTES == 2, "unsupported load width");
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, kLoadNT);
  }
}

// The bits of one scale (fp16 scales in the low half).
template <int SC>
__device__ __forceinline__ uint32_t load_scale_bits(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  if constexpr (SC == PA_SCALE_FP32) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
  } else {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
  }
}

// Block tables and lengths are read-only for a whole launch. Reading them
// through the constant address space lets the compiler use scalar loads for
// the wave-uniform reads even in kernels that store inside their tile loop;
// a scalar load's wait (lgkmcnt) never holds back the K/V loads in flight,
// where a vector load's (vmcnt) would wait for them.
typedef __attribute__((address_space(4))) const int32_t ro_i32;
__device__ __forceinline__ const ro_i32 *ro(const int32_t *ptr) { return (const ro_i32 *)ptr; }

// Compile-time geometry for one (KV dtype, head_dim) instance.
//
// K is fetched in whole rows: consecutive lanes read consecutive 16-byte
// pieces of a (token, kv_head) row, kKLanesPerRow lanes per row, so every
// load instruction covers complete rows (as V's loads do). Rows arrive in a
// per-wave LDS slot (padded by 16 bytes per row, which makes both the row
// writes and the operand reads bank-conflict free) and are read back in the
// MFMA A layout: lane (c, r) takes row r, head-dim elements [32*ks + 8*c, +8)
// for k-step ks. Q uses the same mapping, which is all the reduction needs.
template <int KV, int D>
struct Geo {
  static constexpr int kElem = (KV == PA_KV_FP16 || KV == PA_KV_BF16) ? 2 : 1;  // stored bytes/elem
  static constexpr int kKSteps = D / 32;                    // QK MFMAs per sub-tile (fp16 operands)
  static constexpr int kE = D / 16;                         // V elems per lane row
  static constexpr int kVBytes = kE * kElem;                // V bytes per lane row
  static constexpr int kVWords = (kVBytes + 3) / 4;
  static constexpr int kRowBytes = D * kElem;               // one K/V row
  // A wave iteration covers kNSub 16-token sub-tiles (the code takes any
  // even count). 64-token tiles for 128-byte rows (1-byte KV) were measured
  // 1-3% slower than 32-token ones, so every geometry uses 2.
  static constexpr int kNSub = 2;
  static constexpr int kTT = 16 * kNSub;                    // tokens per tile
  static constexpr int kVRows = 4 * kNSub;                  // V rows per lane
  static constexpr int kKLanesPerRow = kRowBytes / 16;      // 2 .. 32
  static constexpr int kKRowsPerLoad = 64 / kKLanesPerRow;  // rows per instruction
  static constexpr int kKLoads = kTT / kKRowsPerLoad;       // K loads per tile
  static constexpr int kKSlotStride = kRowBytes + 16;       // padded LDS row
  static constexpr int kKSlotBytes = kTT * kKSlotStride;    // per wave
  static constexpr int kScales = 2 * kTT;                   // int8: K and V scales per tile
  // double-buffer the tile registers unless, with the accumulators and the Q
  // operands, they would crowd out the rest (the budget is set by the
  // largest instance that measured best double-buffered: fp16 at D = 128)
  static constexpr int kTileWords = 4 * kKLoads + kVRows * kVWords;
  static constexpr bool kPrefetch = 2 * kTileWords + 4 * kE + 4 * kKSteps <= 176;
};

// Registers of one tile of one wave.
template <int KV, int D>
struct Tile {
  using G = Geo<KV, D>;
  u32x4 k[G::kKLoads];               // K: 16 bytes of row (i*rows_per_load + lane/lanes_per_row)
  uint32_t v[G::kVRows][G::kVWords]; // V row 4c + (e & 3) of sub-tile e >> 2, elems kE*r16..
  float sc[G::kScales / 64];         // int8: scale j*64 + lane of the tile's (K|V, sub-tile, row)
};

// The loop-invariant parts of a wave's tile addresses (one kv head): bases
// at the head, and each lane's byte offsets inside a 16-row sub-tile.
template <int KV, int D>
struct TileAddr {
  const uint8_t *k, *v;    // p.k / p.v + kvh * skh
  const uint8_t *ks, *vs;  // int8: p.ks / p.vs + kvh * scale bytes
  uint32_t k_lane;         // row (lane / kKLanesPerRow) % 16; K load i adds row (i * kKRowsPerLoad) % 16
  uint32_t v_row[4];       // V row load e: row 4c + e % 4, bytes kVBytes * r16 ..
  uint32_t s_lane;         // int8 scale: row r16
  uint32_t s_mask[4];      // int8 scale: all ones in lane group lane / 16, else zero
};

template <int KV, int SC, int D>
__device__ __forceinline__ TileAddr<KV, D> tile_addr(const KParams &p, int kvh, int lane) {
  using G = Geo<KV, D>;
  TileAddr<KV, D> a;
  const uint32_t skt = (uint32_t)p.skt;
  a.k = p.k + (int64_t)kvh * p.skh;
  a.v = p.v + (int64_t)kvh * p.skh;
  a.ks = p.ks + (int64_t)kvh * (SC == PA_SCALE_FP32 ? 4 : 2);
  a.vs = p.vs + (int64_t)kvh * (SC == PA_SCALE_FP32 ? 4 : 2);
  a.k_lane = (uint32_t)((lane / G::kKLanesPerRow) & 15) * skt + 16u * (lane % G::kKLanesPerRow);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    a.v_row[i] = (uint32_t)(4 * (lane >> 4) + i) * skt + (uint32_t)(G::kVBytes * (lane & 15));
  a.s_lane = (uint32_t)(lane & 15) * (uint32_t)p.sst;
#pragma unroll
  for (int g = 0; g < 4; ++g) a.s_mask[g] = (lane >> 4) == g ? ~0u : 0u;
  return a;
}

template <int KV, int D>
struct WaveState {
  using G = Geo<KV, D>;
  f16x8 qop[G::kKSteps];  // Q^T B-operands
  f32x4 acc[G::kE];       // O^T accumulators, one 16x16 block per d-slab
  float m;                // running max (log2 domain) for head column r16
  float l;                // running sum over this lane's tokens
};

// Issue the loads of the tile starting at token n0 (< hi). A tile is two
// 16-row sub-tiles; n0 is a multiple of 32 and pages hold a power of two
// >= 16 rows, so a sub-tile lies in one page and is read as one raw buffer
// from its first row. In the last tile, rows at or past `hi` are either
// read as they are (K rows and K scales: inside the page, finite or not,
// and their scores are replaced by -inf) or read as zeros through the
// buffer's range check (V rows and V scales, which the MFMA multiplies by
// P = 0: zeros keep the products finite). A sub-tile wholly past the end
// re-reads the last one. With `wait_prev`, the K/V loads are issued only
// once the loads issued before them (the tile about to be computed) have
// arrived: one tile in flight per wave instead of two (the block-table
// reads still go ahead).
template <int KV, int SC, int D>
__device__ __forceinline__ void load_tile(Tile<KV, D> &r, const KParams &p, const TileAddr<KV, D> &ta,
                                          const ro_i32 *bt_row, int n0, int hi, int lane,
                                          bool wait_prev = false) {
  using G = Geo<KV, D>;
  constexpr int NS = G::kNSub;
  static_assert(NS == 2 && G::kScales == 64, "one scale per lane covers the tile");
  static_assert(G::kKRowsPerLoad <= 16 || G::kKRowsPerLoad == 32, "K load row layout");
  const uint32_t skt = (uint32_t)p.skt;
  const int page_mask = (1 << p.log2_page) - 1;

  __amdgpu_buffer_rsrc_t rk[NS], rv[NS];
  uint32_t ph[NS], of[NS];
  int rows[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int t0 = min(n0 + 16 * u, (hi - 1) & ~15);
    ph[u] = (uint32_t)min(max(bt_row[(uint32_t)t0 >> p.log2_page], 0), p.num_blocks - 1);
    of[u] = (uint32_t)(t0 & page_mask);
    rows[u] = min(hi - t0, 16);  // valid rows of the sub-tile, >= 1
    const uint64_t row0 = (uint64_t)ph[u] * (uint32_t)p.skn + of[u] * skt;
    rk[u] = page_rsrc(ta.k + row0);
    rv[u] = page_rsrc(ta.v + row0, (int)((uint32_t)rows[u] * skt));
  }
  // int8 scale buffers, made here with the K/V ones. Making them only once
  // the K/V loads are issued keeps the two sets from being live together
  // (no scalar register spills at all), but the compiler then schedules the
  // tile so that C4's decode ran 2.5% slower (183 against 178.5 us).
  [[maybe_unused]] __amdgpu_buffer_rsrc_t rks[NS], rvs[NS];
  if constexpr (KV == PA_KV_INT8) {
    const uint32_t sst = (uint32_t)p.sst;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const uint64_t srow0 = (uint64_t)ph[u] * (uint32_t)p.ssn + of[u] * sst;
      rks[u] = page_rsrc(ta.ks + srow0);
      rvs[u] = page_rsrc(ta.vs + srow0, (int)((uint32_t)rows[u] * sst));
    }
  }
  if (wait_prev) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

#pragma unroll
  for (int i = 0; i < G::kKLoads; ++i) {
    if constexpr (G::kKRowsPerLoad <= 16) {
      // the load's rows lie in sub-tile (i * rows) / 16
      const int u = (i * G::kKRowsPerLoad) >> 4;
      const uint32_t soff = (uint32_t)((i * G::kKRowsPerLoad) & 15) * skt;
      r.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk[u], ta.k_lane, soff, kLoadNT);
    } else {
      // 32 rows per load: lanes 0-31 hold sub-tile 0, lanes 32-63 sub-tile 1;
      // every lane reads its row of both sub-tiles and keeps its own
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rk[0], ta.k_lane, 0, kLoadNT);
      const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rk[1], ta.k_lane, 0, kLoadNT);
      r.k[i] = lane < 32 ? a : b;
    }
  }
#pragma unroll
  for (int e = 0; e < G::kVRows; ++e) buf_load_bytes<G::kVBytes>(r.v[e], rv[e >> 2], ta.v_row[e & 3], 0);
  if constexpr (KV == PA_KV_INT8) {
    // lane group g = lane / 16 holds scale (K | V)[g / 2] of sub-tile g % 2:
    // four loads, each with a uniform buffer, combined by bit masks (a
    // select between the loads would become one load from a per-lane buffer)
    const uint32_t k0 = load_scale_bits<SC>(rks[0], ta.s_lane);
    const uint32_t k1 = load_scale_bits<SC>(rks[1], ta.s_lane);
    const uint32_t v0 = load_scale_bits<SC>(rvs[0], ta.s_lane);
    const uint32_t v1 = load_scale_bits<SC>(rvs[1], ta.s_lane);
    const uint32_t bits = (k0 & ta.s_mask[0]) | (k1 & ta.s_mask[1]) | (v0 & ta.s_mask[2]) | (v1 & ta.s_mask[3]);
    r.sc[0] = SC == PA_SCALE_FP32 ? __builtin_bit_cast(float, bits)
                                  : (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
  }
}

template <int KV, int SC, int D>
__device__ __forceinline__ void compute_tile(WaveState<KV, D> &st, const Tile<KV, D> &r,
                                             const KParams &p, int n0, int hi, int lane,
                                             float *sc_lds, uint8_t *k_lds) {
  using G = Geo<KV, D>;
  constexpr int NS = G::kNSub;
  constexpr int NV = 4 * NS;  // scores per lane: tokens 16u + 4c + i
  const int r16 = lane & 15;
  const int c = lane >> 4;
  const bool tail = n0 + G::kTT > hi;

  // ---- K rows -> LDS slot -> MFMA A layout ----
#pragma unroll
  for (int i = 0; i < G::kKLoads; ++i) {
    const int row = i * G::kKRowsPerLoad + lane / G::kKLanesPerRow;
    *reinterpret_cast<u32x4 *>(k_lds + row * G::kKSlotStride + 16 * (lane % G::kKLanesPerRow)) = r.k[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- int8 scales of this tile into the wave's LDS slot; each lane reads
  // back those of the rows it dequantises (K: its operand row r16 of each
  // sub-tile; V: its tokens {16u + 4c + i} for the P operand), so none are
  // live across the loads ----
  if constexpr (KV == PA_KV_INT8) {
    // (entries 0 .. kTT-1 are K scales, the rest V scales; fp32 scales
    // stored times 2^24, fp16 scales as they are)
#pragma unroll
    for (int j = 0; j < G::kScales / 64; ++j)
      sc_lds[j * 64 + lane] = SC == PA_SCALE_FP32 ? r.sc[j] * kInt8Unit : r.sc[j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- S^T = K Q^T, one 16-token sub-tile at a time ----
  f32x4 sacc[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    // int8: every element of this lane's operand is in row r16 of the
    // sub-tile, so one scale serves them all (fp32 scales: ks8 = s * 2^24,
    // kc8 = -128 * s; fp16 scales: the pair ks2 = (s, s))
    float ks8 = 0.f, kc8 = 0.f;
    uint32_t ks2 = 0;
    if constexpr (KV == PA_KV_INT8) {
      ks8 = sc_lds[16 * u + r16];
      kc8 = ks8 * (-1.0f / 131072.0f);
      if constexpr (SC == PA_SCALE_FP16) ks2 = cvt_pk_f16(ks8, ks8);
    }
#pragma unroll
    for (int ks = 0; ks < G::kKSteps; ++ks) {
      f16x8 kop;
      const uint8_t *src = k_lds + (16 * u + r16) * G::kKSlotStride + (32 * ks + 8 * c) * G::kElem;
      if constexpr (KV == PA_KV_BF16) {
        kop = bf16x8_to_f16x8(*reinterpret_cast<const u32x4 *>(src));
      } else if constexpr (G::kElem == 2) {
        kop = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4 *>(src));
      } else if constexpr (KV == PA_KV_INT8) {
        // the reference's dequantised K, fp16(x * s) per element
        const u32x2 w = *reinterpret_cast<const u32x2 *>(src);
        const uint32_t w0 = w.x ^ kInt8Sign, w1 = w.y ^ kInt8Sign;
        uint32_t dq[4];
        if constexpr (SC == PA_SCALE_FP16) {
          dq[0] = i8pair_fp16_scale(w0, 0, 1, ks2);
          dq[1] = i8pair_fp16_scale(w0, 2, 3, ks2);
          dq[2] = i8pair_fp16_scale(w1, 0, 1, ks2);
          dq[3] = i8pair_fp16_scale(w1, 2, 3, ks2);
        } else {
          dq[0] = i8pair_fp32_scale(perm(w0, w0, pair_sel<KV>(0, 1)), ks8, kc8, ks8, kc8);
          dq[1] = i8pair_fp32_scale(perm(w0, w0, pair_sel<KV>(2, 3)), ks8, kc8, ks8, kc8);
          dq[2] = i8pair_fp32_scale(perm(w1, w1, pair_sel<KV>(0, 1)), ks8, kc8, ks8, kc8);
          dq[3] = i8pair_fp32_scale(perm(w1, w1, pair_sel<KV>(2, 3)), ks8, kc8, ks8, kc8);
        }
        kop = as_f16x8(dq[0], dq[1], dq[2], dq[3]);
      } else {
        const u32x2 w = *reinterpret_cast<const u32x2 *>(src);
        kop = as_f16x8(bytes_to_halves<KV>(w.x, w.x, pair_sel<KV>(0, 1)),
                       bytes_to_halves<KV>(w.x, w.x, pair_sel<KV>(2, 3)),
                       bytes_to_halves<KV>(w.y, w.y, pair_sel<KV>(0, 1)),
                       bytes_to_halves<KV>(w.y, w.y, pair_sel<KV>(2, 3)));
      }
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, st.qop[ks], a, 0, 0, 0);
    }
    sacc[u] = a;
  }
  // the next tile's rows overwrite the slot only after these reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // ---- online softmax over the tokens this lane holds for head r16 ----
  float s[NV];
#pragma unroll
  for (int e = 0; e < NV; ++e) s[e] = sacc[e >> 2][e & 3] * p.qk_scale;
  if (tail) {
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int tok = n0 + 16 * (e >> 2) + 4 * c + (e & 3);
      if (tok >= hi) s[e] = -INFINITY;
    }
  }
  float tmax = s[0];
#pragma unroll
  for (int e = 1; e < NV; ++e) tmax = fmaxf(tmax, s[e]);
  tmax = col_max(tmax);

  const bool need = tmax > st.m + kRescaleLog2;
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(need) != 0, 0)) {
    const float m_new = need ? fmaxf(st.m, tmax) : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int sl = 0; sl < G::kE; ++sl) st.acc[sl] *= alpha;
    st.m = m_new;
  }

  float pr[NV];
#pragma unroll
  for (int e = 0; e < NV; ++e) pr[e] = __builtin_amdgcn_exp2f(s[e] - st.m);
  float lsum = 0.f;
#pragma unroll
  for (int e = 0; e < NV; e += 4) lsum += (pr[e] + pr[e + 1]) + (pr[e + 2] + pr[e + 3]);
  st.l += lsum;

  // ---- O^T += V^T P^T: one MFMA per d-slab and pair of sub-tiles ----
#pragma unroll
  for (int pp = 0; pp < NS / 2; ++pp) {
    f16x8 pop;
#pragma unroll
    for (int e = 0; e < 8; ++e) pop[e] = (_Float16)pr[8 * pp + e];
    if constexpr (G::kElem == 2) {
#pragma unroll
      for (int sl = 0; sl < G::kE; ++sl) {
        uint32_t h[4];
#pragma unroll
        for (int m2 = 0; m2 < 4; ++m2) {
          const int wi = sl >> 1;
          const uint32_t sel = (sl & 1) ? 0x07060302u : 0x05040100u;
          h[m2] = perm(r.v[8 * pp + 2 * m2 + 1][wi], r.v[8 * pp + 2 * m2][wi], sel);
          if constexpr (KV == PA_KV_BF16) h[m2] = bf16x2_to_f16x2(h[m2]);
        }
        const f16x8 vop = as_f16x8(h[0], h[1], h[2], h[3]);
        st.acc[sl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, st.acc[sl], 0, 0, 0);
      }
    } else {
      // int8: element e of the lane's operand is token 16 * (2pp + e / 4)
      // + 4c + e % 4, with V scale vs[e] (fp32 scales: s * 2^24, and
      // vc[e] = -128 * s; fp16 scales: s, and the pairs vs2[m2] = (vs[2m2],
      // vs[2m2 + 1]))
      float vs[8], vc[8];
      uint32_t vs2[4];
      if constexpr (KV == PA_KV_INT8) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const f32x4 vq = *reinterpret_cast<const f32x4 *>(sc_lds + 16 * (NS + 2 * pp + h2) + 4 * c);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            vs[4 * h2 + i] = vq[i];
            vc[4 * h2 + i] = vq[i] * (-1.0f / 131072.0f);
          }
        }
        if constexpr (SC == PA_SCALE_FP16) {
#pragma unroll
          for (int m2 = 0; m2 < 4; ++m2) vs2[m2] = cvt_pk_f16(vs[2 * m2], vs[2 * m2 + 1]);
        }
      }
      // word wi of a row holds head-dim elements 4*wi .. 4*wi+3 of the lane's
      // slab group (int8: sign bits flipped once per word)
      uint32_t vw[8][G::kVWords];
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int w = 0; w < G::kVWords; ++w)
          vw[e][w] = (KV == PA_KV_INT8) ? (r.v[8 * pp + e][w] ^ kInt8Sign) : r.v[8 * pp + e][w];
#pragma unroll
      for (int sl = 0; sl < G::kE; ++sl) {
        const int wi = sl >> 2;
        const uint32_t b = sl & 3;
        uint32_t h[4];
#pragma unroll
        for (int m2 = 0; m2 < 4; ++m2) {
          h[m2] = bytes_to_halves<KV>(vw[2 * m2 + 1][wi], vw[2 * m2][wi], pair_sel<KV>(b, b));
          if constexpr (KV == PA_KV_INT8 && SC == PA_SCALE_FP16) {
            // the two bytes come from two rows: zero-extended halves x + 128,
            // under the exponent byte 0x64 (see i8pair_fp16_scale)
            const f16x2 x2 = __builtin_bit_cast(f16x2, h[m2] | 0x64006400u) -
                             f16x2{(_Float16)1152.0f, (_Float16)1152.0f};
            h[m2] = __builtin_bit_cast(uint32_t, x2 * __builtin_bit_cast(f16x2, vs2[m2]));
          } else if constexpr (KV == PA_KV_INT8) {
            h[m2] = i8pair_fp32_scale(h[m2], vs[2 * m2], vc[2 * m2], vs[2 * m2 + 1], vc[2 * m2 + 1]);
          }
        }
        const f16x8 vop = as_f16x8(h[0], h[1], h[2], h[3]);
        st.acc[sl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, st.acc[sl], 0, 0, 0);
      }
    }
  }
  if constexpr (KV == PA_KV_INT8) {
    // the next tile's scales overwrite the slot only after these reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

// Q^T B-operands of query heads qh0 .. qh0 + nh - 1 of sequence b (lane
// column r16 = head, padded columns are zero).
template <int KV, int D>
__device__ __forceinline__ void load_q(WaveState<KV, D> &st, const KParams &p, int b, int qh0,
                                       int nh, int r16, int c) {
  using G = Geo<KV, D>;
  const bool hv = r16 < nh;
  const uint16_t *qrow = reinterpret_cast<const uint16_t *>(p.q) + (int64_t)b * p.sqb +
                         (int64_t)(qh0 + (hv ? r16 : 0)) * p.sqh;
  // 8 q values from head dim d0 on, as fp16 (bf16 rounded to fp16 first,
  // the reference's q.to(fp16)); zeros for padded heads
  auto q8 = [&](int d0) {
    f16x8 qv = {0, 0, 0, 0, 0, 0, 0, 0};
    if (hv) {
      const u32x4 w = *reinterpret_cast<const u32x4 *>(qrow + d0);
      qv = p.io_bf16 ? bf16x8_to_f16x8(w) : __builtin_bit_cast(f16x8, w);
    }
    return qv;
  };
#pragma unroll
  for (int ks = 0; ks < G::kKSteps; ++ks) st.qop[ks] = q8(32 * ks + 8 * c);
}

template <int KV, int D>
__device__ __forceinline__ void reset_state(WaveState<KV, D> &st) {
  using G = Geo<KV, D>;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int sl = 0; sl < G::kE; ++sl) st.acc[sl] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// One lane's share of a finished row of head h: y[0 .. 4*kE) = O[h][d0 ..)
// (already normalised), L the row's sum of 2^(s - M). Written to `out` of
// sequence b (direct) or as a partial row at element offsets part_off /
// lse_off (the lse by the c == 0 lane).
template <int D>
__device__ __forceinline__ void store_result(const KParams &p, const float *y, float L, float M,
                                             int b, int h, int d0, int c, bool direct,
                                             int64_t part_off, int64_t lse_off) {
  constexpr int kRegs = 4 * (D / 16);
  if (!direct) {
    float *dst = p.part_out + part_off + (int64_t)h * p.sph + d0;
#pragma unroll
    for (int v4 = 0; v4 < kRegs / 4; ++v4) {
      f32x4 t4 = {y[4 * v4], y[4 * v4 + 1], y[4 * v4 + 2], y[4 * v4 + 3]};
      *reinterpret_cast<f32x4 *>(dst + 4 * v4) = t4;
    }
    if (c == 0) p.part_lse[lse_off + (int64_t)h * p.slh] = (L > 0.f) ? M + __log2f(L) : -INFINITY;
  } else {
    uint8_t *dst = p.out + ((int64_t)b * p.sob + (int64_t)h * p.soh + d0) * 2;
    if (p.io_bf16) {
      uint32_t w[kRegs / 2];
#pragma unroll
      for (int e = 0; e < kRegs / 2; ++e)
        w[e] = f32_to_bf16_bits(y[2 * e]) | (f32_to_bf16_bits(y[2 * e + 1]) << 16);
#pragma unroll
      for (int e = 0; e < kRegs / 2; e += 2)
        *reinterpret_cast<u32x2 *>(dst + 4 * e) = u32x2{w[e], w[e + 1]};
    } else if constexpr (kRegs >= 8) {
#pragma unroll
      for (int v8 = 0; v8 < kRegs / 8; ++v8) {
        f16x8 t8;
#pragma unroll
        for (int e = 0; e < 8; ++e) t8[e] = (_Float16)y[8 * v8 + e];
        *reinterpret_cast<f16x8 *>(dst + 16 * v8) = t8;
      }
    } else {
      store_row(dst, y, kRegs, false);
    }
  }
}

// The same result written straight from the accumulators, a few registers at
// a time: acc[sl][i] (sl = 0 .. kE-1) are the kE contiguous head-dim elements
// from 4*kE*c + kE*i, scaled by `inv` on the way out.
template <int D>
__device__ __forceinline__ void store_acc(const KParams &p, const f32x4 *acc, float inv, float L,
                                          float M, int b, int h, int c, bool direct,
                                          int64_t part_off, int64_t lse_off) {
  constexpr int kE = D / 16;
  const int d0 = 4 * kE * c;
  if (!direct) {
    float *dst = p.part_out + part_off + (int64_t)h * p.sph + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (kE >= 4) {
#pragma unroll
        for (int q = 0; q < kE / 4; ++q) {
          const f32x4 t4 = {acc[4 * q][i] * inv, acc[4 * q + 1][i] * inv, acc[4 * q + 2][i] * inv,
                            acc[4 * q + 3][i] * inv};
          *reinterpret_cast<f32x4 *>(dst + kE * i + 4 * q) = t4;
        }
      } else {
#pragma unroll
        for (int sl = 0; sl < kE; ++sl) dst[kE * i + sl] = acc[sl][i] * inv;
      }
    }
    if (c == 0) p.part_lse[lse_off + (int64_t)h * p.slh] = (L > 0.f) ? M + __log2f(L) : -INFINITY;
  } else {
    // kE (even) elements of group i = kE / 2 dwords at byte offset 2 * kE * i
    uint32_t *dst = reinterpret_cast<uint32_t *>(
        p.out + ((int64_t)b * p.sob + (int64_t)h * p.soh + d0) * 2);
    if (p.io_bf16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < kE; e += 2)
          dst[(kE * i + e) / 2] =
              f32_to_bf16_bits(acc[e][i] * inv) | (f32_to_bf16_bits(acc[e + 1][i] * inv) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < kE; e += 2) {
          const f16x2 hh = {(_Float16)(acc[e][i] * inv), (_Float16)(acc[e + 1][i] * inv)};
          dst[(kE * i + e) / 2] = __builtin_bit_cast(uint32_t, hh);
        }
    }
  }
}

// Lane (c, h) holds O[h][4*kE*c + kE*i + sl] in acc[sl][i]; regroup so that
// y[kE*i + sl] is head-dim offset 4*kE*c + kE*i + sl (contiguous), scaled.
template <int D>
__device__ __forceinline__ void regroup(float *y, const float *o, float scale) {
  constexpr int kE = D / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int sl = 0; sl < kE; ++sl) y[kE * i + sl] = o[4 * sl + i] * scale;
}

// Token range [lo, hi) of one split, and how many of the sequence's splits
// hold tokens. chunk = ceil(ceil(T / 32) / S) * 32 tokens, T = the sequence's
// length (the reference's per-sequence rule, triton_decode.py:78-85), or the
// chunk of a max_seq_len-token sequence when max_seq_len > 0 and that is
// larger (ragged batches: long sequences take all S splits, short ones few;
// never below the sequence's own chunk, so no token is dropped).
struct SplitRange {
  int lo, hi, n;
};

__device__ __forceinline__ SplitRange split_range(int seq_len, int num_splits, int max_seq_len,
                                                  int split) {
  const int64_t own = ((int64_t)seq_len + kSplitAlign - 1) / kSplitAlign;
  int64_t ntile_chunk = (own + num_splits - 1) / num_splits;
  if (max_seq_len > 0) {
    const int64_t longest = ((int64_t)max_seq_len + kSplitAlign - 1) / kSplitAlign;
    ntile_chunk = max((longest + num_splits - 1) / num_splits, ntile_chunk);
  }
  const int64_t chunk = max(ntile_chunk, (int64_t)1) * kSplitAlign;  // T = 0 still has one split
  const int64_t lo = min((int64_t)split * chunk, (int64_t)seq_len);
  SplitRange r;
  r.lo = (int)lo;
  r.hi = (int)min(lo + chunk, (int64_t)seq_len);
  r.n = max(1, (int)((seq_len + chunk - 1) / chunk));
  return r;
}

// What a workgroup does with its result:
//   kUnsplit   one workgroup per (b, kv_head, head_tile): fp16 `out`
//   kPartials  one per split: the normalised fp32 partial and its log2-sum-exp
//              for every split, empty ones included (zeros, -inf): the
//              reference's split epilogue (triton_decode.py:169-188)
//   kAuto      as kPartials for the splits that hold tokens; a sequence that
//              fits in one split writes `out` directly, empty splits return at
//              once (the merge kernel skips both)
enum { kUnsplit = 0, kPartials = 1, kAuto = 2 };

// Two workgroups (8 waves) per CU must fit in the register file: the
// double-buffered tiles are sized for that budget.
template <int KV, int SC, int D, int MODE>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
paged_decode_kernel(const KParams p) {
  using G = Geo<KV, D>;
  constexpr int kRegs = 4 * G::kE;  // accumulator floats per lane

  // The K slots are only used inside the tile loop and the wave-merge buffer
  // only after it (behind a barrier), so they share one allocation.
  constexpr int kMergeBytes = (kWaves - 1) * kRegs * 64 * 4;
  constexpr int kSlotsBytes = kWaves * G::kKSlotBytes;
  __shared__ __attribute__((aligned(16))) uint8_t sm_raw[kMergeBytes > kSlotsBytes ? kMergeBytes : kSlotsBytes];
  __shared__ float sm_m[kWaves][16];
  __shared__ float sm_l[kWaves][16];
  __shared__ __attribute__((aligned(16))) float sm_sc[kWaves][G::kScales];
  auto sm_acc = reinterpret_cast<float (*)[kRegs][64]>(sm_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15;
  const int c = lane >> 4;

  // With splits, XCD x (the hardware deals workgroups round-robin to the 8
  // XCDs) takes the contiguous logical range [x * n / 8, (x + 1) * n / 8) of
  // (b, kv_head, head_tile, split) = all splits of a few sequences: measured
  // 3-33% faster on split workloads (ragged most), 2% slower unsplit, so only
  // split launches remap. The tail past a multiple of 8 keeps its index.
  int wg = blockIdx.x;
  if (MODE != kUnsplit) {
    const int n = gridDim.x, full = n - n % 8;
    if (wg < full) wg = (wg % 8) * (full / 8) + wg / 8;
  }
  // wg = ((b * hkv + kvh) * head_tiles + ht) * num_splits + split
  int x = wg;
  const int split = x % p.num_splits;
  x /= p.num_splits;
  const int ht = x % p.head_tiles;
  x /= p.head_tiles;
  const int kvh = x % p.hkv;
  const int b = x / p.hkv;

  const int qh0 = kvh * p.group + ht * 16;
  const int nh = min(16, p.group - ht * 16);

  int seq_len = p.seq_lens[b];
  seq_len = max(0, min(seq_len, p.max_blocks << p.log2_page));

  int lo = 0, hi = seq_len;
  bool direct = true;  // write fp16 `out` (else a split partial)
  if (MODE != kUnsplit) {
    const SplitRange r = split_range(seq_len, p.num_splits, p.max_seq_len, split);
    if (MODE == kAuto && split >= r.n) return;  // an empty split: nothing to read or write
    lo = r.lo;
    hi = r.hi;
    direct = MODE == kAuto && r.n == 1;
  }

  WaveState<KV, D> st;
  reset_state(st);
  load_q(st, p, b, qh0, nh, r16, c);

  const ro_i32 *bt_row = ro(p.bt) + (int64_t)b * p.sbtb;
  const TileAddr<KV, D> addr = tile_addr<KV, SC, D>(p, kvh, lane);
  float *sc_lds = sm_sc[wave];
  uint8_t *k_lds = sm_raw + wave * G::kKSlotBytes;
  const int ntiles = (hi > lo) ? (hi - lo + G::kTT - 1) / G::kTT : 0;
  // this wave's tiles: wave + kWaves * i, i < cnt
  const int cnt = ntiles > wave ? (ntiles - wave + kWaves - 1) / kWaves : 0;
  auto n0_of = [&](int i) { return lo + (wave + kWaves * i) * G::kTT; };
  if (cnt > 0) {
    if constexpr (G::kPrefetch) {
      Tile<KV, D> ta, tb;
      load_tile<KV, SC, D>(ta, p, addr, bt_row, n0_of(0), hi, lane);
      int i = 0;
      for (; i + 2 < cnt; i += 2) {
        load_tile<KV, SC, D>(tb, p, addr, bt_row, n0_of(i + 1), hi, lane);
        compute_tile<KV, SC, D>(st, ta, p, n0_of(i), hi, lane, sc_lds, k_lds);
        load_tile<KV, SC, D>(ta, p, addr, bt_row, n0_of(i + 2), hi, lane);
        compute_tile<KV, SC, D>(st, tb, p, n0_of(i + 1), hi, lane, sc_lds, k_lds);
      }
      if (i + 1 < cnt) {
        load_tile<KV, SC, D>(tb, p, addr, bt_row, n0_of(i + 1), hi, lane);
        compute_tile<KV, SC, D>(st, ta, p, n0_of(i), hi, lane, sc_lds, k_lds);
        compute_tile<KV, SC, D>(st, tb, p, n0_of(i + 1), hi, lane, sc_lds, k_lds);
      } else {
        compute_tile<KV, SC, D>(st, ta, p, n0_of(i), hi, lane, sc_lds, k_lds);
      }
    } else {
      for (int i = 0; i < cnt; ++i) {
        Tile<KV, D> t;
        load_tile<KV, SC, D>(t, p, addr, bt_row, n0_of(i), hi, lane);
        compute_tile<KV, SC, D>(st, t, p, n0_of(i), hi, lane, sc_lds, k_lds);
      }
    }
  }

  // ---- merge the waves through LDS ----
  const float lw = col_sum(st.l);
  if (c == 0) {
    sm_m[wave][r16] = st.m;
    sm_l[wave][r16] = lw;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][r16]);
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float mw = sm_m[w][r16];
    L += (mw == -INFINITY) ? 0.f : sm_l[w][r16] * __builtin_amdgcn_exp2f(mw - M);
  }
  const float f = (st.m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(st.m - M);
  if (wave > 0) {
#pragma unroll
    for (int sl = 0; sl < G::kE; ++sl)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm_acc[wave - 1][4 * sl + i][lane] = st.acc[sl][i] * f;
  }
  __syncthreads();
  if (wave != 0) return;

  float o[kRegs];
#pragma unroll
  for (int sl = 0; sl < G::kE; ++sl)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = st.acc[sl][i] * f;
#pragma unroll
      for (int w = 1; w < kWaves; ++w) a += sm_acc[w - 1][4 * sl + i][lane];
      o[4 * sl + i] = a;
    }
  const float inv = (L > 0.f) ? 1.0f / L : 0.f;
  float y[kRegs];
  regroup<D>(y, o, inv);
  if (r16 >= nh) return;
  store_result<D>(p, y, L, M, b, qh0 + r16, 4 * G::kE * c, c, direct,
                  (int64_t)b * p.spb + (int64_t)split * p.sps, (int64_t)b * p.slb + split);
}

// ----------------------------------------------------------------------------
// Flat (work-balanced) split.
//
// Per (kv_head, head_tile) unit, the batch's 32-token tiles are laid end to
// end in sequence order: sequence b owns flat tiles [cu_b, cu_b + n_b),
// n_b = ceil(T_b / 32). The F = flat_splits waves of the unit take F equal
// contiguous ranges of per = ceil(total / F) tiles, so every wave streams the
// same number of tiles however ragged the lengths are (the classic split gives
// each sequence its own chunks, and a few long sequences then run alone at the
// end of the launch). A wave keeps the tile pipeline going across sequence
// boundaries; when its range leaves a sequence it writes that segment's
// normalised output and log2-sum-exp as partial slot b + j (j = the wave's
// range index), or `out` itself when the segment is the whole sequence.
// Slots are unique: if range j - 1 reached sequence b + 1, sequence b ended
// before range j began. The merge (split_reduce_kernel<D, kMergeFlat>)
// derives the same ranges from seq_lens and folds slots b + j0 .. b + j1.
//
// Equal tile counts are not equal times when a range crosses sequences: each
// sequence a wave starts costs it a new q, a store and a pipeline restart
// (about one fp8 tile at head_dim 128). With flat_cost = c > 0 every
// non-empty sequence is charged c tiles of weight ahead of its first tile:
// sequence b spans weights [cw_b, cw_b + c + n_b), its tile k sits at weight
// cw_b + c + k, and range j takes the tiles whose weights fall in
// [j * per, (j + 1) * per), per = ceil(W / F) over the total weight W. The
// ranges stay contiguous in sequence order (the slot rule above holds); a
// range that covers charges only holds no tiles. c = 0 is the plain split.
// ----------------------------------------------------------------------------

// Tiles of sequence b (its length clamped to the block table).
__device__ __forceinline__ int seq_tiles(const ro_i32 *seq_lens, int b, int max_tokens) {
  const int t = max(0, min(seq_lens[b], max_tokens));
  return (t + kSplitAlign - 1) / kSplitAlign;
}

__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Total flat tiles of the batch (wave-uniform); `len0` receives this lane's
// clamped length of sequence `lane` (0 past the batch).
// seq_lens is scanned kLenChunks chunks of 64 at a time: the chunks' loads
// are all issued before any is used, so up to 512 sequences cost one round
// trip instead of one per 64 (16 chunks made the compiler raise every flat
// instance to 230 VGPRs).
constexpr int kLenChunks = 8;

// Clamped lengths of sequences base + 64 k + lane (k < kLenChunks; 0 past the
// batch), loaded together.
__device__ __forceinline__ void load_len_chunks(const ro_i32 *seq_lens, int batch, int max_tokens,
                                                int base, int lane, int (&len)[kLenChunks]) {
#pragma unroll
  for (int k = 0; k < kLenChunks; ++k) {
    len[k] = 0;
    if (base + 64 * k < batch) {  // wave-uniform
      const int b = base + 64 * k + lane;
      if (b < batch) len[k] = max(0, min(seq_lens[b], max_tokens));
    }
  }
}

__device__ __forceinline__ int len_tiles(int len) { return (len + kSplitAlign - 1) / kSplitAlign; }

__device__ __forceinline__ int flat_total(const ro_i32 *seq_lens, int batch, int max_tokens,
                                          int lane, int &len0) {
  if (batch <= 64) {  // one chunk
    len0 = lane < batch ? max(0, min(seq_lens[lane], max_tokens)) : 0;
    return __builtin_amdgcn_readfirstlane(wave_sum(len_tiles(len0)));
  }
  int total = 0;
  for (int base = 0; base < batch; base += 64 * kLenChunks) {
    int len[kLenChunks];
    load_len_chunks(seq_lens, batch, max_tokens, base, lane, len);
    if (base == 0) len0 = len[0];
    int t = 0;
#pragma unroll
    for (int k = 0; k < kLenChunks; ++k) t += len_tiles(len[k]);
    total += wave_sum(t);
  }
  return __builtin_amdgcn_readfirstlane(total);
}

// A wave's position in its range: sequence b, tile t of b, b's tile count
// and length (all wave-uniform).
struct SeqCursor {
  int b, t, tiles, len;
};

// The sequence holding flat tile f (< total) and f's tile index in it.
// `len0` is this lane's clamped length of sequence `lane` (batch <= 64: the
// values flat_start already loaded), or -1 to load them again.
__device__ __forceinline__ SeqCursor flat_locate(const ro_i32 *seq_lens, int batch, int max_tokens,
                                                 int f, int lane, int len0) {
  SeqCursor cur = {0, 0, 0, 0};
  if (len0 >= 0) {  // batch <= 64: one chunk, already loaded
    const int t = len_tiles(len0);
    const int incl = wave_incl_scan(t, lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > f);
    const int l = hit != 0 ? __builtin_ctzll(hit) : 0;
    cur.b = l;
    cur.t = f - __shfl(incl - t, l);
    cur.len = __shfl(len0, l);
  } else {
    int run = 0;  // tiles of the sequences before this pass
    for (int base = 0; base < batch; base += 64 * kLenChunks) {
      int len[kLenChunks];
      load_len_chunks(seq_lens, batch, max_tokens, base, lane, len);
      // the chunk holding f, from the chunks' tile sums (wave-uniform) ...
      int kk = -1;
#pragma unroll
      for (int k = 0; k < kLenChunks; ++k) {
        const int ck = __builtin_amdgcn_readfirstlane(wave_sum(len_tiles(len[k])));
        if (kk < 0) {
          if (run + ck > f) kk = k;
          else run += ck;
        }
      }
      if (kk < 0) continue;
      // ... then f's sequence inside that chunk
      int lk = 0;
#pragma unroll
      for (int k = 0; k < kLenChunks; ++k)
        if (k == kk) lk = len[k];
      const int t = len_tiles(lk);
      const int incl = wave_incl_scan(t, lane) + run;
      const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > f);
      const int l = hit != 0 ? __builtin_ctzll(hit) : 0;
      cur.b = base + 64 * kk + l;
      cur.t = f - __shfl(incl - t, l);
      cur.len = __shfl(lk, l);
      break;
    }
  }
  cur.b = __builtin_amdgcn_readfirstlane(cur.b);
  cur.t = __builtin_amdgcn_readfirstlane(cur.t);
  cur.len = __builtin_amdgcn_readfirstlane(cur.len);
  cur.tiles = (cur.len + kSplitAlign - 1) / kSplitAlign;
  return cur;
}

// Weight of a sequence of `tiles` tiles under a charge of `cost` tiles per
// non-empty sequence.
__device__ __forceinline__ int seq_weight(int tiles, int cost) { return tiles > 0 ? tiles + cost : 0; }

// Range j of F under a charge of cost > 0 tiles per sequence: its first tile
// (the returned cursor) and its tile count `n` (0: the range holds charges
// only, or lies past the end). Per lane: a = the sequence's tiles whose
// weights lie below the range, e = those below its end; n = sum(e - a).
__device__ __forceinline__ SeqCursor flat_locate_weighted(const ro_i32 *seq_lens, int batch,
                                                          int max_tokens, int F, int j, int cost,
                                                          int lane, int &n) {
  SeqCursor cur = {0, 0, 0, 0};
  n = 0;
  if (batch <= 64) {  // one chunk: one scan gives the weights, the range and its start
    const int len = lane < batch ? max(0, min(seq_lens[lane], max_tokens)) : 0;
    const int t = len_tiles(len);
    const int w = seq_weight(t, cost);
    const int incl = wave_incl_scan(w, lane);
    const int W = __builtin_amdgcn_readlane(incl, 63);
    const int per = max(1, (W + F - 1) / F);
    const int r0 = j * per;
    if (r0 >= W) return cur;
    const int r1 = min(W, r0 + per);
    const int first = incl - w + cost;  // weight of the sequence's tile 0
    const int a = min(max(r0 - first, 0), t), e = min(max(r1 - first, 0), t);
    n = __builtin_amdgcn_readfirstlane(wave_sum(e - a));
    const uint64_t hit = __builtin_amdgcn_ballot_w64(a < t);
    if (n == 0 || hit == 0) {
      n = 0;
      return cur;
    }
    const int l = __builtin_ctzll(hit);
    cur.b = l;
    cur.t = __builtin_amdgcn_readlane(a, l);
    cur.len = __builtin_amdgcn_readlane(len, l);
    cur.tiles = (cur.len + kSplitAlign - 1) / kSplitAlign;
    return cur;
  }
  // total weight, then the range's tiles before and inside it, chunk by chunk
  int W = 0;
  for (int base = 0; base < batch; base += 64 * kLenChunks) {
    int len[kLenChunks];
    load_len_chunks(seq_lens, batch, max_tokens, base, lane, len);
    int s = 0;
#pragma unroll
    for (int k = 0; k < kLenChunks; ++k) s += seq_weight(len_tiles(len[k]), cost);
    W += wave_sum(s);
  }
  W = __builtin_amdgcn_readfirstlane(W);
  const int per = max(1, (W + F - 1) / F);
  const int r0 = j * per;
  if (r0 >= W) return cur;
  const int r1 = min(W, r0 + per);
  int run = 0, start = 0, cnt = 0;  // run: weight of the sequences before this chunk
  for (int base = 0; base < batch && run < r1; base += 64 * kLenChunks) {
    int len[kLenChunks];
    load_len_chunks(seq_lens, batch, max_tokens, base, lane, len);
#pragma unroll
    for (int k = 0; k < kLenChunks; ++k) {
      const int t = len_tiles(len[k]);
      const int w = seq_weight(t, cost);
      const int incl = wave_incl_scan(w, lane) + run;
      const int first = incl - w + cost;
      const int a = min(max(r0 - first, 0), t), e = min(max(r1 - first, 0), t);
      start += wave_sum(a);
      cnt += wave_sum(e - a);
      run = __builtin_amdgcn_readlane(incl, 63);
    }
  }
  n = __builtin_amdgcn_readfirstlane(cnt);
  if (n == 0) return cur;
  return flat_locate(seq_lens, batch, max_tokens, __builtin_amdgcn_readfirstlane(start), lane, -1);
}

// Step to the next flat tile. Only called while the range has another tile,
// so a non-empty sequence follows; the batch bound only guards the reads.
__device__ __forceinline__ void cursor_next(SeqCursor &cur, const ro_i32 *seq_lens, int batch,
                                            int max_tokens) {
  if (++cur.t < cur.tiles) return;
  cur.t = 0;
  while (cur.b + 1 < batch) {
    ++cur.b;
    cur.len = __builtin_amdgcn_readfirstlane(max(0, min(seq_lens[cur.b], max_tokens)));
    cur.tiles = (cur.len + kSplitAlign - 1) / kSplitAlign;
    if (cur.tiles > 0) break;
  }
}

// The flat split launches one wave per SIMD for 2-byte and fp8 caches. With
// two, a SIMD's older wave runs ahead of the younger one (per-wave
// timestamps: the younger finish up to 20% later), and that tail costs more
// than the second wave brings. int8 caches, whose tiles keep one wave busy
// issuing VALU work, launch two per SIMD and balance each pair through LDS
// (in the kernel below). The register budget is that of two waves per SIMD
// for every instance, the budget they were tuned under.
// The flat kernel's arguments: the parameters and, when the host knows the
// lengths (ntab = F > 0), each range's first tile (sequence b in the bits
// from kTabTBits up, tile t below), tile count and the length of b, so that
// no wave scans seq_lens before its first loads.
constexpr int kTabTBits = 20;
constexpr uint32_t kTabTMask = (1u << kTabTBits) - 1;
struct FlatArgs {
  KParams p;
  int32_t ntab;
  uint32_t start[kHostTab];
  uint32_t ntile[kHostTab];
  uint32_t len[kHostTab];
};

template <int KV, int SC, int D>
__global__ void __launch_bounds__(flat_waves<KV>() * 64) __attribute__((amdgpu_waves_per_eu(2)))
paged_decode_flat_kernel(const FlatArgs fa) {
  const KParams &p = fa.p;
  using G = Geo<KV, D>;
  static_assert(G::kTT == kSplitAlign, "flat tiles are the kernel's tiles");
  // the workgroup's W waves take W neighbouring kv heads of one range, so
  // together they read a contiguous W-head stretch of every token row (4
  // consecutive ranges of one kv head instead ran 8-14% slower)
  constexpr int W = flat_waves<KV>();
  __shared__ __attribute__((aligned(16))) uint8_t sm_k[W * G::kKSlotBytes];
  // Two waves per SIMD (int8): waves w and w + 4 share a SIMD, and the SIMD
  // issues for the older one first, so with equal work the younger one ended
  // 24-30 us after its partner at C4 and then ran alone. Each wave posts its
  // finished tile count in sm_done (an extra row of the scale slots, so the
  // other instances keep exactly their LDS), and the one behind runs at
  // issue priority 2 (s_setprio: a scheduling hint; a read before the
  // partner's first post sees whatever the LDS held, which can only change
  // the priority, never a result). Partners then end within ~2 us: C4's
  // decode 171.6 / 171.8 -> 167.8 / 167.6 us (two repetitions, one box; fp16
  // and fp8 unchanged).
  constexpr bool kPairPrio = W == 2 * kFlatWaves;
  __shared__ __attribute__((aligned(16))) float sm_sc[W + (kPairPrio ? 1 : 0)][G::kScales];
  int *const sm_done = kPairPrio ? reinterpret_cast<int *>(&sm_sc[W - 1][0] + G::kScales) : nullptr;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15;
  const int c = lane >> 4;

  // XCD-contiguous workgroup order, as for the classic split launch: an XCD
  // holds neighbouring ranges, i.e. a contiguous stretch of the batch.
  int wg = blockIdx.x;
  {
    const int n = gridDim.x, full = n - n % 8;
    if (wg < full) wg = (wg % 8) * (full / 8) + wg / 8;
  }
  // global wave = j * units + unit: the waves of a workgroup share a range
  // and cover neighbouring kv heads, which read the same pages.
  const int units = p.hkv * p.head_tiles;
  const int gw = wg * W + wave;
  if (gw >= units * p.flat_splits) return;  // no barrier follows: waves are independent
  const int unit = gw % units;
  const int j = gw / units;
  const int kvh = unit / p.head_tiles;
  const int ht = unit % p.head_tiles;
  const int qh0 = kvh * p.group + ht * 16;
  const int nh = min(16, p.group - ht * 16);

  // compute cursor at the range's first tile, and the range's tile count
  // (one pass over seq_lens when the batch fits one wave)
  SeqCursor cc;
  int n;  // this wave's tiles
  if (fa.ntab > 0) {
    n = (int)fa.ntile[j];
    if (n == 0) return;
    const uint32_t st = fa.start[j];
    cc.b = (int)(st >> kTabTBits);
    cc.t = (int)(st & kTabTMask);
    cc.len = (int)fa.len[j];
    cc.tiles = (cc.len + kSplitAlign - 1) / kSplitAlign;
  } else if (p.flat_cost == 0) {
    int len0 = 0;
    const int total = flat_total(ro(p.seq_lens), p.batch, p.max_tokens, lane, len0);
    const int per = max(1, (total + p.flat_splits - 1) / p.flat_splits);
    const int r0 = j * per;
    if (r0 >= total) return;
    n = min(per, total - r0);
    cc = flat_locate(ro(p.seq_lens), p.batch, p.max_tokens, r0, lane, p.batch <= 64 ? len0 : -1);
  } else {
    cc = flat_locate_weighted(ro(p.seq_lens), p.batch, p.max_tokens, p.flat_splits, j, p.flat_cost,
                              lane, n);
    if (n == 0) return;
  }
  if constexpr (kPairPrio) {
    if (lane == 0) __hip_atomic_store(&sm_done[wave], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  SeqCursor lc = cc;                                                        // load cursor
  int seg_t0 = cc.t;  // first tile of the current segment

  WaveState<KV, D> st;
  reset_state(st);
  load_q(st, p, cc.b, qh0, nh, r16, c);

  float *sc_lds = sm_sc[wave];
  uint8_t *k_lds = sm_k + wave * G::kKSlotBytes;
  const TileAddr<KV, D> addr = tile_addr<KV, SC, D>(p, kvh, lane);

  // block-table row of sequence b, in 32 bits (batch * stride_btb < 2^31 is
  // checked on the host): the 64-bit product cost 8 scalar instructions per
  // tile, 2% of C4, whose tiles are issue-bound
  auto bt_of = [&](int b) { return ro(p.bt) + (uint32_t)((uint32_t)b * (uint32_t)p.sbtb); };
  // After computing the wave's i-th tile: close the segment at a sequence
  // end or at the end of the range, then move the compute cursor on.
  auto post = [&](int i) {
    if constexpr (kPairPrio) {
      const int mate = __builtin_amdgcn_readfirstlane(
          __hip_atomic_load(&sm_done[wave ^ kFlatWaves], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      if (lane == 0) __hip_atomic_store(&sm_done[wave], i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (mate > i + 1)
        __builtin_amdgcn_s_setprio(2);
      else
        __builtin_amdgcn_s_setprio(0);
    }
    const bool seq_end = cc.t + 1 == cc.tiles;
    if (seq_end || i + 1 == n) {
      const float L = col_sum(st.l);
      const float inv = (L > 0.f) ? 1.0f / L : 0.f;
      if (r16 < nh) {
        const int slot = cc.b + j;
        store_acc<D>(p, st.acc, inv, L, st.m, cc.b, qh0 + r16, c, seg_t0 == 0 && seq_end,
                     (int64_t)slot * p.spb, (int64_t)slot * p.slb);
      }
      if (i + 1 < n) {
        cursor_next(cc, ro(p.seq_lens), p.batch, p.max_tokens);
        seg_t0 = 0;
        reset_state(st);
        load_q(st, p, cc.b, qh0, nh, r16, c);
      }
    } else {
      ++cc.t;
    }
  };
  auto n0_of = [](const SeqCursor &cur) { return cur.t * G::kTT; };

  if constexpr (G::kPrefetch) {
    // tiles of rows up to 64 bytes (4 KB) keep two in flight at any length:
    // one in flight per wave leaves too few bytes in flight for HBM
    const bool shallow = G::kRowBytes > 64 && n > kDeepTiles;
    Tile<KV, D> ta, tb;
    load_tile<KV, SC, D>(ta, p, addr, bt_of(lc.b), n0_of(lc), lc.len, lane);
    int i = 0;
    for (; i + 2 < n; i += 2) {
      cursor_next(lc, ro(p.seq_lens), p.batch, p.max_tokens);
      load_tile<KV, SC, D>(tb, p, addr, bt_of(lc.b), n0_of(lc), lc.len, lane, shallow);
      compute_tile<KV, SC, D>(st, ta, p, n0_of(cc), cc.len, lane, sc_lds, k_lds);
      post(i);
      cursor_next(lc, ro(p.seq_lens), p.batch, p.max_tokens);
      load_tile<KV, SC, D>(ta, p, addr, bt_of(lc.b), n0_of(lc), lc.len, lane, shallow);
      compute_tile<KV, SC, D>(st, tb, p, n0_of(cc), cc.len, lane, sc_lds, k_lds);
      post(i + 1);
    }
    if (i + 1 < n) {
      cursor_next(lc, ro(p.seq_lens), p.batch, p.max_tokens);
      load_tile<KV, SC, D>(tb, p, addr, bt_of(lc.b), n0_of(lc), lc.len, lane, shallow);
      compute_tile<KV, SC, D>(st, ta, p, n0_of(cc), cc.len, lane, sc_lds, k_lds);
      post(i);
      compute_tile<KV, SC, D>(st, tb, p, n0_of(cc), cc.len, lane, sc_lds, k_lds);
      post(i + 1);
    } else {
      compute_tile<KV, SC, D>(st, ta, p, n0_of(cc), cc.len, lane, sc_lds, k_lds);
      post(i);
    }
  } else {
    for (int i = 0; i < n; ++i) {
      Tile<KV, D> t;
      load_tile<KV, SC, D>(t, p, addr, bt_of(cc.b), n0_of(cc), cc.len, lane);
      compute_tile<KV, SC, D>(st, t, p, n0_of(cc), cc.len, lane, sc_lds, k_lds);
      post(i);
    }
  }
}

// Merge of split partials, one wave per (b, h); lanes cover the head dim.
// The split weights are computed once (lanes over splits) and shared through
// LDS, then every lane walks the splits in a fixed order with 16 independent
// loads in flight, so repeated calls are bit-identical.
constexpr int kReduceChunk = 256;  // splits whose weights are staged at once

// Store one lane's slice of a merged row: acc / wsum (zeros when wsum is 0).
template <int D>
__device__ __forceinline__ void write_merged(const RParams &p, const float *acc, float wsum, int b,
                                             int h, int lane, bool active) {
  constexpr int kPer = D / 64 > 0 ? D / 64 : 1;
  const float inv = (wsum > 0.f) ? 1.0f / wsum : 0.f;
  if (!active) return;
  uint8_t *dst = p.out + ((int64_t)b * p.sob + (int64_t)h * p.soh + lane * kPer) * 2;
  float y[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) y[i] = acc[i] * inv;
  if constexpr (kPer >= 2) {
    store_row(dst, y, kPer, p.io_bf16 != 0);
  } else {
    const uint16_t bits = p.io_bf16 ? (uint16_t)f32_to_bf16_bits(y[0])
                                    : __builtin_bit_cast(uint16_t, (_Float16)y[0]);
    *reinterpret_cast<uint16_t *>(dst) = bits;
  }
}

// What the merge reads:
//   kMergeAll   every split of [B, H, S] partials (pa_split_reduce)
//   kMergeAuto  the partials of a kAuto decode: only the sequence's non-empty
//               splits; sequences held by one split (already written) are
//               skipped
//   kMergeFlat  the slots of a flat decode: sequence b's partials are slots
//               b + j0 .. b + j1 for the ranges j0 .. j1 that cut it;
//               sequences inside one range (already written) are skipped and
//               empty sequences get zeros
enum { kMergeAll = 0, kMergeAuto = 1, kMergeFlat = 2 };

// kMergeWaves waves per workgroup, one (b, h) each; the waves never
// synchronise with each other (each stages its weights in its own LDS row).
constexpr int kMergeWaves = 1;

// Fold S partials of row (b, h) into out: the log2-sum-exps at lse[s *
// lse_step], the normalised rows at part[s * part_step]; lanes cover the
// head dim, `sw` is the wave's LDS row for the split weights. S == 0 (an
// empty sequence) writes zeros.
template <int D>
__device__ __forceinline__ void merge_into_out(const RParams &p, const float *lse, const float *part,
                                               int64_t lse_step, int64_t part_step, int S, int b, int h,
                                               int lane, float *sw) {
  constexpr int kPer = D / 64 > 0 ? D / 64 : 1;  // head-dim elements per lane
  const bool active = lane * kPer < D;
  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) acc[i] = 0.f;
  float wsum = 0.f;

  // Few splits (the common case): every lane loads all log2-sum-exps and its
  // slice of every partial in one round trip and folds them in split order.
  // At most 8 held in registers: the merge's VGPRs set how many of its waves
  // are resident, and 8 measured fastest (C2 3.1 us against 3.9 with 32 at
  // head_dim 128, 3.4 with 16; 4 sends C3's longer sequences to the slow path).
  constexpr int kFast = 64 / kPer > 8 ? 8 : 64 / kPer;
  if (S <= kFast) {
    float ls[kFast], v[kFast][kPer];
#pragma unroll
    for (int s = 0; s < kFast; ++s) {
      ls[s] = -INFINITY;
#pragma unroll
      for (int i = 0; i < kPer; ++i) v[s][i] = 0.f;
      if (s < S) {
        ls[s] = lse[s * lse_step];
        if (active) {
#pragma unroll
          for (int i = 0; i < kPer; ++i) v[s][i] = part[(int64_t)s * part_step + lane * kPer + i];
        }
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < kFast; ++s) m = fmaxf(m, ls[s]);
#pragma unroll
    for (int s = 0; s < kFast; ++s) {
      if (s < S) {
        const float w = (ls[s] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ls[s] - m);
        wsum += w;
#pragma unroll
        for (int i = 0; i < kPer; ++i) acc[i] += w * v[s][i];
      }
    }
    write_merged<D>(p, acc, active ? wsum : 0.f, b, h, lane, active);
    return;
  }

  float m = -INFINITY;
  for (int s = lane; s < S; s += 64) m = fmaxf(m, lse[s * lse_step]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));

  // lane-local partial sums of the weights, combined in a fixed tree below
  for (int s0 = 0; s0 < S; s0 += kReduceChunk) {
    const int n = min(kReduceChunk, S - s0);
    // the previous chunk's weights are read before they are overwritten
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int s = lane; s < n; s += 64) {
      const float ls = lse[(s0 + s) * lse_step];
      const float w = (ls == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ls - m);
      sw[s] = w;
      wsum += w;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (active && m != -INFINITY) {
      const float *src = part + (int64_t)s0 * part_step + lane * kPer;
      int s = 0;
      // 16 partials' loads in flight (8 ran 0.7 us slower over 128 slots)
      for (; s + 16 <= n; s += 16) {
        float v[16][kPer];
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
          for (int i = 0; i < kPer; ++i) v[j][i] = src[(int64_t)(s + j) * part_step + i];
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
          for (int i = 0; i < kPer; ++i) acc[i] += sw[s + j] * v[j][i];
      }
      for (; s < n; ++s)
#pragma unroll
        for (int i = 0; i < kPer; ++i) acc[i] += sw[s] * src[(int64_t)s * part_step + i];
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wsum += __shfl_xor(wsum, o);
  write_merged<D>(p, acc, wsum, b, h, lane, active);
}

template <int D, int KIND>
__global__ void __launch_bounds__(kMergeWaves * 64) split_reduce_kernel(const RParams p) {
  __shared__ float sw_all[kMergeWaves][kReduceChunk];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float *sw = sw_all[wave];
  // XCD-contiguous order, as the split decode launches use: an XCD merges
  // a contiguous stretch of (sequence, head) pairs, whose partials that
  // XCD's ranges wrote (0.3-1.3 us per call at C2, C3 and C5)
  int wg = blockIdx.x;
  {
    const int n = gridDim.x, full = n - n % 8;
    if (wg < full) wg = (wg % 8) * (full / 8) + wg / 8;
  }
  const int bh = wg * kMergeWaves + wave;
  if (bh >= p.batch * p.num_heads) return;
  const int b = bh / p.num_heads;
  const int h = bh % p.num_heads;
  const float *lse = p.part_lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  const float *part = p.part_out + (int64_t)b * p.spb + (int64_t)h * p.sph;
  int64_t lse_step = 1;   // elements between consecutive partials
  int64_t part_step = p.sps;
  int S = p.num_splits;
  if (KIND == kMergeAuto) {
    const int seq_len = max(0, min(p.seq_lens[b], p.max_tokens));
    S = split_range(seq_len, p.num_splits, p.max_seq_len, 0).n;
    if (S <= 1) return;
  } else if (KIND == kMergeFlat) {
    // the decode's ranges: per = ceil(total / F) of weight each, where a
    // non-empty sequence weighs its tiles plus flat_cost
    const int nt = seq_tiles(ro(p.seq_lens), b, p.max_tokens);
    const int cost = p.flat_cost;
    int total = 0, cu = 0;  // all weight, weight before sequence b
    if (p.batch <= 64) {  // one chunk
      const int t = lane < p.batch ? seq_tiles(ro(p.seq_lens), lane, p.max_tokens) : 0;
      total = wave_sum(seq_weight(t, cost));
      cu = wave_sum(lane < b ? seq_weight(t, cost) : 0);
    }
    for (int base = 0; base < p.batch && p.batch > 64; base += 64 * kLenChunks) {
      int len[kLenChunks];
      load_len_chunks(ro(p.seq_lens), p.batch, p.max_tokens, base, lane, len);
      int t = 0, tb = 0;
#pragma unroll
      for (int k = 0; k < kLenChunks; ++k) {
        const int wk = seq_weight(len_tiles(len[k]), cost);
        t += wk;
        tb += base + 64 * k + lane < b ? wk : 0;
      }
      total += wave_sum(t);
      cu += wave_sum(tb);
    }
    S = 0;  // empty sequence: the merge below writes zeros
    if (nt > 0) {
      const int per = max(1, (total + p.num_splits - 1) / p.num_splits);
      const int first = cu + cost;  // weight of b's tile 0
      const int j0 = first / per, j1 = (first + nt - 1) / per;
      if (j0 == j1) return;
      S = j1 - j0 + 1;
      lse = p.part_lse + (int64_t)(b + j0) * p.slb + (int64_t)h * p.slh;
      part = p.part_out + (int64_t)(b + j0) * p.spb + (int64_t)h * p.sph;
      lse_step = p.slb;
      part_step = p.spb;
    }
  }

  merge_into_out<D>(p, lse, part, lse_step, part_step, S, b, h, lane, sw);
}

// The flat split's merge when the host knows the lengths: a table of the
// sequences that need it (cut by a range boundary, or empty), so no wave
// reads seq_lens. Item i: sequence seq[i], its slot count nslot[i] (0 =
// empty, zeros; up to the flat split count) and its first slot slot[i] =
// seq[i] + j0. The items are grouped by the XCD that ran the decode range
// j0 (the host computes it from the decode's XCD-contiguous workgroup
// order), and each group's (item, head) waves run on that XCD, where the
// partials were written: whole calls 0.2-0.3 us faster at C2-C5 than the
// plain XCD-contiguous order over the items.
struct MergeTable {
  RParams r;
  int32_t items;
  int32_t xstart[9];  // items [xstart[x], xstart[x + 1]) run on XCD x
  uint32_t seq[kHostTab];
  uint32_t nslot[kHostTab];
  uint32_t slot[kHostTab];
};
static_assert(sizeof(MergeTable) <= 4096 && sizeof(FlatArgs) <= 4096, "kernel arguments over 4 KB");

template <int D>
__global__ void __launch_bounds__(kMergeWaves * 64) flat_merge_table_kernel(const MergeTable a) {
  const RParams &p = a.r;
  __shared__ float sw_all[kMergeWaves][kReduceChunk];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // workgroup h runs on XCD h % 8 (the hardware deals them round-robin)
  const int x = blockIdx.x % 8, k = (blockIdx.x / 8) * kMergeWaves + wave;
  const int it = a.xstart[x] + k / p.num_heads;
  if (it >= a.xstart[x + 1]) return;
  const int h = k % p.num_heads;
  const int b = (int)a.seq[it], S = (int)a.nslot[it];
  const int64_t slot0 = a.slot[it];
  merge_into_out<D>(p, p.part_lse + slot0 * p.slb + (int64_t)h * p.slh,
                    p.part_out + slot0 * p.spb + (int64_t)h * p.sph, p.slb, p.spb, S, b, h, lane,
                    sw_all[wave]);
}

// ----------------------------------------------------------------------------
// host side: validation, error reporting, dispatch
// ----------------------------------------------------------------------------

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof(msg), fmt, ap);
  va_end(ap);
  return pa_fail(code, "%s", msg);
}

int ok() { return pa_ok(); }

bool aligned(const void *ptr, int a) { return pa_aligned(ptr, a); }

bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

int ilog2(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

// Validates and fills the kernel parameter block. `need_partials` is true when
// the decode kernel will write part_out / part_lse.
int build_params(const pa_decode_args *a, bool need_partials, KParams *kp) {
  if (a == nullptr) return fail(PA_ERR_INVALID, "args is NULL");
  if (!a->q || !a->k_cache || !a->v_cache || !a->out || !a->block_table || !a->seq_lens)
    return fail(PA_ERR_INVALID, "q, k_cache, v_cache, out, block_table and seq_lens must be non-NULL");
  if (a->batch < 0) return fail(PA_ERR_INVALID, "batch %d < 0", a->batch);
  if (a->num_q_heads <= 0 || a->num_kv_heads <= 0)
    return fail(PA_ERR_INVALID, "num_q_heads %d / num_kv_heads %d must be positive",
                a->num_q_heads, a->num_kv_heads);
  if (a->num_q_heads % a->num_kv_heads != 0)
    return fail(PA_ERR_INVALID, "num_q_heads=%d not divisible by num_kv_heads=%d",
                a->num_q_heads, a->num_kv_heads);
  if (a->head_dim <= 0) return fail(PA_ERR_INVALID, "head_dim %d must be positive", a->head_dim);
  if (a->head_dim != 32 && a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return fail(PA_ERR_UNSUPPORTED, "head_dim %d not in (32, 64, 128, 256)", a->head_dim);
  if (a->block_size <= 0) return fail(PA_ERR_INVALID, "block_size %d must be positive", a->block_size);
  if (!is_pow2(a->block_size) || a->block_size < 16 || a->block_size > 256)
    return fail(PA_ERR_UNSUPPORTED, "block_size %d not a power of two in [16, 256]", a->block_size);
  if (a->num_blocks <= 0 || a->max_blocks <= 0)
    return fail(PA_ERR_INVALID, "num_blocks %d / max_blocks %d must be positive", a->num_blocks,
                a->max_blocks);
  if (a->num_splits < 1 || a->num_splits > PA_MAX_SPLITS)
    return fail(PA_ERR_INVALID, "num_splits %d not in [1, %d]", a->num_splits, PA_MAX_SPLITS);
  if (a->max_seq_len < 0) return fail(PA_ERR_INVALID, "max_seq_len %d < 0", a->max_seq_len);
  if ((int64_t)a->max_blocks * a->block_size > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "max_blocks * block_size exceeds 2^31 tokens");
  if (a->io_dtype != PA_IO_FP16 && a->io_dtype != PA_IO_BF16)
    return fail(PA_ERR_UNSUPPORTED, "io_dtype %d unsupported", a->io_dtype);
  if (a->kv_dtype != PA_KV_FP16 && a->kv_dtype != PA_KV_FP8_E5M2 && a->kv_dtype != PA_KV_INT8 &&
      a->kv_dtype != PA_KV_BF16)
    return fail(PA_ERR_INVALID, "kv_dtype %d unknown", a->kv_dtype);
  if (a->kv_dtype == PA_KV_INT8) {
    if (a->scale_dtype != PA_SCALE_FP16 && a->scale_dtype != PA_SCALE_FP32)
      return fail(PA_ERR_INVALID, "int8 KV needs scale_dtype fp16 or fp32, got %d", a->scale_dtype);
    if (!a->k_scale || !a->v_scale) return fail(PA_ERR_INVALID, "int8 KV needs k_scale and v_scale");
    if (a->stride_sn < 0 || a->stride_st < 0)
      return fail(PA_ERR_INVALID, "scale strides must be non-negative");
    const int sb = a->scale_dtype == PA_SCALE_FP32 ? 4 : 2;
    if (a->stride_sn * sb >= (int64_t(1) << 32) || (int64_t)a->block_size * a->stride_st * sb >= (int64_t(1) << 31))
      return fail(PA_ERR_UNSUPPORTED, "scale page stride exceeds 4 GiB or a scale page 2 GiB");
    if (!aligned(a->k_scale, sb) || !aligned(a->v_scale, sb))
      return fail(PA_ERR_INVALID, "scale pointers must be %d-byte aligned", sb);
  } else if (a->scale_dtype != PA_SCALE_NONE) {
    return fail(PA_ERR_INVALID, "scale_dtype must be PA_SCALE_NONE for kv_dtype %d", a->kv_dtype);
  }
  if (a->flat_splits < 0 || a->flat_splits > PA_MAX_FLAT_SPLITS)
    return fail(PA_ERR_INVALID, "flat_splits %d not in [0, %d]", a->flat_splits, PA_MAX_FLAT_SPLITS);
  if (a->flat_seq_cost < 0 || a->flat_seq_cost > PA_MAX_FLAT_SEQ_COST)
    return fail(PA_ERR_INVALID, "flat_seq_cost %d not in [0, %d]", a->flat_seq_cost, PA_MAX_FLAT_SEQ_COST);
  if (a->flat_splits > 0) need_partials = true;
  if (need_partials && (!a->part_out || !a->part_lse))
    return fail(PA_ERR_INVALID, "num_splits > 1 / flat_splits > 0 need part_out and part_lse");

  const int elem = (a->kv_dtype == PA_KV_FP16 || a->kv_dtype == PA_KV_BF16) ? 2 : 1;
  const int64_t strides[] = {a->stride_qb, a->stride_qh, a->stride_kn, a->stride_kt, a->stride_kh,
                             a->stride_ob, a->stride_oh, a->stride_btb};
  for (int64_t s : strides)
    if (s < 0) return fail(PA_ERR_INVALID, "strides must be non-negative");
  if (!aligned(a->q, 16) || (a->stride_qb * 2) % 16 || (a->stride_qh * 2) % 16)
    return fail(PA_ERR_INVALID, "q and its batch/head strides must be 16-byte aligned");
  if (!aligned(a->out, 16) || (a->stride_ob * 2) % 16 || (a->stride_oh * 2) % 16)
    return fail(PA_ERR_INVALID, "out and its batch/head strides must be 16-byte aligned");
  if (!aligned(a->k_cache, 16) || !aligned(a->v_cache, 16) || (a->stride_kn * elem) % 16 ||
      (a->stride_kt * elem) % 16 || (a->stride_kh * elem) % 16)
    return fail(PA_ERR_INVALID, "k_cache/v_cache and their strides must be 16-byte aligned");
  // in-page row offsets are 32-bit in the kernel, and so are the page
  // strides that a block index multiplies
  if ((int64_t)a->block_size * a->stride_kt * elem >= (int64_t(1) << 31))
    return fail(PA_ERR_UNSUPPORTED, "page of %d tokens spans more than 2 GiB", a->block_size);
  if ((int64_t)a->batch * a->stride_btb >= (int64_t(1) << 31))
    return fail(PA_ERR_UNSUPPORTED, "block table of %d rows, row stride %lld, spans 2^31 entries",
                a->batch, (long long)a->stride_btb);
  if (a->stride_kn * elem >= (int64_t(1) << 32))
    return fail(PA_ERR_UNSUPPORTED, "page stride of %lld bytes exceeds 4 GiB",
                (long long)(a->stride_kn * elem));
  // the kernels hold the other strides in 32 bits
  const int64_t big = int64_t(1) << 31;
  if (a->stride_qb >= big || a->stride_qh >= big || a->stride_ob >= big || a->stride_oh >= big ||
      a->stride_kh * elem >= big || a->stride_btb >= big)
    return fail(PA_ERR_UNSUPPORTED, "a q, out, kv-head or block-table stride spans 2^31 elements or bytes");
  if (need_partials) {
    if (a->stride_pb < 0 || a->stride_ph < 0 || a->stride_ps < 0 || a->stride_lb < 0 ||
        a->stride_lh < 0)
      return fail(PA_ERR_INVALID, "workspace strides must be non-negative");
    if (a->stride_pb >= big || a->stride_ph >= big || a->stride_ps >= big || a->stride_lb >= big ||
        a->stride_lh >= big)
      return fail(PA_ERR_UNSUPPORTED, "a workspace stride spans 2^31 elements");
    if (!aligned(a->part_out, 16) || (a->stride_pb * 4) % 16 || (a->stride_ph * 4) % 16 ||
        (a->stride_ps * 4) % 16)
      return fail(PA_ERR_INVALID, "part_out and its strides must be 16-byte aligned");
  }

  const int group = a->num_q_heads / a->num_kv_heads;
  const int head_tiles = (group + PA_MAX_GROUP - 1) / PA_MAX_GROUP;
  const int64_t grid = (int64_t)a->batch * a->num_kv_heads * head_tiles * a->num_splits;
  if (grid > 0x7fffffff) return fail(PA_ERR_UNSUPPORTED, "grid of %lld workgroups too large", (long long)grid);
  if (a->flat_splits > 0) {
    // flat tile counts, range starts and slot indices are 32-bit in the kernel
    const int64_t seq_tiles_max = ((int64_t)a->max_blocks * a->block_size + kSplitAlign - 1) / kSplitAlign;
    if ((int64_t)a->batch * (seq_tiles_max + a->flat_seq_cost) + a->flat_splits > 0x7fffffff)
      return fail(PA_ERR_UNSUPPORTED, "batch * max tiles per sequence too large for the flat split");
    if ((int64_t)a->num_kv_heads * head_tiles * a->flat_splits + kFlatWavesInt8 > 0x7fffffff)
      return fail(PA_ERR_UNSUPPORTED, "flat split grid too large");
  }

  KParams &k = *kp;
  k.q = static_cast<const uint8_t *>(a->q);
  k.k = static_cast<const uint8_t *>(a->k_cache);
  k.v = static_cast<const uint8_t *>(a->v_cache);
  k.ks = static_cast<const uint8_t *>(a->k_scale);
  k.vs = static_cast<const uint8_t *>(a->v_scale);
  k.out = static_cast<uint8_t *>(a->out);
  k.part_out = a->part_out;
  k.part_lse = a->part_lse;
  k.bt = a->block_table;
  k.seq_lens = a->seq_lens;
  k.hkv = a->num_kv_heads;
  k.group = group;
  k.head_tiles = head_tiles;
  k.num_splits = a->num_splits;
  k.num_blocks = a->num_blocks;
  k.max_blocks = a->max_blocks;
  k.log2_page = ilog2(a->block_size);
  k.max_seq_len = a->max_seq_len;
  k.batch = a->batch;
  k.max_tokens = a->max_blocks << k.log2_page;
  k.flat_splits = a->flat_splits;
  k.flat_cost = a->flat_splits > 0 ? a->flat_seq_cost : 0;
  k.sqb = a->stride_qb;
  k.sqh = a->stride_qh;
  k.skn = a->stride_kn * elem;
  k.skt = a->stride_kt * elem;
  k.skh = a->stride_kh * elem;
  const int sb = a->scale_dtype == PA_SCALE_FP32 ? 4 : 2;
  k.ssn = a->stride_sn * sb;
  k.sst = a->stride_st * sb;
  k.sob = a->stride_ob;
  k.soh = a->stride_oh;
  k.spb = a->stride_pb;
  k.sph = a->stride_ph;
  k.sps = a->stride_ps;
  k.slb = a->stride_lb;
  k.slh = a->stride_lh;
  k.sbtb = a->stride_btb;
  k.qk_scale = a->sm_scale * kLog2e;
  k.io_bf16 = a->io_dtype == PA_IO_BF16;
  return PA_OK;
}

// Launch modes beyond the classic kernel's.
constexpr int kFlat = 3;

// Launch tables built on the host from host-side lengths (pa_decode_args.
// seq_lens_host): the flat ranges (FlatArgs) and the merge's sequences
// (MergeTable), the same ranges the kernels would find by scanning seq_lens.
struct HostPlan {
  bool ranges = false;       // fa holds the flat ranges
  bool merge_table = false;  // mt holds every sequence the merge must write
  bool needs_merge = true;   // some sequence is cut or empty
  FlatArgs fa;
  MergeTable mt;
};

template <int KV, int SC, int D>
hipError_t launch_decode_t(const KParams &k, int grid, int mode, hipStream_t st, const HostPlan *hp) {
  const dim3 g(grid), blk(kWaves * 64);
  if (mode == kFlat) {
    constexpr int W = flat_waves<KV>();
    const int flat_grid = (k.hkv * k.head_tiles * k.flat_splits + W - 1) / W;
    if (hp != nullptr && hp->ranges) {
      hipLaunchKernelGGL((paged_decode_flat_kernel<KV, SC, D>), dim3(flat_grid), dim3(W * 64), 0, st, hp->fa);
    } else {
      FlatArgs fa;
      fa.p = k;
      fa.ntab = 0;
      hipLaunchKernelGGL((paged_decode_flat_kernel<KV, SC, D>), dim3(flat_grid), dim3(W * 64), 0, st, fa);
    }
  } else if (mode == kAuto) {
    hipLaunchKernelGGL((paged_decode_kernel<KV, SC, D, kAuto>), g, blk, 0, st, k);
  } else if (mode == kPartials) {
    hipLaunchKernelGGL((paged_decode_kernel<KV, SC, D, kPartials>), g, blk, 0, st, k);
  } else {
    hipLaunchKernelGGL((paged_decode_kernel<KV, SC, D, kUnsplit>), g, blk, 0, st, k);
  }
  return hipGetLastError();
}

template <int KV, int SC>
hipError_t launch_decode_d(const KParams &k, int d, int grid, int mode, hipStream_t st, const HostPlan *hp) {
  switch (d) {
    case 32: return launch_decode_t<KV, SC, 32>(k, grid, mode, st, hp);
    case 64: return launch_decode_t<KV, SC, 64>(k, grid, mode, st, hp);
    case 128: return launch_decode_t<KV, SC, 128>(k, grid, mode, st, hp);
    default: return launch_decode_t<KV, SC, 256>(k, grid, mode, st, hp);
  }
}

hipError_t launch_decode(const KParams &k, const pa_decode_args *a, int mode, hipStream_t st,
                         const HostPlan *hp = nullptr) {
  // the flat launch sizes its own grid from its workgroup width
  const int grid = mode == kFlat ? 0 : a->batch * a->num_kv_heads * k.head_tiles * a->num_splits;
  const int d = a->head_dim;
  if (a->kv_dtype == PA_KV_FP16) return launch_decode_d<PA_KV_FP16, PA_SCALE_NONE>(k, d, grid, mode, st, hp);
  if (a->kv_dtype == PA_KV_BF16) return launch_decode_d<PA_KV_BF16, PA_SCALE_NONE>(k, d, grid, mode, st, hp);
  if (a->kv_dtype == PA_KV_FP8_E5M2)
    return launch_decode_d<PA_KV_FP8_E5M2, PA_SCALE_NONE>(k, d, grid, mode, st, hp);
  if (a->scale_dtype == PA_SCALE_FP32) return launch_decode_d<PA_KV_INT8, PA_SCALE_FP32>(k, d, grid, mode, st, hp);
  return launch_decode_d<PA_KV_INT8, PA_SCALE_FP16>(k, d, grid, mode, st, hp);
}

int check_reduce(const pa_reduce_args *r, RParams *rp) {
  if (r == nullptr) return fail(PA_ERR_INVALID, "args is NULL");
  if (!r->part_out || !r->part_lse || !r->out)
    return fail(PA_ERR_INVALID, "part_out, part_lse and out must be non-NULL");
  if (r->batch < 0 || r->num_heads <= 0 || r->num_splits < 1 || r->num_splits > PA_MAX_SPLITS)
    return fail(PA_ERR_INVALID, "bad sizes batch=%d num_heads=%d num_splits=%d", r->batch,
                r->num_heads, r->num_splits);
  if (r->head_dim != 32 && r->head_dim != 64 && r->head_dim != 128 && r->head_dim != 256)
    return fail(PA_ERR_UNSUPPORTED, "head_dim %d not in (32, 64, 128, 256)", r->head_dim);
  if (r->io_dtype != PA_IO_FP16 && r->io_dtype != PA_IO_BF16)
    return fail(PA_ERR_UNSUPPORTED, "io_dtype %d unsupported", r->io_dtype);
  if (r->stride_pb < 0 || r->stride_ph < 0 || r->stride_ps < 0 || r->stride_lb < 0 ||
      r->stride_lh < 0 || r->stride_ob < 0 || r->stride_oh < 0)
    return fail(PA_ERR_INVALID, "strides must be non-negative");
  if ((int64_t)r->batch * r->num_heads > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "grid too large");
  rp->part_out = r->part_out;
  rp->part_lse = r->part_lse;
  rp->out = static_cast<uint8_t *>(r->out);
  rp->io_bf16 = r->io_dtype == PA_IO_BF16;
  rp->seq_lens = nullptr;
  rp->max_tokens = 0;
  rp->max_seq_len = 0;
  rp->batch = r->batch;
  rp->flat_cost = 0;
  rp->num_heads = r->num_heads;
  rp->num_splits = r->num_splits;
  rp->spb = r->stride_pb;
  rp->sph = r->stride_ph;
  rp->sps = r->stride_ps;
  rp->slb = r->stride_lb;
  rp->slh = r->stride_lh;
  rp->sob = r->stride_ob;
  rp->soh = r->stride_oh;
  return PA_OK;
}

template <int KIND>
hipError_t launch_reduce(const RParams &rp, int batch, int d, hipStream_t st) {
  const int grid = (batch * rp.num_heads + kMergeWaves - 1) / kMergeWaves;
  const dim3 blk(kMergeWaves * 64);
  switch (d) {
    case 32: hipLaunchKernelGGL((split_reduce_kernel<32, KIND>), dim3(grid), blk, 0, st, rp); break;
    case 64: hipLaunchKernelGGL((split_reduce_kernel<64, KIND>), dim3(grid), blk, 0, st, rp); break;
    case 128: hipLaunchKernelGGL((split_reduce_kernel<128, KIND>), dim3(grid), blk, 0, st, rp); break;
    default: hipLaunchKernelGGL((split_reduce_kernel<256, KIND>), dim3(grid), blk, 0, st, rp); break;
  }
  return hipGetLastError();
}

hipError_t launch_merge_table(const MergeTable &mt, int d, hipStream_t st) {
  int most = 0;
  for (int x = 0; x < 8; ++x) most = std::max(most, mt.xstart[x + 1] - mt.xstart[x]);
  const int grid = 8 * ((most * mt.r.num_heads + kMergeWaves - 1) / kMergeWaves);
  const dim3 blk(kMergeWaves * 64);
  switch (d) {
    case 32: hipLaunchKernelGGL((flat_merge_table_kernel<32>), dim3(grid), blk, 0, st, mt); break;
    case 64: hipLaunchKernelGGL((flat_merge_table_kernel<64>), dim3(grid), blk, 0, st, mt); break;
    case 128: hipLaunchKernelGGL((flat_merge_table_kernel<128>), dim3(grid), blk, 0, st, mt); break;
    default: hipLaunchKernelGGL((flat_merge_table_kernel<256>), dim3(grid), blk, 0, st, mt); break;
  }
  return hipGetLastError();
}

// The flat split's ranges and merge list from host-side lengths, exactly as
// the kernels derive them from seq_lens (flat_locate*, kMergeFlat): lengths
// clamped to the block table; sequence b weighs its tiles plus flat_cost when
// non-empty; per = max(1, ceil(W / F)); range j holds the tiles whose weights
// lie in [j * per, (j + 1) * per). Tables that do not fit (more than
// kHostTab ranges or merge entries, a batch over 4096, sequences of 2^20
// tiles) are left off and the kernels scan seq_lens.
//
// `all` (pa_flat_host_plan) receives the complete tables whatever their
// size: ranges[3 j ..] = (first sequence, first tile, tile count) of range j
// (3 F entries), items[3 i ..] = (sequence, first slot, slot count) of the
// i-th sequence the merge writes (3 B entries), and their count.
struct HostPlanOut {
  int32_t *ranges;
  int32_t *items;
  int32_t n_items;
};

void build_host_plan(const pa_decode_args *a, const KParams &k, HostPlan *hp, HostPlanOut *all = nullptr) {
  hp->ranges = hp->merge_table = false;
  hp->needs_merge = true;
  if (a->seq_lens_host == nullptr || a->flat_splits <= 0) return;
  const int F = a->flat_splits, B = a->batch, cost = k.flat_cost;
  const int64_t max_tiles = ((int64_t)k.max_tokens + kSplitAlign - 1) / kSplitAlign;
  int64_t W = 0;
  for (int b = 0; b < B; ++b) {
    const int t = (std::max(0, std::min(a->seq_lens_host[b], k.max_tokens)) + kSplitAlign - 1) / kSplitAlign;
    W += t > 0 ? t + cost : 0;
  }
  const int64_t per = std::max<int64_t>(1, (W + F - 1) / F);
  const bool ranges = F <= kHostTab && B <= (1 << (32 - kTabTBits)) && max_tiles <= (int64_t)kTabTMask;
  FlatArgs &fa = hp->fa;
  MergeTable &mt = hp->mt;
  if (ranges) {
    fa.p = k;
    fa.ntab = F;
    for (int j = 0; j < F; ++j) fa.start[j] = fa.ntile[j] = fa.len[j] = 0;
  }
  if (all != nullptr)
    for (int j = 0; j < 3 * F; ++j) all->ranges[j] = 0;
  int items = 0;
  int64_t cw = 0;
  for (int b = 0; b < B; ++b) {
    const int len = std::max(0, std::min(a->seq_lens_host[b], k.max_tokens));
    const int t = (len + kSplitAlign - 1) / kSplitAlign;
    int64_t S = 0, slot = 0;
    if (t > 0) {
      const int64_t first = cw + cost;  // weight of tile 0
      const int64_t j0 = first / per, j1 = (first + t - 1) / per;
      if (ranges || all != nullptr) {
        for (int64_t j = j0; j <= j1; ++j) {
          const int64_t lo = std::max(first, j * per), hi = std::min(first + t, (j + 1) * per);
          if (ranges) {
            if (fa.ntile[j] == 0) {
              fa.start[j] = ((uint32_t)b << kTabTBits) | (uint32_t)(lo - first);
              fa.len[j] = (uint32_t)len;
            }
            fa.ntile[j] += (uint32_t)(hi - lo);
          }
          if (all != nullptr) {
            int32_t *r = all->ranges + 3 * j;
            if (r[2] == 0) {
              r[0] = b;
              r[1] = (int32_t)(lo - first);
            }
            r[2] += (int32_t)(hi - lo);
          }
        }
      }
      cw += t + cost;
      if (j0 == j1) continue;  // inside one range: the decode pass writes it
      S = j1 - j0 + 1;         // up to F: 32 bits, like the slot index
      slot = b + j0;
    }
    if (items < kHostTab) {
      mt.seq[items] = (uint32_t)b;
      mt.nslot[items] = (uint32_t)S;
      mt.slot[items] = (uint32_t)slot;
    }
    if (all != nullptr) {
      all->items[3 * items] = b;
      all->items[3 * items + 1] = (int32_t)slot;
      all->items[3 * items + 2] = (int32_t)S;
    }
    ++items;
  }
  hp->ranges = ranges;
  hp->needs_merge = items > 0;
  if (items <= kHostTab) {
    hp->merge_table = true;
    mt.items = items;
    // XCD of each item: the one holding the flat decode's logical
    // workgroup of range j0 (unit 0), under the decode's XCD-contiguous order
    const int units = k.hkv * k.head_tiles;
    const int FW = flat_waves_of(a->kv_dtype);
    const int grid = (units * F + FW - 1) / FW, full = grid - grid % 8;
    int xcd[kHostTab], cnt[8] = {0};
    for (int i = 0; i < items; ++i) {
      const int64_t j0 = mt.nslot[i] > 0 ? (int64_t)mt.slot[i] - mt.seq[i] : 0;
      const int64_t L = (j0 * units) / FW;
      xcd[i] = L < full ? (int)(L / (full / 8)) : (int)(L % 8);
      ++cnt[xcd[i]];
    }
    mt.xstart[0] = 0;
    for (int x = 0; x < 8; ++x) mt.xstart[x + 1] = mt.xstart[x] + cnt[x];
    uint32_t s2[kHostTab], n2[kHostTab], o2[kHostTab];
    int pos[8];
    for (int x = 0; x < 8; ++x) pos[x] = mt.xstart[x];
    for (int i = 0; i < items; ++i) {
      const int q = pos[xcd[i]]++;
      s2[q] = mt.seq[i]; n2[q] = mt.nslot[i]; o2[q] = mt.slot[i];
    }
    for (int i = 0; i < items; ++i) { mt.seq[i] = s2[i]; mt.nslot[i] = n2[i]; mt.slot[i] = o2[i]; }
  }
  if (all != nullptr) all->n_items = items;
}

// Whether work launched on `st` now is being captured into a HIP graph (an
// unknown state counts as captured).
bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus s = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &s) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return s != hipStreamCaptureStatusNone;
}

// The host plan of a launch on `st`. Under HIP graph capture there is none:
// the tables would be frozen into the graph's kernel arguments while a replay
// may run on other lengths (a serving loop updates seq_lens in place between
// replays), so the kernels scan seq_lens, which is right for any lengths.
void launch_host_plan(const pa_decode_args *a, const KParams &k, HostPlan *hp, hipStream_t st) {
  if (a->seq_lens_host != nullptr && a->flat_splits > 0 && stream_capturing(st)) {
    hp->ranges = hp->merge_table = false;
    hp->needs_merge = true;
    return;
  }
  build_host_plan(a, k, hp);
}

pa_reduce_args reduce_args_from(const pa_decode_args *a) {
  pa_reduce_args r;
  r.part_out = a->part_out;
  r.part_lse = a->part_lse;
  r.out = a->out;
  r.batch = a->batch;
  r.num_heads = a->num_q_heads;
  r.head_dim = a->head_dim;
  r.num_splits = a->num_splits;
  r.stride_pb = a->stride_pb;
  r.stride_ph = a->stride_ph;
  r.stride_ps = a->stride_ps;
  r.stride_lb = a->stride_lb;
  r.stride_lh = a->stride_lh;
  r.stride_ob = a->stride_ob;
  r.stride_oh = a->stride_oh;
  r.io_dtype = a->io_dtype;
  return r;
}

}  // namespace

namespace {
thread_local char g_err[512] = "";
}  // namespace

// The split partials of pa_decode_noalloc: one array per GPU, loaded with
// the code object and held until the process ends. In host code `scratch`
// only names the symbol for the runtime; kernels get the device address
// that scratch_address() looks up.
static __device__ __align__(256) uint8_t scratch[PA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// This GPU's `scratch` address: hipGetSymbolAddress once per device, with
// the device current, then the kept pointer.
int scratch_address(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pa_fail(PA_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return pa_fail(PA_ERR_UNSUPPORTED, "device %d is beyond the %d the library keeps scratch for", dev,
                   kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return pa_fail(PA_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PA_OK;
}
}  // namespace

int pa_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int pa_ok() {
  g_err[0] = '\0';
  return PA_OK;
}

const char *pa_error_message() { return g_err; }

extern "C" {

int pa_abi_version(void) { return PA_ABI_VERSION; }

const char *pa_last_error(void) { return g_err; }

int pa_decode(const pa_decode_args *a, void *stream) {
  KParams k;
  const bool flat = a != nullptr && a->flat_splits > 0;
  const bool split = a != nullptr && (a->num_splits > 1 || flat);
  int rc = build_params(a, split, &k);
  if (rc != PA_OK) return rc;
  RParams rp;
  pa_reduce_args ra;
  if (split) {
    ra = reduce_args_from(a);
    if (flat) ra.num_splits = 1;  // validated above; the merge reads flat_splits
    rc = check_reduce(&ra, &rp);
    if (rc != PA_OK) return rc;
    rp.seq_lens = a->seq_lens;
    rp.max_tokens = k.max_tokens;
    rp.max_seq_len = a->max_seq_len;
    if (flat) {
      rp.num_splits = a->flat_splits;
      rp.flat_cost = a->flat_seq_cost;
    }
  }
  if (a->batch == 0) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  HostPlan plan;
  if (flat) launch_host_plan(a, k, &plan, st);
  hipError_t e = launch_decode(k, a, flat ? kFlat : split ? kAuto : kUnsplit, st, &plan);
  if (e != hipSuccess) return fail(PA_ERR_HIP, "decode launch failed: %s", hipGetErrorString(e));
  if (split && !(flat && !plan.needs_merge)) {
    if (flat && plan.merge_table) {
      plan.mt.r = rp;
      e = launch_merge_table(plan.mt, a->head_dim, st);
    } else {
      e = flat ? launch_reduce<kMergeFlat>(rp, a->batch, a->head_dim, st)
               : launch_reduce<kMergeAuto>(rp, a->batch, a->head_dim, st);
    }
    if (e != hipSuccess) return fail(PA_ERR_HIP, "reduce launch failed: %s", hipGetErrorString(e));
  }
  return ok();
}

int pa_decode_noalloc(const pa_decode_args *a, void *stream) {
  if (a == nullptr) return fail(PA_ERR_INVALID, "args is NULL");
  pa_decode_args b = *a;
  const bool flat = b.flat_splits > 0;
  const bool split = flat || b.num_splits > 1;
  b.part_out = nullptr;
  b.part_lse = nullptr;
  if (!split) return pa_decode(&b, stream);  // unsplit: no partials, no scratch
  // every argument is validated (with a stand-in workspace address that is
  // never used) before the size check and the first HIP call
  float *const stand_in = reinterpret_cast<float *>(uintptr_t(256));
  b.part_out = stand_in;
  b.part_lse = stand_in;
  b.stride_pb = b.stride_ph = b.stride_ps = b.stride_lb = b.stride_lh = 0;
  KParams k;
  int rc = build_params(&b, true, &k);
  if (rc != PA_OK) return rc;
  // packed partials: flat slots [batch + F, Hq, D] / [batch + F, Hq], or the
  // classic [B, Hq, S, D] / [B, Hq, S] (sizes validated above)
  const int64_t hq = b.num_q_heads, d = b.head_dim, s = flat ? 1 : b.num_splits;
  b.stride_ph = s * d;
  b.stride_pb = hq * s * d;
  b.stride_ps = flat ? 0 : d;
  b.stride_lh = s;
  b.stride_lb = hq * s;
  const int64_t slots = flat ? (int64_t)b.batch + b.flat_splits : (int64_t)b.batch * b.num_splits;
  const int64_t rows = slots * hq;  // < 2^63: slots < 2^33, hq < 2^31
  const int64_t cap = PA_NOALLOC_SCRATCH_BYTES;
  const int64_t lse_off = rows <= cap ? (rows * d * 4 + 255) / 256 * 256 : cap + 1;
  if (rows > cap / (4 * (d + 1)) || lse_off + rows * 4 > cap)
    return fail(PA_ERR_UNSUPPORTED,
                "%s needs %lld partial rows of %lld floats (plus their log-sum-exps), more than the "
                "%lld-byte static scratch of pa_decode_noalloc holds",
                flat ? "this flat split" : "this split", (long long)rows, (long long)d, (long long)cap);
  void *base = nullptr;
  rc = scratch_address(&base);
  if (rc != PA_OK) return rc;
  b.part_out = static_cast<float *>(base);
  b.part_lse = reinterpret_cast<float *>(static_cast<uint8_t *>(base) + lse_off);
  return pa_decode(&b, stream);
}

int pa_decode_partials(const pa_decode_args *a, void *stream) {
  KParams k;
  int rc = build_params(a, true, &k);
  if (rc != PA_OK) return rc;
  if (a->batch == 0) return ok();
  HostPlan plan;
  if (a->flat_splits > 0) launch_host_plan(a, k, &plan, static_cast<hipStream_t>(stream));
  hipError_t e = launch_decode(k, a, a->flat_splits > 0 ? kFlat : kPartials,
                               static_cast<hipStream_t>(stream), &plan);
  if (e != hipSuccess) return fail(PA_ERR_HIP, "decode launch failed: %s", hipGetErrorString(e));
  return ok();
}

int pa_flat_merge(const pa_decode_args *a, void *stream) {
  KParams k;
  int rc = build_params(a, true, &k);
  if (rc != PA_OK) return rc;
  if (a->flat_splits <= 0) return fail(PA_ERR_INVALID, "pa_flat_merge needs flat_splits > 0");
  pa_reduce_args ra = reduce_args_from(a);
  ra.num_splits = 1;
  RParams rp;
  rc = check_reduce(&ra, &rp);
  if (rc != PA_OK) return rc;
  rp.seq_lens = a->seq_lens;
  rp.max_tokens = k.max_tokens;
  rp.num_splits = a->flat_splits;
  rp.flat_cost = a->flat_seq_cost;
  if (a->batch == 0) return ok();
  HostPlan plan;
  launch_host_plan(a, k, &plan, static_cast<hipStream_t>(stream));
  if (!plan.needs_merge) return ok();  // every sequence inside one range: nothing to fold
  hipError_t e;
  if (plan.merge_table) {
    plan.mt.r = rp;
    e = launch_merge_table(plan.mt, a->head_dim, static_cast<hipStream_t>(stream));
  } else {
    e = launch_reduce<kMergeFlat>(rp, a->batch, a->head_dim, static_cast<hipStream_t>(stream));
  }
  if (e != hipSuccess) return fail(PA_ERR_HIP, "reduce launch failed: %s", hipGetErrorString(e));
  return ok();
}

int pa_flat_host_plan(const pa_decode_args *a, int32_t *ranges, int32_t *items, int32_t *n_items,
                      int32_t *in_kernel_args) {
  if (ranges == nullptr || items == nullptr || n_items == nullptr)
    return fail(PA_ERR_INVALID, "ranges, items and n_items must be non-NULL");
  KParams k;
  int rc = build_params(a, true, &k);
  if (rc != PA_OK) return rc;
  if (a->flat_splits <= 0 || a->seq_lens_host == nullptr)
    return fail(PA_ERR_INVALID, "pa_flat_host_plan needs flat_splits > 0 and seq_lens_host");
  HostPlan plan;
  HostPlanOut all = {ranges, items, 0};
  build_host_plan(a, k, &plan, &all);
  *n_items = all.n_items;
  if (in_kernel_args != nullptr)
    *in_kernel_args = (plan.ranges ? PA_HOST_PLAN_RANGES : 0) | (plan.merge_table ? PA_HOST_PLAN_MERGE : 0);
  return ok();
}

int pa_flat_waves_per_simd(int kv_dtype, int scale_dtype, int head_dim, int *out) {
  if (out == nullptr) return fail(PA_ERR_INVALID, "out is NULL");
  *out = 0;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(PA_ERR_UNSUPPORTED, "head_dim %d not in (32, 64, 128, 256)", head_dim);
  const void *fn = nullptr;
  auto pick = [&](auto kv_tag, auto sc_tag) {
    constexpr int KV = decltype(kv_tag)::value, SC = decltype(sc_tag)::value;
    switch (head_dim) {
      case 32:
        fn = reinterpret_cast<const void *>(&paged_decode_flat_kernel<KV, SC, 32>);
        break;
      case 64:
        fn = reinterpret_cast<const void *>(&paged_decode_flat_kernel<KV, SC, 64>);
        break;
      case 128:
        fn = reinterpret_cast<const void *>(&paged_decode_flat_kernel<KV, SC, 128>);
        break;
      default:
        fn = reinterpret_cast<const void *>(&paged_decode_flat_kernel<KV, SC, 256>);
        break;
    }
  };
  using I = int;
  if (kv_dtype == PA_KV_FP16 && scale_dtype == PA_SCALE_NONE)
    pick(std::integral_constant<I, PA_KV_FP16>{}, std::integral_constant<I, PA_SCALE_NONE>{});
  else if (kv_dtype == PA_KV_BF16 && scale_dtype == PA_SCALE_NONE)
    pick(std::integral_constant<I, PA_KV_BF16>{}, std::integral_constant<I, PA_SCALE_NONE>{});
  else if (kv_dtype == PA_KV_FP8_E5M2 && scale_dtype == PA_SCALE_NONE)
    pick(std::integral_constant<I, PA_KV_FP8_E5M2>{}, std::integral_constant<I, PA_SCALE_NONE>{});
  else if (kv_dtype == PA_KV_INT8 && scale_dtype == PA_SCALE_FP16)
    pick(std::integral_constant<I, PA_KV_INT8>{}, std::integral_constant<I, PA_SCALE_FP16>{});
  else if (kv_dtype == PA_KV_INT8 && scale_dtype == PA_SCALE_FP32)
    pick(std::integral_constant<I, PA_KV_INT8>{}, std::integral_constant<I, PA_SCALE_FP32>{});
  else
    return fail(PA_ERR_INVALID, "kv_dtype %d / scale_dtype %d is not a supported pair", kv_dtype,
                scale_dtype);
  int n = 0;
  const int FW = flat_waves_of(kv_dtype);
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, FW * 64, 0);
  if (e != hipSuccess) return fail(PA_ERR_HIP, "occupancy query failed: %s", hipGetErrorString(e));
  *out = n * FW / 4;  // workgroups per CU -> waves per SIMD (4 SIMDs per CU)
  return ok();
}

int pa_split_reduce(const pa_reduce_args *r, void *stream) {
  RParams rp;
  int rc = check_reduce(r, &rp);
  if (rc != PA_OK) return rc;
  if (r->batch == 0) return ok();
  hipError_t e = launch_reduce<kMergeAll>(rp, r->batch, r->head_dim, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PA_ERR_HIP, "reduce launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
