// Paged-KV grouped-query decode attention for MI355X (gfx950, CDNA4).
//
// Replaces the two Triton kernels of the reference
// (ParamThakkar123/paged-decode-attention, pagedattn/triton_decode.py):
//   _paged_decode_kernel  (:33-195)  -> paged_decode_kernel<...>
//   _split_reduce_kernel  (:198-240) -> split_reduce_kernel
// and the launch section of `paged_decode_triton` (:331-376) -> pa_decode.
//
// Work decomposition. One workgroup of kWaves wave64s per
// (batch, kv_head, head_tile, split). The workgroup's token range [lo, hi) is
// cut into 32-token tiles; wave w takes tiles w, w + kWaves, ... Every wave
// keeps its own online-softmax state in VGPRs and the waves are merged once
// through LDS at the end, so a workgroup is a split of kWaves sub-splits that
// costs a single partial write.
//
// Per 32-token tile (two 16-token sub-tiles, each inside one page because the
// page size is a multiple of 16):
//   S^T[tok, h] = K[tok, :] . Q[h, :]   v_mfma_f32_16x16x32_f16, A = K rows
//                                        (lane row = token), B = Q^T (lane
//                                        column = query head of the group)
//   O^T[d, h] += V^T[d, tok] P^T[tok, h] v_mfma_f32_16x16x32_f16, A = V^T,
//                                        B = P^T taken straight from the QK
//                                        accumulator layout (no shuffles)
// K rows are loaded in 16-byte pieces directly into the MFMA A-operand layout.
// V rows are loaded in the natural [tok][d] layout, 16 lanes covering one row
// contiguously, and transposed to [d][tok] pairs in registers with byte
// permutes. All `group` query heads of a kv head share the tile (padded to the
// 16 MFMA columns), so each K/V byte is read from HBM once.
//
// Online softmax in the log2 domain as the reference (triton_decode.py:155-166)
// with one change: the running maximum is only moved when a tile's maximum
// exceeds it by more than kRescaleLog2, so the accumulator rescale is skipped
// on most tiles. This is exact algebra (the normaliser uses the same stale
// maximum); probabilities stay <= 2^kRescaleLog2, far from fp16 overflow.
//
// Quantised KV is dequantised in registers:
//   fp8_e5m2 -> fp16: the e5m2 byte is the high byte of the fp16 pattern.
//   int8 -> fp16 exactly (|x| <= 127), with the per-(token, head) scale folded
//           into the fp32 score (K) and into the probability (V).

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "pagedattn.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;          // waves per workgroup
constexpr int kTile = 32;          // tokens per wave iteration
constexpr float kRescaleLog2 = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;

#ifndef PA_XCD_SWIZZLE
#define PA_XCD_SWIZZLE 0
#endif
#ifndef PA_KV_NONTEMPORAL
#define PA_KV_NONTEMPORAL 1
#endif

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
  int32_t hkv, group, head_tiles, num_splits, num_blocks, max_blocks, log2_page;
  int64_t sqb, sqh;          // elements
  int64_t skn, skt, skh;     // bytes
  int64_t ssn, sst;          // bytes
  int64_t sob, soh;          // elements
  int64_t spb, sph, sps;     // elements
  int64_t slb, slh;          // elements
  int64_t sbtb;              // elements
  float qk_scale;            // sm_scale * log2(e)
};

struct RParams {
  const float *part_out;
  const float *part_lse;
  uint8_t *out;
  int32_t num_heads, num_splits;
  int64_t spb, sph, sps, slb, slh, sob, soh;  // elements
};

__device__ __forceinline__ float wave_max16(float x) {
  // max over the four lanes l, l^16, l^32, l^48 (same MFMA column)
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float wave_sum16(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// 16-bit lane `s` of a packed array of fp16 values held in dwords.
__device__ __forceinline__ uint32_t half_at(const uint32_t *w, int s) {
  return (w[s >> 1] >> ((s & 1) * 16)) & 0xffffu;
}

// Byte `s` of a packed byte array held in dwords.
__device__ __forceinline__ uint32_t byte_at(const uint32_t *w, int s) {
  return (w[s >> 2] >> ((s & 3) * 8)) & 0xffu;
}

// fp16 bit pattern of the value of one stored KV element.
//   KV == PA_KV_FP8_E5M2: exact, the e5m2 byte is the high byte of the fp16.
//   KV == PA_KV_INT8:     1024 + 128 + x as fp16 bits; the caller subtracts
//                         1152 in fp16 afterwards, which is exact.
template <int KV>
__device__ __forceinline__ uint32_t byte_to_half_bits(uint32_t b) {
  if constexpr (KV == PA_KV_FP8_E5M2) {
    return b << 8;
  } else {
    return 0x6400u | (b ^ 0x80u);
  }
}

__device__ __forceinline__ f16x8 bits_to_f16x8(uint32_t w0, uint32_t w1, uint32_t w2,
                                               uint32_t w3) {
  u32x4 u = {w0, w1, w2, w3};
  return __builtin_bit_cast(f16x8, u);
}

template <int KV>
__device__ __forceinline__ f16x8 fix_int8(f16x8 x) {
  if constexpr (KV == PA_KV_INT8) {
    const _Float16 off = (_Float16)1152.0f;
    f16x8 o = {off, off, off, off, off, off, off, off};
    return x - o;
  } else {
    return x;
  }
}

// One K/V load. K and V are streamed exactly once per call, so they may be
// fetched with the non-temporal hint to keep them from displacing reusable
// lines in the caches.
template <typename T>
__device__ __forceinline__ T ld(const uint8_t *p) {
#if PA_KV_NONTEMPORAL
  return __builtin_nontemporal_load(reinterpret_cast<const T *>(p));
#else
  return *reinterpret_cast<const T *>(p);
#endif
}

// Load `BYTES` bytes (2, 4, 8, 16 or 32) of K/V into dwords `w`.
template <int BYTES>
__device__ __forceinline__ void load_bytes(uint32_t *w, const uint8_t *p) {
  if constexpr (BYTES == 32) {
    u32x4 a = ld<u32x4>(p);
    u32x4 b = ld<u32x4>(p + 16);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (BYTES == 16) {
    u32x4 a = ld<u32x4>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (BYTES == 8) {
    u32x2 a = ld<u32x2>(p);
    w[0] = a.x; w[1] = a.y;
  } else if constexpr (BYTES == 4) {
    w[0] = ld<uint32_t>(p);
  } else {
    static_assert(BYTES == 2, "unsupported load width");
    w[0] = ld<uint16_t>(p);
  }
}

template <int BYTES>
__device__ __forceinline__ void zero_words(uint32_t *w) {
#pragma unroll
  for (int i = 0; i < (BYTES + 3) / 4; ++i) w[i] = 0;
}

template <int SC>
__device__ __forceinline__ float load_scale(const uint8_t *p) {
  if constexpr (SC == PA_SCALE_FP32) {
    return *reinterpret_cast<const float *>(p);
  } else {
    return (float)*reinterpret_cast<const _Float16 *>(p);
  }
}

// Compile-time geometry for one (KV dtype, head_dim) instance.
template <int KV, int D>
struct Geo {
  static constexpr int kElem = (KV == PA_KV_FP16) ? 2 : 1;  // stored bytes/elem
  static constexpr int kKSteps = D / 32;                    // QK MFMAs per sub-tile
  static constexpr int kE = D / 16;                         // V elems per lane row
  static constexpr int kVBytes = kE * kElem;                // V bytes per lane row
  static constexpr int kVWords = (kVBytes + 3) / 4;
  // K piece loaded per lane: 16 B for fp16 (one k-step); for 1-byte types one
  // 16-byte piece covers two k-steps (8 B when head_dim == 32).
  static constexpr int kKPieceBytes = (kElem == 2) ? 16 : (D >= 64 ? 16 : 8);
  static constexpr int kKStepsPerPiece = (kElem == 2) ? 1 : (D >= 64 ? 2 : 1);
  static constexpr int kKPieces = kKSteps / kKStepsPerPiece;
};

// Byte offset inside a K row of the piece read by lane group `c` for piece `j`.
// The head-dim index of element e of k-step `ks` for lane group c is
//   2-byte types: 32*ks + 8*c + e
//   1-byte types: 64*(ks/2) + 16*c + 8*(ks%2) + e   (head_dim >= 64)
// Q is loaded with the same mapping, which is all the MFMA reduction needs.
template <int KV, int D>
__device__ __forceinline__ int k_piece_offset(int j, int c) {
  using G = Geo<KV, D>;
  if constexpr (G::kElem == 2) {
    return (32 * j + 8 * c) * 2;
  } else if constexpr (D >= 64) {
    return 64 * j + 16 * c;
  } else {
    return 8 * c;
  }
}

template <int KV, int D>
__device__ __forceinline__ int q_dim_offset(int ks, int c) {
  using G = Geo<KV, D>;
  if constexpr (G::kElem == 2 || D < 64) {
    return 32 * ks + 8 * c;
  } else {
    return 64 * (ks / 2) + 16 * c + 8 * (ks % 2);
  }
}

template <int KV, int SC, int D>
struct WaveState {
  using G = Geo<KV, D>;
  f16x8 qop[G::kKSteps];  // Q^T B-operands
  f32x4 acc[G::kE];       // O^T accumulators, one 16x16 block per d-slab
  float m;                // running max (log2 domain) for head column r16
  float l;                // running sum over this lane's tokens
};

// One 32-token tile for one wave. MASKED handles the range tail.
template <int KV, int SC, int D, bool MASKED>
__device__ __forceinline__ void tile_step(WaveState<KV, SC, D> &st, const KParams &p,
                                          const int32_t *bt_row, int kvh, int n0, int hi,
                                          int lane) {
  using G = Geo<KV, D>;
  const int r16 = lane & 15;
  const int c = lane >> 4;
  const int page_mask = (1 << p.log2_page) - 1;

  // ---- block-table lookup: one entry per 16-token sub-tile (uniform) ----
  int64_t base[2];
  int phys[2], off[2];
  bool sub_live[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int tok0 = n0 + 16 * u;
    sub_live[u] = !MASKED || tok0 < hi;
    phys[u] = 0;
    off[u] = 0;
    if (sub_live[u]) {
      phys[u] = min(max(bt_row[tok0 >> p.log2_page], 0), p.num_blocks - 1);
      off[u] = tok0 & page_mask;
    }
    base[u] = (int64_t)phys[u] * p.skn + (int64_t)off[u] * p.skt + (int64_t)kvh * p.skh;
  }

  // ---- K: lane row = token (16u + r16), 16-byte pieces of the row ----
  uint32_t kw[2][G::kKPieces][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const bool live = sub_live[u] && (!MASKED || (n0 + 16 * u + r16) < hi);
    const uint8_t *row = p.k + base[u] + (int64_t)r16 * p.skt;
#pragma unroll
    for (int j = 0; j < G::kKPieces; ++j) {
      if (live) {
        load_bytes<G::kKPieceBytes>(kw[u][j], row + k_piece_offset<KV, D>(j, c));
      } else {
        zero_words<16>(kw[u][j]);
      }
    }
  }

  // ---- V: lane (c, r16) reads tokens {4c+i, 16+4c+i}, elems [kE*r16, +kE) ----
  uint32_t vw[8][G::kVWords];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int u = e >> 2;
    const int trow = 4 * c + (e & 3);
    const bool live = sub_live[u] && (!MASKED || (n0 + 16 * u + trow) < hi);
    const uint8_t *row = p.v + base[u] + (int64_t)trow * p.skt + G::kVBytes * r16;
    if (live) {
      load_bytes<G::kVBytes>(vw[e], row);
    } else {
      zero_words<G::kVBytes>(vw[e]);
    }
  }

  // ---- int8 scales for this lane's 8 tokens ----
  float ksc[8], vsc[8];
  if constexpr (KV == PA_KV_INT8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int u = e >> 2;
      const int trow = 4 * c + (e & 3);
      const bool live = sub_live[u] && (!MASKED || (n0 + 16 * u + trow) < hi);
      ksc[e] = 0.f;
      vsc[e] = 0.f;
      if (live) {
        const int64_t so = (int64_t)phys[u] * p.ssn + (int64_t)(off[u] + trow) * p.sst +
                           (int64_t)kvh * (SC == PA_SCALE_FP32 ? 4 : 2);
        ksc[e] = load_scale<SC>(p.ks + so);
        vsc[e] = load_scale<SC>(p.vs + so);
      }
    }
  }

  // ---- S^T = K Q^T ----
  f32x4 sacc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < G::kKSteps; ++ks) {
      f16x8 kop;
      if constexpr (G::kElem == 2) {
        const uint32_t *w = kw[u][ks];
        kop = bits_to_f16x8(w[0], w[1], w[2], w[3]);
      } else {
        const int j = ks / G::kKStepsPerPiece;
        const int half = ks % G::kKStepsPerPiece;  // which 8 bytes of the piece
        const uint32_t *w = kw[u][j] + 2 * half;
        uint32_t h[4];
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          const uint32_t b0 = byte_at(w, 2 * q2);
          const uint32_t b1 = byte_at(w, 2 * q2 + 1);
          h[q2] = byte_to_half_bits<KV>(b0) | (byte_to_half_bits<KV>(b1) << 16);
        }
        kop = fix_int8<KV>(bits_to_f16x8(h[0], h[1], h[2], h[3]));
      }
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, st.qop[ks], a, 0, 0, 0);
    }
    sacc[u] = a;
  }

  // ---- online softmax over the 8 tokens this lane holds for head r16 ----
  float s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = sacc[e >> 2][e & 3] * p.qk_scale;
    if constexpr (KV == PA_KV_INT8) x *= ksc[e];
    if constexpr (MASKED) {
      const int tok = n0 + 16 * (e >> 2) + 4 * c + (e & 3);
      if (tok >= hi) x = -INFINITY;
    }
    s[e] = x;
  }
  float tmax = s[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) tmax = fmaxf(tmax, s[e]);
  tmax = wave_max16(tmax);

  const bool need = tmax > st.m + kRescaleLog2;
  if (__builtin_amdgcn_ballot_w64(need) != 0) {
    const float m_new = need ? fmaxf(st.m, tmax) : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int sl = 0; sl < G::kE; ++sl) st.acc[sl] *= alpha;
    st.m = m_new;
  }

  float pr[8];
  float lsum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pr[e] = __builtin_amdgcn_exp2f(s[e] - st.m);
    lsum += pr[e];
  }
  st.l += lsum;

  f16x8 pop;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = pr[e];
    if constexpr (KV == PA_KV_INT8) x *= vsc[e];
    pop[e] = (_Float16)x;
  }

  // ---- O^T += V^T P^T, one MFMA per d-slab ----
#pragma unroll
  for (int sl = 0; sl < G::kE; ++sl) {
    uint32_t h[4];
#pragma unroll
    for (int m2 = 0; m2 < 4; ++m2) {
      if constexpr (G::kElem == 2) {
        h[m2] = half_at(vw[2 * m2], sl) | (half_at(vw[2 * m2 + 1], sl) << 16);
      } else {
        h[m2] = byte_to_half_bits<KV>(byte_at(vw[2 * m2], sl)) |
                (byte_to_half_bits<KV>(byte_at(vw[2 * m2 + 1], sl)) << 16);
      }
    }
    const f16x8 vop = fix_int8<KV>(bits_to_f16x8(h[0], h[1], h[2], h[3]));
    st.acc[sl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, st.acc[sl], 0, 0, 0);
  }
}

// The hardware deals workgroups round-robin to the 8 XCDs (physical index
// p goes to XCD p % 8). Remap so that XCD x runs one contiguous range of
// logical indices: all kv heads and splits of a few sequences then share one
// XCD's L2 and TLBs, and the 8 head rows of each page (adjacent in the NHD
// layout) are fetched by the same XCD. The tail beyond a multiple of 8 keeps
// its index.
__device__ __forceinline__ int xcd_logical(int p, int n) {
#if PA_XCD_SWIZZLE
  constexpr int kXcds = 8;
  const int full = n - n % kXcds;
  if (p >= full) return p;
  const int per = full / kXcds;
  return (p % kXcds) * per + p / kXcds;
#else
  (void)n;
  return p;
#endif
}

template <int KV, int SC, int D, bool SPLIT>
__global__ void __launch_bounds__(kWaves * 64)
paged_decode_kernel(const KParams p) {
  using G = Geo<KV, D>;
  constexpr int kRegs = 4 * G::kE;  // accumulator floats per lane

  __shared__ float sm_m[kWaves][16];
  __shared__ float sm_l[kWaves][16];
  __shared__ float sm_acc[kWaves - 1][kRegs][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15;
  const int c = lane >> 4;

  // logical index = ((b * hkv + kvh) * head_tiles + ht) * num_splits + split
  int x = xcd_logical(blockIdx.x, gridDim.x);
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
  if (SPLIT) {
    const int ntile_all = (seq_len + kTile - 1) / kTile;
    const int chunk = ((ntile_all + p.num_splits - 1) / p.num_splits) * kTile;
    lo = split * chunk;
    hi = min(lo + chunk, seq_len);
  }

  WaveState<KV, SC, D> st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int sl = 0; sl < G::kE; ++sl) st.acc[sl] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const bool hv = r16 < nh;
    const _Float16 *qrow = reinterpret_cast<const _Float16 *>(p.q) + (int64_t)b * p.sqb +
                           (int64_t)(qh0 + (hv ? r16 : 0)) * p.sqh;
#pragma unroll
    for (int ks = 0; ks < G::kKSteps; ++ks) {
      f16x8 qv = {0, 0, 0, 0, 0, 0, 0, 0};
      if (hv) qv = *reinterpret_cast<const f16x8 *>(qrow + q_dim_offset<KV, D>(ks, c));
      st.qop[ks] = qv;
    }
  }

  const int32_t *bt_row = p.bt + (int64_t)b * p.sbtb;
  const int ntiles = (hi > lo) ? (hi - lo + kTile - 1) / kTile : 0;
  for (int t = wave; t < ntiles; t += kWaves) {
    const int n0 = lo + t * kTile;
    if (n0 + kTile <= hi) {
      tile_step<KV, SC, D, false>(st, p, bt_row, kvh, n0, hi, lane);
    } else {
      tile_step<KV, SC, D, true>(st, p, bt_row, kvh, n0, hi, lane);
    }
  }

  // ---- merge the waves through LDS ----
  const float lw = wave_sum16(st.l);
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

  // Lane (c, h) holds O[h][4*kE*c + kE*i + sl] in o[4*sl + i]; regroup so that
  // y[kE*i + sl] is head-dim offset 4*kE*c + kE*i + sl (contiguous).
  float y[kRegs];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int sl = 0; sl < G::kE; ++sl) y[G::kE * i + sl] = o[4 * sl + i] * inv;

  if (r16 >= nh) return;
  const int h = qh0 + r16;
  const int d0 = 4 * G::kE * c;
  if (SPLIT) {
    float *dst = p.part_out + (int64_t)b * p.spb + (int64_t)h * p.sph + (int64_t)split * p.sps + d0;
#pragma unroll
    for (int v4 = 0; v4 < kRegs / 4; ++v4) {
      f32x4 t4 = {y[4 * v4], y[4 * v4 + 1], y[4 * v4 + 2], y[4 * v4 + 3]};
      *reinterpret_cast<f32x4 *>(dst + 4 * v4) = t4;
    }
    if (c == 0) {
      p.part_lse[(int64_t)b * p.slb + (int64_t)h * p.slh + split] =
          (L > 0.f) ? M + __log2f(L) : -INFINITY;
    }
  } else {
    _Float16 *dst = reinterpret_cast<_Float16 *>(p.out) + (int64_t)b * p.sob + (int64_t)h * p.soh + d0;
    if constexpr (kRegs >= 8) {
#pragma unroll
      for (int v8 = 0; v8 < kRegs / 8; ++v8) {
        f16x8 t8;
#pragma unroll
        for (int e = 0; e < 8; ++e) t8[e] = (_Float16)y[8 * v8 + e];
        *reinterpret_cast<f16x8 *>(dst + 8 * v8) = t8;
      }
    } else {
#pragma unroll
      for (int e = 0; e < kRegs; ++e) dst[e] = (_Float16)y[e];
    }
  }
}

// Merge of split partials, one wave per (b, h); lanes cover the head dim.
// Fixed summation order, so repeated calls are bit-identical.
template <int D>
__global__ void __launch_bounds__(64) split_reduce_kernel(const RParams p) {
  constexpr int kPer = D / 64 > 0 ? D / 64 : 1;  // head-dim elements per lane
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / p.num_heads;
  const int h = bh % p.num_heads;
  const float *lse = p.part_lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  const float *part = p.part_out + (int64_t)b * p.spb + (int64_t)h * p.sph;

  float m = -INFINITY;
  for (int s = lane; s < p.num_splits; s += 64) m = fmaxf(m, lse[s]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));

  float wsum = 0.f;
  for (int s = lane; s < p.num_splits; s += 64) {
    const float ls = lse[s];
    wsum += (ls == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ls - m);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wsum += __shfl_xor(wsum, o);

  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) acc[i] = 0.f;
  const bool active = lane * kPer < D;
  if (m != -INFINITY) {
    for (int s = 0; s < p.num_splits; ++s) {
      const float ls = lse[s];
      if (ls == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ls - m);
      if (active) {
        const float *src = part + (int64_t)s * p.sps + lane * kPer;
#pragma unroll
        for (int i = 0; i < kPer; ++i) acc[i] += w * src[i];
      }
    }
  }
  const float inv = (wsum > 0.f) ? 1.0f / wsum : 0.f;
  if (active) {
    _Float16 *dst = reinterpret_cast<_Float16 *>(p.out) + (int64_t)b * p.sob + (int64_t)h * p.soh + lane * kPer;
#pragma unroll
    for (int i = 0; i < kPer; ++i) dst[i] = (_Float16)(acc[i] * inv);
  }
}

// ----------------------------------------------------------------------------
// host side: validation, error reporting, dispatch
// ----------------------------------------------------------------------------

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return PA_OK;
}

bool aligned(const void *ptr, int a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

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
  if (a->io_dtype != PA_IO_FP16) return fail(PA_ERR_UNSUPPORTED, "io_dtype %d unsupported", a->io_dtype);
  if (a->kv_dtype != PA_KV_FP16 && a->kv_dtype != PA_KV_FP8_E5M2 && a->kv_dtype != PA_KV_INT8)
    return fail(PA_ERR_INVALID, "kv_dtype %d unknown", a->kv_dtype);
  if (a->kv_dtype == PA_KV_INT8) {
    if (a->scale_dtype != PA_SCALE_FP16 && a->scale_dtype != PA_SCALE_FP32)
      return fail(PA_ERR_INVALID, "int8 KV needs scale_dtype fp16 or fp32, got %d", a->scale_dtype);
    if (!a->k_scale || !a->v_scale) return fail(PA_ERR_INVALID, "int8 KV needs k_scale and v_scale");
    if (a->stride_sn < 0 || a->stride_st < 0)
      return fail(PA_ERR_INVALID, "scale strides must be non-negative");
    const int sb = a->scale_dtype == PA_SCALE_FP32 ? 4 : 2;
    if (!aligned(a->k_scale, sb) || !aligned(a->v_scale, sb))
      return fail(PA_ERR_INVALID, "scale pointers must be %d-byte aligned", sb);
  } else if (a->scale_dtype != PA_SCALE_NONE) {
    return fail(PA_ERR_INVALID, "scale_dtype must be PA_SCALE_NONE for kv_dtype %d", a->kv_dtype);
  }
  if (need_partials && (!a->part_out || !a->part_lse))
    return fail(PA_ERR_INVALID, "num_splits > 1 needs part_out and part_lse");

  const int elem = (a->kv_dtype == PA_KV_FP16) ? 2 : 1;
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
  if ((int64_t)a->block_size * a->stride_kt * elem >= (int64_t(1) << 31))
    return fail(PA_ERR_UNSUPPORTED, "page of %d tokens spans more than 2 GiB", a->block_size);
  if (need_partials) {
    if (a->stride_pb < 0 || a->stride_ph < 0 || a->stride_ps < 0 || a->stride_lb < 0 ||
        a->stride_lh < 0)
      return fail(PA_ERR_INVALID, "workspace strides must be non-negative");
    if (!aligned(a->part_out, 16) || (a->stride_pb * 4) % 16 || (a->stride_ph * 4) % 16 ||
        (a->stride_ps * 4) % 16)
      return fail(PA_ERR_INVALID, "part_out and its strides must be 16-byte aligned");
  }

  const int group = a->num_q_heads / a->num_kv_heads;
  const int head_tiles = (group + PA_MAX_GROUP - 1) / PA_MAX_GROUP;
  const int64_t grid = (int64_t)a->batch * a->num_kv_heads * head_tiles * a->num_splits;
  if (grid > 0x7fffffff) return fail(PA_ERR_UNSUPPORTED, "grid of %lld workgroups too large", (long long)grid);

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
  return PA_OK;
}

template <int KV, int SC, int D>
hipError_t launch_decode_t(const KParams &k, int grid, bool split, hipStream_t st) {
  if (split) {
    hipLaunchKernelGGL((paged_decode_kernel<KV, SC, D, true>), dim3(grid), dim3(kWaves * 64), 0, st, k);
  } else {
    hipLaunchKernelGGL((paged_decode_kernel<KV, SC, D, false>), dim3(grid), dim3(kWaves * 64), 0, st, k);
  }
  return hipGetLastError();
}

template <int KV, int SC>
hipError_t launch_decode_d(const KParams &k, int d, int grid, bool split, hipStream_t st) {
  switch (d) {
    case 32: return launch_decode_t<KV, SC, 32>(k, grid, split, st);
    case 64: return launch_decode_t<KV, SC, 64>(k, grid, split, st);
    case 128: return launch_decode_t<KV, SC, 128>(k, grid, split, st);
    default: return launch_decode_t<KV, SC, 256>(k, grid, split, st);
  }
}

hipError_t launch_decode(const KParams &k, const pa_decode_args *a, bool split, hipStream_t st) {
  const int grid = a->batch * a->num_kv_heads * k.head_tiles * a->num_splits;
  const int d = a->head_dim;
  if (a->kv_dtype == PA_KV_FP16) return launch_decode_d<PA_KV_FP16, PA_SCALE_NONE>(k, d, grid, split, st);
  if (a->kv_dtype == PA_KV_FP8_E5M2)
    return launch_decode_d<PA_KV_FP8_E5M2, PA_SCALE_NONE>(k, d, grid, split, st);
  if (a->scale_dtype == PA_SCALE_FP32) return launch_decode_d<PA_KV_INT8, PA_SCALE_FP32>(k, d, grid, split, st);
  return launch_decode_d<PA_KV_INT8, PA_SCALE_FP16>(k, d, grid, split, st);
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
  if (r->io_dtype != PA_IO_FP16) return fail(PA_ERR_UNSUPPORTED, "io_dtype %d unsupported", r->io_dtype);
  if (r->stride_pb < 0 || r->stride_ph < 0 || r->stride_ps < 0 || r->stride_lb < 0 ||
      r->stride_lh < 0 || r->stride_ob < 0 || r->stride_oh < 0)
    return fail(PA_ERR_INVALID, "strides must be non-negative");
  if ((int64_t)r->batch * r->num_heads > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "grid too large");
  rp->part_out = r->part_out;
  rp->part_lse = r->part_lse;
  rp->out = static_cast<uint8_t *>(r->out);
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

hipError_t launch_reduce(const RParams &rp, int batch, int d, hipStream_t st) {
  const int grid = batch * rp.num_heads;
  switch (d) {
    case 32: hipLaunchKernelGGL(split_reduce_kernel<32>, dim3(grid), dim3(64), 0, st, rp); break;
    case 64: hipLaunchKernelGGL(split_reduce_kernel<64>, dim3(grid), dim3(64), 0, st, rp); break;
    case 128: hipLaunchKernelGGL(split_reduce_kernel<128>, dim3(grid), dim3(64), 0, st, rp); break;
    default: hipLaunchKernelGGL(split_reduce_kernel<256>, dim3(grid), dim3(64), 0, st, rp); break;
  }
  return hipGetLastError();
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

extern "C" {

int pa_abi_version(void) { return PA_ABI_VERSION; }

const char *pa_last_error(void) { return g_err; }

int pa_decode(const pa_decode_args *a, void *stream) {
  KParams k;
  const bool split = a != nullptr && a->num_splits > 1;
  int rc = build_params(a, split, &k);
  if (rc != PA_OK) return rc;
  RParams rp;
  pa_reduce_args ra;
  if (split) {
    ra = reduce_args_from(a);
    rc = check_reduce(&ra, &rp);
    if (rc != PA_OK) return rc;
  }
  if (a->batch == 0) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = launch_decode(k, a, split, st);
  if (e != hipSuccess) return fail(PA_ERR_HIP, "decode launch failed: %s", hipGetErrorString(e));
  if (split) {
    e = launch_reduce(rp, a->batch, a->head_dim, st);
    if (e != hipSuccess) return fail(PA_ERR_HIP, "reduce launch failed: %s", hipGetErrorString(e));
  }
  return ok();
}

int pa_decode_partials(const pa_decode_args *a, void *stream) {
  KParams k;
  int rc = build_params(a, true, &k);
  if (rc != PA_OK) return rc;
  if (a->batch == 0) return ok();
  hipError_t e = launch_decode(k, a, true, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PA_ERR_HIP, "decode launch failed: %s", hipGetErrorString(e));
  return ok();
}

int pa_split_reduce(const pa_reduce_args *r, void *stream) {
  RParams rp;
  int rc = check_reduce(r, &rp);
  if (rc != PA_OK) return rc;
  if (r->batch == 0) return ok();
  hipError_t e = launch_reduce(rp, r->batch, r->head_dim, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PA_ERR_HIP, "reduce launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
