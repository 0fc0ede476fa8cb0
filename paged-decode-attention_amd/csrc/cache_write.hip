// Paged KV-cache write for MI355X (gfx950): this decode step's K and V rows
// scattered into the NHD pages at slot_mapping, quantised to the cache dtype.
//
// Replaces the KV write that precedes the decode in the reference's vLLM
// path (`reshape_and_cache_flash`, integration/vllm_backend.py:117-122) for
// caches in this library's formats, with the quantisation semantics of
// pagedattn/cache.py:33-48:
//   fp16      copy (bf16 rows into a bf16 cache: copy too)
//   fp8_e5m2  round-to-nearest-even of the fp16 bit pattern to its high byte
//             (e5m2 shares fp16's exponent); overflow rounds to inf and NaN
//             stays NaN, as torch's cast does
//   int8      amax over head_dim (clamped to 1e-6), scale = amax / 127 rounded
//             to the scale type, q = round_half_even(x / scale) clamped to
//             +-127; fp32 IEEE division throughout, so the bytes equal
//             torch's
//
// One (token, kv_head) row per D/8 lanes, 16 bytes (8 fp16) per lane; the
// int8 row maximum is a xor-shuffle reduction inside those lanes.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_errors.h"
#include "pagedattn.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct WParams {
  const uint8_t *key;
  const uint8_t *value;
  uint8_t *kc;
  uint8_t *vc;
  uint8_t *ks;
  uint8_t *vs;
  const int64_t *slots;
  int64_t rows;            // num_tokens * num_kv_heads
  int32_t hkv, block_size;
  int64_t max_slot;        // num_blocks * block_size
  int64_t skt, skh, svt, svh;  // bytes
  int64_t scn, sct, sch;       // bytes
  int64_t ssn, sst;            // bytes
};

// fp16 bit pattern -> e5m2 byte, round to nearest even on the dropped byte.
__device__ __forceinline__ uint32_t half_to_e5m2(uint32_t h) {
  const uint32_t sign = (h >> 8) & 0x80u;
  const uint32_t mag = h & 0x7fffu;
  if (mag > 0x7c00u) return sign | 0x7fu;  // NaN
  return sign | ((mag + 0x7fu + ((mag >> 8) & 1u)) >> 8);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int KV, int SC, int D>
__global__ void __launch_bounds__(256) cache_write_kernel(const WParams p) {
  constexpr int kLanesPerRow = D / 8;  // 8 fp16 (16 bytes) per lane
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / kLanesPerRow;
  const int piece = (int)(gid % kLanesPerRow);
  bool live = row < p.rows;
  const int64_t t = live ? row / p.hkv : 0;
  const int h = live ? (int)(row % p.hkv) : 0;
  const int64_t slot = live ? p.slots[t] : -1;
  live = live && slot >= 0 && slot < p.max_slot;  // uniform across the row's lanes
  const int64_t blk = live ? slot / p.block_size : 0;
  const int64_t off = live ? slot % p.block_size : 0;
  const int64_t cbase = blk * p.scn + off * p.sct + h * p.sch;

#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const uint8_t *src = (which ? p.value : p.key) + t * (which ? p.svt : p.skt) +
                         h * (which ? p.svh : p.skh) + piece * 16;
    uint8_t *dst = which ? p.vc : p.kc;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (live) w = *reinterpret_cast<const u32x4 *>(src);
    uint32_t hv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hv[2 * i] = w[i] & 0xffffu;
      hv[2 * i + 1] = w[i] >> 16;
    }
    if constexpr (KV == PA_KV_FP16 || KV == PA_KV_BF16) {
      if (live) *reinterpret_cast<u32x4 *>(dst + cbase + piece * 16) = w;
    } else if constexpr (KV == PA_KV_FP8_E5M2) {
      uint32_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = half_to_e5m2(hv[i]);
      const u32x2 o = {b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24),
                       b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)};
      if (live) *reinterpret_cast<u32x2 *>(dst + cbase + piece * 8) = o;
    } else {
      float x[8];
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[i] = half_bits_to_float(hv[i]);
        amax = fmaxf(amax, fabsf(x[i]));
      }
#pragma unroll
      for (int o = kLanesPerRow / 2; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
      amax = fmaxf(amax, 1e-6f);
      // IEEE division (the default for float `/` in HIP device code)
      float scale = amax / 127.0f;
      if constexpr (SC == PA_SCALE_FP16) scale = (float)(_Float16)scale;
      // round_half_even(x / scale) with the IEEE quotient's rounding: x times
      // the row's reciprocal is within 1.5 ulp of the correctly rounded
      // quotient, so the two can round to different integers only next to a
      // half-integer; those (rare) elements take the IEEE division
      const float inv = 1.0f / scale;
      uint32_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float q0 = x[i] * inv;
        const float frac = q0 - floorf(q0);
        const float tol = fabsf(q0) * 0x1p-20f + 0x1p-40f;
        float r = rintf(q0);
        if (fabsf(frac - 0.5f) <= tol) r = rintf(x[i] / scale);
        // a zero row with fp16 scales underflows the scale to 0: 0/0 is NaN,
        // which the reference's cast to int8 stores as 0
        const float q = (r != r) ? 0.f : fminf(fmaxf(r, -127.f), 127.f);
        b[i] = (uint32_t)(int32_t)q & 0xffu;
      }
      const u32x2 o = {b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24),
                       b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)};
      if (live) {
        *reinterpret_cast<u32x2 *>(dst + cbase + piece * 8) = o;
        if (piece == 0) {
          uint8_t *s = (which ? p.vs : p.ks) + blk * p.ssn + off * p.sst;
          if constexpr (SC == PA_SCALE_FP16) {
            reinterpret_cast<_Float16 *>(s)[h] = (_Float16)scale;
          } else {
            reinterpret_cast<float *>(s)[h] = scale;
          }
        }
      }
    }
  }
}

template <int KV, int SC>
hipError_t launch_w(const WParams &p, int d, int grid, hipStream_t st) {
  switch (d) {
    case 32: hipLaunchKernelGGL((cache_write_kernel<KV, SC, 32>), dim3(grid), dim3(256), 0, st, p); break;
    case 64: hipLaunchKernelGGL((cache_write_kernel<KV, SC, 64>), dim3(grid), dim3(256), 0, st, p); break;
    case 128: hipLaunchKernelGGL((cache_write_kernel<KV, SC, 128>), dim3(grid), dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((cache_write_kernel<KV, SC, 256>), dim3(grid), dim3(256), 0, st, p); break;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" int pa_cache_write(const pa_cache_write_args *a, void *stream) {
  if (a == nullptr) return pa_fail(PA_ERR_INVALID, "args is NULL");
  if (a->num_tokens < 0) return pa_fail(PA_ERR_INVALID, "num_tokens %d < 0", a->num_tokens);
  if (!a->key || !a->value || !a->k_cache || !a->v_cache || !a->slot_mapping)
    return pa_fail(PA_ERR_INVALID, "key, value, k_cache, v_cache and slot_mapping must be non-NULL");
  if (a->num_kv_heads <= 0 || a->block_size <= 0 || a->num_blocks <= 0)
    return pa_fail(PA_ERR_INVALID, "num_kv_heads %d, block_size %d and num_blocks %d must be positive",
                   a->num_kv_heads, a->block_size, a->num_blocks);
  if (a->head_dim != 32 && a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
    return pa_fail(PA_ERR_UNSUPPORTED, "head_dim %d not in (32, 64, 128, 256)", a->head_dim);
  if (a->kv_dtype != PA_KV_FP16 && a->kv_dtype != PA_KV_FP8_E5M2 && a->kv_dtype != PA_KV_INT8 &&
      a->kv_dtype != PA_KV_BF16)
    return pa_fail(PA_ERR_INVALID, "kv_dtype %d unknown", a->kv_dtype);
  const int64_t strides[] = {a->stride_kt, a->stride_kh, a->stride_vt, a->stride_vh,
                             a->stride_cn, a->stride_ct, a->stride_ch};
  for (int64_t s : strides)
    if (s < 0) return pa_fail(PA_ERR_INVALID, "strides must be non-negative");
  const int elem = (a->kv_dtype == PA_KV_FP16 || a->kv_dtype == PA_KV_BF16) ? 2 : 1;
  const int piece = 8 * elem;  // bytes a lane stores
  if (!pa_aligned(a->key, 16) || !pa_aligned(a->value, 16) || (a->stride_kt * 2) % 16 ||
      (a->stride_kh * 2) % 16 || (a->stride_vt * 2) % 16 || (a->stride_vh * 2) % 16)
    return pa_fail(PA_ERR_INVALID, "key/value and their strides must be 16-byte aligned");
  if (!pa_aligned(a->k_cache, piece) || !pa_aligned(a->v_cache, piece) ||
      (a->stride_cn * elem) % piece || (a->stride_ct * elem) % piece || (a->stride_ch * elem) % piece)
    return pa_fail(PA_ERR_INVALID, "k_cache/v_cache and their strides must be %d-byte aligned", piece);
  int sb = 0;
  if (a->kv_dtype == PA_KV_INT8) {
    if (a->scale_dtype != PA_SCALE_FP16 && a->scale_dtype != PA_SCALE_FP32)
      return pa_fail(PA_ERR_INVALID, "int8 KV needs scale_dtype fp16 or fp32, got %d", a->scale_dtype);
    if (!a->k_scale || !a->v_scale) return pa_fail(PA_ERR_INVALID, "int8 KV needs k_scale and v_scale");
    if (a->stride_sn < 0 || a->stride_st < 0) return pa_fail(PA_ERR_INVALID, "scale strides must be non-negative");
    sb = a->scale_dtype == PA_SCALE_FP32 ? 4 : 2;
    if (!pa_aligned(a->k_scale, sb) || !pa_aligned(a->v_scale, sb))
      return pa_fail(PA_ERR_INVALID, "scale pointers must be %d-byte aligned", sb);
  } else if (a->scale_dtype != PA_SCALE_NONE) {
    return pa_fail(PA_ERR_INVALID, "scale_dtype must be PA_SCALE_NONE for kv_dtype %d", a->kv_dtype);
  }
  const int64_t rows = (int64_t)a->num_tokens * a->num_kv_heads;
  const int64_t lanes = rows * (a->head_dim / 8);
  const int64_t grid = (lanes + 255) / 256;
  if (grid > 0x7fffffff) return pa_fail(PA_ERR_UNSUPPORTED, "too many rows (%lld)", (long long)rows);
  if (rows == 0) return pa_ok();

  WParams p;
  p.key = static_cast<const uint8_t *>(a->key);
  p.value = static_cast<const uint8_t *>(a->value);
  p.kc = static_cast<uint8_t *>(a->k_cache);
  p.vc = static_cast<uint8_t *>(a->v_cache);
  p.ks = static_cast<uint8_t *>(a->k_scale);
  p.vs = static_cast<uint8_t *>(a->v_scale);
  p.slots = a->slot_mapping;
  p.rows = rows;
  p.hkv = a->num_kv_heads;
  p.block_size = a->block_size;
  p.max_slot = (int64_t)a->num_blocks * a->block_size;
  p.skt = a->stride_kt * 2;
  p.skh = a->stride_kh * 2;
  p.svt = a->stride_vt * 2;
  p.svh = a->stride_vh * 2;
  p.scn = a->stride_cn * elem;
  p.sct = a->stride_ct * elem;
  p.sch = a->stride_ch * elem;
  p.ssn = a->stride_sn * sb;
  p.sst = a->stride_st * sb;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int d = a->head_dim;
  hipError_t e;
  if (a->kv_dtype == PA_KV_FP16) e = launch_w<PA_KV_FP16, PA_SCALE_NONE>(p, d, (int)grid, st);
  else if (a->kv_dtype == PA_KV_BF16) e = launch_w<PA_KV_BF16, PA_SCALE_NONE>(p, d, (int)grid, st);
  else if (a->kv_dtype == PA_KV_FP8_E5M2) e = launch_w<PA_KV_FP8_E5M2, PA_SCALE_NONE>(p, d, (int)grid, st);
  else if (a->scale_dtype == PA_SCALE_FP32) e = launch_w<PA_KV_INT8, PA_SCALE_FP32>(p, d, (int)grid, st);
  else e = launch_w<PA_KV_INT8, PA_SCALE_FP16>(p, d, (int)grid, st);
  if (e != hipSuccess) return pa_fail(PA_ERR_HIP, "cache write launch failed: %s", hipGetErrorString(e));
  return pa_ok();
}
