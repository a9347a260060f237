// HBM-streaming kernels of the decode hot path: KV store by slot mapping,
// RMSNorm, fused residual-add + RMSNorm, NeoX RoPE, Qwen3 q/k-norm + RoPE,
// SiLU-and-mul.  All move bf16 in 16-byte vectors (global_load_dwordx4),
// accumulate in fp32 and reduce across lanes with DPP, so each element is
// read once from HBM and written once.
#include "xv_common.h"
#include "xv_kernels.h"

// --------------------------------------------------------------------------
// KV store: one thread moves one 16-byte chunk of K and the matching chunk of V.
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void store_kvcache_kernel(
    const bf16_t* __restrict__ key, int64_t ks_tok, int64_t ks_head,
    const bf16_t* __restrict__ value, int64_t vs_tok, int64_t vs_head,
    bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache,
    int64_t cs_page, int64_t cs_tok, int64_t cs_head, int block_size, const int32_t* __restrict__ slots,
    int total_chunks, int chunks_per_tok, int chunks_per_head) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total_chunks) return;
  const int tok = idx / chunks_per_tok;
  const int c = idx - tok * chunks_per_tok;
  const int32_t slot = slots[tok];
  if (slot < 0) return;  // padding token (slot -1) writes nothing
  const int h = c / chunks_per_head;
  const int d = (c - h * chunks_per_head) * 8;
  const Vec8 kv = load_vec8_nt(key + tok * ks_tok + h * ks_head + d);
  const Vec8 vv = load_vec8_nt(value + tok * vs_tok + h * vs_head + d);
  const int page = slot / block_size;
  const int t = slot - page * block_size;
  const int64_t dst = (int64_t)page * cs_page + (int64_t)t * cs_tok + h * cs_head + d;
  store_vec8_nt(k_cache + dst, kv);
  store_vec8_nt(v_cache + dst, vv);
}

// Tokens whose Hkv*D/8 chunks are a multiple of 64: a unit is 64 chunks of
// one token (its slot and page address are wave uniform), and each wave moves
// U consecutive units.  The 2U 16-byte K/V loads do not depend on the slots,
// so they are issued first and the U slot loads (scalar) travel beside them:
// a wave waits one memory round trip before its stores, not two.
template <int U>
__global__ __launch_bounds__(256) void store_kvcache_wave_kernel(
    const bf16_t* __restrict__ key, int64_t ks_tok, int64_t ks_head,
    const bf16_t* __restrict__ value, int64_t vs_tok, int64_t vs_head,
    bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache,
    int64_t cs_page, int64_t cs_tok, int64_t cs_head, int block_size, const int32_t* __restrict__ slots,
    int num_units, int units_per_tok, int chunks_per_head) {
  const int u0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * U);
  if (u0 >= num_units) return;
  const int lane = threadIdx.x & 63;
  int tok[U];
  int64_t hd[U];
  Vec8 kv[U], vv[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const int u = min(u0 + j, num_units - 1);
    tok[j] = u / units_per_tok;
    const int c = (u - tok[j] * units_per_tok) * 64 + lane;
    const int h = c / chunks_per_head;
    const int d = (c - h * chunks_per_head) * 8;
    hd[j] = h * cs_head + d;
    kv[j] = load_vec8_nt(key + tok[j] * ks_tok + h * ks_head + d);
    vv[j] = load_vec8_nt(value + tok[j] * vs_tok + h * vs_head + d);
  }
  int slot[U];
#pragma unroll
  for (int j = 0; j < U; ++j) slot[j] = __builtin_amdgcn_readfirstlane(slots[tok[j]]);
  // pin the data loads here: the compiler would otherwise sink them into the
  // slot-dependent branches below, behind the slot round trip
#pragma unroll
  for (int j = 0; j < U; ++j) { pin_vec8(kv[j]); pin_vec8(vv[j]); }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    if (u0 + j >= num_units || slot[j] < 0) continue;  // padding token (slot -1) writes nothing
    const int page = slot[j] / block_size;
    const int t = slot[j] - page * block_size;
    const int64_t dst = (int64_t)page * cs_page + (int64_t)t * cs_tok + hd[j];
    store_vec8_nt(k_cache + dst, kv[j]);
    store_vec8_nt(v_cache + dst, vv[j]);
  }
}

extern "C" int xv_store_kvcache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                                const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                                void* k_cache, void* v_cache,
                                int64_t cache_page_stride, int64_t cache_tok_stride, int64_t cache_head_stride,
                                int block_size, const int32_t* slot_mapping, int64_t num_tokens,
                                int num_kv_heads, int head_dim, hipStream_t stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 || block_size <= 0)
    return (int)hipErrorInvalidValue;
  if (!xv_al16(key) || !xv_al16(value) || !xv_al16(k_cache) || !xv_al16(v_cache) ||
      !xv_st8(key_stride_tok) || !xv_st8(key_stride_head) || !xv_st8(value_stride_tok) ||
      !xv_st8(value_stride_head) || !xv_st8(cache_page_stride) || !xv_st8(cache_tok_stride) ||
      !xv_st8(cache_head_stride))
    return (int)hipErrorInvalidValue;  // 16-byte chunks
  if (num_tokens == 0) return 0;
  const int cph = head_dim / 8;
  const int cpt = cph * num_kv_heads;
  if (num_tokens * cpt >= ((int64_t)1 << 31)) return (int)hipErrorInvalidValue;  // 32-bit chunk indices
  if (cpt % 64 == 0) {
    const int upt = cpt / 64;
    const int units = (int)num_tokens * upt;
    // two units per wave once the grid holds more waves than the chip
    // (config 3, 16384 units: 13.8 us against 14.0 with one and 14.1 with four)
    constexpr int kU = 2;
    if (units >= 4096) {
      const int waves = (units + kU - 1) / kU;
      store_kvcache_wave_kernel<kU><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream>>>(
          (const bf16_t*)key, key_stride_tok, key_stride_head, (const bf16_t*)value, value_stride_tok,
          value_stride_head, (bf16_t*)k_cache, (bf16_t*)v_cache, cache_page_stride, cache_tok_stride,
          cache_head_stride, block_size, slot_mapping, units, upt, cph);
    } else {
      store_kvcache_wave_kernel<1><<<dim3((unsigned)((units + 3) / 4)), dim3(256), 0, stream>>>(
          (const bf16_t*)key, key_stride_tok, key_stride_head, (const bf16_t*)value, value_stride_tok,
          value_stride_head, (bf16_t*)k_cache, (bf16_t*)v_cache, cache_page_stride, cache_tok_stride,
          cache_head_stride, block_size, slot_mapping, units, upt, cph);
    }
  } else {
    const int total = (int)(num_tokens * cpt);
    store_kvcache_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream>>>(
        (const bf16_t*)key, key_stride_tok, key_stride_head, (const bf16_t*)value, value_stride_tok,
        value_stride_head, (bf16_t*)k_cache, (bf16_t*)v_cache, cache_page_stride, cache_tok_stride,
        cache_head_stride, block_size, slot_mapping, total, cpt, cph);
  }
  XV_CHECK_LAUNCH();
  return 0;
}

// fp8 (e4m3fn) cache: each bf16 value x is stored as e4m3fn(x * inv_scale)
// (one fp32 multiply, then the hardware's round-to-nearest-even conversion,
// which gives torch's float8_e4m3fn cast of the product: values past the
// format's range become NaN, as there).  Same unit structure as the bf16
// wave kernel: a lane's 16-byte chunk of 8 values becomes 8 bytes.
template <int U>
__global__ __launch_bounds__(256) void store_kvcache_fp8_kernel(
    const bf16_t* __restrict__ key, int64_t ks_tok, int64_t ks_head,
    const bf16_t* __restrict__ value, int64_t vs_tok, int64_t vs_head,
    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    int64_t cs_page, int64_t cs_tok, int64_t cs_head, int block_size, const int32_t* __restrict__ slots,
    int num_units, int units_per_tok, int chunks_per_head, float k_inv, float v_inv) {
  const int u0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * U);
  if (u0 >= num_units) return;
  const int lane = threadIdx.x & 63;
  int tok[U];
  int64_t hd[U];
  Vec8 kv[U], vv[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const int u = min(u0 + j, num_units - 1);
    tok[j] = u / units_per_tok;
    const int c = (u - tok[j] * units_per_tok) * 64 + lane;
    const int h = c / chunks_per_head;
    const int d = (c - h * chunks_per_head) * 8;
    hd[j] = h * cs_head + d;
    kv[j] = load_vec8_nt(key + tok[j] * ks_tok + h * ks_head + d);
    vv[j] = load_vec8_nt(value + tok[j] * vs_tok + h * vs_head + d);
  }
  int slot[U];
#pragma unroll
  for (int j = 0; j < U; ++j) slot[j] = __builtin_amdgcn_readfirstlane(slots[tok[j]]);
#pragma unroll
  for (int j = 0; j < U; ++j) { pin_vec8(kv[j]); pin_vec8(vv[j]); }
  auto to_fp8 = [](const Vec8& x, float inv) {
    float f[8];
    unpack8(x, f);
    uint32_t lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0] * inv, f[1] * inv, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2] * inv, f[3] * inv, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4] * inv, f[5] * inv, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6] * inv, f[7] * inv, hi, true);
    return make_uint2(lo, hi);
  };
#pragma unroll
  for (int j = 0; j < U; ++j) {
    if (u0 + j >= num_units || slot[j] < 0) continue;  // padding token (slot -1) writes nothing
    const int page = slot[j] / block_size;
    const int t = slot[j] - page * block_size;
    const int64_t dst = (int64_t)page * cs_page + (int64_t)t * cs_tok + hd[j];
    *reinterpret_cast<uint2*>(k_cache + dst) = to_fp8(kv[j], k_inv);
    *reinterpret_cast<uint2*>(v_cache + dst) = to_fp8(vv[j], v_inv);
  }
}

extern "C" int xv_store_kvcache_fp8(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                                    const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                                    void* k_cache, void* v_cache,
                                    int64_t cache_page_stride, int64_t cache_tok_stride, int64_t cache_head_stride,
                                    int block_size, const int32_t* slot_mapping, int64_t num_tokens,
                                    int num_kv_heads, int head_dim, float k_scale, float v_scale,
                                    hipStream_t stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 || block_size <= 0)
    return (int)hipErrorInvalidValue;
  if (!(k_scale > 0.0f) || !(v_scale > 0.0f) || !__builtin_isfinite(k_scale) || !__builtin_isfinite(v_scale))
    return (int)hipErrorInvalidValue;
  // bf16 rows as 16-byte chunks; fp8 cache rows as 8-byte pieces
  if (!xv_al16(key) || !xv_al16(value) || ((uintptr_t)k_cache | (uintptr_t)v_cache) & 7 ||
      !xv_st8(key_stride_tok) || !xv_st8(key_stride_head) || !xv_st8(value_stride_tok) ||
      !xv_st8(value_stride_head) || (cache_page_stride | cache_tok_stride | cache_head_stride) & 7)
    return (int)hipErrorInvalidValue;
  if (num_tokens == 0) return 0;
  const int cph = head_dim / 8;
  const int cpt = cph * num_kv_heads;
  if (cpt % 64) return (int)hipErrorInvalidValue;  // whole 64-chunk units per token (Hkv * D a multiple of 512)
  if (num_tokens * cpt >= ((int64_t)1 << 31)) return (int)hipErrorInvalidValue;
  const int upt = cpt / 64;
  const int units = (int)num_tokens * upt;
  const float k_inv = 1.0f / k_scale, v_inv = 1.0f / v_scale;
  constexpr int kU = 2;
  const int waves = (units + kU - 1) / kU;
  store_kvcache_fp8_kernel<kU><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream>>>(
      (const bf16_t*)key, key_stride_tok, key_stride_head, (const bf16_t*)value, value_stride_tok, value_stride_head,
      (uint8_t*)k_cache, (uint8_t*)v_cache, cache_page_stride, cache_tok_stride, cache_head_stride, block_size,
      slot_mapping, units, upt, cph, k_inv, v_inv);
  XV_CHECK_LAUNCH();
  return 0;
}

// Chunked prefill over fp8 pages: every sequence's keys (cached prefix and
// this chunk, already stored) dequantized into bf16 rows at cu_seqlens_k[b]
// + t, the varlen k/v layout xv_prefill_attention reads: bf16(value * scale).
// One thread per 8-value piece of one (token, kv head).
__global__ __launch_bounds__(256) void gather_kv_fp8_kernel(
    const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc, int64_t ps, int64_t ts, int64_t hs,
    const int32_t* __restrict__ bt, int64_t bt_stride, int block_size, const int32_t* __restrict__ cu_k, int hkv,
    float k_scale, float v_scale, bf16_t* __restrict__ ko, bf16_t* __restrict__ vo, int64_t o_st) {
  const int b = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int per_tok = hkv * 16;  // 8-value pieces of a token (D = 128)
  const int t = (int)(idx / per_tok);
  const int k0 = cu_k[b];
  if (t >= cu_k[b + 1] - k0) return;
  const int rem = (int)(idx - (int64_t)t * per_tok), h = rem >> 4, c = rem & 15;
  const int64_t blk = bt[(int64_t)b * bt_stride + t / block_size];
  const int64_t src = blk * ps + (int64_t)(t % block_size) * ts + (int64_t)h * hs + c * 8;
  const uint2 kq = *reinterpret_cast<const uint2*>(kc + src);
  const uint2 vq = *reinterpret_cast<const uint2*>(vc + src);
  auto dq = [](uint2 w, float sc) {
    float f[8];
    const uint32_t ww[2] = {w.x, w.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(ww[j], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(ww[j], true);
      f[4 * j] = lo[0] * sc; f[4 * j + 1] = lo[1] * sc; f[4 * j + 2] = hi[0] * sc; f[4 * j + 3] = hi[1] * sc;
    }
    return pack8(f);
  };
  const int64_t dst = (int64_t)(k0 + t) * o_st + h * 128 + c * 8;
  store_vec8(ko + dst, dq(kq, k_scale));
  store_vec8(vo + dst, dq(vq, v_scale));
}

extern "C" int xv_gather_kv_fp8(const void* k_cache, const void* v_cache, int64_t cache_page_stride,
                                int64_t cache_tok_stride, int64_t cache_head_stride, const int32_t* block_tables,
                                int64_t bt_stride, int block_size, const int32_t* cu_seqlens_k, int batch,
                                int max_seqlen_k, int num_kv_heads, int head_dim, float k_scale, float v_scale,
                                void* k_out, void* v_out, int64_t out_stride_tok, hipStream_t stream) {
  if (head_dim != 128 || batch < 0 || max_seqlen_k < 0 || num_kv_heads <= 0 || block_size <= 0 ||
      batch > 65535 || !(k_scale > 0.0f) || !(v_scale > 0.0f))
    return (int)hipErrorInvalidValue;
  if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 7 || (cache_page_stride | cache_tok_stride | cache_head_stride) & 7 ||
      !xv_al16(k_out) || !xv_al16(v_out) || !xv_st8(out_stride_tok) || out_stride_tok < (int64_t)num_kv_heads * 128)
    return (int)hipErrorInvalidValue;
  if (batch == 0 || max_seqlen_k == 0) return 0;
  const int64_t pieces = (int64_t)max_seqlen_k * num_kv_heads * 16;
  if ((pieces + 255) / 256 > 0x7fffffff) return (int)hipErrorInvalidValue;
  gather_kv_fp8_kernel<<<dim3((unsigned)((pieces + 255) / 256), (unsigned)batch), 256, 0, stream>>>(
      (const uint8_t*)k_cache, (const uint8_t*)v_cache, cache_page_stride, cache_tok_stride, cache_head_stride,
      block_tables, bt_stride, block_size, cu_seqlens_k, num_kv_heads, k_scale, v_scale, (bf16_t*)k_out,
      (bf16_t*)v_out, out_stride_tok);
  XV_CHECK_LAUNCH();
  return 0;
}

// --------------------------------------------------------------------------
// RMSNorm family.  TPR lanes own one row (16 = a DPP row, 64 = a wave); each
// lane keeps up to VPT 8-element vectors of the row in registers.
// --------------------------------------------------------------------------
// Threads per workgroup for TPR lanes per row.
template <int TPR> constexpr int kNormBlock = TPR > 256 ? TPR : 256;

// Sum over the TPR lanes owning a row (TPR >= 128: its waves, through LDS).
template <int TPR>
XV_INLINE float row_sum(float x) {
  if constexpr (TPR == 16) {
    return row16_sum(x);
  } else if constexpr (TPR == 64) {
    return wave_sum(x);
  } else {
    constexpr int W = TPR / 64;  // waves per row
    __shared__ float part[kNormBlock<TPR> / 64];
    x = wave_sum(x);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wave] = x;
    __syncthreads();
    const int w0 = wave / W * W;
    float r = part[w0];
#pragma unroll
    for (int i = 1; i < W; ++i) r += part[w0 + i];
    return r;
  }
}

template <int TPR, int VPT>
__global__ __launch_bounds__(kNormBlock<TPR>) void rmsnorm_kernel(
    const bf16_t* __restrict__ x, int64_t s_outer, int64_t s_inner, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ out, int64_t n_outer, int64_t n_inner, int hidden, float eps) {
  const int rows_per_block = kNormBlock<TPR> / TPR;
  int64_t row = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / TPR;
  int lane = threadIdx.x % TPR;
  int64_t rows = n_outer * n_inner;
  bool active = row < rows;
  int64_t o = active ? row / n_inner : 0;
  int64_t i = active ? row - o * n_inner : 0;
  const bf16_t* xr = x + o * s_outer + i * s_inner;
  int nvec = hidden >> 3;
  float v[VPT][8];
  Vec8 wv[VPT];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (active && vi < nvec) {
      unpack8(load_vec8_nt(xr + vi * 8), v[k]);
      wv[k] = load_vec8(w + vi * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[k][e] * v[k][e];
    }
  }
  ss = row_sum<TPR>(ss);
  if (!active) return;
  float rcp = rsqrtf(ss / (float)hidden + eps);
  bf16_t* orow = out + row * hidden;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (vi < nvec) {
      float wf[8], r[8];
      unpack8(wv[k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = (v[k][e] * rcp) * wf[e];
      store_vec8_nt(orow + vi * 8, pack8(r));
    }
  }
}

template <int TPR, int VPT>
__global__ __launch_bounds__(kNormBlock<TPR>) void fused_add_rmsnorm_kernel(
    bf16_t* __restrict__ x, int64_t xs, bf16_t* __restrict__ res, int64_t rs,
    const bf16_t* __restrict__ w, int64_t rows, int hidden, float eps) {
  const int rows_per_block = kNormBlock<TPR> / TPR;
  int64_t row = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / TPR;
  int lane = threadIdx.x % TPR;
  bool active = row < rows;
  bf16_t* xr = x + (active ? row : 0) * xs;
  bf16_t* rr = res + (active ? row : 0) * rs;
  int nvec = hidden >> 3;
  // all loads (x, residual, weight) issued up front: one memory round trip
  Vec8 xv[VPT], rv[VPT], wv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (active && vi < nvec) {
      xv[k] = load_vec8_nt(xr + vi * 8);
      rv[k] = load_vec8_nt(rr + vi * 8);
      wv[k] = load_vec8(w + vi * 8);
    }
  }
  float v[VPT][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (active && vi < nvec) {
      float a[8], b[8];
      unpack8(xv[k], a);
      unpack8(rv[k], b);
#pragma unroll
      for (int e = 0; e < 8; ++e) { v[k][e] = a[e] + b[e]; ss += v[k][e] * v[k][e]; }
      store_vec8_nt(rr + vi * 8, pack8(v[k]));
    }
  }
  ss = row_sum<TPR>(ss);
  if (!active) return;
  float rcp = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (vi < nvec) {
      float wf[8], r[8];
      unpack8(wv[k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = (v[k][e] * rcp) * wf[e];
      store_vec8_nt(xr + vi * 8, pack8(r));
    }
  }
}

#ifndef XV_NORM_LONG_TPR
#define XV_NORM_LONG_TPR 512  // lanes per row for rows of >= 256 vectors
#endif

template <template <int, int> class Launcher, typename... Args>
static int dispatch_norm(int64_t rows, int hidden, hipStream_t stream, Args... args) {
  if (hidden <= 0 || hidden % 8 || hidden > 16384) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  int nvec = hidden / 8;
  // long rows: a whole workgroup per row keeps each lane's memory chain short
  // and gives many small workgroups (several residency rounds, so loads of
  // one round overlap the reductions of another); short rows: a wave (or a
  // DPP row) per row
  if (nvec >= 256) {
    constexpr int T = XV_NORM_LONG_TPR;
    if (nvec <= T) return Launcher<T, 1>::run(rows, stream, args...);
    if (nvec <= 2 * T) return Launcher<T, 2>::run(rows, stream, args...);
    if (nvec <= 4 * T) return Launcher<T, 4>::run(rows, stream, args...);
    if (nvec <= 8 * T) return Launcher<T, 8>::run(rows, stream, args...);
    return Launcher<T, 16>::run(rows, stream, args...);
  }
  if (nvec <= 16) return Launcher<16, 1>::run(rows, stream, args...);
  if (nvec <= 32) return Launcher<16, 2>::run(rows, stream, args...);
  if (nvec <= 64) return Launcher<16, 4>::run(rows, stream, args...);
  if (nvec <= 128) return Launcher<64, 2>::run(rows, stream, args...);
  if (nvec <= 256) return Launcher<64, 4>::run(rows, stream, args...);
  if (nvec <= 512) return Launcher<64, 8>::run(rows, stream, args...);
  if (nvec <= 1024) return Launcher<64, 16>::run(rows, stream, args...);
  return Launcher<64, 32>::run(rows, stream, args...);
}

template <int TPR, int VPT>
struct RmsLaunch {
  static int run(int64_t rows, hipStream_t stream, const bf16_t* x, int64_t so, int64_t si,
                 const bf16_t* w, bf16_t* out, int64_t no, int64_t ni, int hidden, float eps) {
    constexpr int rpb = kNormBlock<TPR> / TPR;
    int64_t blocks = (rows + rpb - 1) / rpb;
    rmsnorm_kernel<TPR, VPT><<<dim3((unsigned)blocks), dim3(kNormBlock<TPR>), 0, stream>>>(x, so, si, w, out, no, ni,
                                                                                         hidden, eps);
    XV_CHECK_LAUNCH();
    return 0;
  }
};
template <int TPR, int VPT>
struct AddRmsLaunch {
  static int run(int64_t rows, hipStream_t stream, bf16_t* x, int64_t xs, bf16_t* r, int64_t rs,
                 const bf16_t* w, int hidden, float eps) {
    constexpr int rpb = kNormBlock<TPR> / TPR;
    int64_t blocks = (rows + rpb - 1) / rpb;
    fused_add_rmsnorm_kernel<TPR, VPT><<<dim3((unsigned)blocks), dim3(kNormBlock<TPR>), 0, stream>>>(
        x, xs, r, rs, w, rows, hidden, eps);
    XV_CHECK_LAUNCH();
    return 0;
  }
};

// Residual add + RMSNorm whose x arrives as np fp32 partial sums of a
// split-K GEMM (part p of row r at parts + p*part_stride + r*row_stride):
// x = bf16(sum of parts) -- the value the unsplit GEMM would have written --
// then exactly the fused_add_rmsnorm_kernel arithmetic, the result into out.
constexpr int kMaxParts = 8;
template <int TPR, int VPT>
__global__ __launch_bounds__(kNormBlock<TPR>) void fused_add_rmsnorm_parts_kernel(
    const float* __restrict__ parts, int64_t part_stride, int64_t row_stride, int np, bf16_t* __restrict__ out,
    int64_t os, bf16_t* __restrict__ res, int64_t rs, const bf16_t* __restrict__ w, int64_t rows, int hidden,
    float eps) {
  const int rows_per_block = kNormBlock<TPR> / TPR;
  int64_t row = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / TPR;
  int lane = threadIdx.x % TPR;
  bool active = row < rows;
  const float* pr = parts + (active ? row : 0) * row_stride;
  bf16_t* rr = res + (active ? row : 0) * rs;
  int nvec = hidden >> 3;
  float v[VPT][8];
  Vec8 wv[VPT];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (active && vi < nvec) {
      // every part's two float4 and the residual in flight before the first add
      floatx4_t lo[kMaxParts], hi[kMaxParts];
#pragma unroll
      for (int p = 0; p < kMaxParts; ++p) {
        if (p < np) {
          const floatx4_t* src = reinterpret_cast<const floatx4_t*>(pr + p * part_stride + vi * 8);
          lo[p] = __builtin_nontemporal_load(src);
          hi[p] = __builtin_nontemporal_load(src + 1);
        }
      }
      const Vec8 rv = load_vec8_nt(rr + vi * 8);
      wv[k] = load_vec8(w + vi * 8);
      float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < kMaxParts; ++p) {
        if (p < np) {
#pragma unroll
          for (int e = 0; e < 4; ++e) { a[e] += lo[p][e]; a[4 + e] += hi[p][e]; }
        }
      }
      float b[8], xr[8];
      unpack8(pack8(a), xr);  // the GEMM output's bf16 rounding
      unpack8(rv, b);
#pragma unroll
      for (int e = 0; e < 8; ++e) { v[k][e] = xr[e] + b[e]; ss += v[k][e] * v[k][e]; }
      store_vec8_nt(rr + vi * 8, pack8(v[k]));
    }
  }
  ss = row_sum<TPR>(ss);
  if (!active) return;
  float rcp = rsqrtf(ss / (float)hidden + eps);
  bf16_t* orow = out + row * os;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    int vi = lane + k * TPR;
    if (vi < nvec) {
      float wf[8], r[8];
      unpack8(wv[k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = (v[k][e] * rcp) * wf[e];
      store_vec8_nt(orow + vi * 8, pack8(r));
    }
  }
}

template <int TPR, int VPT>
struct AddRmsPartsLaunch {
  static int run(int64_t rows, hipStream_t stream, const float* parts, int64_t pst, int64_t rst, int np, bf16_t* out,
                 int64_t os, bf16_t* r, int64_t rs, const bf16_t* w, int hidden, float eps) {
    constexpr int rpb = kNormBlock<TPR> / TPR;
    int64_t blocks = (rows + rpb - 1) / rpb;
    fused_add_rmsnorm_parts_kernel<TPR, VPT><<<dim3((unsigned)blocks), dim3(kNormBlock<TPR>), 0, stream>>>(
        parts, pst, rst, np, out, os, r, rs, w, rows, hidden, eps);
    XV_CHECK_LAUNCH();
    return 0;
  }
};

extern "C" int xv_rmsnorm(const void* x, int64_t x_stride_outer, int64_t x_stride_inner,
                          const void* weight, void* out, int64_t n_outer, int64_t n_inner,
                          int hidden, float eps, hipStream_t stream) {
  if (n_outer < 0 || n_inner < 0) return (int)hipErrorInvalidValue;
  if (!xv_al16(x) || !xv_al16(weight) || !xv_al16(out) || !xv_st8(x_stride_outer) || !xv_st8(x_stride_inner))
    return (int)hipErrorInvalidValue;
  return dispatch_norm<RmsLaunch>(n_outer * n_inner, hidden, stream, (const bf16_t*)x, x_stride_outer,
                                  x_stride_inner, (const bf16_t*)weight, (bf16_t*)out, n_outer, n_inner,
                                  hidden, eps);
}

extern "C" int xv_fused_add_rmsnorm(void* x, int64_t x_stride, void* residual, int64_t residual_stride,
                                    const void* weight, int64_t rows, int hidden, float eps,
                                    hipStream_t stream) {
  if (rows < 0) return (int)hipErrorInvalidValue;
  if (!xv_al16(x) || !xv_al16(residual) || !xv_al16(weight) || !xv_st8(x_stride) || !xv_st8(residual_stride))
    return (int)hipErrorInvalidValue;
  return dispatch_norm<AddRmsLaunch>(rows, hidden, stream, (bf16_t*)x, x_stride, (bf16_t*)residual,
                                     residual_stride, (const bf16_t*)weight, hidden, eps);
}

extern "C" int xv_fused_add_rmsnorm_parts(const float* parts, int64_t part_stride, int64_t row_stride, int num_parts,
                                          void* out, int64_t out_stride, void* residual, int64_t residual_stride,
                                          const void* weight, int64_t rows, int hidden, float eps,
                                          hipStream_t stream) {
  if (rows < 0 || num_parts < 1 || num_parts > kMaxParts) return (int)hipErrorInvalidValue;
  if (!xv_al16(parts) || (part_stride | row_stride) & 3 || !xv_al16(out) || !xv_al16(residual) ||
      !xv_al16(weight) || !xv_st8(out_stride) || !xv_st8(residual_stride))
    return (int)hipErrorInvalidValue;
  return dispatch_norm<AddRmsPartsLaunch>(rows, hidden, stream, parts, part_stride, row_stride, num_parts,
                                          (bf16_t*)out, out_stride, (bf16_t*)residual, residual_stride,
                                          (const bf16_t*)weight, hidden, eps);
}

// --------------------------------------------------------------------------
// NeoX RoPE (optionally preceded by the per-head RMSNorm of Qwen3).
// 16 lanes (one DPP row) own one head of D = 128: lane j holds elements
// [8j, 8j+8); the rotation partner of lane j is lane j^8 (row_ror:8).
// --------------------------------------------------------------------------
// STORE: k heads go (roped) and v heads go (copied) straight into the paged
// cache at slot_mapping[t] (slot -1: nothing stored), instead of into k_out.
struct CacheDst {
  bf16_t* kc; bf16_t* vc;
  int64_t ps, ts, hs;
  int block_size;
  const int32_t* slots;
  const bf16_t* v; int64_t vs_tok, vs_head;
  float k_inv = 1.0f, v_inv = 1.0f;  // fp8 caches: 1 / scale
};

// Eight bf16 values x -> e4m3fn(x * inv) as 8 bytes (the fp8 KV store's rule).
XV_INLINE uint2 vec8_to_fp8(const Vec8& x, float inv) {
  float f[8];
  unpack8(x, f);
  uint32_t lo = 0, hi = 0;
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0] * inv, f[1] * inv, lo, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2] * inv, f[3] * inv, lo, true);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4] * inv, f[5] * inv, hi, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6] * inv, f[7] * inv, hi, true);
  return make_uint2(lo, hi);
}

// One wave per token: 16-lane row r of the wave handles heads r, r+4, r+8, ...
// The token's position, its fp32 cos/sin row, the norm weights and the slot
// are fetched once per lane; all head loads of a row (up to kRopeBatch) are
// issued before the first is used.
#ifndef XV_ROPE_BATCH
#define XV_ROPE_BATCH 6
#endif
#ifndef XV_ROPE_ROWS
#define XV_ROPE_ROWS 8  // 16-lane rows per token (two waves)
#endif
constexpr int kRopeBatch = XV_ROPE_BATCH;
constexpr int kRopeRows = XV_ROPE_ROWS;

template <bool NORM, bool STORE, bool F8 = false>
__global__ __launch_bounds__(256) void rope_kernel(
    const bf16_t* __restrict__ q, int64_t qs_tok, int64_t qs_head,
    const bf16_t* __restrict__ k, int64_t ks_tok, int64_t ks_head,
    const bf16_t* __restrict__ qw, const bf16_t* __restrict__ kw, float eps,
    const int64_t* __restrict__ positions, const float* __restrict__ cos_sin,
    bf16_t* __restrict__ q_out, bf16_t* __restrict__ k_out,
    int64_t num_tokens, int hq, int hkv, CacheDst cd) {
  constexpr int D = 128;
  const int64_t tok = ((int64_t)blockIdx.x * 16 + (threadIdx.x >> 4)) / kRopeRows;
  if (tok >= num_tokens) return;
  const int row = (threadIdx.x >> 4) % kRopeRows, lane = threadIdx.x & 15;
  const int nrot = hq + hkv;                       // heads normed and rotated
  const int heads = nrot + (STORE ? hkv : 0);      // STORE: v heads follow, copied
  const int64_t pos = positions[tok];
  const float* cs = cos_sin + pos * D + (lane & 7) * 8;
  const float4 c0 = *reinterpret_cast<const float4*>(cs);
  const float4 c1 = *reinterpret_cast<const float4*>(cs + 4);
  const float4 s0 = *reinterpret_cast<const float4*>(cs + D / 2);
  const float4 s1 = *reinterpret_cast<const float4*>(cs + D / 2 + 4);
  const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  float wq[8], wk[8];
  if constexpr (NORM) {
    unpack8(load_vec8(qw + lane * 8), wq);
    unpack8(load_vec8(kw + lane * 8), wk);
  }
  int32_t slot = 0;
  int64_t cache_off = 0;
  if constexpr (STORE) {
    slot = cd.slots[tok];
    const int page = slot / cd.block_size, t = slot - page * cd.block_size;
    cache_off = (int64_t)page * cd.ps + (int64_t)t * cd.ts + lane * 8;
  }
  for (int h0 = row; h0 < heads; h0 += kRopeRows * kRopeBatch) {
    Vec8 xv[kRopeBatch];
#pragma unroll
    for (int j = 0; j < kRopeBatch; ++j) {
      const int h = h0 + kRopeRows * j;
      if (h >= heads) break;
      const bf16_t* src = h < hq ? q + tok * qs_tok + (int64_t)h * qs_head
                        : h < nrot ? k + tok * ks_tok + (int64_t)(h - hq) * ks_head
                                   : cd.v + tok * cd.vs_tok + (int64_t)(h - nrot) * cd.vs_head;
      xv[j] = load_vec8_nt(src + lane * 8);
    }
#pragma unroll
    for (int j = 0; j < kRopeBatch; ++j) {
      const int h = h0 + kRopeRows * j;
      if (h >= heads) break;
      if (STORE && h >= nrot) {  // v head: plain copy into the cache
        if (slot >= 0) {
          const int64_t off = cache_off + (int64_t)(h - nrot) * cd.hs;
          if constexpr (F8) *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(cd.vc) + off) = vec8_to_fp8(xv[j], cd.v_inv);
          else store_vec8_nt(cd.vc + off, xv[j]);
        }
        continue;
      }
      const bool is_q = h < hq;
      float x[8];
      unpack8(xv[j], x);
      if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
        ss = row16_sum(ss);
        const float rcp = rsqrtf(ss / (float)D + eps);
        // round to bf16 between the norm and the rotation, as the two separate ops do
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = bf16_to_f32(f32_to_bf16((x[e] * rcp) * (is_q ? wq[e] : wk[e])));
      }
      float r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float partner = dpp_f<0x128>(x[e]);  // row_ror:8 -> lane j^8
        r[e] = lane < 8 ? x[e] * c[e] - partner * sn[e] : x[e] * c[e] + partner * sn[e];
      }
      if (is_q) {
        store_vec8_nt(q_out + (tok * hq + h) * D + lane * 8, pack8(r));
      } else if constexpr (STORE) {
        if (slot >= 0) {
          const int64_t off = cache_off + (int64_t)(h - hq) * cd.hs;
          // fp8: the roped k rounded to bf16 first, as the unfused store sees it
          if constexpr (F8) *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(cd.kc) + off) = vec8_to_fp8(pack8(r), cd.k_inv);
          else store_vec8_nt(cd.kc + off, pack8(r));
        }
      } else {
        store_vec8_nt(k_out + (tok * hkv + (h - hq)) * D + lane * 8, pack8(r));
      }
    }
  }
}

template <bool NORM, bool STORE, bool F8 = false>
static int launch_rope_t(const void* q, int64_t qst, int64_t qsh, const void* k, int64_t kst, int64_t ksh,
                         const void* qw, const void* kw, float eps, const int64_t* positions, const float* cs,
                         void* q_out, void* k_out, int64_t T, int hq, int hkv, const CacheDst& cd,
                         hipStream_t stream) {
  // rows and weights move as 16-byte vectors, the fp32 table as float4
  if (!xv_al16(q) || !xv_al16(k) || !xv_al16(qw) || !xv_al16(kw) || !xv_al16(cs) || !xv_al16(q_out) ||
      !xv_al16(k_out) || !xv_st8(qst) || !xv_st8(qsh) || !xv_st8(kst) || !xv_st8(ksh))
    return (int)hipErrorInvalidValue;
  if (STORE && (!xv_al16(cd.kc) || !xv_al16(cd.vc) || !xv_al16(cd.v) || !xv_st8(cd.ps) || !xv_st8(cd.ts) ||
                !xv_st8(cd.hs) || !xv_st8(cd.vs_tok) || !xv_st8(cd.vs_head)))
    return (int)hipErrorInvalidValue;  // (fp8 caches: 8-byte pieces, the same element strides suffice)
  const unsigned blocks = (unsigned)((T * kRopeRows + 15) / 16);
  rope_kernel<NORM, STORE, F8><<<blocks, 256, 0, stream>>>((const bf16_t*)q, qst, qsh, (const bf16_t*)k, kst, ksh,
                                                       (const bf16_t*)qw, (const bf16_t*)kw, eps, positions, cs,
                                                       (bf16_t*)q_out, (bf16_t*)k_out, T, hq, hkv, cd);
  XV_CHECK_LAUNCH();
  return 0;
}

static int launch_rope(bool norm, const void* q, int64_t qst, int64_t qsh, const void* k, int64_t kst,
                       int64_t ksh, const void* qw, const void* kw, float eps, const int64_t* positions,
                       const float* cs, void* q_out, void* k_out, int64_t T, int hq, int hkv, int D,
                       hipStream_t stream) {
  if (D != 128 || hq <= 0 || hkv < 0 || T < 0) return (int)hipErrorInvalidValue;
  if (T == 0) return 0;
  CacheDst cd = {};
  return norm ? launch_rope_t<true, false>(q, qst, qsh, k, kst, ksh, qw, kw, eps, positions, cs, q_out, k_out, T, hq,
                                           hkv, cd, stream)
              : launch_rope_t<false, false>(q, qst, qsh, k, kst, ksh, qw, kw, eps, positions, cs, q_out, k_out, T,
                                            hq, hkv, cd, stream);
}

extern "C" int xv_qk_norm_rope_store(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                     const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                                     const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                                     const void* q_weight, const void* k_weight, float eps,
                                     const int64_t* positions, const float* cos_sin_cache, void* q_out,
                                     void* k_cache, void* v_cache, int64_t cache_page_stride,
                                     int64_t cache_tok_stride, int64_t cache_head_stride, int block_size,
                                     const int32_t* slot_mapping, int64_t num_tokens, int num_q_heads,
                                     int num_kv_heads, int head_dim, hipStream_t stream) {
  if (head_dim != 128 || num_q_heads <= 0 || num_kv_heads <= 0 || num_tokens < 0 || block_size <= 0)
    return (int)hipErrorInvalidValue;
  if (num_tokens == 0) return 0;
  CacheDst cd;
  cd.kc = (bf16_t*)k_cache; cd.vc = (bf16_t*)v_cache;
  cd.ps = cache_page_stride; cd.ts = cache_tok_stride; cd.hs = cache_head_stride; cd.block_size = block_size;
  cd.slots = slot_mapping; cd.v = (const bf16_t*)v; cd.vs_tok = v_stride_tok; cd.vs_head = v_stride_head;
  return launch_rope_t<true, true>(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, q_weight, k_weight,
                                   eps, positions, cos_sin_cache, q_out, nullptr, num_tokens, num_q_heads,
                                   num_kv_heads, cd, stream);
}

extern "C" int xv_qk_norm_rope_store_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                         const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                                         const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                                         const void* q_weight, const void* k_weight, float eps,
                                         const int64_t* positions, const float* cos_sin_cache, void* q_out,
                                         void* k_cache, void* v_cache, int64_t cache_page_stride,
                                         int64_t cache_tok_stride, int64_t cache_head_stride, int block_size,
                                         const int32_t* slot_mapping, int64_t num_tokens, int num_q_heads,
                                         int num_kv_heads, int head_dim, float k_scale, float v_scale,
                                         hipStream_t stream) {
  if (head_dim != 128 || num_q_heads <= 0 || num_kv_heads <= 0 || num_tokens < 0 || block_size <= 0)
    return (int)hipErrorInvalidValue;
  if (!(k_scale > 0.0f) || !(v_scale > 0.0f) || !__builtin_isfinite(k_scale) || !__builtin_isfinite(v_scale))
    return (int)hipErrorInvalidValue;
  if (num_tokens == 0) return 0;
  CacheDst cd;
  cd.kc = (bf16_t*)k_cache; cd.vc = (bf16_t*)v_cache;
  cd.ps = cache_page_stride; cd.ts = cache_tok_stride; cd.hs = cache_head_stride; cd.block_size = block_size;
  cd.slots = slot_mapping; cd.v = (const bf16_t*)v; cd.vs_tok = v_stride_tok; cd.vs_head = v_stride_head;
  cd.k_inv = 1.0f / k_scale; cd.v_inv = 1.0f / v_scale;
  return launch_rope_t<true, true, true>(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, q_weight,
                                         k_weight, eps, positions, cos_sin_cache, q_out, nullptr, num_tokens,
                                         num_q_heads, num_kv_heads, cd, stream);
}

extern "C" int xv_rotary_embedding(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                   const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                                   const int64_t* positions, const float* cos_sin_cache,
                                   void* q_out, void* k_out, int64_t num_tokens,
                                   int num_q_heads, int num_kv_heads, int head_dim, hipStream_t stream) {
  return launch_rope(false, q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, nullptr, nullptr,
                     0.f, positions, cos_sin_cache, q_out, k_out, num_tokens, num_q_heads, num_kv_heads,
                     head_dim, stream);
}

extern "C" int xv_qk_norm_rope(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                               const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                               const void* q_weight, const void* k_weight, float eps,
                               const int64_t* positions, const float* cos_sin_cache,
                               void* q_out, void* k_out, int64_t num_tokens,
                               int num_q_heads, int num_kv_heads, int head_dim, hipStream_t stream) {
  return launch_rope(true, q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, q_weight, k_weight,
                     eps, positions, cos_sin_cache, q_out, k_out, num_tokens, num_q_heads, num_kv_heads,
                     head_dim, stream);
}

// --------------------------------------------------------------------------
// SiLU-and-mul: one thread per 8 outputs.
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void silu_and_mul_kernel(const bf16_t* __restrict__ x, int64_t xs,
                                                           bf16_t* __restrict__ out, int64_t os,
                                                           int64_t total_vec, int vec_per_row, int inter) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total_vec) return;
  int64_t row = idx / vec_per_row;
  int c = (int)(idx - row * vec_per_row) * 8;
  const bf16_t* xr = x + row * xs;
  float g[8], u[8], r[8];
  unpack8(load_vec8_nt(xr + c), g);
  unpack8(load_vec8_nt(xr + inter + c), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = g[e] * __builtin_amdgcn_rcpf(1.0f + __expf(-g[e])) * u[e];
  store_vec8_nt(out + row * os + c, pack8(r));
}

extern "C" int xv_silu_and_mul(const void* x, int64_t x_stride, void* out, int64_t out_stride,
                               int64_t num_tokens, int inter_size, hipStream_t stream) {
  if (num_tokens < 0 || inter_size <= 0 || inter_size % 8) return (int)hipErrorInvalidValue;
  if (!xv_al16(x) || !xv_al16(out) || !xv_st8(x_stride) || !xv_st8(out_stride)) return (int)hipErrorInvalidValue;
  if (num_tokens == 0) return 0;
  int vpr = inter_size / 8;
  int64_t total = num_tokens * vpr;
  silu_and_mul_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, stream>>>(
      (const bf16_t*)x, x_stride, (bf16_t*)out, out_stride, total, vpr, inter_size);
  XV_CHECK_LAUNCH();
  return 0;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// --------------------------------------------------------------------------
// Streaming copy: the measurement yardstick for the kernels above (what a
// plain read-once / write-once transfer of the same byte count reaches on this
// part), not part of the decode path.
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                          int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}
// A grid of 1024 workgroups, four 16-byte vectors per lane per round.
__global__ __launch_bounds__(256) void stream_copy_grid_kernel(const u32x4_t* __restrict__ src,
                                                               u32x4_t* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 1024;
  for (int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x; base < n; base += stride) {
    u32x4_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (base + 256 * j < n) v[j] = __builtin_nontemporal_load(src + base + 256 * j);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (base + 256 * j < n) __builtin_nontemporal_store(v[j], dst + base + 256 * j);
  }
}

extern "C" int xv_stream_copy(const void* src, void* dst, int64_t bytes, int shape, hipStream_t stream) {
  if (bytes < 0 || bytes % 16 || !xv_al16(src) || !xv_al16(dst) || (shape != 0 && shape != 1))
    return (int)hipErrorInvalidValue;
  const int64_t n = bytes / 16;
  if (n == 0) return 0;
  if (shape == 0) {
    if ((n + 255) / 256 > 0x7fffffff) return (int)hipErrorInvalidValue;
    stream_copy_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, stream>>>((const u32x4_t*)src, (u32x4_t*)dst, n);
  } else {
    stream_copy_grid_kernel<<<dim3(1024), 256, 0, stream>>>((const u32x4_t*)src, (u32x4_t*)dst, n);
  }
  XV_CHECK_LAUNCH();
  return 0;
}
