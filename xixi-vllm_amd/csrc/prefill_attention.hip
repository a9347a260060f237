// Varlen causal prefill attention (chunked prefill / cached prefix) for gfx950.
//
// Workgroup = 8 waves over one (sequence, kv head, query block); wave w serves
// query head kvh*G + w%G for the 16 query tokens (w/G)*16 .. +16 of the block,
// so the block holds 16*8/G tokens and every K/V tile staged in LDS is shared
// by all G heads of the kv group.  Per 64-key tile and wave:
//   S^T = K Q^T   16 x v_mfma_f32_16x16x32_bf16 (A = K rows from LDS, B = Q^T
//                 held in VGPRs); lane (q = lane%16, g) holds keys 16m+4g+r of
//                 its own query, so the online softmax is in-lane plus two
//                 cross-row shuffles and the O rescale needs no shuffle;
//   O^T += V^T P^T  16 x v_mfma_f32_16x16x32_bf16 (A = V^T read transposed with
//                 ds_read_b64_tr_b16, B = P^T straight from the S^T layout).
// K/V tiles are double buffered: the next tile's global loads are in flight
// while the current tile is computed.  Causal masking is bottom-right aligned
// (query i of q_len sees keys j <= k_len - q_len + i); fully masked tiles are
// skipped.  Keys come from dense rows or through the paged block table.
#include "xv_common.h"
#include "xv_kernels.h"
#include <math.h>

namespace {

constexpr int kD = 128;
constexpr int kKeys = 64;        // keys per tile
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kKPitch = 272;     // LDS bytes per K row (ds_read_b128 rows, padded)
constexpr int kVPitch = 288;     // LDS bytes per V row (transposed reads, padded)
constexpr int kKBytes = kKeys * kKPitch;
constexpr int kVBytes = kKeys * kVPitch;

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4;

struct PrefillArgs {
  const bf16_t* q; int64_t q_st, q_sh;
  const bf16_t* k; const bf16_t* v; int64_t kv_st, kv_sh;
  const bf16_t* kc; const bf16_t* vc; int64_t page_stride, tok_stride, head_stride;
  const int32_t* bt; int64_t bt_stride;
  const int32_t* cu_q; const int32_t* cu_k;
  bf16_t* out; int64_t out_st;
  int hq, hkv, block_size;
  float scale_log2;
};

XV_INLINE bf16x8_t as_bf16x8(const Vec8& v) {
  bf16x8_t r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// Global address of key row j (kv head kvh) of sequence b, or nullptr past k_len.
XV_INLINE const bf16_t* key_row(const PrefillArgs& a, const bf16_t* dense, const bf16_t* paged, int b, int kvh,
                                int j, int k0, int k_len) {
  if (j >= k_len) return nullptr;
  if (a.bt) {
    const int page = a.bt[(int64_t)b * a.bt_stride + j / a.block_size];
    return paged + (int64_t)page * a.page_stride + (int64_t)(j % a.block_size) * a.tok_stride +
           (int64_t)kvh * a.head_stride;
  }
  return dense + (int64_t)(k0 + j) * a.kv_st + (int64_t)kvh * a.kv_sh;
}

// Each of the 512 threads moves 2 x 16 B of K and of V for a 64-key tile.
struct TileRegs {
  Vec8 k[2], v[2];
};

XV_INLINE void tile_load(TileRegs& r, const PrefillArgs& a, int b, int kvh, int key0, int k0, int k_len) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = threadIdx.x + u * kThreads;  // chunk id in [0, 1024): key = c/16, 16B chunk = c%16
    const int j = key0 + (c >> 4);
    const int off = (c & 15) * 8;
    const bf16_t* kr = key_row(a, a.k, a.kc, b, kvh, j, k0, k_len);
    const bf16_t* vr = key_row(a, a.v, a.vc, b, kvh, j, k0, k_len);
    if (kr) {
      r.k[u] = load_vec8(kr + off);
      r.v[u] = load_vec8(vr + off);
    } else {  // past the sequence: zeros (never NaN garbage)
      r.k[u].w[0] = r.k[u].w[1] = r.k[u].w[2] = r.k[u].w[3] = 0u;
      r.v[u] = r.k[u];
    }
  }
}

XV_INLINE void tile_store(const TileRegs& r, char* kl, char* vl) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = threadIdx.x + u * kThreads;
    const int row = c >> 4, ch = c & 15;
    *reinterpret_cast<uint4*>(kl + row * kKPitch + ch * 16) = make_uint4(r.k[u].w[0], r.k[u].w[1], r.k[u].w[2], r.k[u].w[3]);
    *reinterpret_cast<uint4*>(vl + row * kVPitch + ch * 16) = make_uint4(r.v[u].w[0], r.v[u].w[1], r.v[u].w[2], r.v[u].w[3]);
  }
}

template <int G>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
  constexpr int R = kWaves / G;      // 16-token row blocks per workgroup
  constexpr int kBlockQ = 16 * R;    // query tokens per workgroup
  __shared__ __attribute__((aligned(16))) char lds[2 * (kKBytes + kVBytes)];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int b = blockIdx.z, kvh = blockIdx.y;
  const int q0 = a.cu_q[b], q_len = a.cu_q[b + 1] - q0;
  const int k0 = a.cu_k[b], k_len = a.cu_k[b + 1] - k0;
  const int qb0 = blockIdx.x * kBlockQ;
  if (qb0 >= q_len) return;
  const int head = kvh * G + wave % G;
  const int qrow0 = qb0 + (wave / G) * 16;  // first query (within the sequence) of this wave
  const int my_q = qrow0 + i;               // the query of this lane's column
  const int shift = k_len - q_len;          // bottom-right alignment

  // keys needed by the whole workgroup: up to the last query of the block
  const int q_last = min(qb0 + kBlockQ, q_len) - 1;
  const int kv_end = min(k_len, shift + q_last + 1);
  const int ntiles = (kv_end + kKeys - 1) / kKeys;

  // Q^T operand: column = query my_q, k-chunk 4s+g
  bf16x8_t qb[4];
  {
    const int qi = min(my_q, q_len - 1);
    const bf16_t* qp = a.q + (int64_t)(q0 + qi) * a.q_st + (int64_t)head * a.q_sh + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = as_bf16x8(load_vec8(qp + 32 * s));
  }

  floatx4_t o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const int my_kend = shift + my_q + 1;  // this query sees keys [0, my_kend)
  const int wave_kend = min(k_len, shift + min(qrow0 + 15, q_len - 1) + 1);

  TileRegs tr;
  if (ntiles > 0) {
    tile_load(tr, a, b, kvh, 0, k0, k_len);
    tile_store(tr, lds, lds + kKBytes);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    char* kl = lds + (t & 1) * (kKBytes + kVBytes);
    char* vl = kl + kKBytes;
    if (t + 1 < ntiles) tile_load(tr, a, b, kvh, (t + 1) * kKeys, k0, k_len);
    const int key0 = t * kKeys;
    if (key0 < wave_kend) {
      // ---- S^T for the 4 key sub-tiles ----
      floatx4_t sc[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        sc[m] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        const char* kr = kl + (16 * m + i) * kKPitch + 16 * g;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint4 kv = *reinterpret_cast<const uint4*>(kr + 64 * s);
          Vec8 kk; kk.w[0] = kv.x; kk.w[1] = kv.y; kk.w[2] = kv.z; kk.w[3] = kv.w;
          sc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kk), qb[s], sc[m], 0, 0, 0);
        }
      }
      // ---- mask, online softmax (lane = one query, keys 16m+4g+r) ----
      float mx = -INFINITY;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = key0 + 16 * m + 4 * g + r;
          const float v = (key < my_kend) ? sc[m][r] * a.scale_log2 : -INFINITY;
          sc[m][r] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
      short pb[4][4];
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = (m_new == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sc[m][r] - m_new);
          psum += p;
          pb[m][r] = (short)f32_to_bf16(p);
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int n = 0; n < 8; ++n) o[n] *= alpha;
      // ---- O^T += V^T P^T, 32 keys per MFMA (sub-tiles m, m+1) ----
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        bf16x8_t pbv;
        {
          short tmp[8] = {pb[2 * h2][0], pb[2 * h2][1], pb[2 * h2][2], pb[2 * h2][3],
                          pb[2 * h2 + 1][0], pb[2 * h2 + 1][1], pb[2 * h2 + 1][2], pb[2 * h2 + 1][3]};
          __builtin_memcpy(&pbv, tmp, 16);
        }
        const char* vb0 = vl + (32 * h2 + 4 * g + (i >> 2)) * kVPitch + 8 * (i & 3);
        const char* vb1 = vb0 + 16 * kVPitch;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb0 + 32 * n));
          short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb1 + 32 * n));
          short tmp[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          bf16x8_t va;
          __builtin_memcpy(&va, tmp, 16);
          o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pbv, o[n], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // everyone done with buffer t&1 ... and (t+1)&1 is free
    if (t + 1 < ntiles) {
      char* kn = lds + ((t + 1) & 1) * (kKBytes + kVBytes);
      tile_store(tr, kn, kn + kKBytes);
    }
    __syncthreads();
  }

  // ---- normalise and write: lane holds O[my_q][16n + 4g + r] ----
  float lsum = l_run;
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  if (my_q >= q_len) return;
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  bf16_t* op = a.out + (int64_t)(q0 + my_q) * a.out_st + (int64_t)head * kD + 4 * g;
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    uint2 w = make_uint2(pack_bf16x2(o[n][0] * inv, o[n][1] * inv), pack_bf16x2(o[n][2] * inv, o[n][3] * inv));
    *reinterpret_cast<uint2*>(op + 16 * n) = w;
  }
}

}  // namespace

extern "C" int xv_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                    const void* k, const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                                    const void* k_cache, const void* v_cache,
                                    int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                    const int32_t* block_tables, int64_t bt_stride,
                                    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                    void* out, int64_t out_stride_tok,
                                    int batch, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                                    int head_dim, int block_size, float scale, hipStream_t stream) {
  if (head_dim != kD || batch < 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || max_seqlen_q < 0)
    return (int)hipErrorInvalidValue;
  const int group = num_q_heads / num_kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8) return (int)hipErrorInvalidValue;
  if (block_tables) {
    if (!k_cache || !v_cache || block_size <= 0) return (int)hipErrorInvalidValue;
  } else if (!k || !v) {
    return (int)hipErrorInvalidValue;
  }
  if (batch == 0 || max_seqlen_q == 0) return 0;
  PrefillArgs a;
  a.q = (const bf16_t*)q; a.q_st = q_stride_tok; a.q_sh = q_stride_head;
  a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.kv_st = kv_stride_tok; a.kv_sh = kv_stride_head;
  a.kc = (const bf16_t*)k_cache; a.vc = (const bf16_t*)v_cache;
  a.page_stride = page_stride; a.tok_stride = tok_stride; a.head_stride = head_stride;
  a.bt = block_tables; a.bt_stride = bt_stride;
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k;
  a.out = (bf16_t*)out; a.out_st = out_stride_tok;
  a.hq = num_q_heads; a.hkv = num_kv_heads; a.block_size = block_size;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int block_q = 16 * (kWaves / group);
  dim3 grid((unsigned)((max_seqlen_q + block_q - 1) / block_q), (unsigned)num_kv_heads, (unsigned)batch);
  switch (group) {
    case 1: prefill_kernel<1><<<grid, kThreads, 0, stream>>>(a); break;
    case 2: prefill_kernel<2><<<grid, kThreads, 0, stream>>>(a); break;
    case 4: prefill_kernel<4><<<grid, kThreads, 0, stream>>>(a); break;
    default: prefill_kernel<8><<<grid, kThreads, 0, stream>>>(a); break;
  }
  XV_CHECK_LAUNCH();
  return 0;
}
