// Paged GQA decode attention for gfx950.
//
// Work unit: one wave64 workgroup per (sequence, group of GW query heads
// sharing one kv head, KV split of `pps` 16-token pages).  The wave streams
// its pages straight from HBM into registers in the operand layout of
// v_mfma_f32_16x16x32_bf16, so no LDS is used:
//   lane = 16*g + t  (t = token within the page, g = 0..3)
//   K/V: lane loads 16-byte chunks c = 4*s + g (s = 0..3) of token row t, i.e.
//        for each s the four lanes of a token read 64 contiguous bytes.
//   Q:   A operand, row i = lane%16 holds query head i % GW (rows replicated),
//        same chunk mapping, so MFMA step s contracts d in chunk 4s+g.
//   S = Q K^T lands as acc[r] = S[row 4g+r][token t]  ->  head r % GW.
// Every lane therefore holds the scores of its own token for all GW heads,
// and P.V runs on the VALU against the V chunks the same lane loaded:
//   o[h][d = 8*(4s+g)+e] += p[h] * v[s][e].
// Softmax is online in the exp2 domain with the running max reduced over the
// 16 tokens of a page by DPP (identical in all four lane rows).  The 16 token
// lanes are summed once at the end of the split with DPP row reductions.
// Splits of one (sequence, head) are merged by a second kernel through an
// fp32 workspace holding normalised partial outputs and their log2-sum-exp.
#include "xv_common.h"
#include "../../include/xv_kernels.h"
#include <math.h>
#include <stdlib.h>

namespace {

constexpr int kD = 128;
constexpr int kPage = 16;

struct DecodeArgs {
  const bf16_t* q; int64_t q_st, q_sh;
  const bf16_t* kc; const bf16_t* vc;
  int64_t page_stride, tok_stride, head_stride;
  const int32_t* bt; int64_t bt_stride;
  const int32_t* seqlens;
  bf16_t* out; int64_t out_st;
  float* ws_o; float* ws_lse;
  int hq, hkv, group, pps, max_splits;
  float scale_log2;
};

struct PageRegs {
  Vec8 k[4];
  Vec8 v[4];
};

XV_INLINE void load_page(PageRegs& r, const DecodeArgs& a, int page, int kvh, int t, int g) {
  int64_t base = (int64_t)page * a.page_stride + (int64_t)t * a.tok_stride + (int64_t)kvh * a.head_stride;
  const bf16_t* kp = a.kc + base + 8 * g;
  const bf16_t* vp = a.vc + base + 8 * g;
#pragma unroll
  for (int s = 0; s < 4; ++s) r.k[s] = load_vec8_nt(kp + 32 * s);
#pragma unroll
  for (int s = 0; s < 4; ++s) r.v[s] = load_vec8_nt(vp + 32 * s);
}

XV_INLINE bf16x8_t as_bf16x8(const Vec8& v) {
  bf16x8_t r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

template <int GW>
struct SplitState {
  float m[GW];
  float l[GW];
  float o[GW][4][8];
};

template <int GW>
XV_INLINE void process_page(SplitState<GW>& st, PageRegs& r, const bf16x8_t (&qa)[4], int tok_idx,
                            int ctx, bool last, float scale_log2) {
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[s], as_bf16x8(r.k[s]), acc, 0, 0, 0);
  const bool valid = tok_idx < ctx;
  if (last && !valid) {
    // cache rows past the sequence end may hold anything (even NaN): zero them
#pragma unroll
    for (int s = 0; s < 4; ++s) r.v[s].w[0] = r.v[s].w[1] = r.v[s].w[2] = r.v[s].w[3] = 0u;
  }
#pragma unroll
  for (int h = 0; h < GW; ++h) {
    float sc = valid ? acc[h] * scale_log2 : -INFINITY;
    float mx = row16_max(sc);
    float m_new = fmaxf(st.m[h], mx);
    if (m_new > st.m[h]) {
      float alpha = __builtin_amdgcn_exp2f(st.m[h] - m_new);
      st.l[h] *= alpha;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) st.o[h][s][e] *= alpha;
      st.m[h] = m_new;
    }
    float p = __builtin_amdgcn_exp2f(sc - m_new);
    st.l[h] += p;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        st.o[h][s][2 * w] += p * bf16lo(r.v[s].w[w]);
        st.o[h][s][2 * w + 1] += p * bf16hi(r.v[s].w[w]);
      }
    }
  }
}

template <int GW>
__global__ __launch_bounds__(64) void paged_decode_kernel(DecodeArgs a) {
  const int lane = threadIdx.x;
  const int t = lane & 15, g = lane >> 4;
  const int hgroups = a.hkv * (a.group / GW);
  const int b = blockIdx.x / hgroups;
  const int hg = blockIdx.x - b * hgroups;
  const int kvh = hg / (a.group / GW);
  const int head0 = kvh * a.group + (hg - kvh * (a.group / GW)) * GW;
  const int split = blockIdx.y;
  const int ctx = a.seqlens[b];
  const int npages = (ctx + kPage - 1) / kPage;
  const int nsplit = (npages + a.pps - 1) / a.pps;

  if (ctx <= 0) {
    // padding row: defined zero output, written once by split 0
    if (split == 0 && t < GW) {
      bf16_t* o = a.out + (int64_t)b * a.out_st + (int64_t)(head0 + t) * kD + 8 * g;
      Vec8 z; z.w[0] = z.w[1] = z.w[2] = z.w[3] = 0u;
#pragma unroll
      for (int s = 0; s < 4; ++s) store_vec8(o + 32 * s, z);
    }
    return;
  }
  if (split >= nsplit) return;
  const int p0 = split * a.pps;
  const int np = min(a.pps, npages - p0);

  // page ids of this split, one per lane, broadcast with readlane
  int pid = 0;
  if (lane < np) pid = a.bt[(int64_t)b * a.bt_stride + p0 + lane];

  bf16x8_t qa[4];
  {
    const bf16_t* qp = a.q + (int64_t)b * a.q_st + (int64_t)(head0 + (t % GW)) * a.q_sh + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qa[s] = as_bf16x8(load_vec8(qp + 32 * s));
  }

  SplitState<GW> st;
#pragma unroll
  for (int h = 0; h < GW; ++h) {
    st.m[h] = -INFINITY;
    st.l[h] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) st.o[h][s][e] = 0.f;
  }

  PageRegs r0, r1;
  load_page(r0, a, __builtin_amdgcn_readlane(pid, 0), kvh, t, g);
  for (int i = 0; i < np; i += 2) {
    if (i + 1 < np) load_page(r1, a, __builtin_amdgcn_readlane(pid, i + 1), kvh, t, g);
    process_page<GW>(st, r0, qa, (p0 + i) * kPage + t, ctx, p0 + i == npages - 1, a.scale_log2);
    if (i + 1 >= np) break;
    if (i + 2 < np) load_page(r0, a, __builtin_amdgcn_readlane(pid, i + 2), kvh, t, g);
    process_page<GW>(st, r1, qa, (p0 + i + 1) * kPage + t, ctx, p0 + i + 1 == npages - 1, a.scale_log2);
  }

  // sum the 16 token lanes of each row
#pragma unroll
  for (int h = 0; h < GW; ++h) {
    st.l[h] = row16_sum(st.l[h]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) st.o[h][s][e] = row16_sum(st.o[h][s][e]);
  }

#pragma unroll
  for (int h = 0; h < GW; ++h) {
    if (t != h) continue;
    const float inv = 1.0f / st.l[h];
    if (nsplit == 1) {
      bf16_t* o = a.out + (int64_t)b * a.out_st + (int64_t)(head0 + h) * kD + 8 * g;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = st.o[h][s][e] * inv;
        store_vec8(o + 32 * s, pack8(v));
      }
    } else {
      const int64_t row = ((int64_t)b * a.hq + head0 + h) * a.max_splits + split;
      float* o = a.ws_o + row * kD + 8 * g;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float4 v0 = make_float4(st.o[h][s][0] * inv, st.o[h][s][1] * inv, st.o[h][s][2] * inv, st.o[h][s][3] * inv);
        float4 v1 = make_float4(st.o[h][s][4] * inv, st.o[h][s][5] * inv, st.o[h][s][6] * inv, st.o[h][s][7] * inv);
        *reinterpret_cast<float4*>(o + 32 * s) = v0;
        *reinterpret_cast<float4*>(o + 32 * s + 4) = v1;
      }
      if (g == 0) a.ws_lse[row] = st.m[h] + __log2f(st.l[h]);
    }
  }
}

// Merge the split partials of one (sequence, query head): 64 lanes x 2 dims.
__global__ __launch_bounds__(64) void merge_splits_kernel(DecodeArgs a) {
  const int b = blockIdx.x / a.hq;
  const int h = blockIdx.x - b * a.hq;
  const int ctx = a.seqlens[b];
  const int npages = (ctx + kPage - 1) / kPage;
  const int nsplit = (npages + a.pps - 1) / a.pps;
  if (nsplit <= 1) return;
  const int64_t row0 = ((int64_t)b * a.hq + h) * a.max_splits;
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, a.ws_lse[row0 + s]);
  float den = 0.f, o0 = 0.f, o1 = 0.f;
  const int d = threadIdx.x * 2;
  for (int s = 0; s < nsplit; ++s) {
    float w = __builtin_amdgcn_exp2f(a.ws_lse[row0 + s] - mx);
    float2 v = *reinterpret_cast<const float2*>(a.ws_o + (row0 + s) * kD + d);
    den += w;
    o0 += w * v.x;
    o1 += w * v.y;
  }
  const float inv = 1.0f / den;
  *reinterpret_cast<uint32_t*>(a.out + (int64_t)b * a.out_st + (int64_t)h * kD + d) = pack_bf16x2(o0 * inv, o1 * inv);
}

int pages_per_split() {
  static int pps = [] {
    const char* e = getenv("XV_DECODE_PAGES_PER_SPLIT");
    int v = e ? atoi(e) : 16;
    if (v < 1) v = 1;
    if (v > 64) v = 64;
    return v;
  }();
  return pps;
}

}  // namespace

extern "C" size_t xv_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                                 int max_blocks_per_seq, int block_size, int head_dim) {
  (void)num_kv_heads; (void)block_size;
  if (batch <= 0 || max_blocks_per_seq <= 0) return 0;
  const int ms = (max_blocks_per_seq + pages_per_split() - 1) / pages_per_split();
  return (size_t)batch * num_q_heads * ms * ((size_t)head_dim + 1) * sizeof(float);
}

extern "C" int xv_paged_decode_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                         const void* k_cache, const void* v_cache,
                                         int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                         const int32_t* block_tables, int64_t bt_stride,
                                         const int32_t* cache_seqlens,
                                         void* out, int64_t out_stride_tok,
                                         void* workspace, size_t workspace_bytes,
                                         int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                         int block_size, int max_blocks_per_seq, float scale,
                                         hipStream_t stream) {
  if (head_dim != kD || block_size != kPage || batch < 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads || max_blocks_per_seq <= 0)
    return (int)hipErrorInvalidValue;
  const int group = num_q_heads / num_kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  const int pps = pages_per_split();
  const int max_splits = (max_blocks_per_seq + pps - 1) / pps;
  const size_t need = xv_paged_decode_workspace_size(batch, num_q_heads, num_kv_heads, max_blocks_per_seq,
                                                     block_size, head_dim);
  if (max_splits > 1 && (workspace == nullptr || workspace_bytes < need)) return (int)hipErrorInvalidValue;
  DecodeArgs a;
  a.q = (const bf16_t*)q; a.q_st = q_stride_tok; a.q_sh = q_stride_head;
  a.kc = (const bf16_t*)k_cache; a.vc = (const bf16_t*)v_cache;
  a.page_stride = page_stride; a.tok_stride = tok_stride; a.head_stride = head_stride;
  a.bt = block_tables; a.bt_stride = bt_stride; a.seqlens = cache_seqlens;
  a.out = (bf16_t*)out; a.out_st = out_stride_tok;
  a.ws_o = (float*)workspace;
  a.ws_lse = a.ws_o ? a.ws_o + (size_t)batch * num_q_heads * max_splits * kD : nullptr;
  a.hq = num_q_heads; a.hkv = num_kv_heads; a.group = group; a.pps = pps; a.max_splits = max_splits;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int gw = group >= 4 ? 4 : group;
  dim3 grid((unsigned)(batch * num_kv_heads * (group / gw)), (unsigned)max_splits);
  switch (gw) {
    case 1: paged_decode_kernel<1><<<grid, 64, 0, stream>>>(a); break;
    case 2: paged_decode_kernel<2><<<grid, 64, 0, stream>>>(a); break;
    default: paged_decode_kernel<4><<<grid, 64, 0, stream>>>(a); break;
  }
  XV_CHECK_LAUNCH();
  if (max_splits > 1) {
    merge_splits_kernel<<<dim3((unsigned)(batch * num_q_heads)), 64, 0, stream>>>(a);
    XV_CHECK_LAUNCH();
  }
  return 0;
}
