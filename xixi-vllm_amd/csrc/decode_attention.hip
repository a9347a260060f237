// Paged GQA decode attention for gfx950.
//
// Work unit: one wave64 workgroup per (sequence, kv head, KV split of `pps`
// 16-token pages); all G = Hq/Hkv query heads of the kv head are served by
// the one pass over the pages.  Per page:
//   K (HBM -> VGPR) is the A operand of S^T = K Q^T on v_mfma_f32_16x16x32_bf16:
//     lane = 16*g + i: row i = token i, MFMA step s contracts d-chunk 4s+g, so
//     the four lanes of a token read 64 contiguous bytes per load instruction.
//   Q^T is the B operand: column c = lane%16 holds query head c % G.
//   S^T lands as acc[r] = S[head c%G][token 4g+r]; the online softmax reduces
//   the 4 tokens in-lane and the 4 lane rows with two cross-row shuffles.
//   P (bf16) is then already the A operand of O = P V on
//   v_mfma_f32_16x16x16_bf16 (row = head, k = token 4g+j): no shuffle.
//   V (HBM -> VGPR -> LDS, rows padded to 288 B) is read back transposed with
//   ds_read_b64_tr_b16 as the B operand (k = token, column = d), 8 d-tiles.
//   O accumulates in the MFMA output layout: 8 tiles x 4 fp32 per lane.
// Splits of one (sequence, head) are merged by a second kernel through an
// fp32 workspace holding normalised partial outputs and their log2-sum-exp.
#include "xv_common.h"
#include "../../include/xv_kernels.h"
#include <math.h>
#include <stdlib.h>

namespace {

constexpr int kD = 128;
constexpr int kPage = 16;
constexpr int kLdsRow = 288;  // bytes per V row in LDS (256 + 32 pad: conflict-free transposed reads)

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4;

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
  for (int s = 0; s < 4; ++s) r.k[s] = load_vec8(kp + 32 * s);
#pragma unroll
  for (int s = 0; s < 4; ++s) r.v[s] = load_vec8(vp + 32 * s);
}

XV_INLINE bf16x8_t as_bf16x8(const Vec8& v) {
  bf16x8_t r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

struct SplitState {
  float m;      // running max (log2 domain) of head c%G, identical across lane rows
  float l;      // lane-local sum of p over this lane's tokens
  floatx4_t o[8];  // O tile n: rows 4g+r (head (4g+r)%G), column d = 16n + lane%16
};

template <int G>
XV_INLINE void process_page(SplitState& st, PageRegs& r, char* lds, const bf16x8_t (&qb)[4], int page_tok0,
                            int ctx, bool last, float scale_log2, int lane) {
  const int i = lane & 15, g = lane >> 4;
  // ---- V -> LDS (zero rows past the sequence end: they may hold NaN) ----
  if (last && page_tok0 + i >= ctx) {
#pragma unroll
    for (int s = 0; s < 4; ++s) r.v[s].w[0] = r.v[s].w[1] = r.v[s].w[2] = r.v[s].w[3] = 0u;
  }
#pragma unroll
  for (int s = 0; s < 4; ++s)
    *reinterpret_cast<uint4*>(lds + i * kLdsRow + 16 * (4 * s + g)) =
        make_uint4(r.v[s].w[0], r.v[s].w[1], r.v[s].w[2], r.v[s].w[3]);
  // ---- S^T = K Q^T ----
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(r.k[s]), qb[s], acc, 0, 0, 0);
  // ---- online softmax for head c%G over tokens 4g..4g+3 ----
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = (page_tok0 + 4 * g + j < ctx) ? acc[j] * scale_log2 : -INFINITY;
  float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(st.m, mx);
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
  st.m = m_new;
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(sc[j] - m_new);
  st.l = st.l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  short4_t pa;
#pragma unroll
  for (int j = 0; j < 4; ++j) pa[j] = (short)f32_to_bf16(p[j]);
  // rescale O rows: row 4g+rr holds head (4g+rr)%G, whose alpha sits in lane (row base)|head
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int hsrc = (4 * g + rr) % G;
    const float ar = __shfl(alpha, (lane & 48) | hsrc);
#pragma unroll
    for (int n = 0; n < 8; ++n) st.o[n][rr] *= ar;
  }
  // No barrier: the workgroup is one wave and a wave's LDS operations complete
  // in order, so the transposed reads below see the rows just written (the
  // compiler keeps the order: both access the same __shared__ array).  A
  // __syncthreads here would also wait for the prefetched page.
  // ---- O += P V, V^T tiles read transposed from LDS ----
  const int rowt = 4 * g + (i >> 2);
  const char* vb = lds + rowt * kLdsRow + 8 * (i & 3);
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    short4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb + 32 * n));
    st.o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vt, st.o[n], 0, 0, 0);
  }
}

template <int G, int NBUF, int WPB>
__global__ __launch_bounds__(64 * WPB) void paged_decode_kernel(DecodeArgs a, int units) {
  __shared__ __attribute__((aligned(16))) char lds_all[WPB][kPage * kLdsRow];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  char* lds = lds_all[wave];
  const int i = lane & 15, g = lane >> 4;
  // unit = split * (B*Hkv) + (b*Hkv + kvh): the waves of a workgroup are
  // independent units (no intra-workgroup synchronisation anywhere)
  const int unit = blockIdx.x * WPB + wave;
  if (unit >= units) return;
  const int bh_count = units / a.max_splits;
  const int split = unit / bh_count;
  const int bh = unit - split * bh_count;
  const int b = bh / a.hkv;
  const int kvh = bh - b * a.hkv;
  const int head0 = kvh * G;
  const int ctx = a.seqlens[b];
  const int npages = (ctx + kPage - 1) / kPage;
  const int nsplit = (npages + a.pps - 1) / a.pps;

  if (ctx <= 0) {
    // padding row: defined zero output, written once by split 0
    if (split == 0) {
      for (int e = lane; e < G * kD / 2; e += 64)
        reinterpret_cast<uint32_t*>(a.out + (int64_t)b * a.out_st + (int64_t)head0 * kD)[e] = 0u;
    }
    return;
  }
  if (split >= nsplit) return;
  const int p0 = split * a.pps;
  const int np = min(a.pps, npages - p0);

  // page ids of this split, one per lane, broadcast with readlane
  int pid = 0;
  if (lane < np) pid = a.bt[(int64_t)b * a.bt_stride + p0 + lane];

  bf16x8_t qb[4];
  {
    const bf16_t* qp = a.q + (int64_t)b * a.q_st + (int64_t)(head0 + (i % G)) * a.q_sh + 8 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s) qb[s] = as_bf16x8(load_vec8(qp + 32 * s));
  }

  SplitState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int n = 0; n < 8; ++n) st.o[n] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  // NBUF page buffers: NBUF-1 pages always in flight ahead of the one being
  // processed.  Prefetches are issued unconditionally (clamped to the split's
  // last page) so the outstanding-load count is the same on every path and
  // the compiler's vmcnt waits stay partial.
  PageRegs r[NBUF];
#pragma unroll
  for (int k = 0; k < NBUF - 1; ++k) load_page(r[k], a, __builtin_amdgcn_readlane(pid, min(k, np - 1)), kvh, i, g);
  for (int it = 0; it < np; it += NBUF) {
#pragma unroll
    for (int u = 0; u < NBUF; ++u) {
      load_page(r[(u + NBUF - 1) % NBUF], a, __builtin_amdgcn_readlane(pid, min(it + u + NBUF - 1, np - 1)), kvh, i, g);
      if (it + u < np)
        process_page<G>(st, r[u], lds, qb, (p0 + it + u) * kPage, ctx, p0 + it + u == npages - 1, a.scale_log2, lane);
    }
  }

  // total p-sum of head c%G, then fetch it for the heads of this lane's O rows
  float lsum = st.l;
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  // rows 4g+rr with 4g+rr < G hold distinct heads; the others are replicas
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int row = 4 * g + rr;
    const int hsrc = row % G;
    const float lh = __shfl(lsum, hsrc);
    const float mh = __shfl(st.m, hsrc);
    if (row >= G) continue;
    const float inv = 1.0f / lh;
    const int head = head0 + row;
    if (nsplit == 1) {
      bf16_t* o = a.out + (int64_t)b * a.out_st + (int64_t)head * kD + i;
#pragma unroll
      for (int n = 0; n < 8; ++n) o[16 * n] = (bf16_t)f32_to_bf16(st.o[n][rr] * inv);
    } else {
      const int64_t wrow = ((int64_t)b * a.hq + head) * a.max_splits + split;
      float* o = a.ws_o + wrow * kD + i;
#pragma unroll
      for (int n = 0; n < 8; ++n) o[16 * n] = st.o[n][rr] * inv;
      if (i == 0) a.ws_lse[wrow] = mh + __log2f(lh);
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

// Launch variants (page buffers x waves per workgroup); 0 is the default.
int decode_variant() {
  static int v = [] {
    const char* e = getenv("XV_DECODE_VARIANT");
    return e ? atoi(e) : 0;
  }();
  return v;
}

template <int G>
void launch_group(const DecodeArgs& a, int units, int variant, hipStream_t stream) {
  switch (variant) {
    case 1: paged_decode_kernel<G, 2, 1><<<units, 64, 0, stream>>>(a, units); break;
    case 2: paged_decode_kernel<G, 3, 1><<<units, 64, 0, stream>>>(a, units); break;
    case 3: paged_decode_kernel<G, 2, 4><<<(units + 3) / 4, 256, 0, stream>>>(a, units); break;
    default: paged_decode_kernel<G, 3, 4><<<(units + 3) / 4, 256, 0, stream>>>(a, units); break;
  }
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
  const int units = batch * num_kv_heads * max_splits;
  const int variant = decode_variant();
  switch (group) {
    case 1: launch_group<1>(a, units, variant, stream); break;
    case 2: launch_group<2>(a, units, variant, stream); break;
    case 4: launch_group<4>(a, units, variant, stream); break;
    default: launch_group<8>(a, units, variant, stream); break;
  }
  XV_CHECK_LAUNCH();
  if (max_splits > 1) {
    merge_splits_kernel<<<dim3((unsigned)(batch * num_q_heads)), 64, 0, stream>>>(a);
    XV_CHECK_LAUNCH();
  }
  return 0;
}
