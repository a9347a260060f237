// Varlen causal prefill attention (chunked prefill / cached prefix) for gfx950.
//
// Workgroup = 4 waves over one (sequence, query block, kv head): the waves
// serve min(G, 4) query heads of the kv group x 32 queries each, so every
// 64-key K/V tile staged in LDS is shared by all of them.  Per tile and wave
// (32 queries x 64 keys), all on v_mfma_f32_32x32x16_bf16:
//   S^T = K Q^T      2 key tiles x 8 d-steps; A = K rows from LDS
//                    (ds_read_b128), B = Q^T held in VGPRs.  Lane l holds query
//                    l%32 and keys 8j + 4(l/32) + r of each 32-key tile, so the
//                    online softmax is in-lane plus one cross-half exchange.
//   O^T += V^T P^T   4 d-tiles x 4 key-steps; A = V^T read transposed from LDS
//                    (ds_read_b64_tr_b16), B = P^T straight from the S^T
//                    registers: each key-step takes the lane's 8 consecutive
//                    accumulators, and V^T is read in the same key order.
// K and V tiles travel HBM -> LDS by LDS-DMA (buffer_load ... lds), whole
// 256-byte rows, into swizzled images (16-byte chunk c of row r at slot
// c ^ swz(r)) that keep the K and V^T reads free of bank conflicts on the
// 64-bank LDS.  The softmax runs in the exp2 domain with the scale folded
// into one FMA, masks only on tiles that cross the diagonal and rescales O
// lazily (only when a query's running max grew by more than 2^8).  Tiles
// are double buffered: the next tile's loads are in flight while the current
// one is computed; one barrier per tile.  Causal masking is bottom-right
// aligned (query i of q_len sees keys j <= k_len - q_len + i) and applied only
// on tiles that cross a wave's diagonal; tiles past it are skipped.  Rows past
// k_len read as zeros (bounded buffer resources), so unused cache slots never
// reach P.V.
#include "xv_common.h"
#include "xv_kernels.h"
#include <math.h>
#include <type_traits>

namespace {

constexpr int kD = 128;
constexpr int kKeys = 64;                  // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = kKeys * kD * 2;      // bytes of one K (or V) tile
constexpr int kBuf = 2 * kTile;            // K then V
constexpr float kLazy = 8.0f;
const xv_bf16x2 kOnes = {(__bf16)1.0f, (__bf16)1.0f};

typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

struct PrefillArgs {
  const bf16_t* q; int64_t q_st, q_sh;
  const bf16_t* k; const bf16_t* v; int64_t kv_st, kv_sh;
  const bf16_t* kc; const bf16_t* vc; int64_t page_stride, tok_stride, head_stride;
  const int32_t* bt; int64_t bt_stride; int block_size;
  const int32_t* cu_q; const int32_t* cu_k;
  bf16_t* out; int64_t out_st;
  int hq, hkv, qblocks, batch;
  float scale_log2;
};

XV_INLINE int swz_k(int r) { return r & 15; }
// V^T reads: a 32-lane group reads 4 rows x 4 chunks (one 64-byte d-tile):
// chunk 4n + j of row r sits at slot 4(n ^ (r & 3)) + j, 16 distinct slots.
XV_INLINE int swz_v(int r) { return (r & 3) << 2; }

XV_INLINE __amdgpu_buffer_rsrc_t rsrc(const bf16_t* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* q = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Wave w moves keys key0+16w .. +15 of the tile (one cache page when paged):
// 4 LDS-DMA instructions for K and/or 4 for V, each 4 whole rows.
template <bool PAGED, bool DO_K, bool DO_V>
XV_INLINE void load_rows(char* buf, const PrefillArgs& a, int b, int kvh, int key0, int k0, int k_len,
                         int64_t page_off, int wave, int lane) {
  const int j0 = key0 + 16 * wave;
  const int valid = min(16, k_len - j0);
  const bf16_t *kb, *vb;
  int64_t rs;  // row stride (elements)
  if (PAGED) {
    const int64_t off = page_off + (int64_t)kvh * a.head_stride;
    kb = a.kc + off; vb = a.vc + off; rs = a.tok_stride;
  } else {
    const int64_t off = (int64_t)(k0 + j0) * a.kv_st + (int64_t)kvh * a.kv_sh;
    kb = a.k + off; vb = a.v + off; rs = a.kv_st;
  }
  const uint32_t bytes = valid > 0 ? (uint32_t)(((int64_t)(valid - 1) * rs + kD) * 2) : 0u;
  const __amdgpu_buffer_rsrc_t rk = rsrc(kb, bytes), rv = rsrc(vb, bytes);
  const int slot = lane & 15;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int r = 4 * s + (lane >> 4);  // row within the wave's 16
    const int R = 16 * wave + r;        // row within the tile
    const int vo_k = (int)(r * rs * 2) + ((slot ^ swz_k(R)) << 4);
    const int vo_v = (int)(r * rs * 2) + ((slot ^ swz_v(R)) << 4);
    if (DO_K)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(buf + (16 * wave + 4 * s) * 256), 16, vo_k, 0, 0, 0);
    if (DO_V)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(buf + kTile + (16 * wave + 4 * s) * 256), 16, vo_v,
                                               0, 0, 0);
  }
}

// Per-lane LDS addresses, fixed for the whole kernel; tile, buffer and row
// offsets go into the instructions' immediate offsets.
//   K A-operand of d-step s (any key tile mt): row l%32 (+32mt), d-chunk 2s + l/32.
//   V^T A-operand of d-tile n: rows 4(l/32) + (l%16)/4 (+16ks + 8half),
//   chunk 4n + 2((l/16)%2) + (l%4)/2, 8-byte half l%2 -- swizzled slot
//   4(n ^ row%4) + chunk%4.
struct LdsAddr {
  uint32_t k[8];
  uint32_t v[4];
};
XV_INLINE LdsAddr lds_addr(const char* lds, int lane) {
  LdsAddr a;
  const uint32_t base = (uint32_t)reinterpret_cast<uintptr_t>(lds);
  const int l32 = lane & 31, h = lane >> 5, q = lane >> 4, i = lane & 15;
#pragma unroll
  for (int s = 0; s < 8; ++s) a.k[s] = base + l32 * 256 + (((2 * s + h) ^ swz_k(l32)) << 4);
  const int row = 4 * h + (i >> 2);
  const int cl = 2 * (q & 1) + ((i & 3) >> 1);
#pragma unroll
  for (int n = 0; n < 4; ++n) a.v[n] = base + kTile + row * 256 + (((4 * n + cl) ^ swz_v(row)) << 4) + 8 * (i & 1);
  return a;
}

// All 16 K A-operands of a tile (kf[8mt + s]) in two asm blocks: the reads
// are issued together and only the first eight are waited for; k_wait_rest
// completes the other eight (passed through it, so nothing reads them
// earlier).
template <int PAR>
XV_INLINE void read_k16(bf16x8_t (&kf)[16], const LdsAddr& ad) {
  __asm__ __volatile__(
      "ds_read_b128 %0, %16 offset:%24\n\t"
      "ds_read_b128 %1, %17 offset:%24\n\t"
      "ds_read_b128 %2, %18 offset:%24\n\t"
      "ds_read_b128 %3, %19 offset:%24\n\t"
      "ds_read_b128 %4, %20 offset:%24\n\t"
      "ds_read_b128 %5, %21 offset:%24\n\t"
      "ds_read_b128 %6, %22 offset:%24\n\t"
      "ds_read_b128 %7, %23 offset:%24\n\t"
      "ds_read_b128 %8, %16 offset:%25\n\t"
      "ds_read_b128 %9, %17 offset:%25\n\t"
      "ds_read_b128 %10, %18 offset:%25\n\t"
      "ds_read_b128 %11, %19 offset:%25\n\t"
      "ds_read_b128 %12, %20 offset:%25\n\t"
      "ds_read_b128 %13, %21 offset:%25\n\t"
      "ds_read_b128 %14, %22 offset:%25\n\t"
      "ds_read_b128 %15, %23 offset:%25\n\t"
      "s_waitcnt lgkmcnt(8)"
      : "=&v"(kf[0]), "=&v"(kf[1]), "=&v"(kf[2]), "=&v"(kf[3]), "=&v"(kf[4]), "=&v"(kf[5]), "=&v"(kf[6]),
        "=&v"(kf[7]), "=&v"(kf[8]), "=&v"(kf[9]), "=&v"(kf[10]), "=&v"(kf[11]), "=&v"(kf[12]), "=&v"(kf[13]),
        "=&v"(kf[14]), "=&v"(kf[15])
      : "v"(ad.k[0]), "v"(ad.k[1]), "v"(ad.k[2]), "v"(ad.k[3]), "v"(ad.k[4]), "v"(ad.k[5]), "v"(ad.k[6]),
        "v"(ad.k[7]), "n"(PAR * kBuf), "n"(PAR * kBuf + 32 * 256)
      : "memory");
}
XV_INLINE void k_wait_rest(bf16x8_t (&kf)[16]) {
  __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                       : "+v"(kf[8]), "+v"(kf[9]), "+v"(kf[10]), "+v"(kf[11]), "+v"(kf[12]), "+v"(kf[13]),
                         "+v"(kf[14]), "+v"(kf[15])
                       :
                       : "memory");
}

// V^T A-operands of key-steps KS0, KS0+1 for all four d-tiles: lane l holds
// d = 32n + l%32 and keys 16ks + 4(l/32) + {0..3} and +8 (ks = 2mt + kk), two
// transposed reads of 4 rows each; t[4n + 2(ks-KS0) + half].  The 16 reads are
// issued together and the first eight (d-tiles 0, 1) waited for;
// vt_wait_rest completes the others.
typedef short short4_t __attribute__((ext_vector_type(4)));
template <int PAR, int KS0>
XV_INLINE void read_vt_ks2(short4_t (&t)[16], const LdsAddr& ad) {
  constexpr int o0 = PAR * kBuf + (16 * KS0) * 256;
  __asm__ __volatile__(
      "ds_read_b64_tr_b16 %0, %16 offset:%20\n\t"
      "ds_read_b64_tr_b16 %1, %16 offset:%21\n\t"
      "ds_read_b64_tr_b16 %2, %16 offset:%22\n\t"
      "ds_read_b64_tr_b16 %3, %16 offset:%23\n\t"
      "ds_read_b64_tr_b16 %4, %17 offset:%20\n\t"
      "ds_read_b64_tr_b16 %5, %17 offset:%21\n\t"
      "ds_read_b64_tr_b16 %6, %17 offset:%22\n\t"
      "ds_read_b64_tr_b16 %7, %17 offset:%23\n\t"
      "ds_read_b64_tr_b16 %8, %18 offset:%20\n\t"
      "ds_read_b64_tr_b16 %9, %18 offset:%21\n\t"
      "ds_read_b64_tr_b16 %10, %18 offset:%22\n\t"
      "ds_read_b64_tr_b16 %11, %18 offset:%23\n\t"
      "ds_read_b64_tr_b16 %12, %19 offset:%20\n\t"
      "ds_read_b64_tr_b16 %13, %19 offset:%21\n\t"
      "ds_read_b64_tr_b16 %14, %19 offset:%22\n\t"
      "ds_read_b64_tr_b16 %15, %19 offset:%23\n\t"
      "s_waitcnt lgkmcnt(8)"
      : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7]),
        "=&v"(t[8]), "=&v"(t[9]), "=&v"(t[10]), "=&v"(t[11]), "=&v"(t[12]), "=&v"(t[13]), "=&v"(t[14]),
        "=&v"(t[15])
      : "v"(ad.v[0]), "v"(ad.v[1]), "v"(ad.v[2]), "v"(ad.v[3]), "n"(o0), "n"(o0 + 8 * 256), "n"(o0 + 16 * 256),
        "n"(o0 + 24 * 256)
      : "memory");
}
XV_INLINE void vt_wait_rest(short4_t (&t)[16]) {
  __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                       : "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]), "+v"(t[12]), "+v"(t[13]), "+v"(t[14]),
                         "+v"(t[15])
                       :
                       : "memory");
}
// A-operand of d-tile n, key-step KS0 + j from read_vt_ks2's registers
// (a whole-vector shuffle of the two 64-bit halves: composing it from 16-bit
// elements leaves a no-op bit-field insert per register in front of the MFMA)
typedef short short8_t __attribute__((ext_vector_type(8)));
XV_INLINE bf16x8_t vt_operand(const short4_t (&t)[16], int n, int j) {
  const short8_t r = __builtin_shufflevector(t[4 * n + 2 * j], t[4 * n + 2 * j + 1], 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, r);
}

// Sequence of dispatch slot j: sequences in descending causal work
// q_len * (k_len - q_len) + q_len * (q_len + 1) / 2 (ties: lower index
// first), so the costliest sequences' blocks are dispatched first and the
// cheapest ones finish the grid.  Each sequence's blocks stay together in the
// dispatch order (they share K/V tiles in L2).  Batches above 64 keep their
// own order.
XV_INLINE int seq_by_work(const int* cu_q, const int* cu_k, int batch, int j) {
  if (batch > 64) return j;
  const int lane = threadIdx.x & 63;
  int64_t w = -1;
  if (lane < batch) {
    const int ql = cu_q[lane + 1] - cu_q[lane], kl = cu_k[lane + 1] - cu_k[lane];
    w = (int64_t)ql * (kl - ql) + (int64_t)ql * (ql + 1) / 2;
  }
  int pos = 0;
  for (int t = 0; t < batch; ++t) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)w, t);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)w >> 32), t);
    const int64_t wt = (int64_t)(((uint64_t)hi << 32) | lo);
    pos += (wt > w || (wt == w && t < lane)) ? 1 : 0;
  }
  const uint64_t m = __ballot(lane < batch && pos == j);
  return __builtin_amdgcn_readfirstlane(__builtin_ctzll(m));
}

template <int G, bool PAGED>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(PrefillArgs a) {
  constexpr int GW = G < 4 ? G : 4;   // query heads per workgroup
  constexpr int QS = 4 / GW;          // 32-query sub-blocks per workgroup
  constexpr int kBlockQ = 32 * QS;
  __shared__ __attribute__((aligned(16))) char lds[2 * kBuf];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps per-wave values scalar
  const int l32 = lane & 31, h = lane >> 5;
  // XCD-aware order: workgroups go round-robin to the 8 XCDs, so with the head
  // slot fastest every XCD serves the same kv head(s) and keeps their K/V tiles
  // in its own L2; each head carries the same work, which balances the XCDs.
  const int hsel = blockIdx.x, rank = blockIdx.y;
  const int b = seq_by_work(a.cu_q, a.cu_k, a.batch, blockIdx.z);
  // group 8: two slots per kv head (query heads 0-3 and 4-7), slot = half * Hkv
  // + kvh, so both halves of a kv head land on the same XCD
  const int kvh = G == 8 ? hsel % a.hkv : hsel;
  const int head = G == 8 ? kvh * 8 + (hsel / a.hkv) * 4 + wave : kvh * G + wave % GW;
  const int q0 = a.cu_q[b], q_len = a.cu_q[b + 1] - q0;
  const int k0 = a.cu_k[b], k_len = a.cu_k[b + 1] - k0;
  // rank from the sequence's own end: the last (longest) block of the causal
  // triangle is dispatched first, then the next-to-last, ...
  const int qb0 = ((q_len + kBlockQ - 1) / kBlockQ - 1 - rank) * kBlockQ;
  if (qb0 < 0) return;
  const int shift = k_len - q_len;  // bottom-right alignment
  const int qw0 = qb0 + (wave / GW) * 32;  // the wave's first query
  const int my_q = qw0 + l32;
  const int kv_end = min(k_len, shift + min(qb0 + kBlockQ, q_len));  // keys the block needs
  const int ntiles = (kv_end + kKeys - 1) / kKeys;
  const bool active = qw0 < q_len;
  const int wave_kend = active ? min(k_len, shift + min(qw0 + 32, q_len)) : 0;  // keys any query of the wave sees
  const int wave_kfull = shift + qw0 + 1;  // keys every query of the wave sees
  const int my_kend = shift + my_q + 1;

  // Q^T B-operands: lane holds query my_q, d = 16s + 8(l/32) .. +7
  bf16x8_t qb[8];
  {
    const int qi = min(my_q, q_len - 1);
    const bf16_t* qp = a.q + (int64_t)(q0 + qi) * a.q_st + (int64_t)head * a.q_sh + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const Vec8 v = load_vec8(qp + 16 * s);
      __builtin_memcpy(&qb[s], &v, 16);
    }
  }
  floatx16_t o[4];
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[n][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // element offset of the 16 keys j .. j + 15 (a 16-aligned run inside one
  // cache block of block_size tokens): block bt[j / BS], token j % BS
  auto page_of = [&](int t) -> int64_t {
    if (!PAGED) return 0;
    const int j = t * kKeys + 16 * wave;
    if (j >= k_len) return 0;
    const int blk = j / a.block_size;
    const int64_t page = __builtin_amdgcn_readfirstlane(a.bt[(int64_t)b * a.bt_stride + blk]);
    return page * a.page_stride + (int64_t)(j - blk * a.block_size) * a.tok_stride;
  };
  const LdsAddr ad = lds_addr(lds, lane);
  // S^T of one tile from K buffer PAR
  auto s_tile = [&](auto par_tag, floatx16_t (&s)[2]) {
    constexpr int PAR = decltype(par_tag)::value;
    bf16x8_t kf[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) s[0][r] = s[1][r] = 0.f;
    read_k16<PAR>(kf, ad);
#pragma unroll
    for (int u = 0; u < 8; ++u) s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[u], qb[u], s[0], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);  // the wait below stays behind these MFMAs
    k_wait_rest(kf);
#pragma unroll
    for (int u = 0; u < 8; ++u) s[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[8 + u], qb[u], s[1], 0, 0, 0);
  };
  // online softmax of tile t's scores s -> P (bf16), O and l rescaled as needed
  auto softmax = [&](int t, floatx16_t (&s)[2], bf16x8_t (&pb)[2][2]) {
    const int key0 = t * kKeys;
    // (on raw scores: scale > 0 keeps the order; p = exp2(s*scale - m*scale))
    if (key0 + kKeys > wave_kfull) {  // the tile crosses some query's diagonal
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
          s[mt][r] = key < my_kend ? s[mt][r] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mt][r]);
    mx = xor32_max(mx) * a.scale_log2;  // running max in the exp2 domain
    // lazy rescale: the max used for exp2 moves only when it grew by more
    // than kLazy (p <= 2^kLazy meanwhile; exact after the final 1/l)
    if (mx > m_run + kLazy) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - mx);  // 0 on the first tile
      m_run = mx;
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < 4; ++n) o[n] *= alpha;
    }
    const float nm = m_run == -INFINITY ? 0.f : -m_run;  // fully masked so far: p = 0
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mt][8 * kk + 2 * e], a.scale_log2, nm));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mt][8 * kk + 2 * e + 1], a.scale_log2, nm));
          w[e] = pack_bf16x2(p0, p1);
          // the row sum takes the bf16 values P.V multiplies
          l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(xv_bf16x2, w[e]), kOnes, l_run, false);
        }
        __builtin_memcpy(&pb[mt][kk], w, 16);
      }
  };
  // O^T += V^T P^T from V buffer PAR
  auto pv_tile = [&](auto par_tag, const bf16x8_t (&pb)[2][2]) {
    constexpr int PAR = decltype(par_tag)::value;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {  // key-steps 2k2, 2k2+1 (= key tile mt = k2)
      short4_t vt[16];
      if (k2 == 0) read_vt_ks2<PAR, 0>(vt, ad); else read_vt_ks2<PAR, 2>(vt, ad);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int n = 0; n < 2; ++n)
          o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt_operand(vt, n, j), pb[k2][j], o[n], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      vt_wait_rest(vt);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int n = 2; n < 4; ++n)
          o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt_operand(vt, n, j), pb[k2][j], o[n], 0, 0, 0);
    }
  };

  // Software pipeline, one tile deep: iteration t computes S(t+1) from K
  // buffer (t+1)&1 while the softmax of tile t (scores from the previous
  // iteration) runs on the VALU, then O += P(t) V(t) from V buffer t&1.  K
  // therefore runs a tile ahead of V: iteration t loads K(t+2) into the K
  // buffer S(t) used and V(t+1) into the V buffer P(t-1) V(t-1) used, both
  // freed by the barrier at its top.
  int64_t pv_page = ntiles > 1 ? page_of(1) : 0, pk_page = ntiles > 2 ? page_of(2) : 0;
  if (ntiles > 0) load_rows<PAGED, true, true>(lds, a, b, kvh, 0, k0, k_len, page_of(0), wave, lane);
  if (ntiles > 1) load_rows<PAGED, true, false>(lds + kBuf, a, b, kvh, kKeys, k0, k_len, pv_page, wave, lane);
  __asm__ __volatile__("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // scores of even tiles in s_even, of odd tiles in s_odd (no copies)
  floatx16_t s_even[2], s_odd[2];
  if (ntiles > 0 && 0 < wave_kend) s_tile(std::integral_constant<int, 0>{}, s_even);
  auto iter = [&](auto par_tag, int t, floatx16_t (&sc)[2], floatx16_t (&sn)[2]) {
    constexpr int PAR = decltype(par_tag)::value;  // t & 1
    __asm__ __volatile__("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // K(t+1) and V(t) are in LDS; every wave is done with iteration t-1
    if (t + 2 < ntiles) load_rows<PAGED, true, false>(lds + PAR * kBuf, a, b, kvh, (t + 2) * kKeys, k0, k_len, pk_page, wave, lane);
    if (t + 1 < ntiles) load_rows<PAGED, false, true>(lds + (1 - PAR) * kBuf, a, b, kvh, (t + 1) * kKeys, k0, k_len, pv_page, wave, lane);
    pv_page = pk_page;
    if (t + 3 < ntiles) pk_page = page_of(t + 3);
    if (t + 1 < ntiles && (t + 1) * kKeys < wave_kend) s_tile(std::integral_constant<int, 1 - PAR>{}, sn);
    if (t * kKeys < wave_kend) {
      bf16x8_t pb[2][2];
      // the softmax is the serial link between MFMA phases: at raised issue
      // priority it runs ahead of the other wave on this SIMD, whose MFMAs
      // fill the gaps (measured +3-5 % over equal priority)
      __builtin_amdgcn_s_setprio(1);
      softmax(t, sc, pb);
      __builtin_amdgcn_s_setprio(0);
      pv_tile(par_tag, pb);
    }
  };
  for (int t = 0; t < ntiles; t += 2) {
    iter(std::integral_constant<int, 0>{}, t, s_even, s_odd);
    if (t + 1 < ntiles) iter(std::integral_constant<int, 1>{}, t + 1, s_odd, s_even);
  }
  // ---- normalise and write: lane holds O[my_q][32n + 8j + 4(l/32) + r] ----
  const float lsum = xor32_sum(l_run);
  if (!active || my_q >= q_len) return;
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  bf16_t* op = a.out + (int64_t)(q0 + my_q) * a.out_st + (int64_t)head * kD + 4 * h;
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint2 w = make_uint2(pack_bf16x2(o[n][4 * j] * inv, o[n][4 * j + 1] * inv),
                                 pack_bf16x2(o[n][4 * j + 2] * inv, o[n][4 * j + 3] * inv));
      *reinterpret_cast<uint2*>(op + 32 * n + 8 * j) = w;
    }
}

template <int G>
void launch(const PrefillArgs& a, dim3 grid, hipStream_t stream) {
  if (a.bt) prefill_kernel<G, true><<<grid, kThreads, 0, stream>>>(a);
  else prefill_kernel<G, false><<<grid, kThreads, 0, stream>>>(a);
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
    if (!k_cache || !v_cache || block_size <= 0 || block_size % 16) return (int)hipErrorInvalidValue;
    // K/V rows move by 16-byte LDS-DMA
    if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15 || (page_stride | tok_stride | head_stride) & 7)
      return (int)hipErrorInvalidValue;
  } else {
    if (!k || !v) return (int)hipErrorInvalidValue;
    if (((uintptr_t)k | (uintptr_t)v) & 15 || (kv_stride_tok | kv_stride_head) & 7) return (int)hipErrorInvalidValue;
  }
  // q rows are read as 16-byte vectors, out is written as 8-byte pieces
  if ((uintptr_t)q & 15 || (q_stride_tok | q_stride_head) & 7 || (uintptr_t)out & 7 || out_stride_tok & 3)
    return (int)hipErrorInvalidValue;
  if (batch == 0 || max_seqlen_q == 0) return 0;
  PrefillArgs a;
  a.q = (const bf16_t*)q; a.q_st = q_stride_tok; a.q_sh = q_stride_head;
  a.k = (const bf16_t*)k; a.v = (const bf16_t*)v; a.kv_st = kv_stride_tok; a.kv_sh = kv_stride_head;
  a.kc = (const bf16_t*)k_cache; a.vc = (const bf16_t*)v_cache;
  a.page_stride = page_stride; a.tok_stride = tok_stride; a.head_stride = head_stride;
  a.bt = block_tables; a.bt_stride = bt_stride; a.block_size = block_size;
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k;
  a.out = (bf16_t*)out; a.out_st = out_stride_tok;
  a.hq = num_q_heads; a.hkv = num_kv_heads; a.batch = batch;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int gw = group < 4 ? group : 4;
  const int block_q = 32 * (4 / gw);
  a.qblocks = (max_seqlen_q + block_q - 1) / block_q;
  if (a.qblocks > 65535 || batch > 65535) return (int)hipErrorInvalidValue;  // grid y / z limits
  const dim3 grid((unsigned)(num_kv_heads * (group == 8 ? 2 : 1)), (unsigned)a.qblocks, (unsigned)batch);
  switch (group) {
    case 1: launch<1>(a, grid, stream); break;
    case 2: launch<2>(a, grid, stream); break;
    case 4: launch<4>(a, grid, stream); break;
    default: launch<8>(a, grid, stream); break;
  }
  XV_CHECK_LAUNCH();
  return 0;
}
