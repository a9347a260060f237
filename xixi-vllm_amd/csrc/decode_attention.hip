// Paged GQA decode attention for gfx950.
//
// Work split ("stream-K" over pages): the (sequence, kv head, page) space is
// flattened in that order and cut into equal contiguous ranges of L pages,
// one per resident single-wave workgroup, so every wave streams the same
// number of pages and the whole grid is resident at once (no dispatch rounds,
// no tail of late units).  A range may cover several (sequence, kv head)
// segments; a segment cut by range boundaries yields one partial per wave,
// merged by a second kernel through a workspace (normalised partial output
// in bf16 + fp32 log2-sum-exp).  The merge weights and sums in fp32.  A segment inside one range is written directly.
// All G = Hq/Hkv query heads of a kv head are served by one pass.  Per page:
//   K and V go HBM -> LDS by LDS-DMA, whole 256-byte rows per instruction,
//   into a swizzled image (conflict-free reads below).
//   K (LDS -> VGPR) is the A operand of S^T = K Q^T on v_mfma_f32_16x16x32_bf16:
//     lane = 16*g + i: row i = token i, MFMA step s contracts d-chunk 4s+g.
//   Q^T is the B operand: column c = lane%16 holds query head c % G.
//   S^T lands as acc[r] = S[head c%G][token 4g+r]; the online softmax reduces
//   the 4 tokens in-lane and the 4 lane rows with two cross-row shuffles.
//   P (bf16) is then already the A operand of O = P V on
//   v_mfma_f32_16x16x16_bf16 (row = head, k = token 4g+j): no shuffle.
//   V is read from LDS transposed with ds_read_b64_tr_b16 as the B operand
//   (k = token, column = d), 8 d-tiles.
//   O accumulates in the MFMA output layout: 8 tiles x 4 fp32 per lane.
#include "xv_common.h"
#include "xv_kernels.h"
#include <math.h>
#include <stdlib.h>
#include <mutex>
#include <type_traits>

namespace {

constexpr int kD = 128;
constexpr int kPage = 16;
constexpr int kVPageBytes = 4096;  // one page's V rows of one kv head in LDS
#ifndef XV_DECODE_WAVES_PER_CU
#define XV_DECODE_WAVES_PER_CU 4  // one wave per SIMD: no oldest-first starvation between waves
#endif

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
  bf16_t* ws_ob;  // the partial rows, bf16, kD per row (in ws_o's region)
  int* ws_nparts;  // partials per (sequence, kv head), written by the wave holding the segment's last page
  int batch, hq, hkv, group;
  int nsub;       // 16-token pages per cache block (block_size / 16)
  int lmin;       // minimum pages per wave range for any table of the launch's width (host bound)
  int max_parts;  // partial slots per (sequence, head) in the workspace
  int nwaves;     // workgroups of the main kernel (the range count)
  float scale_log2;
  float v_scale;  // fp8 pages: the V dequantisation scale, applied to the output (1 for bf16 pages)
  // Cascade (shared-prefix) decode; pre_tokens == nullptr otherwise.  Row b's
  // first pre_tokens[b] tokens were attended by the prefix pass, whose
  // partials (normalised output, log2-sum-exp) sit at pre_o / pre_lse slot
  // (chunk * batch + b) * hq + h; bt and seqlens then describe the
  // suffix only, and every suffix segment of such a row leaves a partial.
  const int32_t* pre_tokens;
  int pre_chunk_pages;  // prefix pages per prefix-pass chunk
  const bf16_t* pre_o; const float* pre_lse;  // prefix outputs in bf16 (halves the pass's store traffic)
};

// Both K and V of a page travel HBM -> LDS by LDS-DMA (buffer_load ... lds:
// lane l's 16 bytes land at base + 16*l), so no page data passes through
// VGPRs before it is needed and the compiler never has to wait for a page
// load: the only wait on page data is the explicit vmcnt in process_page.
//
// LDS image of one page of one kv head (4 KB for K, 4 KB for V): token t's
// 256-byte row at t*256, its 16-byte chunk c in slot c ^ swz(t).  The swizzle
// makes the 16 tokens of a K read (same chunk) and the 8 tokens of each half
// of a transposed V read land in distinct banks.
// Load instruction s (0..3) moves tokens 4s..4s+3 as four whole 256-byte rows
// (lane l: token 4s + l/16, slot l%16, i.e. chunk (l%16) ^ swz(t)), so every
// instruction reads full rows whatever the page layout ([BS][Hkv][D] as the
// reference pool, or [Hkv][BS][D]).  The page base is wave uniform (a scalar
// buffer resource per page) covering only the page's valid rows: rows past
// the sequence end read as zeros, so garbage (even NaN) in unused cache slots
// never reaches P.V.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kPageLds = 2 * kVPageBytes;  // K then V

constexpr int kNontemporal = 2;  // buffer instruction cache-policy bits: nt

XV_INLINE int swz(int t) { return ((t & 7) << 1) | (t >> 3); }
// fp8 page image: token r's 128-byte row at r * 128, 16-byte piece p in slot
// p ^ swz8(r), so the 16 tokens of a K read (same piece) and the V conversion
// reads hit distinct banks.
XV_INLINE int swz8(int r) { return (r & 7) ^ (r >> 3); }
constexpr int kF8Half = 2048;  // V rows of an fp8 page image start here

// base and bytes are wave uniform: readfirstlane lets the compiler keep the
// resource in SGPRs (otherwise it emits a per-lane "waterfall" loop).
XV_INLINE __amdgpu_buffer_rsrc_t page_rsrc(const bf16_t* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* q = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Per-lane offsets, fixed for the whole kernel.
struct LaneOffsets {
  int g[4];  // global byte offset of load instruction s within a page
  int g8[2];  // fp8 pages: global byte offset of load instruction s (8 rows of 128 bytes each)
  uint32_t k8[2];  // fp8 pages: LDS offsets of this lane's two K pieces (its S^T A operands)
  uint32_t v8[2];  // fp8 pages: LDS offsets of the two pieces of a tensor this lane widens to bf16 (widen_unit_f8)
  uint32_t vt8[4];  // fp8 pages: LDS offsets of this lane's transposed byte reads of V (O tiles 2m, 2m+1)
  uint32_t k[4];  // LDS byte offset of this lane's K A-operand chunk for MFMA step s
  uint32_t v[8];  // LDS byte offset (V half) of this lane's transposed read for O tile n
};

XV_INLINE LaneOffsets lane_offsets(int64_t tok_stride, int lane) {
  LaneOffsets o;
  const int i = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int t = 4 * s + g;
    o.g[s] = (int)(t * tok_stride * 2) + ((i ^ swz(t)) << 4);
    // K A operand of step s: row = token i, d-chunk 4s + g
    o.k[s] = (uint32_t)(i * 256 + (((4 * s + g) ^ swz(i)) << 4));
  }
  // fp8 rows (tok_stride in bytes): instruction s moves tokens 8s .. 8s+7;
  // lane l fills slot l%8 of token r = 8s + l/8 with piece (l%8) ^ swz8(r)
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int r = 8 * s + (lane >> 3);
    o.g8[s] = (int)(r * tok_stride) + (((lane & 7) ^ swz8(r)) << 4);
  }
  // K: lane (g, i) takes token i's values 32g .. 32g+31 (pieces 2g, 2g+1):
  // MFMA step s contracts d-chunk 4g + s (q is read in the same order).
  // Widening a tensor to bf16: lane l converts token l/4's values 32(l%4) .. +31.
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    o.k8[h] = (uint32_t)(i * 128 + (((2 * g + h) ^ swz8(i)) << 4));
    const int r = lane >> 2, p = 2 * (lane & 3) + h;
    o.v8[h] = (uint32_t)(kF8Half + r * 128 + ((p ^ swz8(r)) << 4));
  }
  // fp8 V read transposed by bytes (ds_read_b64_tr_b8: in each 16-lane group
  // output lane i's byte j is byte i % 8 of the 8 bytes input lane 2j + i / 8
  // addresses): input lane (g, L) addresses token 4g + (j % 4), j = L / 2, of
  // 16-byte piece 2m + j / 4, half L % 2; output lane (g, i) then holds tokens
  // 4g .. 4g+3 of columns 16(2m) + i (bytes 0..3) and 16(2m+1) + i (bytes
  // 4..7): the B operands of O tiles 2m and 2m + 1.
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int j = (lane & 15) >> 1, r = 4 * g + (j & 3), piece = 2 * m + (j >> 2);
    o.vt8[m] = (uint32_t)(kF8Half + r * 128 + ((piece ^ swz8(r)) << 4) + 8 * (lane & 1));
  }
  // V B operand of tile n: lane (g, i) supplies token 4g + i/4, columns
  // 16n + 4(i%4) .. +3 = chunk 2n + (i%4)/2, bytes 8*(i%2) of it
  const int t = 4 * g + (i >> 2);
#pragma unroll
  for (int n = 0; n < 8; ++n)
    o.v[n] = (uint32_t)(kVPageBytes + t * 256 + (((2 * n + ((i & 3) >> 1)) ^ swz(t)) << 4) + 8 * (i & 1));
  return o;
}

// One 16-token page: tokens 16*sub .. 16*sub + 15 of cache block `page`.
// (A is any argument record with the cache fields kc, vc and strides.)
template <typename A>
XV_INLINE void issue_page(char* buf, const A& a, int page, int sub, int kvh, int valid_rows,
                          const LaneOffsets& lo) {
  const int64_t base =
      (int64_t)page * a.page_stride + (int64_t)sub * kPage * a.tok_stride + (int64_t)kvh * a.head_stride;
  const uint32_t bytes = (uint32_t)(((int64_t)(valid_rows - 1) * a.tok_stride + kD) * 2);
  const __amdgpu_buffer_rsrc_t rk = page_rsrc(a.kc + base, bytes);
  const __amdgpu_buffer_rsrc_t rv = page_rsrc(a.vc + base, bytes);
  // KV is streamed once per call: nontemporal (cache policy nt), which on
  // this part raises the streaming rate of the page pattern by ~12 %
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(buf + 1024 * s), 16, lo.g[s], 0, 0, kNontemporal);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(buf + kVPageBytes + 1024 * s), 16, lo.g[s], 0, 0,
                                             kNontemporal);
  }
}

// The same page with fp8 (e4m3fn) K and V, strides in bytes: rows of 128
// bytes, two LDS-DMA instructions of eight whole rows per tensor, K at buf
// and V at buf + kF8PageBytes / 2 (token r's row at r * 128).  Rows past the
// sequence end read as zeros, as above.
template <typename A>
XV_INLINE void issue_page_f8(char* buf, const A& a, int page, int sub, int kvh, int valid_rows,
                             const LaneOffsets& lo) {
  const int64_t base =
      (int64_t)page * a.page_stride + (int64_t)sub * kPage * a.tok_stride + (int64_t)kvh * a.head_stride;
  const uint32_t bytes = (uint32_t)((int64_t)(valid_rows - 1) * a.tok_stride + kD);
  const __amdgpu_buffer_rsrc_t rk =
      page_rsrc(reinterpret_cast<const bf16_t*>(reinterpret_cast<const char*>(a.kc) + base), bytes);
  const __amdgpu_buffer_rsrc_t rv =
      page_rsrc(reinterpret_cast<const bf16_t*>(reinterpret_cast<const char*>(a.vc) + base), bytes);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(buf + 1024 * s), 16, lo.g8[s], 0, 0, kNontemporal);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(buf + kF8Half + 1024 * s), 16, lo.g8[s], 0, 0,
                                             kNontemporal);
  }
}

// 16 fp8 (e4m3fn) values -> 16 bf16 (exact: every e4m3fn value is a bf16).
XV_INLINE void fp8x16_to_bf16(const u32x4_t& w, uint32_t (&o)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], true);
    o[2 * k] = pack_bf16x2(lo[0], lo[1]);
    o[2 * k + 1] = pack_bf16x2(hi[0], hi[1]);
  }
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

constexpr float kLazy = 8.0f;

// Value of head (4g+RR)%G -- the head of O row 4g+RR -- for a per-head value
// that is equal across the four 16-lane rows: lane (4g+RR)%G of this row.
// G == 16 is the cascade prefix pass: 16 distinct query rows per tile, so
// row 4g+RR's value sits in lane 4g+RR of the 16-lane row, which depends on g.
template <int G, int RR>
XV_INLINE float head_of_row(float x, int g) {
  if constexpr (G == 16) return __shfl(x, 20 * g + RR);
  else if constexpr (G == 8) return (g & 1) ? row_bcast<(4 + RR) % 8>(x) : row_bcast<RR % 8>(x);
  else return row_bcast<RR % G>(x);
}

// O row 4g+RR *= alpha of its head.
template <int G, int RR>
XV_INLINE void rescale_row(SplitState& st, float alpha, int g) {
  const float ar = head_of_row<G, RR>(alpha, g);
#pragma unroll
  for (int n = 0; n < 8; ++n) st.o[n][RR] *= ar;
}

// K (A operands of S^T) and transposed V (B operands of O) of one page from
// its LDS image.  VM >= 0: first wait until at most VM vector-memory
// operations are outstanding (the page's LDS-DMA); the wait and the reads are
// one asm block so that the compiler, which cannot tell the LDS buffers apart,
// adds no wait of its own on the loads in flight.  VM < 0: no vmcnt wait (the
// caller already waited and synchronised the workgroup).
struct PageRegs {
  bf16x8_t kr[4];
  short4_t vt[8];
};
template <int VM, bool WAIT = true>
XV_INLINE void read_page(PageRegs& pr, const char* buf, const LaneOffsets& lo) {
  const uint32_t b0 = (uint32_t)reinterpret_cast<uintptr_t>(buf);
#define XV_PAGE_READS                                                                                   \
  "ds_read_b128 %0, %12\n\t"                                                                            \
  "ds_read_b128 %1, %13\n\t"                                                                            \
  "ds_read_b128 %2, %14\n\t"                                                                            \
  "ds_read_b128 %3, %15\n\t"                                                                            \
  "ds_read_b64_tr_b16 %4, %16\n\t"                                                                      \
  "ds_read_b64_tr_b16 %5, %17\n\t"                                                                      \
  "ds_read_b64_tr_b16 %6, %18\n\t"                                                                      \
  "ds_read_b64_tr_b16 %7, %19\n\t"                                                                      \
  "ds_read_b64_tr_b16 %8, %20\n\t"                                                                      \
  "ds_read_b64_tr_b16 %9, %21\n\t"                                                                      \
  "ds_read_b64_tr_b16 %10, %22\n\t"                                                                     \
  "ds_read_b64_tr_b16 %11, %23\n\t"
#define XV_PAGE_OPERANDS                                                                                \
  : "=&v"(pr.kr[0]), "=&v"(pr.kr[1]), "=&v"(pr.kr[2]), "=&v"(pr.kr[3]), "=&v"(pr.vt[0]), "=&v"(pr.vt[1]), \
    "=&v"(pr.vt[2]), "=&v"(pr.vt[3]), "=&v"(pr.vt[4]), "=&v"(pr.vt[5]), "=&v"(pr.vt[6]), "=&v"(pr.vt[7])  \
  : "v"(b0 + lo.k[0]), "v"(b0 + lo.k[1]), "v"(b0 + lo.k[2]), "v"(b0 + lo.k[3]), "v"(b0 + lo.v[0]),       \
    "v"(b0 + lo.v[1]), "v"(b0 + lo.v[2]), "v"(b0 + lo.v[3]), "v"(b0 + lo.v[4]), "v"(b0 + lo.v[5]),       \
    "v"(b0 + lo.v[6]), "v"(b0 + lo.v[7])
  if constexpr (VM >= 0 && WAIT) {
    __asm__ __volatile__("s_waitcnt vmcnt(%24)\n\t" XV_PAGE_READS "s_waitcnt lgkmcnt(0)" XV_PAGE_OPERANDS, "n"(VM)
                         : "memory");
  } else if constexpr (VM >= 0) {
    __asm__ __volatile__("s_waitcnt vmcnt(%24)\n\t" XV_PAGE_READS XV_PAGE_OPERANDS, "n"(VM) : "memory");
  } else {
    __asm__ __volatile__(XV_PAGE_READS "s_waitcnt lgkmcnt(0)" XV_PAGE_OPERANDS : "memory");
  }
#undef XV_PAGE_READS
#undef XV_PAGE_OPERANDS
}

// 4 fp8 (e4m3fn) values -> 4 bf16 (exact).
XV_INLINE short4_t fp8x4_to_bf16(uint32_t w) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  const uint32_t a = pack_bf16x2(lo[0], lo[1]), b = pack_bf16x2(hi[0], hi[1]);
  short4_t r;
  r[0] = (short)(a & 0xffffu);
  r[1] = (short)(a >> 16);
  r[2] = (short)(b & 0xffffu);
  r[3] = (short)(b >> 16);
  return r;
}

// The operands of an fp8 page straight from its raw image: the lane's two K
// pieces (its S^T A operands: token i's values 32g .. 32g+31, so MFMA step s
// contracts d-chunk 4g + s) and V by four transposed byte reads, in one asm
// block with one wait; both convert to bf16 in registers.  VM as in read_page.
template <int VM>
XV_INLINE void read_page_f8t(PageRegs& pr, const char* buf, const LaneOffsets& lo) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const uint32_t b0 = (uint32_t)reinterpret_cast<uintptr_t>(buf);
  u32x4_t k0, k1;
  u32x2_t v[4];
  __asm__ __volatile__(
      "s_waitcnt vmcnt(%6)\n\t"
      "ds_read_b128 %0, %7\n\t"
      "ds_read_b128 %1, %8\n\t"
      "ds_read_b64_tr_b8 %2, %9\n\t"
      "ds_read_b64_tr_b8 %3, %10\n\t"
      "ds_read_b64_tr_b8 %4, %11\n\t"
      "ds_read_b64_tr_b8 %5, %12\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(k0), "=&v"(k1), "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "n"(VM), "v"(b0 + lo.k8[0]), "v"(b0 + lo.k8[1]), "v"(b0 + lo.vt8[0]), "v"(b0 + lo.vt8[1]),
        "v"(b0 + lo.vt8[2]), "v"(b0 + lo.vt8[3])
      : "memory");
  uint32_t o[2][8];
  fp8x16_to_bf16(k0, o[0]);
  fp8x16_to_bf16(k1, o[1]);
#pragma unroll
  for (int j = 0; j < 4; ++j) __builtin_memcpy(&pr.kr[j], &o[j >> 1][4 * (j & 1)], 16);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    pr.vt[2 * m] = fp8x4_to_bf16(v[m][0]);
    pr.vt[2 * m + 1] = fp8x4_to_bf16(v[m][1]);
  }
}

// One tensor (K or V) of an fp8 page image at `raw` (its 16 rows of 128
// bytes) widened to the bf16 page layout at `dst` (row t at t * 256, chunk c
// in slot c ^ swz(t), as the LDS-DMA of a bf16 page leaves it): lane l
// converts token l / 4's values 32 (l % 4) .. +31.
XV_INLINE void widen_unit_f8(const char* raw, char* dst, const LaneOffsets& lo, int lane) {
  const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(raw + (lo.v8[0] - kF8Half));
  const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(raw + (lo.v8[1] - kF8Half));
  uint32_t o[2][8];
  fp8x16_to_bf16(w0, o[0]);
  fp8x16_to_bf16(w1, o[1]);
  const int r = lane >> 2, q = lane & 3;
  char* row = dst + r * 256;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t* v = &o[j >> 1][4 * (j & 1)];
    *reinterpret_cast<uint4*>(row + (((4 * q + j) ^ swz(r)) << 4)) = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// S^T = K Q^T, the online softmax update and O += P V for one page already
// in registers.  Tokens at page_tok0 + t >= ctx are masked.
template <int G>
XV_INLINE void page_math(SplitState& st, const PageRegs& pr, const bf16x8_t (&qb)[4], int page_tok0, int ctx,
                         float scale_log2, int lane) {
  const int g = lane >> 4;
  const bf16x8_t (&kr)[4] = pr.kr;
  const short4_t (&vt)[8] = pr.vt;
  // ---- S^T = K Q^T ----
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kr[s], qb[s], acc, 0, 0, 0);
  // ---- online softmax for head c%G over tokens 4g..4g+3 ----
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = (page_tok0 + 4 * g + j < ctx) ? acc[j] * scale_log2 : -INFINITY;
  float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  mx = xor32_max(xor16_max(mx));
  // Lazy rescaling: the running max used for exp2 only moves when some head's
  // max grew by more than kLazy (p <= 2^kLazy meanwhile, exact after the
  // final 1/l).  Random or trained logits settle within a few pages, after
  // which the O rescale (32 accumulator reads/writes) is skipped.
  const float m_new = fmaxf(st.m, mx);
  if (__any(m_new > st.m + kLazy)) {
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.m = m_new;
    st.l *= alpha;
    rescale_row<G, 0>(st, alpha, g);
    rescale_row<G, 1>(st, alpha, g);
    rescale_row<G, 2>(st, alpha, g);
    rescale_row<G, 3>(st, alpha, g);
  }
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(sc[j] - st.m);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  short4_t pa;
#pragma unroll
  for (int j = 0; j < 4; ++j) pa[j] = (short)f32_to_bf16(p[j]);
  // ---- O += P V ----
#pragma unroll
  for (int n = 0; n < 8; ++n) st.o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vt[n], st.o[n], 0, 0, 0);
}

// Two pages whose LDS images sit kPairStride bytes apart (consecutive ring
// slots or bf16 images), read in one asm block with one wait: the second
// page's addresses are the first's plus an immediate offset.
constexpr int kPairStride = kPageLds;
XV_INLINE void read_page_pair(PageRegs& p0, PageRegs& p1, const char* buf, const LaneOffsets& lo) {
  const uint32_t b0 = (uint32_t)reinterpret_cast<uintptr_t>(buf);
  static_assert(kPairStride == 8192, "the offsets below are kPairStride");
  __asm__ __volatile__(
      "ds_read_b128 %0, %24\n\t"
      "ds_read_b128 %1, %25\n\t"
      "ds_read_b128 %2, %26\n\t"
      "ds_read_b128 %3, %27\n\t"
      "ds_read_b64_tr_b16 %4, %28\n\t"
      "ds_read_b64_tr_b16 %5, %29\n\t"
      "ds_read_b64_tr_b16 %6, %30\n\t"
      "ds_read_b64_tr_b16 %7, %31\n\t"
      "ds_read_b64_tr_b16 %8, %32\n\t"
      "ds_read_b64_tr_b16 %9, %33\n\t"
      "ds_read_b64_tr_b16 %10, %34\n\t"
      "ds_read_b64_tr_b16 %11, %35\n\t"
      "ds_read_b128 %12, %24 offset:8192\n\t"
      "ds_read_b128 %13, %25 offset:8192\n\t"
      "ds_read_b128 %14, %26 offset:8192\n\t"
      "ds_read_b128 %15, %27 offset:8192\n\t"
      "ds_read_b64_tr_b16 %16, %28 offset:8192\n\t"
      "ds_read_b64_tr_b16 %17, %29 offset:8192\n\t"
      "ds_read_b64_tr_b16 %18, %30 offset:8192\n\t"
      "ds_read_b64_tr_b16 %19, %31 offset:8192\n\t"
      "ds_read_b64_tr_b16 %20, %32 offset:8192\n\t"
      "ds_read_b64_tr_b16 %21, %33 offset:8192\n\t"
      "ds_read_b64_tr_b16 %22, %34 offset:8192\n\t"
      "ds_read_b64_tr_b16 %23, %35 offset:8192\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(p0.kr[0]), "=&v"(p0.kr[1]), "=&v"(p0.kr[2]), "=&v"(p0.kr[3]), "=&v"(p0.vt[0]), "=&v"(p0.vt[1]),
        "=&v"(p0.vt[2]), "=&v"(p0.vt[3]), "=&v"(p0.vt[4]), "=&v"(p0.vt[5]), "=&v"(p0.vt[6]), "=&v"(p0.vt[7]),
        "=&v"(p1.kr[0]), "=&v"(p1.kr[1]), "=&v"(p1.kr[2]), "=&v"(p1.kr[3]), "=&v"(p1.vt[0]), "=&v"(p1.vt[1]),
        "=&v"(p1.vt[2]), "=&v"(p1.vt[3]), "=&v"(p1.vt[4]), "=&v"(p1.vt[5]), "=&v"(p1.vt[6]), "=&v"(p1.vt[7])
      : "v"(b0 + lo.k[0]), "v"(b0 + lo.k[1]), "v"(b0 + lo.k[2]), "v"(b0 + lo.k[3]), "v"(b0 + lo.v[0]),
        "v"(b0 + lo.v[1]), "v"(b0 + lo.v[2]), "v"(b0 + lo.v[3]), "v"(b0 + lo.v[4]), "v"(b0 + lo.v[5]),
        "v"(b0 + lo.v[6]), "v"(b0 + lo.v[7])
      : "memory");
}

// page_math over two pages as one 32-token step (tokens 0..15 from p0,
// 16..31 from p1; tokens >= ntok masked): one softmax update, the two S^T
// products and the two P V products as independent MFMA chains.
template <int G>
XV_INLINE void page_math_pair(SplitState& st, const PageRegs& p0, const PageRegs& p1, const bf16x8_t (&qb)[4],
                              int ntok, float scale_log2, int lane) {
  const int g = lane >> 4;
  floatx4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p0.kr[s], qb[s], a0, 0, 0, 0);
    a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p1.kr[s], qb[s], a1, 0, 0, 0);
  }
  float sc[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = (4 * g + j < ntok) ? a0[j] * scale_log2 : -INFINITY;
    sc[4 + j] = (16 + 4 * g + j < ntok) ? a1[j] * scale_log2 : -INFINITY;
  }
  float mx = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
  mx = xor32_max(xor16_max(mx));
  const float m_new = fmaxf(st.m, mx);
  if (__any(m_new > st.m + kLazy)) {  // lazy rescaling, as in page_math
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.m = m_new;
    st.l *= alpha;
    rescale_row<G, 0>(st, alpha, g);
    rescale_row<G, 1>(st, alpha, g);
    rescale_row<G, 2>(st, alpha, g);
    rescale_row<G, 3>(st, alpha, g);
  }
  float p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(sc[j] - st.m);
  st.l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  short4_t pa0, pa1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pa0[j] = (short)f32_to_bf16(p[j]);
    pa1[j] = (short)f32_to_bf16(p[4 + j]);
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) st.o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa0, p0.vt[n], st.o[n], 0, 0, 0);
#pragma unroll
  for (int n = 0; n < 8; ++n) st.o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa1, p1.vt[n], st.o[n], 0, 0, 0);
}

// VMEM operations one page issue makes: 4 LDS-DMA instructions each for K
// and V, or 2 each for fp8 pages.
template <bool F8> constexpr int kPageOps = F8 ? 4 : 8;

template <int G, int NB, bool F8>
XV_INLINE void process_page(SplitState& st, const char* buf, const LaneOffsets& lo, const bf16x8_t (&qb)[4],
                            int page_tok0, int ctx, float scale_log2, int lane) {
  // The page arrived by LDS-DMA; the VMEM operations of each of the NB-1
  // pages issued after it may still be in flight: vmcnt(ops*(NB-1)) waits
  // exactly for this page.
  PageRegs pr;
  if constexpr (F8) {
    read_page_f8t<kPageOps<true> * (NB - 1)>(pr, buf, lo);
  } else {
    read_page<kPageOps<false> * (NB - 1)>(pr, buf, lo);
  }
  page_math<G>(st, pr, qb, page_tok0, ctx, scale_log2, lane);
}

// Stream positions per half of the page-id table.
constexpr int kIdWindow = 128;

// Uniform position of a page in the flat (sequence, kv head, page) space.
struct Cursor {
  int b, kvh, pg;  // sequence, kv head, 16-token page within the sequence
  int sub;         // pg modulo the 16-token pages of a cache block
  int npb, ctx;    // pages and tokens of sequence b
};

// The next page of the flat space.  Sequences without pages (cache_seqlens
// 0) hold no flat positions and are stepped over; the caller only advances
// while a next page exists, and the loop is bounded by the batch regardless.
XV_INLINE void advance(Cursor& c, const int* pref, const int* sl, int hkv, int batch, int nsub) {
  if (++c.pg < c.npb) {
    if (++c.sub == nsub) c.sub = 0;
    return;
  }
  c.pg = 0;
  c.sub = 0;
  if (++c.kvh < hkv) return;
  c.kvh = 0;
  do {
    ++c.b;
    c.npb = __builtin_amdgcn_readfirstlane(pref[c.b + 1] - pref[c.b]);
  } while (c.npb == 0 && c.b < batch - 1);
  c.ctx = __builtin_amdgcn_readfirstlane(sl[c.b]);
}

// Sequence holding flat page f: the largest b with hkv*pref[b] <= f.
XV_INLINE int seq_of(const int* pref, int batch, int hkv, int64_t f) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)hkv * pref[mid] <= f) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// q rows of one (sequence, kv head): G rows of 256 B in LDS, row h at h*256.
// One LDS-DMA instruction moves 4 rows (1 KB); rows past G read as zeros.
template <int G> constexpr int kQSlot = G <= 4 ? 1024 : G * 256;
template <int G> constexpr int kBufBytes = kPageLds + kQSlot<G>;
// fp8 pages: 2 KB of K and 2 KB of V per page buffer, the q slot after them,
// plus one bf16 image per wave that each page is converted into
constexpr int kF8PageBytes = kPageLds / 2;
template <int G, bool F8> constexpr int kPageBufBytes = F8 ? kF8PageBytes : kPageLds;
template <int G, bool F8> constexpr int kBufBytesT = kPageBufBytes<G, F8> + kQSlot<G>;
// Page buffers per wave: 4 (3 at G = 8) keeps four waves' LDS within a CU.
template <int G> constexpr int kNbufG = G <= 4 ? 4 : 3;
// fp8 pages: two waves per SIMD with two page buffers each.  One wave per
// SIMD left the fp8 kernel paced by its per-page chain (page wait, LDS reads,
// conversion, V image round trip, math; 93 us at config 2, 69 us with the
// math removed); a second wave on the SIMD overlaps one wave's chain with
// the other's, 66 us.  The buffers shrink to fit eight waves' LDS in a CU.
// (V now reaches its B operands by transposed byte reads of the raw page,
// without the image round trip: 66 us as well; three waves per SIMD 82 us,
// three buffers 68 us.)
#ifndef XV_F8_WPE
#define XV_F8_WPE 2
#endif
#ifndef XV_F8_NB
#define XV_F8_NB 2
#endif
template <int G, bool F8> constexpr int kNbufT = (F8 && XV_F8_NB > 0) ? XV_F8_NB : kNbufG<G>;

template <int G>
XV_INLINE void issue_q(char* slot, const DecodeArgs& a, int b, int kvh, int lane) {
  const bf16_t* base = a.q + (int64_t)b * a.q_st + (int64_t)kvh * G * a.q_sh;
  const uint32_t bytes = (uint32_t)(((int64_t)(G - 1) * a.q_sh + kD) * 2);
  const __amdgpu_buffer_rsrc_t rq = page_rsrc(base, bytes);
#pragma unroll
  for (int j = 0; j < (G + 3) / 4; ++j) {
    const int row = 4 * j + (lane >> 4);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(slot + 1024 * j), 16,
                                             (int)(row * a.q_sh * 2) + ((lane & 15) << 4), 0, 0, 0);
  }
}

// Q^T B operand of MFMA step s from the q slot: column i holds head i % G,
// k = d-chunk 4s + g.  The slot arrived with the page it was issued with:
// the same vmcnt as that page's wait covers it.
// F8: step s contracts d-chunk 4g + s instead (the fp8 path's K order).
template <int G, int NB, int OPS, bool F8 = false>
XV_INLINE void read_q(bf16x8_t (&qb)[4], const char* slot, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const uint32_t a0 = (uint32_t)reinterpret_cast<uintptr_t>(slot) + (i % G) * 256 + g * (F8 ? 64 : 16);
  constexpr int st = F8 ? 16 : 64;  // bytes between steps
  __asm__ __volatile__(
      "s_waitcnt vmcnt(%5)\n\t"
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %4 offset:%7\n\t"
      "ds_read_b128 %3, %4 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(qb[0]), "=&v"(qb[1]), "=&v"(qb[2]), "=&v"(qb[3])
      : "v"(a0), "n"(OPS * (NB - 1)), "n"(st), "n"(2 * st), "n"(3 * st)
      : "memory");
}

// Write the finished segment (b, kvh): bf16 output if this wave covered the
// whole segment, else the normalised partial (bf16, as the output is) and its log2-sum-exp in slot
// part.  The O rows go through LDS `stage` (kQSlot<G> bytes: the q slot of
// the page buffer in hand, free once its q is in registers) and leave as
// whole 16-byte pieces, a few store instructions per segment instead of one
// per 16-column tile and row block.
template <int G>
XV_INLINE void finish_segment(const DecodeArgs& a, const SplitState& st, int b, int kvh, bool full, int part,
                              int lane, char* stage) {
  static_assert(G * kD * 2 <= kQSlot<G>, "the q slot stages the segment's G bf16 output rows");
  const int i = lane & 15, g = lane >> 4;
  // total p-sum of head c%G over the four rows
  const float lsum = xor32_sum(xor16_sum(st.l));
  float inv[4], lse[4];
  auto row_consts = [&](auto rr_tag) {
    constexpr int RR = decltype(rr_tag)::value;
    const float lh = head_of_row<G, RR>(lsum, g);
    inv[RR] = a.v_scale / lh;
    lse[RR] = head_of_row<G, RR>(st.m, g) + __log2f(lh);
  };
  row_consts(std::integral_constant<int, 0>{});
  row_consts(std::integral_constant<int, 1>{});
  row_consts(std::integral_constant<int, 2>{});
  row_consts(std::integral_constant<int, 3>{});
  // the wave's own LDS writes precede its reads (rows past G are replicas: not written)
  auto wave_sync = [] {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
  };
  const int head0 = kvh * G;
  if (full) {
    uint16_t* s16 = reinterpret_cast<uint16_t*>(stage);  // row r (head head0 + r) at r * 256 B
#pragma unroll
    for (int RR = 0; RR < 4; ++RR) {
      const int row = 4 * g + RR;
      if (row < G) {
#pragma unroll
        for (int nn = 0; nn < 8; ++nn) s16[row * kD + 16 * nn + i] = (uint16_t)f32_to_bf16(st.o[nn][RR] * inv[RR]);
      }
    }
    wave_sync();
    // the G heads' rows are contiguous in the output row of sequence b
    char* dst = reinterpret_cast<char*>(a.out + (int64_t)b * a.out_st + (int64_t)head0 * kD);
    constexpr int kBytes = G * kD * 2;
#pragma unroll
    for (int k = 0; k < (kBytes + 1023) / 1024; ++k) {
      const int off = 1024 * k + 16 * lane;
      if (off < kBytes) *reinterpret_cast<uint4*>(dst + off) = *reinterpret_cast<const uint4*>(stage + off);
    }
    return;
  }
  // bf16 partial rows (256 B each, max_parts rows apart per head)
  uint16_t* s16 = reinterpret_cast<uint16_t*>(stage);
  float* s32 = reinterpret_cast<float*>(stage);
  const int64_t wrow0 = ((int64_t)b * a.hq + head0) * a.max_parts + part;  // head h: + h * max_parts
#pragma unroll
  for (int RR = 0; RR < 4; ++RR) {
    const int row = 4 * g + RR;
    if (row < G) {
#pragma unroll
      for (int nn = 0; nn < 8; ++nn) s16[row * kD + 16 * nn + i] = (uint16_t)f32_to_bf16(st.o[nn][RR] * inv[RR]);
    }
  }
  wave_sync();
  {
    constexpr int kBytes = G * kD * 2;
#pragma unroll
    for (int k = 0; k < (kBytes + 1023) / 1024; ++k) {
      const int off = 1024 * k + 16 * lane;
      if (off < kBytes) {
        const int r = off / (kD * 2), w = off % (kD * 2);
        char* dst = reinterpret_cast<char*>(a.ws_ob + (wrow0 + (int64_t)r * a.max_parts) * kD) + w;
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(stage + off);
      }
    }
  }
  wave_sync();  // the stage's reads are done before the log2-sum-exps overwrite it
#pragma unroll
  for (int RR = 0; RR < 4; ++RR) {
    const int row = 4 * g + RR;
    if (i == 0 && row < G) s32[row] = lse[RR];
  }
  wave_sync();
  if (lane < G) a.ws_lse[wrow0 + (int64_t)lane * a.max_parts] = s32[lane];
}

XV_INLINE void reset(SplitState& st) {
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int n = 0; n < 8; ++n) st.o[n] = floatx4_t{0.f, 0.f, 0.f, 0.f};
}

// Page ids of the wave's stream live in a double-buffered LDS table of
// kIdWindow positions per half, filled by LDS-DMA from the block table (lane l
// fetches position base + l, base + 64 + l).  The half for window k+1 is
// requested when the issue side enters window k, kIdWindow pages before its
// first use: every page wait in between (vmcnt in process_page) orders it.
// Positions past the range fetch entry 0 (never used).
XV_INLINE void load_window(char* half, const DecodeArgs& a, __amdgpu_buffer_rsrc_t rbt, const int* pref, int64_t f0,
                           int base, int n, int lane) {
#pragma unroll
  for (int j = 0; j < kIdWindow / 64; ++j) {
    const int y = base + 64 * j + lane;
    int off = 0;
    if (y < n) {
      const int64_t f = f0 + y;
      const int b = seq_of(pref, a.batch, a.hkv, f);
      const int npb = pref[b + 1] - pref[b];
      const int r = (int)(f - (int64_t)a.hkv * pref[b]);
      const int kvh = r / npb;
      off = (int)(((int64_t)b * a.bt_stride + (r - kvh * npb) / a.nsub) * 4);  // the page's cache block
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rbt, (lds_void*)(half + 256 * j), 4, off, 0, 0, 0);
  }
}

// Page ids of stream positions y0 .. y0+3 (clamped to n-1) from the table,
// with one LDS wait for the four (an asm read: the compiler does not order
// LDS-DMA writes against plain LDS reads).
struct Ids4 {
  int v[4];
};
XV_INLINE uint32_t id_addr(const char* tab, int y) {
  return (uint32_t)reinterpret_cast<uintptr_t>(tab) + ((y / kIdWindow) & 1) * (kIdWindow * 4) + (y % kIdWindow) * 4;
}
XV_INLINE Ids4 lookup4(const char* tab, int y0, int n) {
  int r0, r1, r2, r3;
  __asm__ __volatile__(
      "ds_read_b32 %0, %4\n\t"
      "ds_read_b32 %1, %5\n\t"
      "ds_read_b32 %2, %6\n\t"
      "ds_read_b32 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(id_addr(tab, min(y0, n - 1))), "v"(id_addr(tab, min(y0 + 1, n - 1))),
        "v"(id_addr(tab, min(y0 + 2, n - 1))), "v"(id_addr(tab, min(y0 + 3, n - 1)))
      : "memory");
  Ids4 r;
  r.v[0] = __builtin_amdgcn_readfirstlane(r0);
  r.v[1] = __builtin_amdgcn_readfirstlane(r1);
  r.v[2] = __builtin_amdgcn_readfirstlane(r2);
  r.v[3] = __builtin_amdgcn_readfirstlane(r3);
  return r;
}

constexpr int kMaxBatch = 256;  // sequences per launch (larger batches are launched in chunks)

#ifndef XV_DECODE_WPE
#define XV_DECODE_WPE 1  // waves per SIMD the register budget is fitted to
#endif

// Pages per wave range, from the launch's actual page counts: a segment of
// np pages touches at most ceil(np / L) + 1 ranges, so L >= ceil(max np /
// (max_parts - 1)) keeps every segment's partials within its workspace slots
// (the host's lmin is the same bound for the widest table the block-table
// width allows; rows far shorter than the table, such as the suffixes of a
// cascade decode, get ranges sized to what they hold).  At least
// kMinRangePages pages keep the page pipeline busy.
constexpr int kMinRangePages = 4;
XV_INLINE int range_pages(const DecodeArgs& a, int64_t total, int max_np) {
  const int64_t per = (total + a.nwaves - 1) / a.nwaves;
  const int need = (max_np + a.max_parts - 2) / (a.max_parts - 1);
  return (int)max((int64_t)max(kMinRangePages, need), per);
}


template <int G, bool F8 = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(F8 ? XV_F8_WPE : XV_DECODE_WPE,
                                                                      F8 ? XV_F8_WPE : XV_DECODE_WPE))) void paged_decode_kernel(DecodeArgs a) {
  constexpr int NB = kNbufT<G, F8>;
  constexpr int BUF = kBufBytesT<G, F8>;
  constexpr int QOFF = kPageBufBytes<G, F8>;  // the q slot within a page buffer
  __shared__ __attribute__((aligned(16))) char lds[NB * BUF];
  __shared__ int pref[kMaxBatch + 1];  // pages of sequences 0..b-1
  __shared__ int sl[kMaxBatch];        // cache_seqlens
  __shared__ __attribute__((aligned(16))) char idtab[2 * kIdWindow * 4];
  const int lane = threadIdx.x;
  // prefix sums of the page counts (every wave computes them)
  int carry = 0, max_np = 0;
  for (int c = 0; c < a.batch; c += 64) {
    const int b = c + lane;
    const int ctx = b < a.batch ? max(a.seqlens[b], 0) : 0;
    const int np = (ctx + kPage - 1) / kPage;
    max_np = max(max_np, np);
    int inc = np;
    // inclusive scan by DPP: within 16-lane rows, then across rows
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x111, 0xf, 0xf, true);  // row_shr:1
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x112, 0xf, 0xf, true);  // row_shr:2
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x114, 0xf, 0xf, true);  // row_shr:4
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x118, 0xf, 0xf, true);  // row_shr:8
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x142, 0xa, 0xf, true);  // row_bcast:15 into rows 1, 3
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x143, 0xc, 0xf, true);  // row_bcast:31 into rows 2, 3
    if (b < a.batch) {
      pref[b + 1] = carry + inc;
      sl[b] = ctx;
    }
    carry += __builtin_amdgcn_readlane(inc, 63);
  }
  if (lane == 0) pref[0] = 0;
  __syncthreads();  // single wave: orders the LDS writes before the reads
  max_np = (int)wave_max((float)max_np);  // page counts are exact in fp32 (below 2^24)
  const int64_t total = (int64_t)a.hkv * carry;
  const int L = range_pages(a, total, max_np);
  const int64_t f0 = (int64_t)blockIdx.x * L;
  const int n = (int)max((int64_t)0, min(f0 + L, total) - f0);  // pages of this wave's range
  if (n == 0) return;
  const LaneOffsets offs = lane_offsets(a.tok_stride, lane);

  // cursor at the range's first page
  Cursor c0;
  c0.b = __builtin_amdgcn_readfirstlane(seq_of(pref, a.batch, a.hkv, f0));
  c0.npb = __builtin_amdgcn_readfirstlane(pref[c0.b + 1] - pref[c0.b]);
  c0.ctx = __builtin_amdgcn_readfirstlane(sl[c0.b]);
  {
    const int r = (int)(f0 - (int64_t)a.hkv * pref[c0.b]);
    c0.kvh = __builtin_amdgcn_readfirstlane(r / c0.npb);
    c0.pg = __builtin_amdgcn_readfirstlane(r - c0.kvh * c0.npb);
    c0.sub = __builtin_amdgcn_readfirstlane(c0.pg % a.nsub);
  }
  Cursor ic = c0, pc = c0;  // issue and process cursors
  const __amdgpu_buffer_rsrc_t rbt =
      page_rsrc(reinterpret_cast<const bf16_t*>(a.bt), (uint32_t)((int64_t)a.batch * a.bt_stride * 4));
  // the first window only: the second is requested once the first pages are
  // in flight (it is read kIdWindow - NB positions later)
  load_window(idtab, a, rbt, pref, f0, 0, n, lane);
  __asm__ __volatile__("s_waitcnt vmcnt(0)" ::: "memory");  // nothing else in flight yet
  int issued = -1;  // last stream position issued

  // One page (and, at a segment start, its q rows) into buffer `slot`.
  // Positions past the range are clamped to its last page (a harmless
  // re-read), so every call issues the same 8 page loads; the wait in
  // process_page relies on that count.
  auto issue = [&](int y, int slot, int page_id) {
    char* buf = lds + slot * BUF;
    if (y > issued) {
      const bool newseg = issued < 0 || (advance(ic, pref, sl, a.hkv, a.batch, a.nsub), ic.pg == 0);
      issued = y;
      if (y % kIdWindow == 0 && y > 0)  // entering window k: request window k+1
        load_window(idtab + ((y / kIdWindow + 1) & 1) * (kIdWindow * 4), a, rbt, pref, f0, y + kIdWindow, n, lane);
      if (newseg) issue_q<G>(buf + QOFF, a, ic.b, ic.kvh, lane);
    }
    if constexpr (F8) issue_page_f8(buf, a, page_id, ic.sub, ic.kvh, min(kPage, ic.ctx - ic.pg * kPage), offs);
    else issue_page(buf, a, page_id, ic.sub, ic.kvh, min(kPage, ic.ctx - ic.pg * kPage), offs);
  };

  SplitState st;
  reset(st);
  bf16x8_t qb[4];
  auto finish = [&](const Cursor& c, char* stage) {
    const int64_t seg0 = (int64_t)a.hkv * pref[c.b] + (int64_t)c.kvh * c.npb;
    // a row with a shared prefix always leaves a partial: the merge combines it with the prefix pass's
    const bool pre = a.pre_tokens != nullptr && __builtin_amdgcn_readfirstlane(a.pre_tokens[c.b]) > 0;
    const bool full = seg0 >= f0 && seg0 + c.npb <= f0 + n && !pre;
    const int part = (int)(blockIdx.x - seg0 / L);
    finish_segment<G>(a, st, c.b, c.kvh, full, part, lane, stage);
    if (lane == 0 && seg0 + c.npb <= f0 + n) a.ws_nparts[c.b * a.hkv + c.kvh] = full ? 1 : part + 1;
  };
  auto process = [&](int x, int slot) {
    char* buf = lds + slot * BUF;
    if (x > 0) {
      const Cursor prev = pc;
      advance(pc, pref, sl, a.hkv, a.batch, a.nsub);
      if (pc.pg == 0) {
        // the new segment's q first: its slot then stages the finished one
        read_q<G, NB, kPageOps<F8>, F8>(qb, buf + QOFF, lane);
        finish(prev, buf + QOFF);
        reset(st);
      }
    } else {
      read_q<G, NB, kPageOps<F8>, F8>(qb, buf + QOFF, lane);
    }
    process_page<G, NB, F8>(st, buf, offs, qb, pc.pg * kPage, pc.ctx, a.scale_log2, lane);
  };

  static_assert(NB <= 8, "at most eight ids per lookup");
  // ids of positions y0 .. y0 + 7 (the second four only when NB needs them)
  auto lookup = [&](int y0, int (&v)[8]) {
    const Ids4 a4 = lookup4(idtab, y0, n);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = a4.v[k];
    if constexpr (NB > 4) {
      const Ids4 b4 = lookup4(idtab, y0 + 4, n);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 + k] = b4.v[k];
    }
  };
  {
    int ids[8];
    lookup(0, ids);
#pragma unroll
    for (int k = 0; k < NB - 1; ++k) issue(min(k, n - 1), k, ids[k]);
  }
  // window 1; every page wait before its first use orders it
  load_window(idtab + kIdWindow * 4, a, rbt, pref, f0, kIdWindow, n, lane);
  for (int x0 = 0; x0 < n; x0 += NB) {
    // ids of the NB positions issued in this round; window k+1 of the table
    // was requested when the issue side entered window k, at least
    // kIdWindow - 2*NB positions before any of them
    int ids[8];
    lookup(x0 + NB - 1, ids);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      issue(min(x0 + u + NB - 1, n - 1), (u + NB - 1) % NB, ids[u]);
      if (x0 + u < n) process(x0 + u, u);
    }
  }
  // the last processed buffer's q slot: its q is in registers, and no DMA
  // targets it any more (q only comes with a segment's first page)
  finish(pc, lds + ((n - 1) % NB) * BUF + QOFF);
}

// Cascade decode: prefix-pass partials per (sequence, query head).
constexpr int kCascMaxChunks = 32;

// Weighted merge of n partials of one (sequence, query head) by one wave:
// lane j holds partial j's weight (j < 64, then j - 64, j - 128 in two more
// registers); four groups of 16 lanes take every fourth partial, 8 dims per
// lane, 32 partials per batch of loads with two batches in flight, and the
// groups are summed by lane swaps.  part_vals(j, i, lo, hi) loads values
// 8i .. 8i + 7 of partial j, part_lse(j) is its log2-sum-exp; n <= kMergeMaxParts.
constexpr int kMergeMaxParts = 192;
// lse_lane: partial `lane`'s log2-sum-exp when the caller loaded it already
// (HAVE_LANE), so that it need not wait for a load after learning n.
template <bool HAVE_LANE, typename PV, typename PL>
XV_INLINE void merge_general(int n, PV part_vals, PL part_lse, float lse_lane, bf16_t* orow, int lane) {
  const float la = lane < n ? (HAVE_LANE ? lse_lane : part_lse(lane)) : -INFINITY;
  const float lb = 64 + lane < n ? part_lse(64 + lane) : -INFINITY;
  const float lc = 128 + lane < n ? part_lse(128 + lane) : -INFINITY;
  const float mx = wave_max(fmaxf(la, fmaxf(lb, lc)));
  const float wa = lane < n ? __builtin_amdgcn_exp2f(la - mx) : 0.f;
  const float wb = 64 + lane < n ? __builtin_amdgcn_exp2f(lb - mx) : 0.f;
  const float wc = 128 + lane < n ? __builtin_amdgcn_exp2f(lc - mx) : 0.f;
  const float den = wave_sum(wa + wb + wc);
  const int g = lane >> 4, i = lane & 15;  // group g: partials g, g + 4, ...; dims 8i .. 8i + 7
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto load = [&](float4 (&v)[8][2], int j0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      part_vals(min(j0 + 4 * k + g, n - 1), i, v[k][0], v[k][1]);
    }
  };
  auto fold = [&](const float4 (&v)[8][2], int j0) {
    // partial j's weight sits in lane j mod 64 of the register of its
    // 64-block; a batch (32 partials from j0, a multiple of 32) lies in one
    // block, and group g's partial of step k is j0 + 4k + g: four lane reads
    // into scalars, one per group
    const float wsrc = j0 < 64 ? wa : j0 < 128 ? wb : wc;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = j0 + 4 * k + g;
      const int s0 = (j0 + 4 * k) & 63;
      const float w0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsrc), s0));
      const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsrc), s0 + 1));
      const float w2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsrc), s0 + 2));
      const float w3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsrc), s0 + 3));
      const float w = j < n ? (g == 0 ? w0 : g == 1 ? w1 : g == 2 ? w2 : w3) : 0.f;
      acc[0] += w * v[k][0].x; acc[1] += w * v[k][0].y; acc[2] += w * v[k][0].z; acc[3] += w * v[k][0].w;
      acc[4] += w * v[k][1].x; acc[5] += w * v[k][1].y; acc[6] += w * v[k][1].z; acc[7] += w * v[k][1].w;
    }
  };
  float4 va[8][2], vb[8][2];
  load(va, 0);
  for (int j0 = 0; j0 < n; j0 += 64) {
    if (j0 + 32 < n) load(vb, j0 + 32);
    fold(va, j0);
    if (j0 + 32 < n) {
      if (j0 + 64 < n) load(va, j0 + 64);
      fold(vb, j0 + 32);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = xor32_sum(xor16_sum(acc[e]));
  if (g == 0) {
    const float inv = 1.0f / den;
    uint32_t* o = reinterpret_cast<uint32_t*>(orow + 8 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(acc[2 * e] * inv, acc[2 * e + 1] * inv);
  }
}

// Merge the partials of one (sequence, query head) with one wave.  Also
// writes the zero output of padding rows (cache_seqlens 0).  The partial
// count comes from the main kernel.  The count, the sequence length, the
// first kFastParts partials (the common splits, 2 dims per lane) and the
// log2-sum-exp of partial `lane` are loaded together, so a merge of up to
// kFastParts partials costs one memory round trip.  More partials take
// merge_general.  Cascade rows (a shared prefix) merge the suffix partials
// with the prefix pass's chunk partials.
constexpr int kFastParts = 4;  // partial counts merged from the first memory round trip
__global__ __launch_bounds__(64) void merge_parts_kernel(DecodeArgs a) {
  const int b = blockIdx.x / a.hq;
  const int h = blockIdx.x - b * a.hq;
  const int lane = threadIdx.x;
  const int d = lane * 2;
  const int64_t row0 = ((int64_t)b * a.hq + h) * a.max_parts;
  const int ctx = a.seqlens[b];
  int n = a.ws_nparts[b * a.hkv + h / a.group];  // stale when ctx <= 0: not used then
  bf16_t* orow = a.out + (int64_t)b * a.out_st + (int64_t)h * kD;
  if (a.pre_tokens != nullptr) {
    const int pre_pages = a.pre_tokens[b] / kPage;
    if (pre_pages > 0) {
      n = ctx > 0 ? n : 0;
      const int npre = (pre_pages + a.pre_chunk_pages - 1) / a.pre_chunk_pages;
      // partial j >= n: prefix chunk j - n, rows chunk-major
      const int64_t cstride = (int64_t)a.batch * a.hq, prow = (int64_t)b * a.hq + h;
      merge_general<false>(
          n + npre,
          [&](int j, int i, float4& lo, float4& hi) {
            float f[8];  // suffix and prefix chunk partials are bf16
            unpack8(load_vec8(j < n ? a.ws_ob + (row0 + j) * kD + 8 * i : a.pre_o + ((j - n) * cstride + prow) * kD + 8 * i),
                    f);
            lo = make_float4(f[0], f[1], f[2], f[3]);
            hi = make_float4(f[4], f[5], f[6], f[7]);
          },
          [&](int j) { return j < n ? a.ws_lse[row0 + j] : a.pre_lse[(j - n) * cstride + prow]; }, 0.f, orow,
          lane);
      return;
    }
  }
  // speculative: the first kFastParts rows (clamped to max_parts - 1: rows
  // below max_parts exist in every workspace, and max_parts >= 2)
  float lf[kFastParts];
  float2 vf[kFastParts];
#pragma unroll
  for (int r = 0; r < kFastParts; ++r) {
    const int64_t row = row0 + min(r, a.max_parts - 1);
    lf[r] = a.ws_lse[row];
    const uint32_t u = *reinterpret_cast<const uint32_t*>(a.ws_ob + row * kD + d);
    vf[r] = make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
  }
  const float lmine = lane < a.max_parts ? a.ws_lse[row0 + lane] : -INFINITY;
  if (ctx <= 0) {
    *reinterpret_cast<uint32_t*>(orow + d) = 0u;
    return;
  }
  if (n <= 1) return;
  if (n <= kFastParts) {
    float mx = lf[0];
#pragma unroll
    for (int r = 1; r < kFastParts; ++r) mx = r < n ? fmaxf(mx, lf[r]) : mx;
    float den = 0.f, ox = 0.f, oy = 0.f;
#pragma unroll
    for (int r = 0; r < kFastParts; ++r) {
      if (r >= n) break;  // rows past n hold stale data (even NaN): never touched
      const float w = __builtin_amdgcn_exp2f(lf[r] - mx);
      den += w;
      ox += w * vf[r].x;
      oy += w * vf[r].y;
    }
    const float inv = 1.0f / den;
    *reinterpret_cast<uint32_t*>(orow + d) = pack_bf16x2(ox * inv, oy * inv);
    return;
  }
  merge_general<true>(
      n,
      [&](int j, int i, float4& lo, float4& hi) {
        float f[8];
        unpack8(load_vec8(a.ws_ob + (row0 + j) * kD + 8 * i), f);
        lo = make_float4(f[0], f[1], f[2], f[3]);
        hi = make_float4(f[4], f[5], f[6], f[7]);
      },
      [&](int j) { return a.ws_lse[row0 + j]; }, lmine, orow, lane);
}

// Minimum pages per wave range.  It bounds the partials per (sequence, head),
// parts = ceil(max_blocks / lmin) + 1, by P: at most 129, and fewer when the
// workspace for batch x q heads x P partials would pass kPartBudget.  Small
// batches of long sequences thus still fill every wave slot, and at least four
// pages per range keep the page pipeline busy (two: B 1 x 2048 11.4 us, four: 10.7).
constexpr int kMaxParts = 129;
constexpr size_t kPartBudget = (size_t)32 << 20;
static_assert(kMaxParts <= kMergeMaxParts, "the merge holds at most kMergeMaxParts weights per head");
int min_range_pages(int batch, int num_q_heads, int max_blocks_per_seq) {
  const size_t per_part = (size_t)max(batch, 1) * max(num_q_heads, 1) * (kD + 1) * sizeof(float);
  const int P = (int)max((size_t)3, min((size_t)kMaxParts, kPartBudget / per_part));
  return max(kMinRangePages, (max_blocks_per_seq + P - 2) / (P - 1));
}

// ---------------------------------------------------------------------------
// Cascade (shared-prefix) decode, prefix pass.  The sequences of a group share
// their first P tokens: the same cache blocks, as a prefix cache maps them.
// Instead of every member streaming those pages, one workgroup per (prefix
// chunk, kv head, group) reads the chunk's pages once and attends the whole
// group's query rows to them: R = members x G rows (at most kCascRows), in
// 16-row tiles on the MFMA columns (each column its own row, G = 16 in the
// page math), one tile per wave.  The chunk's pages stream through a ring of
// four quarters (4 pages each, 32 KB of bf16 pages) by LDS-DMA, three
// quarters in flight while the tiles run over the fourth; the page ids are
// fetched into LDS once.  Each row's normalised chunk output and its
// log2-sum-exp go to the prefix partial slots, which the merge combines with
// the row's suffix partials.  The same workgroups write the suffix view of
// every row (block-table rows shifted past the prefix blocks, suffix
// lengths) for the suffix decode.
constexpr int kCascRows = 128;
constexpr int kCascWaves = kCascRows / 16;  // one 16-row tile per wave
constexpr int kCascSub = 16;                // pages in the ring (128 KB of bf16 pages)
constexpr int kCascQuarter = kCascSub / 4;  // pages per quarter: one (page, K or V) unit per wave
// fp8 pages: the ring holds raw pages (4 KB each), and two bf16 images of a
// quarter (4 pages in the bf16 page layout), which the workgroup's waves fill
// together, one (page, K or V) unit each, and then all read.
constexpr int kCascMaxChunkPages = 2048;  // pages per prefix chunk (kCascMaxChunks of them: 1M-token prefixes)
template <bool F8> constexpr int kCascLds = F8 ? kCascSub * (kPageLds / 2) + 2 * kCascQuarter * kPageLds
                                               : kCascSub * kPageLds;

struct CascadeArgs {
  const bf16_t* q; int64_t q_st, q_sh;
  const bf16_t* kc; const bf16_t* vc;
  int64_t page_stride, tok_stride, head_stride;
  const int32_t* bt; int64_t bt_stride;
  const int32_t* seqlens;
  int nsub, block_size, batch, max_blocks;
  const int4* grp_info;     // per group: first index into grp_rows, rows, first row, prefix tokens
  const int32_t* grp_rows;  // batch rows of each group
  const int32_t* pre_tokens;
  int num_groups, hq, hkv, chunk_pages, num_chunks;
  bf16_t* pre_o; float* pre_lse;
  int32_t* sbt; int32_t* ssl;  // suffix view: [batch, max_blocks] block table, [batch] lengths
  float scale_log2;
  float v_scale;  // fp8 pages: the V dequantisation scale, applied to the output (1 for bf16 pages)
};

XV_INLINE void cascade_suffix_view(const CascadeArgs& a, int v, int nview) {
  for (int b = v; b < a.batch; b += nview) {
    const int pre = max(a.pre_tokens[b], 0);
    const int skip = pre / a.block_size;
    for (int j = threadIdx.x; j < a.max_blocks; j += blockDim.x)
      a.sbt[(int64_t)b * a.max_blocks + j] = j + skip < a.max_blocks ? a.bt[(int64_t)b * a.bt_stride + j + skip] : -1;
    if (threadIdx.x == 0) a.ssl[b] = max(a.seqlens[b] - pre, 0);
  }
}

// LDS-DMA instructions of one (page, K or V) unit.
template <bool F8> constexpr int kUnitOps = F8 ? 2 : 4;
template <int N>
XV_INLINE void wait_vm() { __asm__ __volatile__("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int G, bool F8 = false>
__global__ __launch_bounds__(kCascWaves * 64) void cascade_prefix_kernel(CascadeArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[kCascLds<F8>];
  __shared__ int ids[kCascMaxChunkPages];  // the chunk's page ids
  __shared__ int rowb[kCascRows];          // batch row of each tile row
  constexpr int kUnitPage = F8 ? kPageLds / 2 : kPageLds;  // LDS bytes of one page (K then V)
  // Workgroup w: (chunk, group, kv head), chunk fastest, so the workgroups of
  // empty groups (a graph records a fixed group count) are interleaved with
  // working ones instead of forming a tail of their own.  Every workgroup
  // also writes the suffix view of rows w, w + grid, ... (the launch has at
  // least min(batch, 64) workgroups); workgroups of their own for the view
  // would hold this kernel's LDS too and push prefix work into a second round.
  const int w = (int)blockIdx.x;
  if (w >= a.num_groups * a.num_chunks * a.hkv) {
    cascade_suffix_view(a, w, gridDim.x);
    return;
  }
  const int c = w % a.num_chunks, grp = (w / a.num_chunks) % a.num_groups,
            kvh = w / (a.num_chunks * a.num_groups);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // one record gives everything the page loads need: the page ids are one
  // round trip away, the q rows two (their batch rows first)
  const int4 info = a.grp_info[grp];
  const int r0 = __builtin_amdgcn_readfirstlane(info.x);
  const int nm = __builtin_amdgcn_readfirstlane(min(info.y, kCascRows / G));
  if (nm <= 0) {
    cascade_suffix_view(a, w, gridDim.x);
    return;
  }
  const int b0 = __builtin_amdgcn_readfirstlane(info.z);
  const int npages = __builtin_amdgcn_readfirstlane(info.w) / kPage;
  const int p0 = c * a.chunk_pages, p1 = min(npages, p0 + a.chunk_pages);
  if (p0 >= p1) {
    cascade_suffix_view(a, w, gridDim.x);
    return;
  }
  const int R = nm * G;
  const LaneOffsets offs = lane_offsets(a.tok_stride, lane);
  const int i = lane & 15, g = lane >> 4;
  const bool active = wave * 16 < R;  // this wave's tile holds rows
  const uint32_t bytes = (uint32_t)(((int64_t)(kPage - 1) * a.tok_stride + kD) * (F8 ? 1 : 2));
  const int np = p1 - p0;
  // the chunk's page ids, fetched once into LDS (every issue then reads its
  // id there instead of waiting on memory)
  for (int k = threadIdx.x; k < np; k += kCascWaves * 64)
    ids[k] = a.bt[(int64_t)b0 * a.bt_stride + (p0 + k) / a.nsub];
  // Quarter q of the chunk: pages 4q .. 4q + 3 in ring slot q % 4 (slot
  // pages 4 (q % 4) ..); wave w moves page 4q + w / 2, its K rows (w even) or
  // V rows (w odd).  Pages past the chunk's end read its last page again
  // (never used), so every issue counts the same kUnitOps instructions.
  auto issue_quarter = [&](int q) {
    const int k = min(4 * q + (wave >> 1), np - 1);
    const int p = p0 + k;
    const int id = __builtin_amdgcn_readfirstlane(ids[k]);
    const int64_t base = (int64_t)id * a.page_stride + (int64_t)(p % a.nsub) * kPage * a.tok_stride +
                         (int64_t)kvh * a.head_stride;
    const bf16_t* src = (wave & 1) ? a.vc : a.kc;
    char* const slot = lds + (4 * (q & 3) + (wave >> 1)) * kUnitPage;
    if constexpr (F8) {  // element strides are byte strides
      const __amdgpu_buffer_rsrc_t r =
          page_rsrc(reinterpret_cast<const bf16_t*>(reinterpret_cast<const char*>(src) + base), bytes);
      char* dst = slot + ((wave & 1) ? kF8Half : 0);
#pragma unroll
      for (int s = 0; s < 2; ++s)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + 1024 * s), 16, offs.g8[s], 0, 0, kNontemporal);
    } else {
      const __amdgpu_buffer_rsrc_t r = page_rsrc(src + base, bytes);
      char* dst = slot + ((wave & 1) ? kVPageBytes : 0);
#pragma unroll
      for (int s = 0; s < 4; ++s)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + 1024 * s), 16, offs.g[s], 0, 0, kNontemporal);
    }
  };
  // Q^T B operand of the wave's tile: column i = row 16 w + i, k = d-chunk 4s + g
  // (fp8 pages are widened to the bf16 page layout first: the same order)
  bf16x8_t qb[4];
  {
    const int row = wave * 16 + i;
    if (row < R) {
      const int b = a.grp_rows[r0 + row / G];
      if (g == 0) rowb[row] = b;  // for the output rows (ordered by the loop's barriers)
      const bf16_t* qr = a.q + (int64_t)b * a.q_st + (int64_t)(kvh * G + row % G) * a.q_sh;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const Vec8 v = load_vec8(qr + (4 * s + g) * 8);
        __builtin_memcpy(&qb[s], &v, 16);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) qb[s] = bf16x8_t{};
    }
  }
  SplitState st;
  reset(st);
  constexpr int kOps = kUnitOps<F8>;
  static_assert(2 * kCascQuarter == kCascWaves, "one (page, K or V) unit of a quarter per wave");
  char* const img0 = lds + kCascSub * kUnitPage;  // fp8 pages: the two quarter images
  const int Q = (np + 3) / 4;
  __syncthreads();  // the id table
  // Three quarters in flight ahead of the one the tiles run over.  Step t
  // waits for quarter t (the quarters issued after it, at most two, may
  // still be in flight) and, past the barrier that every wave reaches only
  // once done with quarter t - 1, refills that quarter's slot with quarter t + 3.
  for (int q = 0; q < min(Q, 3); ++q) issue_quarter(q);
  for (int t = 0; t < Q; ++t) {
    if (t + 2 < Q) wait_vm<2 * kOps>();
    else if (t + 1 < Q) wait_vm<kOps>();
    else wait_vm<0>();
    __syncthreads();
    if (t + 3 < Q) issue_quarter(t + 3);
    const int k0 = 4 * t, kn = min(np, k0 + 4);
    char* const ring = lds + 4 * (t & 3) * kUnitPage;
    // fp8 pages: wave w widens unit w of the quarter (page k0 + w / 2, K or
    // V) into image t % 2; the first barrier of step t - 1 ordered every read
    // of that image (step t - 2) before these writes
    char* const img = img0 + (t & 1) * kCascQuarter * kPageLds;
    if constexpr (F8) {
      // every unit, also past the chunk's end (a re-read page): the pair
      // steps below read whole pairs, masked but finite
      const int half = (wave & 1) ? kF8Half : 0;
      widen_unit_f8(ring + (wave >> 1) * kUnitPage + half, img + (wave >> 1) * kPageLds + 2 * half, offs, lane);
      __syncthreads();
    }
    if (active) {
      // pages in pairs: 32-token steps; a pair's missing second page (odd
      // count) is a re-read page, masked
      const char* const src = F8 ? img : ring;
      static_assert(kPairStride == kPageLds && (F8 || kUnitPage == kPageLds), "pair slots are kPairStride apart");
      for (int k = k0; k < kn; k += 2) {
        PageRegs pr0, pr1;
        read_page_pair(pr0, pr1, src + (k - k0) * kPageLds, offs);
        page_math_pair<16>(st, pr0, pr1, qb, k + 1 < kn ? 2 * kPage : kPage, a.scale_log2, lane);
      }
    }
  }
  __syncthreads();  // the output tiles below reuse the ring
  cascade_suffix_view(a, w, gridDim.x);  // every wave (the view loops over the workgroup's threads)
  if (!active) return;
  // Rows 16 w + 4 g + RR of O, normalised, go through LDS (the page buffers
  // are free now) so that each row's 512 bytes leave as whole 16-byte pieces:
  // the wave's 16 x 128 fp32 tile at w * 16 * kORow floats, rows padded to
  // kORow floats to spread the banks.
  constexpr int kORow = kD + 4;
  static_assert(kCascWaves * 16 * kORow * 4 <= kCascLds<F8>, "the output tiles fit the page buffers");
  float* tile = reinterpret_cast<float*>(lds) + wave * 16 * kORow;
  const float lsum = xor32_sum(xor16_sum(st.l));
  auto put = [&](auto rr_tag) {
    constexpr int RR = decltype(rr_tag)::value;
    const float lh = head_of_row<16, RR>(lsum, g);
    const float mh = head_of_row<16, RR>(st.m, g);
    const float inv = a.v_scale / lh;
    float* o = tile + (4 * g + RR) * kORow + i;
#pragma unroll
    for (int nn = 0; nn < 8; ++nn) o[16 * nn] = st.o[nn][RR] * inv;
    const int row = wave * 16 + 4 * g + RR;
    if (i == 0 && row < R) {
      const int b = rowb[row];
      a.pre_lse[((int64_t)c * a.batch + b) * a.hq + kvh * G + row % G] = mh + __log2f(lh);
    }
  };
  put(std::integral_constant<int, 0>{});
  put(std::integral_constant<int, 1>{});
  put(std::integral_constant<int, 2>{});
  put(std::integral_constant<int, 3>{});
  // wave-private region: the wave's own LDS writes precede its reads
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  // lane l: rows 4k + l / 16, values 8 (l % 16) .. +7, stored as 8 bf16
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int rt = 4 * k + (lane >> 4);
    const int row = wave * 16 + rt;
    if (row >= R) break;
    const int b = rowb[row];
    const float* src = tile + rt * kORow + 8 * (lane & 15);
    const float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
    const float f[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    store_vec8(a.pre_o + (((int64_t)c * a.batch + b) * a.hq + kvh * G + row % G) * kD + 8 * (lane & 15), pack8(f));
  }
}

template <bool F8>
int occupancy(int group) {
  int per_cu = 0;
  switch (group) {
    case 1: hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_kernel<1, F8>, 64, 0); break;
    case 2: hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_kernel<2, F8>, 64, 0); break;
    case 4: hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_kernel<4, F8>, 64, 0); break;
    default: hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_kernel<8, F8>, 64, 0); break;
  }
  return per_cu;
}
int waves_for(int group, bool f8 = false) {
  // resident single-wave workgroups: CUs x per-CU occupancy (queried once per device)
  static int cached[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int slot = (group == 1 ? 0 : group == 2 ? 1 : group == 4 ? 2 : 3) + (f8 ? 4 : 0);
  if (cached[slot]) return cached[slot];
  int dev = 0, cus = 0;
  hipGetDevice(&dev);
  hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  int per_cu = f8 ? occupancy<true>(group) : occupancy<false>(group);
#if XV_DECODE_WAVES_PER_CU > 0
  per_cu = min(per_cu, XV_DECODE_WAVES_PER_CU * (f8 ? XV_F8_WPE : 1));
#endif
  cached[slot] = max(1, cus) * max(1, per_cu);
  return cached[slot];
}

}  // namespace

// Workspace layout: [partial counts int32, B*Hkv, padded to 256 B][partial outputs: bf16 rows of kD in a region
// sized for fp32][partial log2-sum-exp fp32]
size_t counter_bytes(int batch, int num_kv_heads) { return ((size_t)batch * num_kv_heads * 4 + 255) / 256 * 256; }

// Workspace of one launch of `batch` <= kMaxBatch sequences; max_pages counts
// 16-token pages per sequence.
size_t chunk_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int max_pages) {
  const int lmin = min_range_pages(batch, num_q_heads, max_pages);
  const int parts = (max_pages + lmin - 1) / lmin + 1;
  return counter_bytes(batch, num_kv_heads) + (size_t)batch * num_q_heads * parts * ((size_t)kD + 1) * sizeof(float);
}

// 16-token pages per sequence for a block table of max_blocks cache blocks.
int64_t pages_per_seq(int max_blocks_per_seq, int block_size) {
  return (int64_t)max_blocks_per_seq * (block_size > 0 && block_size % kPage == 0 ? block_size / kPage : 1);
}

// The largest one-launch workspace over every batch up to `batch` (launches
// take at most kMaxBatch sequences).  The need of a single batch size is not
// monotone (the partial budget lets small batches keep more partials), so the
// query takes the maximum: the result never decreases with the batch, and a
// workspace sized for the largest batch serves every smaller one.  Callers that
// capture graphs for several batch sizes rely on this: their workspace is
// allocated once, before the first (largest) capture.
extern "C" size_t xv_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                                 int max_blocks_per_seq, int block_size, int head_dim) {
  (void)head_dim;
  const int64_t pages = pages_per_seq(max_blocks_per_seq, block_size);
  if (batch <= 0 || pages <= 0 || pages > INT32_MAX || num_kv_heads <= 0) return 256;
  size_t need = 256;
  for (int b = 1; b <= min(batch, kMaxBatch); ++b)
    need = max(need, chunk_workspace_bytes(b, num_q_heads, num_kv_heads, (int)pages));
  return need;
}

namespace {

// One launch pair (main kernel + merge) over batch <= kMaxBatch sequences,
// arguments already validated.
struct CascadeParts {  // the prefix pass's partials for the merge (pre_tokens == nullptr: none)
  const int32_t* pre_tokens = nullptr;
  int chunk_pages = 1;
  const bf16_t* pre_o = nullptr;
  const float* pre_lse = nullptr;
};

int decode_chunk(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                 const void* v_cache, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                 const int32_t* block_tables, int64_t bt_stride, const int32_t* cache_seqlens, void* out,
                 int64_t out_stride_tok, void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
                 int num_kv_heads, int nsub, int max_pages, float scale, hipStream_t stream,
                 const CascadeParts& cp = CascadeParts(), bool f8 = false, float v_scale = 1.0f) {
  const size_t need = chunk_workspace_bytes(batch, num_q_heads, num_kv_heads, max_pages);
  if (workspace == nullptr || workspace_bytes < need) return (int)hipErrorInvalidValue;
  const int group = num_q_heads / num_kv_heads;
  DecodeArgs a;
  a.q = (const bf16_t*)q; a.q_st = q_stride_tok; a.q_sh = q_stride_head;
  a.kc = (const bf16_t*)k_cache; a.vc = (const bf16_t*)v_cache;
  a.page_stride = page_stride; a.tok_stride = tok_stride; a.head_stride = head_stride;
  a.bt = block_tables; a.bt_stride = bt_stride; a.seqlens = cache_seqlens;
  a.out = (bf16_t*)out; a.out_st = out_stride_tok;
  const int lmin = min_range_pages(batch, num_q_heads, max_pages);
  a.max_parts = (max_pages + lmin - 1) / lmin + 1;
  a.ws_nparts = (int*)workspace;
  a.ws_o = (float*)((char*)workspace + counter_bytes(batch, num_kv_heads));
  a.ws_lse = a.ws_o + (size_t)batch * num_q_heads * a.max_parts * kD;
  a.ws_ob = reinterpret_cast<bf16_t*>(a.ws_o);
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads; a.group = group; a.lmin = lmin; a.nsub = nsub;
  // ranges: enough to fill the resident wave slots, never more than needed at lmin pages each
  const int64_t max_total = (int64_t)batch * num_kv_heads * max_pages;
  a.nwaves = (int)min((int64_t)waves_for(group, f8), (max_total + lmin - 1) / lmin);
  a.scale_log2 = scale * 1.4426950408889634f;
  a.v_scale = v_scale;
  a.pre_tokens = cp.pre_tokens; a.pre_chunk_pages = cp.chunk_pages; a.pre_o = cp.pre_o; a.pre_lse = cp.pre_lse;
  if (f8) {
    switch (group) {
      case 1: paged_decode_kernel<1, true><<<a.nwaves, 64, 0, stream>>>(a); break;
      case 2: paged_decode_kernel<2, true><<<a.nwaves, 64, 0, stream>>>(a); break;
      case 4: paged_decode_kernel<4, true><<<a.nwaves, 64, 0, stream>>>(a); break;
      default: paged_decode_kernel<8, true><<<a.nwaves, 64, 0, stream>>>(a); break;
    }
  } else {
    switch (group) {
      case 1: paged_decode_kernel<1><<<a.nwaves, 64, 0, stream>>>(a); break;
      case 2: paged_decode_kernel<2><<<a.nwaves, 64, 0, stream>>>(a); break;
      case 4: paged_decode_kernel<4><<<a.nwaves, 64, 0, stream>>>(a); break;
      default: paged_decode_kernel<8><<<a.nwaves, 64, 0, stream>>>(a); break;
    }
  }
  XV_CHECK_LAUNCH();
  merge_parts_kernel<<<dim3((unsigned)(batch * num_q_heads)), 64, 0, stream>>>(a);
  XV_CHECK_LAUNCH();
  return 0;
}

// Argument checks shared by both entry points (host only, no device call).
int decode_check(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                 const void* v_cache, int64_t page_stride, int64_t tok_stride, int64_t head_stride, void* out,
                 int64_t out_stride_tok, int batch, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                 int max_blocks_per_seq, bool f8 = false) {
  if (head_dim != kD || block_size <= 0 || block_size % kPage || batch < 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads || max_blocks_per_seq <= 0)
    return (int)hipErrorInvalidValue;
  const int group = num_q_heads / num_kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8) return (int)hipErrorInvalidValue;
  const int64_t max_pages = pages_per_seq(max_blocks_per_seq, block_size);
  if (max_pages > (1 << 24)) return (int)hipErrorInvalidValue;  // 256M tokens per sequence
  // rows move by 16-byte LDS-DMA: aligned bases, strides in whole 16-byte units
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15 || (q_stride_tok | q_stride_head) & 7 ||
      (page_stride | tok_stride | head_stride) & (f8 ? 15 : 7))  // cache strides in elements: 2 or 1 bytes
    return (int)hipErrorInvalidValue;
  if ((uintptr_t)out & 3 || out_stride_tok & 1) return (int)hipErrorInvalidValue;  // bf16 pairs stored as 4 bytes
  return 0;
}

// Checks, then the launches in chunks of kMaxBatch sequences, in stream order
// on the same workspace.
int decode_run(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
               const void* v_cache, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
               const int32_t* block_tables, int64_t bt_stride, const int32_t* cache_seqlens, void* out,
               int64_t out_stride_tok, void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
               int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq, float scale,
               hipStream_t stream, bool f8 = false, float k_scale = 1.0f, float v_scale = 1.0f) {
  const int rc0 = decode_check(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride,
                               head_stride, out, out_stride_tok, batch, num_q_heads, num_kv_heads, head_dim,
                               block_size, max_blocks_per_seq, f8);
  if (rc0 || batch == 0) return rc0;
  const int64_t max_pages = pages_per_seq(max_blocks_per_seq, block_size);
  for (int c0 = 0; c0 < batch; c0 += kMaxBatch) {
    const int rc = decode_chunk(
        (const bf16_t*)q + (int64_t)c0 * q_stride_tok, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride,
        tok_stride, head_stride, block_tables + (int64_t)c0 * bt_stride, bt_stride, cache_seqlens + c0,
        (bf16_t*)out + (int64_t)c0 * out_stride_tok, out_stride_tok, workspace, workspace_bytes,
        min(kMaxBatch, batch - c0), num_q_heads, num_kv_heads, block_size / kPage, (int)max_pages,
        f8 ? scale * k_scale : scale, stream, CascadeParts(), f8, f8 ? v_scale : 1.0f);
    if (rc) return rc;
  }
  return 0;
}

}  // namespace

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
  return decode_run(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride, head_stride,
                    block_tables, bt_stride, cache_seqlens, out, out_stride_tok, workspace, workspace_bytes, batch,
                    num_q_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, stream);
}

// fp8 (e4m3fn) K/V pages: the same kernels with a per-page conversion to bf16
// in LDS; k_scale multiplies the scores (folded into the softmax scale) and
// v_scale the output.
extern "C" int xv_paged_decode_attention_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                             const void* k_cache, const void* v_cache,
                                             int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                             const int32_t* block_tables, int64_t bt_stride,
                                             const int32_t* cache_seqlens,
                                             void* out, int64_t out_stride_tok,
                                             void* workspace, size_t workspace_bytes,
                                             int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                             int block_size, int max_blocks_per_seq, float scale,
                                             float k_scale, float v_scale, hipStream_t stream) {
  if (!(k_scale > 0.0f) || !(v_scale > 0.0f) || !isfinite(k_scale) || !isfinite(v_scale))
    return (int)hipErrorInvalidValue;
  return decode_run(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride, head_stride,
                    block_tables, bt_stride, cache_seqlens, out, out_stride_tok, workspace, workspace_bytes, batch,
                    num_q_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, stream, true,
                    k_scale, v_scale);
}

// ---------------------------------------------------------------------------
// Cascade (shared-prefix) decode entry point.
namespace {
size_t al256(size_t x) { return (x + 255) / 256 * 256; }
struct CascadeLayout {
  size_t sbt, ssl, lse, o, dec, total;
};
CascadeLayout cascade_layout(int batch, int num_q_heads, int num_kv_heads, int max_blocks_per_seq, int block_size) {
  CascadeLayout L;
  L.sbt = 0;
  L.ssl = al256((size_t)batch * max_blocks_per_seq * 4);
  L.lse = L.ssl + al256((size_t)batch * 4);
  L.o = L.lse + al256((size_t)batch * num_q_heads * kCascMaxChunks * 4);
  L.dec = L.o + al256((size_t)batch * num_q_heads * kCascMaxChunks * kD * 2);
  L.total = L.dec + chunk_workspace_bytes(batch, num_q_heads, num_kv_heads,
                                          (int)pages_per_seq(max_blocks_per_seq, block_size));
  return L;
}
}  // namespace

extern "C" size_t xv_cascade_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                                   int max_blocks_per_seq, int block_size, int head_dim) {
  (void)head_dim;
  const int64_t pages = pages_per_seq(max_blocks_per_seq, block_size);
  if (batch <= 0 || pages <= 0 || pages > INT32_MAX || num_kv_heads <= 0 || num_q_heads <= 0) return 256;
  size_t need = 256;
  for (int b = 1; b <= min(batch, kMaxBatch); ++b)  // never decreases with the batch
    need = max(need, cascade_layout(b, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size).total);
  return need;
}

namespace {
int cascade_run(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                const void* v_cache, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                const int32_t* block_tables, int64_t bt_stride, const int32_t* cache_seqlens,
                const int32_t* prefix_tokens, const int32_t* group_info, const int32_t* group_rows, int num_groups,
                int max_prefix_blocks, void* out, int64_t out_stride_tok, void* workspace, size_t workspace_bytes,
                int batch, int num_q_heads, int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq,
                float scale, hipStream_t stream, bool f8, float k_scale, float v_scale) {
  const int rc0 = decode_check(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride,
                               head_stride, out, out_stride_tok, batch, num_q_heads, num_kv_heads, head_dim,
                               block_size, max_blocks_per_seq, f8);
  if (rc0) return rc0;
  if (batch > kMaxBatch || num_groups < 0 || num_groups > 65535 || max_prefix_blocks < 0 ||
      max_prefix_blocks > max_blocks_per_seq || !prefix_tokens || (num_groups > 0 && (!group_info || !group_rows)) ||
      ((uintptr_t)group_info & 15))
    return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  const CascadeLayout Lw = cascade_layout(batch, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size);
  if (workspace == nullptr || workspace_bytes < Lw.total || (uintptr_t)workspace & 255)
    return (int)hipErrorInvalidValue;
  char* ws = (char*)workspace;
  int32_t* sbt = (int32_t*)(ws + Lw.sbt);
  int32_t* ssl = (int32_t*)(ws + Lw.ssl);
  float* pre_lse = (float*)(ws + Lw.lse);
  bf16_t* pre_o = (bf16_t*)(ws + Lw.o);
  const int nsub = block_size / kPage;
  const int group = num_q_heads / num_kv_heads;
  // 1. the prefix pass (at most kCascMaxChunks chunks of the longest prefix),
  //    whose workgroups also write the suffix view of every row
  const int max_pre_pages = max_prefix_blocks * nsub;
  const int chunk_pages = max(4, (max_pre_pages + kCascMaxChunks - 1) / kCascMaxChunks);
  if (chunk_pages > kCascMaxChunkPages) return (int)hipErrorInvalidValue;  // prefixes beyond 1M tokens
  {
    CascadeArgs c;
    c.q = (const bf16_t*)q; c.q_st = q_stride_tok; c.q_sh = q_stride_head;
    c.kc = (const bf16_t*)k_cache; c.vc = (const bf16_t*)v_cache;
    c.page_stride = page_stride; c.tok_stride = tok_stride; c.head_stride = head_stride;
    c.bt = block_tables; c.bt_stride = bt_stride; c.seqlens = cache_seqlens;
    c.nsub = nsub; c.block_size = block_size; c.batch = batch; c.max_blocks = max_blocks_per_seq;
    c.grp_info = (const int4*)group_info; c.grp_rows = group_rows; c.pre_tokens = prefix_tokens;
    c.num_groups = max_pre_pages > 0 ? num_groups : 0;
    c.hq = num_q_heads; c.hkv = num_kv_heads; c.chunk_pages = chunk_pages;
    c.pre_o = pre_o; c.pre_lse = pre_lse; c.sbt = sbt; c.ssl = ssl;
    c.scale_log2 = (f8 ? scale * k_scale : scale) * 1.4426950408889634f;
    c.v_scale = f8 ? v_scale : 1.0f;
    c.num_chunks = max(1, (max_pre_pages + chunk_pages - 1) / chunk_pages);
    const dim3 grid((unsigned)max(c.num_groups * c.num_chunks * num_kv_heads, min(batch, 64)));
    if (f8) {
      switch (group) {
        case 1: cascade_prefix_kernel<1, true><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
        case 2: cascade_prefix_kernel<2, true><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
        case 4: cascade_prefix_kernel<4, true><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
        default: cascade_prefix_kernel<8, true><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
      }
    } else {
      switch (group) {
        case 1: cascade_prefix_kernel<1><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
        case 2: cascade_prefix_kernel<2><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
        case 4: cascade_prefix_kernel<4><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
        default: cascade_prefix_kernel<8><<<grid, kCascWaves * 64, 0, stream>>>(c); break;
      }
    }
    XV_CHECK_LAUNCH();
  }
  // 3. the suffix decode and the merge of suffix and prefix partials
  CascadeParts cp;
  cp.pre_tokens = prefix_tokens; cp.chunk_pages = chunk_pages; cp.pre_o = pre_o; cp.pre_lse = pre_lse;
  return decode_chunk(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride, head_stride, sbt,
                      max_blocks_per_seq, ssl, out, out_stride_tok, ws + Lw.dec, Lw.total - Lw.dec, batch,
                      num_q_heads, num_kv_heads, nsub, (int)pages_per_seq(max_blocks_per_seq, block_size),
                      f8 ? scale * k_scale : scale, stream, cp, f8, f8 ? v_scale : 1.0f);
}
}  // namespace

extern "C" int xv_cascade_decode_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                           const void* k_cache, const void* v_cache,
                                           int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                           const int32_t* block_tables, int64_t bt_stride,
                                           const int32_t* cache_seqlens, const int32_t* prefix_tokens,
                                           const int32_t* group_info, const int32_t* group_rows,
                                           int num_groups, int max_prefix_blocks,
                                           void* out, int64_t out_stride_tok,
                                           void* workspace, size_t workspace_bytes,
                                           int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                           int block_size, int max_blocks_per_seq, float scale,
                                           hipStream_t stream) {
  return cascade_run(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride, head_stride,
                     block_tables, bt_stride, cache_seqlens, prefix_tokens, group_info, group_rows, num_groups,
                     max_prefix_blocks, out, out_stride_tok, workspace, workspace_bytes, batch, num_q_heads,
                     num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, stream, false, 1.0f, 1.0f);
}

// The same on fp8 (e4m3fn) K/V pages, scales as in xv_paged_decode_attention_fp8.
extern "C" int xv_cascade_decode_attention_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                               const void* k_cache, const void* v_cache,
                                               int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                               const int32_t* block_tables, int64_t bt_stride,
                                               const int32_t* cache_seqlens, const int32_t* prefix_tokens,
                                               const int32_t* group_info, const int32_t* group_rows,
                                               int num_groups, int max_prefix_blocks,
                                               void* out, int64_t out_stride_tok,
                                               void* workspace, size_t workspace_bytes,
                                               int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                               int block_size, int max_blocks_per_seq, float scale,
                                               float k_scale, float v_scale, hipStream_t stream) {
  if (!(k_scale > 0.0f) || !(v_scale > 0.0f) || !isfinite(k_scale) || !isfinite(v_scale))
    return (int)hipErrorInvalidValue;
  return cascade_run(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride, head_stride,
                     block_tables, bt_stride, cache_seqlens, prefix_tokens, group_info, group_rows, num_groups,
                     max_prefix_blocks, out, out_stride_tok, workspace, workspace_bytes, batch, num_q_heads,
                     num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, stream, true, k_scale, v_scale);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the workspace is `scratch`, a file-scope device
// array of kScratchBytes that every GPU the library runs on holds until the
// process ends.  Host code never uses the array's name as an address (on the
// host it is only a stand-in): the device address is looked up once per
// device with hipGetSymbolAddress, with that device current, and kept per
// device.  The decode kernels need no initial workspace contents (counts and
// partials are written before they are read), so nothing is cleared.  All
// calls on one device share its array: calls that overlap on one GPU (other
// streams, other threads) race.
constexpr size_t kScratchBytes = (size_t)48 << 20;
__device__ __align__(256) char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first
// call per device).
hipError_t scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return hipSuccess;
}
}  // namespace

extern "C" int xv_paged_decode_attention_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                                 const void* k_cache, const void* v_cache,
                                                 int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                                 const int32_t* block_tables, int64_t bt_stride,
                                                 const int32_t* cache_seqlens,
                                                 void* out, int64_t out_stride_tok,
                                                 int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                                 int block_size, int max_blocks_per_seq, float scale,
                                                 hipStream_t stream) {
  // arguments and the workspace this call needs, checked before the device is touched
  const int rc0 = decode_check(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride,
                               head_stride, out, out_stride_tok, batch, num_q_heads, num_kv_heads, head_dim,
                               block_size, max_blocks_per_seq);
  if (rc0 || batch == 0) return rc0;
  if (xv_paged_decode_workspace_size(batch, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size, head_dim) >
      kScratchBytes)
    return (int)hipErrorInvalidValue;
  void* ws = nullptr;
  const hipError_t e = scratch_ptr(&ws);
  if (e != hipSuccess) return (int)e;
  return decode_run(q, q_stride_tok, q_stride_head, k_cache, v_cache, page_stride, tok_stride, head_stride,
                    block_tables, bt_stride, cache_seqlens, out, out_stride_tok, ws, kScratchBytes, batch,
                    num_q_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, scale, stream);
}
