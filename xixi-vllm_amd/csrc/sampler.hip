// Vocab-wide sampler for gfx950: greedy argmax, temperature / top-k / top-p /
// min-p with an explicit uniform per row.  Four launch shapes share the
// arithmetic below: one 1024-thread workgroup per row (sample_kernel), the
// all-greedy argmax over several workgroups per row (greedy_segment_kernel),
// the sampled path over several workgroups per row for batches of up to
// kSegMaxBatch rows (seg_stats / seg_hist / row_finish), and for calls whose every
// top_k is at most 64 a two-launch top-k path (seg_topk / row_topk); all give
// the same ids.
//
// Greedy rows follow torch.argmax, the reference's greedy: the lowest NaN id
// if the row holds a NaN, else the largest logit at its lowest id.  Sampled
// rows drop NaN logits (the reference's softmax would turn the whole row NaN).
// Candidates are ordered by descending logit, ties by ascending id.  Every
// candidate's probability mass is an exact int64
//   q = trunc(2^40 * 2^d),  d = (l * (1/T) - x_max) * log2 e  (<= 0)
// with a fixed Taylor exp2 (explicit FMAs) shared with the C restatement of the
// oracle, so kept sets, masses and token ids are bit-identical to it.
//
// Fast path (every row whose boundary fits in LDS):
//   1. one pass: max and min keys;
//   2. one pass: q of every candidate, binned by distance below the max,
//      bucket = min(255, floor(-bs d)) with bs = 16 buckets per binary order,
//      or finer for rows spanning less than 255/16 orders (per-wave LDS
//      histograms of counts and masses, the far bucket in registers);
//   3. the buckets give the bucket holding each cut-off: top-k (by count),
//      top-p (first bucket whose inclusive mass exceeds floor(top_p * mass of
//      the top-k set)), min-p (bucket of the smallest key whose probability
//      reaches min_p of the largest); only the earliest such bucket's
//      candidates are gathered to LDS and bitonic-sorted, which gives the exact
//      boundary candidate (key, id) and the kept mass M;
//   4. one pass: inverse CDF in ascending id order, exp only for kept ids:
//      the first kept id whose inclusive mass exceeds floor(u * M).
// A boundary bucket larger than LDS falls back to an exact row-wide two-level
// (high byte, low byte) radix select over LDS histograms.
#include "xv_common.h"
#include "xv_kernels.h"
#include <math.h>

#pragma clang fp contract(off)


namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int64_t kTieAll = 0x7fffffffffffffffll;
constexpr int kBuckets = 256;
constexpr int kMaxCand = 8192;  // candidates of one bucket sorted in LDS

XV_INLINE float sampler_exp2(float x) {
  if (!(x > -125.0f)) return 0.0f;
  float n = __builtin_rintf(x);
  float f = x - n;
  float p = 1.5252733646775596e-05f;
  p = __builtin_fmaf(p, f, 1.5403529687318951e-04f);
  p = __builtin_fmaf(p, f, 1.3333557872101665e-03f);
  p = __builtin_fmaf(p, f, 9.6181286498904228e-03f);
  p = __builtin_fmaf(p, f, 5.5504109710454941e-02f);
  p = __builtin_fmaf(p, f, 2.4022650718688965e-01f);
  p = __builtin_fmaf(p, f, 6.9314718246459961e-01f);
  p = __builtin_fmaf(p, f, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

XV_INLINE uint32_t order_key(uint32_t b) {  // 0 is reserved for NaN / padding
  if ((b & 0x7fffu) > 0x7f80u) return 0u;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
XV_INLINE uint32_t key_to_bits(uint32_t k) { return (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu); }

// d = (l / T - x_max) * log2 e, evaluated as the oracle does
XV_INLINE float log2_ratio(uint32_t bits, float inv_t, float zmax) {
  float z = bf16_to_f32(bits) * inv_t;
  float d = z - zmax;
  return d * 1.44269502162933349609375f;
}
XV_INLINE float exp_of(uint32_t bits, float inv_t, float zmax) { return sampler_exp2(log2_ratio(bits, inv_t, zmax)); }
// e is in [0, 1] (exp2 of d <= 0; NaN gives 0), so the product converts as
// an unsigned value: the same integer, without the signed conversion's sign
// handling (about half its instructions).
XV_INLINE int64_t mass_of(float e) { return (int64_t)(uint64_t)(e * 1099511627776.0f); }
// Bucket of a candidate d below the max: floor(-d * bs), the last bucket
// holding everything further.  bs is per row (bucket_scale); any bs > 0 keeps
// the buckets monotone in the key, which is all the boundary search needs.
XV_INLINE int bucket_of(float d, float bs) {
  const float u = -d * bs;  // >= 0 for every candidate (d <= 0); NaN -> last bucket
  return u < 255.0f ? (u > 0.0f ? (int)u : 0) : 255;
}
// 16 buckets per binary order, finer when the row spans less than 255/16
// orders below its max (near-flat rows), so that the smallest candidate lands
// in the last bucket and the row spreads over all of them.
XV_INLINE float bucket_scale(float dmin) {
  return (-dmin * 16.0f >= 255.0f || !(-dmin > 1e-30f)) ? 16.0f : 255.0f / -dmin;
}

// Load the 8 logits of thread t in tile j (bits, 0xffff = NaN for padding).
XV_INLINE void load8(const bf16_t* row, int V, int base, bool vec_ok, uint32_t (&bits)[8]) {
  if (vec_ok && base + 8 <= V) {
    Vec8 v = load_vec8(row + base);
#pragma unroll
    for (int k = 0; k < 4; ++k) { bits[2 * k] = v.w[k] & 0xffffu; bits[2 * k + 1] = v.w[k] >> 16; }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) bits[k] = (base + k < V) ? (uint32_t)row[base + k] : 0xffffu;
  }
}

// Apply f(bits, id) to every id of this thread's contiguous range
// [t*C, t*C + C), C a multiple of 8: chunks of kChunk 16-byte loads are issued
// together, so a pass over the row costs a few memory round trips, not one
// per vector.  Thread order is id order.
constexpr int kChunk = 8;
XV_INLINE int range_len(int V) { return ((V + kThreads - 1) / kThreads + 7) / 8 * 8; }
// Apply f(bits, id) to the ids of a coalesced, lane-interleaved layout: in
// step c, vector v of thread t is id 8*((c*kChunk + v)*kThreads + t).  Ids
// ascend within a thread.  Order across threads is not id order.
template <typename F>
XV_INLINE void for_each_strided(const bf16_t* row, int V, bool vec_ok, F&& f) {
  const int nvec = (V + 7) / 8;
  for (int c = 0; c * kChunk * kThreads < nvec; ++c) {
    uint32_t bits[kChunk][8];
#pragma unroll
    for (int v = 0; v < kChunk; ++v) {
      const int vi = (c * kChunk + v) * kThreads + threadIdx.x;
      if (vi < nvec) load8(row, V, vi * 8, vec_ok, bits[v]);
    }
#pragma unroll
    for (int v = 0; v < kChunk; ++v) {
      const int vi = (c * kChunk + v) * kThreads + threadIdx.x;
      if (vi < nvec)
#pragma unroll
        for (int k = 0; k < 8; ++k) f(bits[v][k], vi * 8 + k);
    }
  }
}

template <int CH = kChunk, typename F>
XV_INLINE void for_each_elem(const bf16_t* row, int V, bool vec_ok, F&& f) {
  const int C = range_len(V);
  const int i0 = threadIdx.x * C, i1 = min(V, i0 + C);
  for (int c = i0; c < i1; c += 8 * CH) {
    uint32_t bits[CH][8];
#pragma unroll
    for (int v = 0; v < CH; ++v)
      if (c + 8 * v < i1) load8(row, V, c + 8 * v, vec_ok, bits[v]);
#pragma unroll
    for (int v = 0; v < CH; ++v)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int id = c + 8 * v + k;
        if (id < i1) f(bits[v][k], id);
      }
  }
}

struct Shared {
  uint32_t red_u[kWaves];
  float red_f[kWaves];
  int64_t red_l[kWaves];
  int64_t red_l2[kWaves];
  uint32_t cnt[256];
  unsigned long long mass[256];
  // broadcast slots
  uint32_t b_key;
  int64_t b_tie;
  int64_t b_id;
  int64_t b_total;
  int b_hb;
  int b_int[8];
  int64_t b_long[8];
};

// LDS of the fast path: per-wave bucket histograms, then the candidate list
struct FastShared {
  uint32_t wcnt[kWaves][kBuckets];
  unsigned long long wmass[kWaves][kBuckets];
  unsigned long long cand[kMaxCand];  // (key << 32) | (0xffffffff - id), sorted descending
  int ncand;
};

// x[lane ^ S] in registers, no LDS round trip: DPP within a 16-lane row for
// S = 1, 2 (quad_perm), 8 (row_ror:8) and 4 (row_ror:4 for lanes with bit 2
// set, row_ror:12 for the others: row_ror:n reads lane (i - n) mod 16), the
// gfx950 row-swap permutes for 16 and 32 (each result holds x[lane] in one
// half of the rows and x[lane ^ S] in the other).
template <int CTRL>
XV_INLINE uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
}
template <int S>
XV_INLINE uint32_t xor_lane(uint32_t x) {
  const int lane = threadIdx.x & 63;
  if constexpr (S == 1) return dpp_u<0xB1>(x);
  else if constexpr (S == 2) return dpp_u<0x4E>(x);
  else if constexpr (S == 4) { const uint32_t a = dpp_u<0x124>(x), b = dpp_u<0x12C>(x); return (lane & 4) ? a : b; }
  else if constexpr (S == 8) return dpp_u<0x128>(x);
  else if constexpr (S == 16) { const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false); return (lane & 16) ? r[0] : r[1]; }
  else { static_assert(S == 32, "xor by a power of two below 64"); const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false); return (lane & 32) ? r[0] : r[1]; }
}
template <int S>
XV_INLINE unsigned long long xor_lane64(unsigned long long x) {
  return ((unsigned long long)xor_lane<S>((uint32_t)(x >> 32)) << 32) | xor_lane<S>((uint32_t)x);
}
XV_INLINE unsigned long long xor_lane64(unsigned long long x, int s) {  // s a constant after unrolling
  switch (s) {
    case 1: return xor_lane64<1>(x);
    case 2: return xor_lane64<2>(x);
    case 4: return xor_lane64<4>(x);
    case 8: return xor_lane64<8>(x);
    case 16: return xor_lane64<16>(x);
    default: return xor_lane64<32>(x);
  }
}
// Wave-wide reductions through the register permutes above (the shuffles
// they replace each took an LDS round trip, two for 64-bit values).
XV_INLINE uint32_t wave_max_u(uint32_t x) {
  x = max(x, xor_lane<1>(x));
  x = max(x, xor_lane<2>(x));
  x = max(x, xor_lane<4>(x));
  x = max(x, xor_lane<8>(x));
  x = max(x, xor_lane<16>(x));
  return max(x, xor_lane<32>(x));
}
XV_INLINE uint32_t wave_min_u(uint32_t x) {
  x = min(x, xor_lane<1>(x));
  x = min(x, xor_lane<2>(x));
  x = min(x, xor_lane<4>(x));
  x = min(x, xor_lane<8>(x));
  x = min(x, xor_lane<16>(x));
  return min(x, xor_lane<32>(x));
}
XV_INLINE float wave_maxf(float x) {
  x = fmaxf(x, __uint_as_float(xor_lane<1>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xor_lane<2>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xor_lane<4>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xor_lane<8>(__float_as_uint(x))));
  x = fmaxf(x, __uint_as_float(xor_lane<16>(__float_as_uint(x))));
  return fmaxf(x, __uint_as_float(xor_lane<32>(__float_as_uint(x))));
}
XV_INLINE int64_t wave_min_l(int64_t x) {
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) {
    const int64_t y = (int64_t)xor_lane64(x, sh);
    x = y < x ? y : x;
  }
  return x;
}
XV_INLINE unsigned long long wave_max_ull(unsigned long long x) {
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) {
    const unsigned long long y = xor_lane64(x, sh);
    x = y > x ? y : x;
  }
  return x;
}


// x[lane - S] within the lane's 16-lane row (0 for the first S lanes of a
// row), and the cross-row broadcasts of lane 15 (into rows 1, 3) and lane 31
// (into rows 2, 3); other lanes get 0.
template <int CTRL, int ROWS>
XV_INLINE uint64_t dpp64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)x, CTRL, ROWS, 0xf, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(x >> 32), CTRL, ROWS, 0xf, true);
  return ((uint64_t)hi << 32) | lo;
}
XV_INLINE int64_t wave_sum_l(int64_t x) {
  x += (int64_t)xor_lane64<1>((uint64_t)x);
  x += (int64_t)xor_lane64<2>((uint64_t)x);
  x += (int64_t)xor_lane64<4>((uint64_t)x);
  x += (int64_t)xor_lane64<8>((uint64_t)x);
  x += (int64_t)xor_lane64<16>((uint64_t)x);
  x += (int64_t)xor_lane64<32>((uint64_t)x);
  return x;
}
// Inclusive prefix sum over the wave's lanes: within rows by row_shr 1, 2, 4,
// 8, then row 1 and 3 add lane 15 of the row before, rows 2 and 3 lane 31.
XV_INLINE int64_t wave_incl_scan_l(int64_t x) {
  x += (int64_t)dpp64<0x111, 0xf>((uint64_t)x);
  x += (int64_t)dpp64<0x112, 0xf>((uint64_t)x);
  x += (int64_t)dpp64<0x114, 0xf>((uint64_t)x);
  x += (int64_t)dpp64<0x118, 0xf>((uint64_t)x);
  x += (int64_t)dpp64<0x142, 0xa>((uint64_t)x);
  x += (int64_t)dpp64<0x143, 0xc>((uint64_t)x);
  return x;
}

XV_INLINE uint32_t block_max_u(Shared& s, uint32_t x) {
  x = wave_max_u(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.red_u[w] = x;
  __syncthreads();
  uint32_t r = s.red_u[0];
  for (int i = 1; i < kWaves; ++i) r = max(r, s.red_u[i]);
  return r;
}
XV_INLINE uint32_t block_min_u(Shared& s, uint32_t x) {
  x = wave_min_u(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.red_u[w] = x;
  __syncthreads();
  uint32_t r = s.red_u[0];
  for (int i = 1; i < kWaves; ++i) r = min(r, s.red_u[i]);
  return r;
}
XV_INLINE float block_maxf(Shared& s, float x) {
  x = wave_maxf(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.red_f[w] = x;
  __syncthreads();
  float r = s.red_f[0];
  for (int i = 1; i < kWaves; ++i) r = fmaxf(r, s.red_f[i]);
  return r;
}
XV_INLINE int64_t block_sum_l(Shared& s, int64_t x) {
  x = wave_sum_l(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.red_l[w] = x;
  __syncthreads();
  int64_t r = 0;
  for (int i = 0; i < kWaves; ++i) r += s.red_l[i];
  return r;
}
// Exclusive prefix sum over the block (thread order); *total gets the block sum.
XV_INLINE int64_t block_excl_scan(Shared& s, int64_t x, int64_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t inc = wave_incl_scan_l(x);
  __syncthreads();
  if (lane == 63) s.red_l[w] = inc;
  __syncthreads();
  int64_t before = 0, tot = 0;
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) before += s.red_l[i];
    tot += s.red_l[i];
  }
  *total = tot;
  return before + inc - x;
}

// Two exclusive prefix sums over the block at once (one pair of barriers).
XV_INLINE void block_excl_scan2(Shared& s, int64_t x, int64_t y, int64_t* ex, int64_t* ey, int64_t* tx,
                                int64_t* ty) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t ix = wave_incl_scan_l(x), iy = wave_incl_scan_l(y);
  __syncthreads();
  if (lane == 63) {
    s.red_l[w] = ix;
    s.red_l2[w] = iy;
  }
  __syncthreads();
  int64_t bx = 0, by = 0, sx = 0, sy = 0;
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) {
      bx += s.red_l[i];
      by += s.red_l2[i];
    }
    sx += s.red_l[i];
    sy += s.red_l2[i];
  }
  *ex = bx + ix - x;
  *ey = by + iy - y;
  *tx = sx;
  *ty = sy;
}

struct Boundary {
  uint32_t key;  // kept: key > key, or key == key with tie index <= tie
  int64_t tie;   // kTieAll: every tie of `key` kept
};
XV_INLINE bool earlier(const Boundary& a, const Boundary& b) {
  return a.key > b.key || (a.key == b.key && a.tie < b.tie);
}

// Call f(bits, id) for every slot of a lane-interleaved layout like that of
// for_each_strided (kChunkAll vectors per step) on every lane of every wave: slots at or past V come as
// 0xffff (key 0), so f may use wave-wide operations.
constexpr int kChunkAll = 8;
template <typename F>
XV_INLINE void for_each_strided_all(const bf16_t* row, int V, bool vec_ok, F&& f) {
  const int nvec = (V + 7) / 8;
  for (int c = 0; c * kChunkAll * kThreads < nvec; ++c) {
    uint32_t w[kChunkAll][4];  // packed pairs, low half first
#pragma unroll
    for (int v = 0; v < kChunkAll; ++v) {
      const int base = ((c * kChunkAll + v) * kThreads + threadIdx.x) * 8;
      if (vec_ok && base + 8 <= V) {
        const Vec8 x = load_vec8(row + base);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[v][k] = x.w[k];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          w[v][k] = (base + 2 * k < V ? (uint32_t)row[base + 2 * k] : 0xffffu) |
                    (base + 2 * k + 1 < V ? (uint32_t)row[base + 2 * k + 1] : 0xffffu) << 16;
      }
    }
#pragma unroll
    for (int v = 0; v < kChunkAll; ++v)
#pragma unroll
      for (int k = 0; k < 8; ++k)
        f((w[v][k >> 1] >> (16 * (k & 1))) & 0xffffu, ((c * kChunkAll + v) * kThreads + threadIdx.x) * 8 + k);
  }
}

// Add one count (CNT) and the mass m (MASS) to bin `bin` of the LDS
// histograms for every lane with `on`.  The lanes of each of the wave's first
// four distinct bins are summed first and added with one atomic per
// histogram: near-flat rows put nearly every candidate into two or three
// high-byte bins, where per-lane atomics to one address serialise.  Lanes of
// further bins add their own.  Called by the whole wave.
template <bool CNT, bool MASS>
XV_INLINE void hist_add(uint32_t* cnt, unsigned long long* mass, bool on, int bin, int64_t m) {
  const int lane = threadIdx.x & 63;
  bool pending = on;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const unsigned long long todo = __ballot(pending);
    if (todo == 0ull) break;
    const int lead = __builtin_ctzll(todo);
    const int lb = __shfl(bin, lead);
    const bool mine = pending && bin == lb;
    const unsigned long long mm = __ballot(mine);
    const int64_t sm = MASS ? wave_sum_l(mine ? m : 0) : 0;
    if (lane == lead) {
      if (CNT) atomicAdd(&cnt[lb], (uint32_t)__popcll(mm));
      if (MASS) atomicAdd(&mass[lb], (unsigned long long)sm);
    }
    pending = pending && !mine;
  }
  if (pending) {
    if (CNT) atomicAdd(&cnt[bin], 1u);
    if (MASS) atomicAdd(&mass[bin], (unsigned long long)m);
  }
}

XV_INLINE void clear_hist(Shared& s) {
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += kThreads) { s.cnt[i] = 0; s.mass[i] = 0; }
  __syncthreads();
}

// Exact cut-offs by a two-level (high byte, low byte) radix select over LDS
// histograms of the whole row: the fallback when the boundary bucket of the
// fast path holds more candidates than LDS does (very flat distributions).
// Histogram passes read the row in chunks of kChunk vectors per thread (a few
// memory round trips per pass).
XV_INLINE void general_boundary(Shared& s, const bf16_t* row, int V, bool vec_ok, float inv_t, float zmax,
                                int top_k, float top_p, float min_p, bool use_k, bool use_p, bool use_m,
                                Boundary& bd_out, int64_t& id_cut_out, int64_t& M_out) {
  const int t = threadIdx.x;
  Boundary bd = {1u, kTieAll};
  if (use_k || use_p || use_m) {
    // ---- pass 2: high-byte histogram of counts and masses; min-p key ----
    clear_hist(s);
    uint32_t kmin_p = 0xffffffffu;
    for_each_strided_all(row, V, vec_ok, [&](uint32_t bits, int) {
      const uint32_t key = order_key(bits);
      const float e = exp_of(bits, inv_t, zmax);
      if (use_m && key && e >= min_p) kmin_p = min(kmin_p, key);
      hist_add<true, true>(s.cnt, s.mass, key != 0, (int)(key >> 8), mass_of(e));
    });
    kmin_p = use_m ? block_min_u(s, kmin_p) : 0u;
    __syncthreads();

    // boundary of top-k (by count), and total mass of the top-k set
    int64_t total_k = 0;
    if (t == 0) {
      int64_t tot = 0;
      for (int i = 0; i < 256; ++i) tot += (int64_t)s.mass[i];
      s.b_total = tot;
      if (use_k) {
        int64_t c = 0;
        int hb = 255;
        for (; hb > 0; --hb) {
          if (c + s.cnt[hb] > (uint32_t)(top_k - 1)) break;
          c += s.cnt[hb];
        }
        s.b_hb = hb;
        s.b_tie = c;  // count above the bin
      }
    }
    __syncthreads();
    Boundary bk = {1u, kTieAll};
    if (use_k) {
      // ---- pass 3: low-byte histogram inside the top-k high bin ----
      const int hb = s.b_hb;
      const int64_t c_above = s.b_tie;
      clear_hist(s);
      for_each_strided_all(row, V, vec_ok, [&](uint32_t bits, int) {
        const uint32_t key = order_key(bits);
        hist_add<true, false>(s.cnt, s.mass, key != 0 && (int)(key >> 8) == hb, (int)(key & 255), 0);
      });
      __syncthreads();
      if (t == 0) {
        int64_t c = c_above;
        int lb = 255;
        for (; lb > 0; --lb) {
          if (c + s.cnt[lb] > top_k - 1) break;
          c += s.cnt[lb];
        }
        s.b_key = ((uint32_t)hb << 8) | (uint32_t)lb;
        s.b_tie = (int64_t)(top_k - 1) - c;
      }
      __syncthreads();
      bk.key = s.b_key;
      bk.tie = s.b_tie;
      // mass of the top-k set: everything above the boundary key plus tie_k+1 copies
      int64_t above = 0;
      for_each_strided(row, V, vec_ok, [&](uint32_t bits, int) {
        if (order_key(bits) > bk.key) above += mass_of(exp_of(bits, inv_t, zmax));
      });
      above = block_sum_l(s, above);
      total_k = above + (bk.tie + 1) * mass_of(exp_of(key_to_bits(bk.key), inv_t, zmax));
    } else {
      total_k = s.b_total;
    }

    Boundary bp = {1u, kTieAll};
    if (use_p) {
      // ---- pass 4: first rank whose inclusive mass exceeds floor(top_p * total_k) ----
      const int64_t thr = (int64_t)floor((double)top_p * (double)total_k);
      if (use_k) {
        // pass 3 reused the histograms: rebuild the high-byte masses
        clear_hist(s);
        for_each_strided_all(row, V, vec_ok, [&](uint32_t bits, int) {
          const uint32_t key = order_key(bits);
          hist_add<false, true>(s.cnt, s.mass, key != 0, (int)(key >> 8), mass_of(exp_of(bits, inv_t, zmax)));
        });
      }
      __syncthreads();
      if (t == 0) {
        int64_t m = 0;
        int hb = 255;
        bool found = false;
        for (; hb >= 0; --hb) {
          if (m + (int64_t)s.mass[hb] > thr) { found = true; break; }
          m += (int64_t)s.mass[hb];
        }
        s.b_hb = found ? hb : -1;
        s.b_total = m;
      }
      __syncthreads();
      const int hb = s.b_hb;
      const int64_t m_above = s.b_total;
      if (hb >= 0) {
        clear_hist(s);
        for_each_strided_all(row, V, vec_ok, [&](uint32_t bits, int) {
          const uint32_t key = order_key(bits);
          const bool in = key != 0 && (int)(key >> 8) == hb;
          hist_add<false, true>(s.cnt, s.mass, in, (int)(key & 255), in ? mass_of(exp_of(bits, inv_t, zmax)) : 0);
        });
        __syncthreads();
        if (t == 0) {
          int64_t m = m_above;
          int lb = 255;
          for (; lb > 0; --lb) {
            if (m + (int64_t)s.mass[lb] > thr) break;
            m += (int64_t)s.mass[lb];
          }
          const uint32_t key = ((uint32_t)hb << 8) | (uint32_t)lb;
          const int64_t q = mass_of(exp_of(key_to_bits(key), inv_t, zmax));
          s.b_key = key;
          s.b_tie = q > 0 ? (thr - m) / q : kTieAll;
        }
        __syncthreads();
        bp.key = s.b_key;
        bp.tie = s.b_tie;
      }
    }
    bd = bk;
    if (earlier(bp, bd)) bd = bp;
    if (use_m && kmin_p != 0xffffffffu) {
      Boundary bm = {kmin_p, kTieAll};
      if (earlier(bm, bd)) bd = bm;
    }
  }

  // ---- pass 5: kept mass, and the id of the last kept tie of the boundary key ----
  // Thread t owns the contiguous ids of for_each_elem, so one block scan of the
  // per-thread tie counts ranks the ties in id order.  Every tie has the same
  // mass q.
  int64_t above = 0, nt = 0;
  for_each_elem(row, V, vec_ok, [&](uint32_t bits, int) {
    const uint32_t key = order_key(bits);
    if (key > bd.key) above += mass_of(exp_of(bits, inv_t, zmax));
    nt += key == bd.key;
  });
  int64_t ties;
  const int64_t r0 = block_excl_scan(s, nt, &ties);
  const int64_t kept_ties = bd.tie == kTieAll ? ties : min(ties, bd.tie + 1);
  const int64_t q = kept_ties ? mass_of(exp_of(key_to_bits(bd.key), inv_t, zmax)) : 0;
  const int64_t M = block_sum_l(s, above) + kept_ties * q;
  if (t == 0) s.b_id = kTieAll;
  __syncthreads();
  if (bd.tie != kTieAll && bd.tie >= r0 && bd.tie < r0 + nt) {
    int64_t r = r0;
    for_each_elem<2>(row, V, vec_ok, [&](uint32_t bits, int id) {  // one thread: few registers
      if (order_key(bits) == bd.key) {
        if (r == bd.tie) s.b_id = id;
        ++r;
      }
    });
  }
  __syncthreads();
  id_cut_out = s.b_id;
  __syncthreads();  // every thread has read b_id before it is reset
  bd_out = bd;
  M_out = M;
}

XV_INLINE int64_t block_min_l(Shared& s, int64_t x) {
  x = wave_min_l(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.red_l[w] = x;
  __syncthreads();
  int64_t r = s.red_l[0];
  for (int i = 1; i < kWaves; ++i) r = s.red_l[i] < r ? s.red_l[i] : r;
  return r;
}

XV_INLINE uint32_t cand_key(unsigned long long c) { return (uint32_t)(c >> 32); }
XV_INLINE int64_t cand_id(unsigned long long c) { return (int64_t)(0xffffffffu - (uint32_t)(c & 0xffffffffu)); }
XV_INLINE int64_t cand_mass(unsigned long long c, float inv_t, float zmax) {
  return mass_of(exp_of(key_to_bits(cand_key(c)), inv_t, zmax));
}

// Bitonic sort of fs.cand[0, n) descending (n <= kMaxCand), padding with
// zeros up to the next power of two; the padding sorts last.
XV_INLINE void sort_cand_desc(FastShared& fs, int n) {
  const int t = threadIdx.x;
  int np2 = 1;
  while (np2 < n) np2 <<= 1;
  for (int i = n + t; i < np2; i += kThreads) fs.cand[i] = 0ull;  // padding sorts last
  __syncthreads();
  for (int size = 2; size <= np2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < np2 / 2; i += kThreads) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const unsigned long long a = fs.cand[lo], b = fs.cand[hi];
        const bool desc = (lo & size) == 0;
        if (desc ? (a < b) : (a > b)) { fs.cand[lo] = b; fs.cand[hi] = a; }
      }
      __syncthreads();
    }
  }
}

// Gather the candidates of bucket `target` into fs.cand and bitonic-sort them
// descending (key descending, id ascending).  Returns the count; a count above
// kMaxCand means the bucket did not fit (nothing sorted).
XV_INLINE int gather_bucket(FastShared& fs, const bf16_t* row, int V, bool vec_ok, float inv_t,
                            float zmax, float bs, int target, int target_lo = -1) {
  if (target_lo < 0) target_lo = target;  // gather buckets target_lo .. target
  const int t = threadIdx.x;
  __syncthreads();
  if (t == 0) fs.ncand = 0;
  __syncthreads();
  for_each_strided(row, V, vec_ok, [&](uint32_t bits, int id) {
    const uint32_t key = order_key(bits);
    if (!key) return;
    const int bkt = bucket_of(log2_ratio(bits, inv_t, zmax), bs);
    if (bkt < target_lo || bkt > target) return;
    const int slot = atomicAdd(&fs.ncand, 1);
    if (slot < kMaxCand)
      fs.cand[slot] = ((unsigned long long)key << 32) | (unsigned long long)(0xffffffffu - (uint32_t)id);
  });
  __syncthreads();
  const int n = fs.ncand;
  if (n > kMaxCand) return n;
  sort_cand_desc(fs, n);
  return n;
}

// Sum of the masses of the first m sorted candidates.
XV_INLINE int64_t list_mass_prefix(Shared& s, const FastShared& fs, int n, int64_t m, float inv_t, float zmax) {
  const int per = (n + kThreads - 1) / kThreads;
  const int i0 = threadIdx.x * per, i1 = min(n, i0 + per);
  int64_t sum = 0;
  for (int i = i0; i < i1; ++i)
    if (i < m) sum += cand_mass(fs.cand[i], inv_t, zmax);
  return block_sum_l(s, sum);
}

// First sorted index whose inclusive mass (plus base) exceeds thr, n if none.
XV_INLINE int64_t list_first_exceed(Shared& s, const FastShared& fs, int n, int64_t base, int64_t thr, float inv_t,
                                    float zmax) {
  const int per = (n + kThreads - 1) / kThreads;
  const int i0 = threadIdx.x * per, i1 = min(n, i0 + per);
  int64_t local = 0;
  for (int i = i0; i < i1; ++i) local += cand_mass(fs.cand[i], inv_t, zmax);
  int64_t tot;
  int64_t cum = base + block_excl_scan(s, local, &tot);
  int64_t found = n;
  for (int i = i0; i < i1; ++i) {
    cum += cand_mass(fs.cand[i], inv_t, zmax);
    if (cum > thr) { found = i; break; }
  }
  return block_min_l(s, found);
}

// Number of sorted candidates with key >= kmin (a prefix of the list).
XV_INLINE int64_t list_count_ge(Shared& s, const FastShared& fs, int n, uint32_t kmin) {
  int64_t c = 0;
  for (int i = threadIdx.x; i < n; i += kThreads) c += cand_key(fs.cand[i]) >= kmin;
  return block_sum_l(s, c);
}

// Smallest key whose probability reaches min_p of the largest (0xffffffff:
// none).  Only candidates within half a binary order of the threshold need an
// exp: below that their probability is certainly under min_p.
XV_INLINE uint32_t minp_key(Shared& s, const bf16_t* row, int V, bool vec_ok, float inv_t, float zmax,
                            float min_p) {
  const float d_lo = __log2f(min_p) - 0.5f;
  uint32_t kminp = 0xffffffffu;
  for_each_strided(row, V, vec_ok, [&](uint32_t bits, int) {
    const uint32_t key = order_key(bits);
    if (!key) return;
    const float d = log2_ratio(bits, inv_t, zmax);
    if (d >= d_lo && sampler_exp2(d) >= min_p) kminp = min(kminp, key);
  });
  return block_min_u(s, kminp);
}

// Fast path with top-k: bucket counts only (no exp), then every candidate of
// the buckets up to the one holding rank k-1 is gathered and sorted; the
// top-k set, its mass, the top-p and min-p cuts all come from that list.
XV_INLINE bool topk_boundary(Shared& s, FastShared& fs, const bf16_t* row, int V, bool vec_ok,
                             float inv_t, float zmax, float bs, int top_k, float top_p, float min_p, bool use_p, bool use_m,
                             uint32_t& key_cut, int64_t& id_cut, int64_t& M, int& list_kept) {
  const int t = threadIdx.x, w = t >> 6;
  for (int i = t; i < kWaves * kBuckets; i += kThreads) (&fs.wcnt[0][0])[i] = 0u;
  __syncthreads();
  int64_t far_c = 0;
  for_each_strided(row, V, vec_ok, [&](uint32_t bits, int) {
    if (!order_key(bits)) return;
    const int bkt = bucket_of(log2_ratio(bits, inv_t, zmax), bs);
    if (bkt < kBuckets - 1) atomicAdd(&fs.wcnt[w][bkt], 1u);
    else far_c += 1;
  });
  far_c = block_sum_l(s, far_c);
  __syncthreads();
  if (t < kBuckets) {
    uint32_t c = 0;
    for (int ww = 0; ww < kWaves; ++ww) c += fs.wcnt[ww][t];
    if (t == kBuckets - 1) c += (uint32_t)far_c;
    s.cnt[t] = c;
  }
  __syncthreads();
  int bk = kBuckets;
  int64_t upto = 0;  // candidates in buckets 0..bk
  {
    int64_t c = 0;
    for (int bkt = 0; bkt < kBuckets; ++bkt) {
      c += s.cnt[bkt];
      if (c >= top_k) { bk = bkt; upto = c; break; }
    }
  }
  if (bk >= kBuckets - 1 || upto > kMaxCand) return false;  // rank k-1 far out or too many: exact row-wide path
  const uint32_t kminp = use_m ? minp_key(s, row, V, vec_ok, inv_t, zmax, min_p) : 0xffffffffu;
  const int n = gather_bucket(fs, row, V, vec_ok, inv_t, zmax, bs, bk, 0);
  if (n > kMaxCand) return false;
  const int64_t total_k = list_mass_prefix(s, fs, n, top_k, inv_t, zmax);
  int64_t jcut = (int64_t)top_k - 1;
  if (use_p) {
    const int64_t thr = (int64_t)floor((double)top_p * (double)total_k);
    jcut = min(jcut, list_first_exceed(s, fs, n, 0, thr, inv_t, zmax));
  }
  if (use_m && kminp != 0xffffffffu && kminp >= cand_key(fs.cand[n - 1]))
    jcut = min(jcut, list_count_ge(s, fs, n, kminp) - 1);
  if (jcut >= n) jcut = n - 1;
  if (jcut < 0) jcut = 0;
  const unsigned long long edge = fs.cand[jcut];
  key_cut = cand_key(edge);
  id_cut = cand_id(edge);
  M = list_mass_prefix(s, fs, n, jcut + 1, inv_t, zmax);
  list_kept = (int)jcut + 1;  // the kept set is exactly fs.cand[0, jcut]
  return true;
}

// Fast path: kept set = key > key_cut, or key == key_cut and id <= id_cut;
// M = its mass.  Returns false when a boundary bucket overflowed the list.
XV_INLINE bool fast_boundary(Shared& s, FastShared& fs, const bf16_t* row, int V, bool vec_ok,
                             float inv_t, float zmax, float bs, int top_k, float top_p, float min_p, bool use_k, bool use_p,
                             bool use_m, uint32_t& key_cut, int64_t& id_cut, int64_t& M, int& list_kept) {
  const int t = threadIdx.x, w = t >> 6;
  if (use_k) return topk_boundary(s, fs, row, V, vec_ok, inv_t, zmax, bs, top_k, top_p, min_p, use_p, use_m,
                                  key_cut, id_cut, M, list_kept);
  // ---- pass 2: every candidate's mass, binned by distance below the max ----
  for (int i = t; i < kWaves * kBuckets; i += kThreads) {
    (&fs.wcnt[0][0])[i] = 0u;
    (&fs.wmass[0][0])[i] = 0ull;
  }
  __syncthreads();
  int64_t far_c = 0, far_m = 0;
  uint32_t kminp = 0xffffffffu;
  for_each_strided(row, V, vec_ok, [&](uint32_t bits, int) {
    const uint32_t key = order_key(bits);
    if (!key) return;
    const float d = log2_ratio(bits, inv_t, zmax);
    const float e = sampler_exp2(d);
    const int64_t q = mass_of(e);
    const int bkt = bucket_of(d, bs);
    if (bkt < kBuckets - 1) {
      atomicAdd(&fs.wcnt[w][bkt], 1u);
      atomicAdd(&fs.wmass[w][bkt], (unsigned long long)q);
    } else {
      far_c += 1;
      far_m += q;
    }
    if (use_m && e >= min_p) kminp = min(kminp, key);
  });
  far_c = block_sum_l(s, far_c);
  far_m = block_sum_l(s, far_m);
  if (use_m) kminp = block_min_u(s, kminp);
  __syncthreads();
  if (t < kBuckets) {
    uint32_t c = 0;
    unsigned long long m = 0;
    for (int ww = 0; ww < kWaves; ++ww) { c += fs.wcnt[ww][t]; m += fs.wmass[ww][t]; }
    if (t == kBuckets - 1) { c += (uint32_t)far_c; m += (unsigned long long)far_m; }
    s.cnt[t] = c;
    s.mass[t] = m;
  }
  __syncthreads();
  int64_t total = 0;
  for (int bkt = 0; bkt < kBuckets; ++bkt) total += (int64_t)s.mass[bkt];
  key_cut = 1u;
  id_cut = kTieAll;
  M = total;
  if (!(use_k || use_p || use_m)) return true;

  // ---- bucket of each cut-off ----
  int bk = kBuckets;
  int64_t ck_before = 0, mk_before = 0;
  if (use_k) {
    int64_t c = 0, m = 0;
    for (int bkt = 0; bkt < kBuckets; ++bkt) {
      if (c + s.cnt[bkt] >= (uint32_t)top_k) { bk = bkt; ck_before = c; mk_before = m; break; }
      c += s.cnt[bkt];
      m += (int64_t)s.mass[bkt];
    }
  }
  int64_t total_k = total;
  int nk = 0;
  if (bk < kBuckets) {
    if (s.cnt[bk] > (uint32_t)kMaxCand) return false;  // known before gathering
    nk = gather_bucket(fs, row, V, vec_ok, inv_t, zmax, bs, bk);
    if (nk > kMaxCand) return false;
    total_k = mk_before + list_mass_prefix(s, fs, nk, top_k - ck_before, inv_t, zmax);
  }
  int bp = kBuckets;
  int64_t thr = 0, mp_before = 0;
  if (use_p) {
    thr = (int64_t)floor((double)top_p * (double)total_k);
    int64_t m = 0;
    for (int bkt = 0; bkt < kBuckets; ++bkt) {
      if (m + (int64_t)s.mass[bkt] > thr) { bp = bkt; mp_before = m; break; }
      m += (int64_t)s.mass[bkt];
    }
  }
  int bm = kBuckets;
  if (use_m && kminp != 0xffffffffu) bm = bucket_of(log2_ratio(key_to_bits(kminp), inv_t, zmax), bs);
  const int bf = min(bk, min(bp, bm));
  if (bf >= kBuckets) return true;  // no cut-off limits the row: everything kept
  int n = nk;
  if (bf != bk) {
    if (s.cnt[bf] > (uint32_t)kMaxCand) return false;
    n = gather_bucket(fs, row, V, vec_ok, inv_t, zmax, bs, bf);
    if (n > kMaxCand) return false;
  }
  // ---- exact cut inside the boundary bucket ----
  int64_t jcut = kTieAll;
  if (bk == bf) jcut = min(jcut, (int64_t)top_k - ck_before - 1);
  if (bp == bf) jcut = min(jcut, list_first_exceed(s, fs, n, mp_before, thr, inv_t, zmax));
  if (bm == bf) jcut = min(jcut, list_count_ge(s, fs, n, kminp) - 1);
  if (jcut >= n) jcut = n - 1;
  if (jcut < 0) jcut = 0;
  int64_t m_before = 0;
  for (int bkt = 0; bkt < bf; ++bkt) m_before += (int64_t)s.mass[bkt];
  const unsigned long long edge = fs.cand[jcut];
  key_cut = cand_key(edge);
  id_cut = cand_id(edge);
  M = m_before + list_mass_prefix(s, fs, n, jcut + 1, inv_t, zmax);
  return true;
}

// Inverse-CDF draw over a kept set held as the sorted list fs.cand[0, n):
// re-key it as (~id << 32 | key), so that the descending sort puts ids in
// ascending order, then scan its masses.  Returns the first id whose inclusive
// mass exceeds rdraw (kTieAll: none).
XV_INLINE int64_t list_draw(Shared& s, FastShared& fs, int n, float inv_t, float zmax, int64_t rdraw) {
  const int t = threadIdx.x;
  __syncthreads();
  for (int i = t; i < n; i += kThreads) {
    const unsigned long long c = fs.cand[i];
    fs.cand[i] = ((unsigned long long)(0xffffffffu - (uint32_t)cand_id(c)) << 32) | cand_key(c);
  }
  __syncthreads();
  sort_cand_desc(fs, n);
  auto entry_mass = [&](unsigned long long c) {
    return mass_of(exp_of(key_to_bits((uint32_t)(c & 0xffffffffu)), inv_t, zmax));
  };
  const int per = (n + kThreads - 1) / kThreads;
  const int j0 = t * per, j1 = min(n, j0 + per);
  int64_t local = 0;
  for (int j = j0; j < j1; ++j) local += entry_mass(fs.cand[j]);
  int64_t tot;
  int64_t cum = block_excl_scan(s, local, &tot);
  int64_t found = kTieAll;
  for (int j = j0; j < j1; ++j) {
    cum += entry_mass(fs.cand[j]);
    if (cum > rdraw) { found = 0xffffffffu - (uint32_t)(fs.cand[j] >> 32); break; }
  }
  return block_min_l(s, found);
}

// The draw point floor(u * M), clamped to [0, M).
XV_INLINE int64_t draw_point(float u, int64_t M) {
  int64_t r = (int64_t)((double)u * (double)M);
  if (r >= M) r = M - 1;
  if (r < 0) r = 0;
  return r;
}

// The draw's answer when no candidate has mass.  A scaled row maximum z_max
// that is not finite (a largest logit of +inf or -inf, or a finite one past
// fp32's range once divided by the temperature) makes d = z - z_max NaN at
// the largest key (inf - inf), whose exp2 is 0, and -inf below it: every
// mass is 0, and the draw takes the first candidate in rank order, the
// lowest id holding the largest key.  With a finite z_max the largest logit
// has mass 2^40 and is always kept, so this is the only way the kept mass is 0.
XV_INLINE int64_t lowest_id_of_key(Shared& s, const bf16_t* row, int V, bool vec_ok, uint32_t key) {
  uint32_t first = 0xffffffffu;
  for_each_strided(row, V, vec_ok, [&](uint32_t bits, int id) {
    if (id < V && order_key(bits) == key) first = min(first, (uint32_t)id);
  });
  first = block_min_u(s, first);
  return first == 0xffffffffu ? 0 : (int64_t)first;
}

// The whole sampler for row b by one kThreads workgroup.
XV_INLINE void sample_row(Shared& s, FastShared& fs, int b, const bf16_t* __restrict__ logits, int64_t stride, int V,
                          const float* __restrict__ temps, const float* __restrict__ top_ps,
                          const int32_t* __restrict__ top_ks, const float* __restrict__ min_ps,
                          const float* __restrict__ uniforms, int flags, int64_t* __restrict__ out_ids) {
  const int t = threadIdx.x;
  const bf16_t* row = logits + (int64_t)b * stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const float temp = temps ? temps[b] : 1.0f;
  const bool greedy = (flags & XV_SAMPLE_ALL_GREEDY) || temp <= 1e-5f;

  // ---- greedy (torch.argmax): the lowest NaN id if the row holds a NaN,
  // else the max value and the lowest index holding it ----
  if (greedy) {
    // one pass: the lane's max, its lowest id and its lowest NaN id, then the block's
    float fm = -INFINITY;
    uint32_t best = 0xffffffffu, nan_id = 0xffffffffu;
    for_each_strided(row, V, vec_ok, [&](uint32_t bits, int id) {
      if (!order_key(bits)) {
        if (id < V) nan_id = min(nan_id, (uint32_t)id);  // ids past V are padding
        return;
      }
      const float v = bf16_to_f32(bits);
      if (v > fm) { fm = v; best = (uint32_t)id; }  // ids ascend within a lane: keeps the lowest
    });
    nan_id = block_min_u(s, nan_id);
    const float gm = block_maxf(s, fm);
    best = block_min_u(s, fm == gm ? best : 0xffffffffu);
    if (nan_id != 0xffffffffu) best = nan_id;
    if (t == 0) out_ids[b] = best == 0xffffffffu ? 0 : (int64_t)best;
    return;
  }

  // ---- pass 1: the largest key ----
  uint32_t kmax = 0, kmin = 0xffffffffu;
  for_each_strided(row, V, vec_ok, [&](uint32_t bits, int) {
    const uint32_t key = order_key(bits);
    kmax = max(kmax, key);
    if (key) kmin = min(kmin, key);
  });
  kmax = block_max_u(s, kmax);
  kmin = block_min_u(s, kmin);
  const float inv_t = 1.0f / temp;
  const float zmax = bf16_to_f32(key_to_bits(kmax)) * inv_t;
  if (kmax && !__builtin_isfinite(zmax)) {  // no mass anywhere
    const int64_t id = lowest_id_of_key(s, row, V, vec_ok, kmax);
    if (t == 0) out_ids[b] = id;
    return;
  }
  const float bs = kmax ? bucket_scale(log2_ratio(key_to_bits(kmin), inv_t, zmax)) : 16.0f;

  const float top_p = ((flags & XV_SAMPLE_USE_TOP_P) && top_ps) ? top_ps[b] : 1.0f;
  const float min_p = ((flags & XV_SAMPLE_USE_MIN_P) && min_ps) ? min_ps[b] : 0.0f;
  const bool use_p = top_p < 1.0f;
  const bool use_m = min_p > 0.0f;
  // a min-p above 1 keeps the first candidate alone (as row_params)
  const int top_k = min_p > 1.0f ? 1 : ((flags & XV_SAMPLE_USE_TOP_K) && top_ks) ? top_ks[b] : V;
  const bool use_k = top_k > 0 && top_k < V;

  uint32_t key_cut;
  int64_t id_cut, M;
  int list_kept = 0;  // > 0: the kept set is the sorted list prefix fs.cand[0, list_kept)
  if (!fast_boundary(s, fs, row, V, vec_ok, inv_t, zmax, bs, top_k, top_p, min_p, use_k, use_p, use_m,
                     key_cut, id_cut, M, list_kept)) {
    list_kept = 0;
    Boundary bd;
    general_boundary(s, row, V, vec_ok, inv_t, zmax, top_k, top_p, min_p, use_k, use_p, use_m, bd, id_cut,
                     M);
    key_cut = bd.key;
  }

  // ---- last pass: inverse-CDF draw in ascending id order (exp for kept ids only) ----
  // Thread t owns the contiguous ids [t*C, t*C + C), C a multiple of 8, so one
  // block scan orders the whole row.
  const float u = uniforms ? uniforms[b] : 0.5f;
  const int64_t rdraw = draw_point(u, M);
  if (list_kept > 0) {
    const int64_t found = list_draw(s, fs, list_kept, inv_t, zmax, rdraw);
    if (t == 0) out_ids[b] = found == kTieAll ? 0 : found;
    return;
  }
  const int C = ((V + kThreads - 1) / kThreads + 7) / 8 * 8;
  const int i0 = t * C, i1 = min(V, i0 + C);
  auto kept_mass = [&](uint32_t bits, int id) -> int64_t {
    const uint32_t key = order_key(bits);
    const bool kept = key && (key > key_cut || (key == key_cut && (int64_t)id <= id_cut));
    return kept ? mass_of(exp_of(bits, inv_t, zmax)) : 0;
  };
  int64_t mine = 0;
  for_each_elem(row, V, vec_ok, [&](uint32_t bits, int id) { mine += kept_mass(bits, id); });
  __syncthreads();
  if (t == 0) s.b_id = -1;
  int64_t tot;
  int64_t cum = block_excl_scan(s, mine, &tot);
  if (cum <= rdraw && rdraw < cum + mine) {
    for (int i = i0; i < i1 && s.b_id < 0; i += 8) {
      uint32_t bits[8];
      load8(row, V, i, vec_ok, bits);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (i + k >= i1) break;
        cum += kept_mass(bits[k], i + k);
        if (cum > rdraw) { s.b_id = i + k; break; }
      }
    }
  }
  __syncthreads();
  if (t == 0) out_ids[b] = s.b_id >= 0 ? s.b_id : 0;
}

__global__ __launch_bounds__(kThreads) void sample_kernel(const bf16_t* __restrict__ logits, int64_t stride, int V,
                                                          const float* __restrict__ temps,
                                                          const float* __restrict__ top_ps,
                                                          const int32_t* __restrict__ top_ks,
                                                          const float* __restrict__ min_ps,
                                                          const float* __restrict__ uniforms, int flags,
                                                          int64_t* __restrict__ out_ids) {
  __shared__ Shared s;
  __shared__ FastShared fs;
  sample_row(s, fs, blockIdx.x, logits, stride, V, temps, top_ps, top_ks, min_ps, uniforms, flags, out_ids);
}

// ---------------------------------------------------------------------------
// All-greedy batches over several workgroups per row (a small batch would
// leave most CUs idle with one workgroup per row).  A lane keeps the largest
// order key of its ids (-0 folded into +0, which torch.argmax treats as equal)
// and the lowest id holding it, and its lowest NaN id, as the one-workgroup
// path does with float compares.  Each workgroup
// then folds its best into the row's 64-bit slot with one atomic max of
//   order key << 32 | (2^32 - 1 - id)      (greedy_word: NaN above every value)
// (as torch.argmax: a NaN wins, then the largest logit, among equals the lowest id) and counts
// itself in the row's arrival counter; the last workgroup of the row writes the id
// and clears both words for the next call.  Every atomic is awaited before
// the next one is issued, so the count is only bumped after the workgroup's
// max has been performed.  Atomics on one cache line serialise, so each row
// has its own line and is cut into at most 32 segments.
// A lane's greedy candidate as one word that an integer max orders like
// torch.argmax: key << 32 | (2^32 - 1 - id).  A NaN (nid >= 0, the lane's
// lowest NaN id) takes key 0xffff, above every value's order key (at most
// 0xff80, +inf); otherwise the lane's max value fm at its lowest id bid.  0
// means no candidate.
XV_INLINE unsigned long long greedy_word(float fm, int bid, int nid) {
  if (nid >= 0) return (0xffffull << 32) | (0xffffffffu - (uint32_t)nid);
  if (bid < 0) return 0ull;
  const uint32_t fb = __float_as_uint(fm) >> 16;
  return ((unsigned long long)order_key(fb == 0x8000u ? 0u : fb) << 32) | (0xffffffffu - (uint32_t)bid);
}

constexpr int kGreedyThreads = 256;
constexpr int kGreedyUnroll = 2;  // 8-id vectors per lane per step (2, 4, 6, 8, 16 measured)
constexpr int kGreedyLine = 16;  // u64 words per row: its slot, then its arrival counter, one 128-byte line

__global__ __launch_bounds__(kGreedyThreads) void greedy_segment_kernel(const bf16_t* __restrict__ logits,
                                                                        int64_t stride, int V, int seg_len,
                                                                        unsigned long long* __restrict__ slots,
                                                                        unsigned int* __restrict__ arrivals,
                                                                        int64_t* __restrict__ out_ids) {
  const int b = blockIdx.y;
  const bf16_t* row = logits + (int64_t)b * stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int beg = blockIdx.x * seg_len, end = min(V, beg + seg_len);
  // The lane's best as an order key with -0 folded into +0 (torch.argmax
  // treats them as equal), its lowest id, and its lowest NaN id.  A vector's
  // keys are computed two per packed op; only a vector whose largest key
  // beats the lane's best is searched id by id, and a vector holding a NaN
  // or padding (keys outside [0x7f, 0xff80]) goes id by id as well.
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  const u16x2 top2 = {(unsigned short)0x8000u, (unsigned short)0x8000u}, one2 = {(unsigned short)1u, (unsigned short)1u};
  uint32_t bk = 0;
  int bid = -1, nid = -1;
  constexpr int step = kGreedyThreads * 8;
  for (int i0 = beg + threadIdx.x * 8; i0 < end; i0 += kGreedyUnroll * step) {
    uint32_t w[kGreedyUnroll][4];
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u) {
      const int i = i0 + u * step;
      if (i < end && vec_ok && i + 8 <= end) {
        const Vec8 x = load_vec8(row + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[u][k] = x.w[k];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          w[u][k] = (i + 2 * k < end ? (uint32_t)row[i + 2 * k] : 0xffffu) |
                    (i + 2 * k + 1 < end ? (uint32_t)row[i + 2 * k + 1] : 0xffffu) << 16;
      }
    }
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u) {
      const int i = i0 + u * step;
      if (i >= end) break;
      uint32_t kk[4];
      u16x2 hi2 = {(unsigned short)0u, (unsigned short)0u}, lo2 = {(unsigned short)0xffffu, (unsigned short)0xffffu};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        u16x2 w2 = __builtin_bit_cast(u16x2, w[u][k]);
        w2 = w2 * __builtin_elementwise_min(w2 ^ top2, one2);  // -0 (0x8000) -> +0
        const u16x2 sg = __builtin_bit_cast(u16x2, (s16x2)(__builtin_bit_cast(s16x2, w2) >> (short)15));
        const u16x2 k2 = w2 ^ (sg | top2);
        kk[k] = __builtin_bit_cast(uint32_t, k2);
        hi2 = __builtin_elementwise_max(hi2, k2);
        lo2 = __builtin_elementwise_min(lo2, k2);
      }
      const uint32_t vmax = max((uint32_t)hi2.x, (uint32_t)hi2.y), vmin = min((uint32_t)lo2.x, (uint32_t)lo2.y);
      if (vmax > 0xff80u || vmin < 0x7fu) {  // NaN or padding: id by id
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t key = (kk[k >> 1] >> (16 * (k & 1))) & 0xffffu;
          const bool real = i + k < end;
          const bool nan = real && (key > 0xff80u || key < 0x7fu);
          nid = (nid < 0 && nan) ? i + k : nid;
          const bool better = real && !nan && key > bk;
          bid = better ? i + k : bid;
          bk = better ? key : bk;
        }
      } else if (vmax > bk) {  // the lowest id holding the vector's largest key
        int first = 7;
#pragma unroll
        for (int k = 7; k >= 0; --k) first = ((kk[k >> 1] >> (16 * (k & 1))) & 0xffffu) == vmax ? k : first;
        bk = vmax;
        bid = i + first;
      }
    }
  }
  unsigned long long best = 0;
  if (nid >= 0) best = (0xffffull << 32) | (0xffffffffu - (uint32_t)nid);
  else if (bid >= 0) best = ((unsigned long long)bk << 32) | (0xffffffffu - (uint32_t)bid);
  best = wave_max_ull(best);
  __shared__ unsigned long long wbest[kGreedyThreads / 64];
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kGreedyThreads / 64; ++w) best = wbest[w] > best ? wbest[w] : best;
    const unsigned int waves = gridDim.x;  // arrivals per row: one per workgroup
    // returning atomics: each result is awaited before the next is issued
    unsigned long long seen = 0;
    unsigned long long* slot = slots + (int64_t)b * kGreedyLine;
    unsigned int* arrival = arrivals + (int64_t)b * 2 * kGreedyLine;
    if (best) seen = __hip_atomic_fetch_max(slot, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // (a slot never holds all ones -- keys fit 16 bits -- so the increment is 1,
    // but it depends on the max's result, which keeps the two in order)
    const unsigned int inc = seen == ~0ull ? 0u : 1u;
    const unsigned int n = __hip_atomic_fetch_add(arrival, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n == waves - 1) {
      const unsigned long long c = __hip_atomic_fetch_max(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      out_ids[b] = c ? (int64_t)(0xffffffffu - (uint32_t)c) : 0;  // (a row always has a candidate)
      __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(arrival, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}


// ---------------------------------------------------------------------------
// Sampled rows over several workgroups per row (batches given a workspace).
//
// A row is cut into R segments of whole 8-id vectors, one kSegThreads
// workgroup each, and the one-workgroup algorithm above runs as three
// launches (a launch boundary makes one kernel's global writes visible to the
// next, across XCDs):
//   1. seg_stats:  per segment, the largest and smallest key and the greedy best;
//   2. seg_hist:   per segment, bucket counts and masses, the min-p key, and the
//                  segment's total mass (its kept mass when the row has no cut);
//   3. row_finish: per row, one 1024-thread workgroup: the summed histograms
//                  give the bucket(s) holding the cut-offs (greedy and all-NaN
//                  rows finish here); the workgroup gathers those buckets'
//                  candidates from the row into LDS, makes the exact cut (by
//                  per-key counts, or a sort) and the kept mass (top-k rows
//                  draw from the list and finish), then draws: the segment
//                  holding floor(u * M), then the id in it.  A row whose
//                  buckets hold more candidates than LDS runs sample_row.
//                  Each segment's kept mass follows without another pass over
//                  the logits: its masses of the buckets before the cut's
//                  bucket (every candidate there is kept) plus its candidates
//                  up to the cut (exact integer sums of the same per-candidate
//                  masses).
// Buckets, masses, cuts and the draw are those of the one-workgroup path, so
// the ids are identical to it.

constexpr int kSegThreads = 256;
constexpr int kSegWaves = kSegThreads / 64;
#ifndef XV_SEG_MAX
#define XV_SEG_MAX 32
#endif
#ifndef XV_SEG_CHUNK
#define XV_SEG_CHUNK 4
#endif
#ifndef XV_SEG_TARGET
#define XV_SEG_TARGET 2048
#endif
constexpr int kMaxSegs = XV_SEG_MAX;
constexpr int kSegChunk = XV_SEG_CHUNK;
// Rows of the multi-workgroup sampled path; larger batches take one workgroup
// per row.  Up to 512 rows the path measured faster than one workgroup per row
// (top-p 0.9 at V 151936: 103 against 233 us at 192 rows, 241 against 465 at
// 512; its workspace holds kMaxCand candidates per row, 64 KB).
constexpr int kSegMaxBatch = 512;

enum : int { kPlanDone = 0, kPlanGather = 1, kPlanDraw = 2, kPlanFallback = 3 };

struct __attribute__((aligned(128))) RowPlan {
  int status;
  int use_k;           // the list is the top-k candidates (draw from the list)
  int cut_p, cut_m;    // the top-p / min-p cut falls in the gathered bucket
  uint32_t kminp;      // min-p key (0xffffffff: none)
  uint32_t key_cut;
  uint32_t klo, khi;   // keys of buckets lo..hi: exactly [klo, khi]
  float zmax, inv_t;
  int64_t thr, mp_before, m_before, id_cut, M;
};

struct SegArgs {
  const bf16_t* logits;
  int64_t stride;
  int V, R, seg_len, flags;
  const float* temps;
  const float* top_ps;
  const int32_t* top_ks;
  const float* min_ps;
  const float* uniforms;
  int64_t* out_ids;
  uint32_t* seg_kmax;           // [B * R]
  uint32_t* seg_kmin;           // [B * R]
  uint32_t* seg_minp;           // [B * R]
  unsigned long long* seg_best; // [B * R] greedy (key << 32 | ~id)
  int64_t* seg_kept;            // [B * R]
  uint32_t* seg_cnt;            // [B * R * kBuckets]
  unsigned long long* seg_mass; // [B * R * kBuckets]
  unsigned long long* cand;     // [B * cand_stride]
  int64_t cand_stride;          // candidates per row: kMaxCand, or R * kTopList on the top-k path
};

struct RowParams {
  bool greedy, use_k, use_p, use_m;
  int top_k;
  float temp, top_p, min_p;
};
XV_INLINE RowParams row_params(const SegArgs& a, int b) {
  RowParams p;
  p.temp = a.temps[b];
  p.greedy = p.temp <= 1e-5f;
  p.top_k = ((a.flags & XV_SAMPLE_USE_TOP_K) && a.top_ks) ? a.top_ks[b] : a.V;
  p.top_p = ((a.flags & XV_SAMPLE_USE_TOP_P) && a.top_ps) ? a.top_ps[b] : 1.0f;
  p.min_p = ((a.flags & XV_SAMPLE_USE_MIN_P) && a.min_ps) ? a.min_ps[b] : 0.0f;
  // No candidate reaches a min-p above 1 (the largest logit's ratio is
  // exactly 1), and the kept set is then the first candidate alone, as a
  // top-k of 1 keeps it.
  if (p.min_p > 1.0f) p.top_k = 1;
  p.use_k = p.top_k > 0 && p.top_k < a.V;
  p.use_p = p.top_p < 1.0f;
  p.use_m = p.min_p > 0.0f;
  return p;
}

// f(bits, id) for every id of segment [beg, end) on every lane: vector vi of
// the segment is (c * kSegChunk + v) * kSegThreads + t; ids ascend within a
// lane; slots outside the segment come as 0xffff (key 0).
template <typename F>
XV_INLINE void for_seg_chunks(const bf16_t* row, bool vec_ok, int beg, int end, F&& f) {
  const int nvec = (end - beg + 7) / 8;
  for (int c = 0; c * kSegChunk * kSegThreads < nvec; ++c) {
    uint32_t w[kSegChunk][4];
#pragma unroll
    for (int v = 0; v < kSegChunk; ++v) {
      const int base = beg + ((c * kSegChunk + v) * kSegThreads + (int)threadIdx.x) * 8;
      if (vec_ok && base + 8 <= end) {
        const Vec8 x = load_vec8(row + base);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[v][k] = x.w[k];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          w[v][k] = (base + 2 * k < end ? (uint32_t)row[base + 2 * k] : 0xffffu) |
                    (base + 2 * k + 1 < end ? (uint32_t)row[base + 2 * k + 1] : 0xffffu) << 16;
      }
    }
    f(w, c);
  }
}
template <typename F>
XV_INLINE void for_seg(const bf16_t* row, bool vec_ok, int beg, int end, F&& f) {
  for_seg_chunks(row, vec_ok, beg, end, [&](const uint32_t (&w)[kSegChunk][4], int c) {
#pragma unroll
    for (int v = 0; v < kSegChunk; ++v) {
      const int base = beg + ((c * kSegChunk + v) * kSegThreads + (int)threadIdx.x) * 8;
#pragma unroll
      for (int k = 0; k < 8; ++k) f((w[v][k >> 1] >> (16 * (k & 1))) & 0xffffu, base + k);
    }
  });
}

// f(word) for every 32-bit word (two ids, the lower in the low half) of the
// segment's vectors, in for_seg's order; slots outside the segment come as
// 0xffff halves.
template <typename F>
XV_INLINE void for_seg_words(const bf16_t* row, bool vec_ok, int beg, int end, F&& f) {
  for_seg_chunks(row, vec_ok, beg, end, [&](const uint32_t (&w)[kSegChunk][4], int) {
#pragma unroll
    for (int v = 0; v < kSegChunk; ++v)
#pragma unroll
      for (int k = 0; k < 4; ++k) f(w[v][k]);
  });
}

struct SegRed {
  unsigned long long u[kSegWaves];
  int64_t l[kSegWaves];
};
XV_INLINE uint32_t seg_max_u(SegRed& r, uint32_t x) {
  x = wave_max_u(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) r.u[threadIdx.x >> 6] = x;
  __syncthreads();
  uint32_t m = (uint32_t)r.u[0];
  for (int i = 1; i < kSegWaves; ++i) m = max(m, (uint32_t)r.u[i]);
  return m;
}
XV_INLINE uint32_t seg_min_u(SegRed& r, uint32_t x) {
  x = wave_min_u(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) r.u[threadIdx.x >> 6] = x;
  __syncthreads();
  uint32_t m = (uint32_t)r.u[0];
  for (int i = 1; i < kSegWaves; ++i) m = min(m, (uint32_t)r.u[i]);
  return m;
}
XV_INLINE unsigned long long seg_max_ull(SegRed& r, unsigned long long x) {
  x = wave_max_ull(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) r.u[threadIdx.x >> 6] = x;
  __syncthreads();
  unsigned long long m = r.u[0];
  for (int i = 1; i < kSegWaves; ++i) m = r.u[i] > m ? r.u[i] : m;
  return m;
}
XV_INLINE int64_t seg_sum_l(SegRed& r, int64_t x) {
  x = wave_sum_l(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) r.l[threadIdx.x >> 6] = x;
  __syncthreads();
  int64_t m = 0;
  for (int i = 0; i < kSegWaves; ++i) m += r.l[i];
  return m;
}
XV_INLINE int64_t seg_min_l(SegRed& r, int64_t x) {
  x = wave_min_l(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) r.l[threadIdx.x >> 6] = x;
  __syncthreads();
  int64_t m = r.l[0];
  for (int i = 1; i < kSegWaves; ++i) m = r.l[i] < m ? r.l[i] : m;
  return m;
}
// Inclusive prefix sum over the workgroup (thread order).
XV_INLINE int64_t seg_incl_scan(SegRed& r, int64_t x) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  x = wave_incl_scan_l(x);
  __syncthreads();
  if (lane == 63) r.l[w] = x;
  __syncthreads();
  for (int i = 0; i < w; ++i) x += r.l[i];
  return x;
}

// Row max / min keys from the segment stats, and the row constants.
struct RowConsts {
  uint32_t kmax, kmin;
  float inv_t, zmax, bs;
};
// From lane values already loaded (segment `lane` of the row, or 0 / ~0).
XV_INLINE RowConsts row_consts_of(uint32_t kmax_lane, uint32_t kmin_lane, float temp) {
  RowConsts c;
  c.kmax = wave_max_u(kmax_lane);
  c.kmin = wave_min_u(kmin_lane);
  c.inv_t = 1.0f / temp;
  c.zmax = bf16_to_f32(key_to_bits(c.kmax)) * c.inv_t;
  c.bs = c.kmax ? bucket_scale(log2_ratio(key_to_bits(c.kmin), c.inv_t, c.zmax)) : 16.0f;
  return c;
}
XV_INLINE RowConsts row_consts(const SegArgs& a, int b, float temp) {
  // every wave reduces the R <= 64 segment values itself: one load per lane
  RowConsts c;
  const int lane = threadIdx.x & 63;
  c.kmax = wave_max_u(lane < a.R ? a.seg_kmax[b * a.R + lane] : 0u);
  c.kmin = wave_min_u(lane < a.R ? a.seg_kmin[b * a.R + lane] : 0xffffffffu);
  c.inv_t = 1.0f / temp;
  c.zmax = bf16_to_f32(key_to_bits(c.kmax)) * c.inv_t;
  c.bs = c.kmax ? bucket_scale(log2_ratio(key_to_bits(c.kmin), c.inv_t, c.zmax)) : 16.0f;
  return c;
}

__global__ __launch_bounds__(kSegThreads) void seg_stats_kernel(SegArgs a) {
  __shared__ SegRed red;
  const int b = blockIdx.y, r = blockIdx.x;
  const bf16_t* row = a.logits + (int64_t)b * a.stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int beg = r * a.seg_len, end = min(a.V, beg + a.seg_len);
  if (a.temps[b] <= 1e-5f) {  // greedy row: the segment's best (torch.argmax: NaN, else value; lowest id)
    float fm = -INFINITY;
    int bid = -1, nid = -1;
    for_seg(row, vec_ok, beg, end, [&](uint32_t bits, int id) {
      const float v = bf16_to_f32(bits);  // NaN (and padding) never compares greater
      const bool better = v > fm;         // ids ascend within a lane: keeps the lowest
      fm = better ? v : fm;
      bid = better ? id : bid;
      nid = (nid < 0 && id < end && !order_key(bits)) ? id : nid;
    });
    unsigned long long best = greedy_word(fm, bid, nid);
    best = seg_max_ull(red, best);
    if (threadIdx.x == 0) a.seg_best[b * a.R + r] = best;
    return;
  }
  // Order keys two per packed op (x ^ 0x8000, or ~x for a set sign bit):
  // finite keys lie in [0x7f, 0xff80], padding (0xffff) gives key 0, and
  // the smallest key is taken as min(key - 1) + 1 so that key 0 wraps above
  // every other.  NaN bits land outside [0x7f, 0xff80]; a lane that holds
  // one redoes its ids one at a time with order_key (NaN: key 0).
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  const u16x2 top2 = {(unsigned short)0x8000u, (unsigned short)0x8000u}, one2 = {(unsigned short)1u, (unsigned short)1u};
  u16x2 hi2 = {(unsigned short)0u, (unsigned short)0u}, lo2 = {(unsigned short)0xffffu, (unsigned short)0xffffu};
  for_seg_words(row, vec_ok, beg, end, [&](uint32_t wd) {
    const u16x2 w2 = __builtin_bit_cast(u16x2, wd);
    const u16x2 sg = __builtin_bit_cast(u16x2, (s16x2)(__builtin_bit_cast(s16x2, w2) >> (short)15));
    const u16x2 k2 = w2 ^ (sg | top2);
    hi2 = __builtin_elementwise_max(hi2, k2);
    lo2 = __builtin_elementwise_min(lo2, (u16x2)(k2 - one2));
  });
  uint32_t kmax = max((uint32_t)hi2.x, (uint32_t)hi2.y);
  const uint32_t km1 = min((uint32_t)lo2.x, (uint32_t)lo2.y);
  uint32_t kmin = km1 == 0xffffu ? 0xffffffffu : km1 + 1u;
  if (kmax > 0xff80u || kmin < 0x7fu) {
    kmax = 0;
    kmin = 0xffffffffu;
    for_seg(row, vec_ok, beg, end, [&](uint32_t bits, int) {
      const uint32_t key = order_key(bits);
      kmax = max(kmax, key);
      kmin = min(kmin, key ? key : 0xffffffffu);
    });
  }
  kmax = seg_max_u(red, kmax);
  kmin = seg_min_u(red, kmin);
  if (threadIdx.x == 0) {
    a.seg_kmax[b * a.R + r] = kmax;
    a.seg_kmin[b * a.R + r] = kmin;
  }
}

__global__ __launch_bounds__(kSegThreads) void seg_hist_kernel(SegArgs a) {
  __shared__ SegRed red;
  __shared__ uint32_t wcnt[kSegWaves][kBuckets];
  __shared__ unsigned long long wmass[kSegWaves][kBuckets];
  const int b = blockIdx.y, r = blockIdx.x, t = threadIdx.x, w = t >> 6;
  const RowParams p = row_params(a, b);
  if (p.greedy) return;
  const RowConsts rc = row_consts(a, b, p.temp);
  const bf16_t* row = a.logits + (int64_t)b * a.stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int beg = r * a.seg_len, end = min(a.V, beg + a.seg_len);
  for (int i = t; i < kSegWaves * kBuckets; i += kSegThreads) {
    (&wcnt[0][0])[i] = 0u;
    (&wmass[0][0])[i] = 0ull;
  }
  __syncthreads();
  int64_t far_c = 0, far_m = 0;
  uint32_t kminp = 0xffffffffu;
  if (p.use_k) {
    // counts only: the sorted top-k list gives every mass the cut needs; the
    // min-p key needs an exp only within half a binary order of its threshold
    const float d_lo = __log2f(p.min_p) - 0.5f;
    for_seg(row, vec_ok, beg, end, [&](uint32_t bits, int) {
      const uint32_t key = order_key(bits);
      if (!key) return;
      const float d = log2_ratio(bits, rc.inv_t, rc.zmax);
      const int bkt = bucket_of(d, rc.bs);
      if (bkt < kBuckets - 1) atomicAdd(&wcnt[w][bkt], 1u);
      else far_c += 1;
      if (p.use_m && d >= d_lo && sampler_exp2(d) >= p.min_p) kminp = min(kminp, key);
    });
  } else {
    for_seg(row, vec_ok, beg, end, [&](uint32_t bits, int) {
      const uint32_t key = order_key(bits);
      if (!key) return;
      const float d = log2_ratio(bits, rc.inv_t, rc.zmax);
      const float e = sampler_exp2(d);
      const int64_t q = mass_of(e);
      const int bkt = bucket_of(d, rc.bs);
      if (bkt < kBuckets - 1) {
        atomicAdd(&wcnt[w][bkt], 1u);
        atomicAdd(&wmass[w][bkt], (unsigned long long)q);
      } else {
        far_c += 1;
        far_m += q;
      }
      if (p.use_m && e >= p.min_p) kminp = min(kminp, key);
    });
  }
  far_c = seg_sum_l(red, far_c);
  far_m = seg_sum_l(red, far_m);
  kminp = seg_min_u(red, kminp);
  __syncthreads();
  const int64_t o = ((int64_t)b * a.R + r) * kBuckets;
  static_assert(kSegThreads == kBuckets, "one thread per bucket");
  uint32_t c = 0;
  unsigned long long m = 0;
  for (int ww = 0; ww < kSegWaves; ++ww) { c += wcnt[ww][t]; m += wmass[ww][t]; }
  if (t == kBuckets - 1) { c += (uint32_t)far_c; m += (unsigned long long)far_m; }
  a.seg_cnt[o + t] = c;
  if (!p.use_k) a.seg_mass[o + t] = m;  // top-k rows take their masses from the list
  // the segment's total mass: its kept mass if the row has no cut (rows with
  // a cut take theirs from the cut; top-k rows never reach the draw)
  const int64_t total = seg_sum_l(red, p.use_k ? 0 : (int64_t)m);
  if (t == 0) {
    a.seg_minp[b * a.R + r] = kminp;
    a.seg_kept[b * a.R + r] = total;
  }
}

// List operations on at most 64 candidates held one per lane, by one wave
// (no workgroup barriers).
//
// Bitonic sort of the wave, descending; zeros (padding) sort last.
XV_INLINE unsigned long long wave_sort_desc(unsigned long long c) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const unsigned long long o = xor_lane64(c, stride);
      const bool take_max = ((lane & size) == 0) == ((lane & stride) == 0);
      c = take_max ? (o > c ? o : c) : (o < c ? o : c);
    }
  return c;
}
// 32-bit forms of the list operations, for lists whose words order as the
// 64-bit candidate words do (a segment's key << 13 | (8191 - offset of the id
// in the segment), the row merge's key << 16 | index): each compare-exchange
// stage then moves and selects one register, not two.
XV_INLINE uint32_t xor_lane(uint32_t x, int s) {  // s a constant after unrolling
  switch (s) {
    case 1: return xor_lane<1>(x);
    case 2: return xor_lane<2>(x);
    case 4: return xor_lane<4>(x);
    case 8: return xor_lane<8>(x);
    case 16: return xor_lane<16>(x);
    default: return xor_lane<32>(x);
  }
}
XV_INLINE uint32_t wave_sort_desc32(uint32_t c) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t o = xor_lane(c, stride);
      const bool take_max = ((lane & size) == 0) == ((lane & stride) == 0);
      c = take_max ? max(o, c) : min(o, c);
    }
  return c;
}
template <int S>
XV_INLINE uint32_t merge_stage32(uint32_t c) {  // the larger to the lane with bit S clear
  const uint32_t o = xor_lane<S>(c);
  return (threadIdx.x & S) ? min(o, c) : max(o, c);
}
// Top 64 of two lists sorted descending (lane j holds element j of each):
// the elementwise max against the reversed second list is bitonic and holds
// the top 64; six compare-exchange stages sort it descending.  y[63 - lane]
// is row_mirror (lane i of a row reads lane 15 - i), then the row swaps.
XV_INLINE uint32_t merge_top64_32(uint32_t x, uint32_t y) {
  const uint32_t c = max(x, xor_lane<32>(xor_lane<16>(dpp_u<0x140>(y))));
  return merge_stage32<1>(merge_stage32<2>(merge_stage32<4>(merge_stage32<8>(merge_stage32<16>(merge_stage32<32>(c))))));
}

// First lane whose predicate holds, `none` if no lane's does.
XV_INLINE int64_t wave_first(bool pred, int64_t none) {
  const unsigned long long m = __ballot(pred);
  return m ? (int64_t)__builtin_ctzll(m) : none;
}

// The cut of a list of n <= 64 candidates, wave 0 alone: the same cut, kept
// mass and draw as the workgroup list functions.
// c: this lane's candidate (0 past n), in any order unless `sorted` says the
// lanes hold the list sorted descending already.
// segk: per segment in LDS, the kept mass of the buckets before the cut's
// (rows without top-k; the list's part is added here).
XV_INLINE void row_cut_wave_list(const SegArgs& a, RowPlan& plan, const RowParams& p, int b, int n,
                                 unsigned long long c, unsigned long long* segk, bool sorted = false) {
  const int lane = threadIdx.x & 63;
  const float inv_t = plan.inv_t, zmax = plan.zmax;
  if (!sorted) c = wave_sort_desc(c);
  const int64_t q = lane < n ? cand_mass(c, inv_t, zmax) : 0;
  const int64_t incl = wave_incl_scan_l(q);
  const uint32_t key = cand_key(c);
  const uint32_t kminp = plan.kminp;
  int64_t jcut;
  if (plan.use_k) {
    const int64_t total_k = wave_sum_l(lane < p.top_k ? q : 0);
    jcut = (int64_t)p.top_k - 1;
    if (p.use_p) {
      const int64_t thr = (int64_t)floor((double)p.top_p * (double)total_k);
      jcut = min(jcut, wave_first(lane < n && incl > thr, n));
    }
    const uint32_t last = cand_key(__shfl(c, n - 1));
    if (p.use_m && kminp != 0xffffffffu && kminp >= last)
      jcut = min(jcut, (int64_t)__popcll(__ballot(lane < n && key >= kminp)) - 1);
  } else {
    jcut = kTieAll;
    if (plan.cut_p) jcut = min(jcut, wave_first(lane < n && plan.mp_before + incl > plan.thr, n));
    if (plan.cut_m) jcut = min(jcut, (int64_t)__popcll(__ballot(lane < n && key >= kminp)) - 1);
  }
  if (jcut >= n) jcut = n - 1;
  if (jcut < 0) jcut = 0;
  const unsigned long long edge = __shfl(c, (int)jcut);
  const int64_t m_list = wave_sum_l(lane <= jcut ? q : 0);
  if (plan.use_k) {
    // the kept list in ascending id order: re-keyed (~id << 32 | key), sorted descending
    const float u = a.uniforms ? a.uniforms[b] : 0.5f;
    const int64_t rdraw = draw_point(u, m_list);
    // no mass in the list (z_max not finite, see lowest_id_of_key): its first candidate
    const int64_t first = cand_id(__shfl(c, 0));
    int64_t fid;
    if (a.V <= (1 << 26)) {
      // 32-bit words (0x3ffffff - id) << 6 | lane, sorted descending: ids
      // ascending, each word naming the lane that holds its mass
      uint32_t e = lane <= jcut ? (0x3ffffffu - (uint32_t)cand_id(c)) << 6 | (uint32_t)lane : 0u;
      e = wave_sort_desc32(e);
      const int64_t qe = (int64_t)__shfl((long long)q, (int)(e & 63u));
      const int64_t ie = wave_incl_scan_l(lane <= jcut ? qe : 0);
      const int64_t fi = wave_first(lane <= jcut && ie > rdraw, -1);
      const uint32_t ef = __shfl(e, fi < 0 ? 0 : (int)fi);
      fid = fi < 0 ? first : (int64_t)(0x3ffffffu - (ef >> 6));
    } else {
      unsigned long long e =
          lane <= jcut ? ((unsigned long long)(0xffffffffu - (uint32_t)cand_id(c)) << 32) | cand_key(c) : 0ull;
      e = wave_sort_desc(e);
      const int64_t qe = lane <= jcut ? mass_of(exp_of(key_to_bits((uint32_t)(e & 0xffffffffu)), inv_t, zmax)) : 0;
      const int64_t ie = wave_incl_scan_l(qe);
      const int64_t fi = wave_first(lane <= jcut && ie > rdraw, -1);
      const unsigned long long ef = __shfl(e, fi < 0 ? 0 : (int)fi);
      fid = fi < 0 ? first : (int64_t)(0xffffffffu - (uint32_t)(ef >> 32));
    }
    if (lane == 0) {
      a.out_ids[b] = fid;
      plan.status = kPlanDone;
    }
    return;
  }
  // each segment's kept mass: its earlier buckets plus its listed candidates up to the cut
  if (lane <= jcut) atomicAdd(&segk[cand_id(c) / a.seg_len], (unsigned long long)q);
  if (lane == 0) {
    plan.key_cut = cand_key(edge);
    plan.id_cut = cand_id(edge);
    plan.M = plan.m_before + m_list;
    plan.status = kPlanDraw;
  }
}

// The cut of a gathered bucket list of a row without top-k, by per-key counts
// instead of a sort.  A candidate's mass depends on its key alone and the
// list's order is key descending, ties by ascending id, so a prefix of the
// list is a key plus the number of that key's lowest ids, and the mass before
// a key is a sum of count x mass over the keys above it.  Bin j of the count
// array holds key khi - j.  Returns false, having written nothing, when the
// keys span more bins than the array holds or the cut splits a tie group of
// more than kTieRank ids (the sort then takes the list); the result is the
// sort's in every other case.
constexpr int kKeyBins = kWaves * kBuckets;  // the per-wave histograms' LDS, unused here
constexpr int kTieRank = 512;
XV_INLINE bool row_cut_by_keys(const SegArgs& a, RowPlan& plan, Shared& s, FastShared& fs, int n,
                               uint32_t* tie_ids, unsigned long long* segk) {
  const int t = threadIdx.x;
  const uint32_t klo = plan.klo, khi = plan.khi;
  if (khi < klo || khi - klo >= (uint32_t)kKeyBins) return false;
  const int K = (int)(khi - klo) + 1;
  const float inv_t = plan.inv_t, zmax = plan.zmax;
  uint32_t* kcnt = &fs.wcnt[0][0];
  for (int j = t; j < K; j += kThreads) kcnt[j] = 0u;
  __syncthreads();
  for (int i = t; i < n; i += kThreads) atomicAdd(&kcnt[khi - cand_key(fs.cand[i])], 1u);
  __syncthreads();
  constexpr int kPerT = kKeyBins / kThreads;  // consecutive bins of one thread
  static_assert(kPerT * kThreads == kKeyBins, "bins per thread");
  const int j0 = t * kPerT;
  uint32_t c[kPerT];
  int64_t m[kPerT];
  int64_t local = 0;
  int64_t first = kTieAll, last = -1;  // present bins of this thread
#pragma unroll
  for (int k = 0; k < kPerT; ++k) {
    const int j = j0 + k;
    c[k] = j < K ? kcnt[j] : 0u;
    m[k] = c[k] ? mass_of(exp_of(key_to_bits(khi - (uint32_t)j), inv_t, zmax)) : 0;
    local += (int64_t)c[k] * m[k];
    if (c[k]) {
      first = first < j ? first : j;
      last = j;
    }
  }
  int64_t list_mass;  // unused
  const int64_t before = block_excl_scan(s, local, &list_mass);  // mass of the bins before this thread's
  // cut position (bin << 32 | ties kept): kTieAll keeps the whole list, -1 only its first candidate
  int64_t pos = kTieAll;
  if (plan.cut_p) {  // first candidate whose inclusive mass (after the earlier buckets') exceeds thr
    const int64_t thr = plan.thr;
    int64_t cum = plan.mp_before + before, found = kTieAll;
#pragma unroll
    for (int k = 0; k < kPerT; ++k) {
      const int64_t w = (int64_t)c[k] * m[k];
      if (found == kTieAll && c[k] && cum + w > thr) {
        int64_t i = m[k] > 0 ? (thr - cum) / m[k] + 1 : 1;
        i = i < 1 ? 1 : (i > (int64_t)c[k] ? (int64_t)c[k] : i);
        found = ((int64_t)(j0 + k) << 32) | i;
      }
      cum += w;
    }
    pos = block_min_l(s, found);
  }
  if (plan.cut_m) {  // the candidates with key >= kminp, a prefix of the list
    const uint32_t kminp = plan.kminp;
    int64_t lastm = -1;
    if (kminp <= khi) {
      const int64_t jm = (int64_t)(khi - kminp);
#pragma unroll
      for (int k = 0; k < kPerT; ++k)
        if (c[k] && j0 + k <= jm) lastm = ((int64_t)(j0 + k) << 32) | c[k];
    }
    lastm = -block_min_l(s, -lastm);
    pos = lastm < pos ? lastm : pos;
  }
  int jc;
  int64_t ic;
  if (pos == kTieAll) {  // (uniform branches: the block reductions run on every thread)
    jc = (int)-block_min_l(s, -last);
    ic = kTieAll;
  } else if (pos < 0) {
    jc = (int)block_min_l(s, first);
    ic = 1;
  } else {
    jc = (int)(pos >> 32);
    ic = pos & 0xffffffffll;
  }
  const uint32_t key_cut = khi - (uint32_t)jc;
  const int64_t cnt_c = kcnt[jc];
  if (ic >= cnt_c) ic = kTieAll;
  int64_t id_cut = kTieAll;
  if (ic != kTieAll) {
    // the ic-th smallest id of key_cut: each of its ids counts the smaller ones
    if (cnt_c > kTieRank) return false;
    __syncthreads();
    if (t == 0) fs.ncand = 0;
    __syncthreads();
    for (int i = t; i < n; i += kThreads) {
      const unsigned long long e = fs.cand[i];
      if (cand_key(e) == key_cut) tie_ids[atomicAdd(&fs.ncand, 1)] = (uint32_t)cand_id(e);
    }
    __syncthreads();
    const int nt = fs.ncand, nt4 = (nt + 3) & ~3;
    if (t >= nt && t < nt4) tie_ids[t] = 0xffffffffu;
    __syncthreads();
    if (t < nt) {
      const uint32_t mine = tie_ids[t];
      const uint4* v = reinterpret_cast<const uint4*>(tie_ids);
      int rank = 0;
      for (int q = 0; q < nt4 / 4; ++q) {
        const uint4 x = v[q];
        rank += (x.x < mine) + (x.y < mine) + (x.z < mine) + (x.w < mine);
      }
      if (rank == ic - 1) s.b_id = mine;
    }
    __syncthreads();
    id_cut = s.b_id;
  }
  // kept mass of the list: the bins before jc, and ic (or all) ties of jc
  if (jc >= j0 && jc < j0 + kPerT) {
    int64_t kept = plan.m_before + before;
#pragma unroll
    for (int k = 0; k < kPerT; ++k)
      if (j0 + k < jc) kept += (int64_t)c[k] * m[k];
      else if (j0 + k == jc) kept += (ic == kTieAll ? (int64_t)c[k] : ic) * m[k];
    s.b_total = kept;
  }
  for (int i = t; i < n; i += kThreads) {
    const unsigned long long e = fs.cand[i];
    const uint32_t key = cand_key(e);
    const int64_t id = cand_id(e);
    if (key > key_cut || (key == key_cut && id <= id_cut))
      atomicAdd(&segk[id / a.seg_len], (unsigned long long)cand_mass(e, inv_t, zmax));
  }
  __syncthreads();
  if (t == 0) {
    plan.key_cut = key_cut;
    plan.id_cut = id_cut;
    plan.M = s.b_total;
    plan.status = kPlanDraw;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Top-k path, for calls whose every row has 1 <= top_k <= kTopList (the
// caller's max_top_k; greedy rows too, since a row's argmax is its first
// candidate).  The order of candidates (key descending, id ascending) does not
// depend on the temperature, so a row's top kTopList candidates are the top
// kTopList of its segments' own top kTopList lists, and they hold everything
// a top-k row's cut and draw need: the row max (the first candidate), the
// masses of the top-k set, the min-p key within it.  Two launches and one pass
// over the logits:
//   seg_topk: per segment, its top kTopList candidates, sorted, into the row's
//             list (each wave selects from its own ids, wave 0 merges);
//   row_topk: per row, a tree of pairwise merges of the sorted segment lists
//             (bitonic, in registers, one wave per merge), then the argmax
//             (greedy rows) or the cut and draw of row_cut_wave (top-k rows).
// A row that does not meet the bound runs sample_row, so ids never depend on
// the caller's claim.
constexpr int kTopList = 64;
constexpr int kTopVecs = 4;  // 8-id vectors per thread in registers: segments of up to 8192 ids

XV_INLINE int wave_incl_scan_i(int x) { return (int)wave_incl_scan_l(x); }

// Each wave selects the top kTopList of its own ids (vectors v * kSegThreads
// + 64 w + lane of the segment, ids ascending in (v, lane, k) order) with no
// workgroup barrier: its largest key, a wave-private LDS histogram of the
// 256 keys below it (keys further down never touch LDS), the threshold key T
// from a scan of that histogram (a bit-by-bit count over all keys when fewer
// than kTopList lie that close), then a compaction by per-lane masks into a
// 32-bit list it sorts.  Wave 0 merges the four sorted wave lists and writes
// the segment's list as 64-bit candidate words.
__global__ __launch_bounds__(kSegThreads) void seg_topk_kernel(SegArgs a) {
  static_assert(kMaxSegs * kTopList <= kMaxCand, "the segment lists fit the row's list");
  __shared__ uint32_t hist[kSegWaves][256];
  static_assert(kTopVecs * 8 * kSegThreads <= 8192, "segment offsets fit the 13 bits of a list entry");
  __shared__ uint32_t wl[kSegWaves][kTopList];
  __shared__ uint4 kst[kTopVecs][kSegThreads];  // each thread's keys, packed as in kw
  const int b = blockIdx.y, r = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const bf16_t* row = a.logits + (int64_t)b * a.stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int beg = r * a.seg_len, end = min(a.V, beg + a.seg_len);
  const int nv = ((end - beg + 7) / 8 + kSegThreads - 1) / kSegThreads;  // <= kTopVecs (checked by the host)
  // Whole 16-byte vectors first, every load issued before any is used; then
  // the ids of a partial vector (at most one lane) or of an unaligned row.
  uint32_t kw[kTopVecs][4];
#pragma unroll
  for (int v = 0; v < kTopVecs; ++v) {
    const int base = beg + (v * kSegThreads + t) * 8;
#pragma unroll
    for (int k = 0; k < 4; ++k) kw[v][k] = 0xffffffffu;
    if (v < nv && vec_ok && base + 8 <= end) {
      const Vec8 y = load_vec8(row + base);
#pragma unroll
      for (int k = 0; k < 4; ++k) kw[v][k] = y.w[k];
    }
  }
#pragma unroll
  for (int v = 0; v < kTopVecs; ++v) {
    const int base = beg + (v * kSegThreads + t) * 8;
    if (v < nv && !(vec_ok && base + 8 <= end) && base < end) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        kw[v][k] = (base + 2 * k < end ? (uint32_t)row[base + 2 * k] : 0xffffu) |
                   (base + 2 * k + 1 < end ? (uint32_t)row[base + 2 * k + 1] : 0xffffu) << 16;
    }
  }
  // Order keys, two per packed 16-bit op: x ^ 0x8000 for a sign bit of 0,
  // ~x for 1 (order_key's map on non-NaN values).  Finite keys lie in
  // [0x7f, 0xff80]; NaN bits land outside, as do the padding words (0xffff
  // gives key 0).  A lane holding any such key redoes them one at a time:
  // NaN takes key 0 (dropped), except in a greedy row, which is
  // torch.argmax: its NaNs (real ids only) take key 0xffff, above every value,
  // so the list's first entry is the lowest NaN id when there is one.
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  const u16x2 top2 = {(unsigned short)0x8000u, (unsigned short)0x8000u};
  u16x2 hi2 = {(unsigned short)0u, (unsigned short)0u}, lo2 = {(unsigned short)0xffffu, (unsigned short)0xffffu};
#pragma unroll
  for (int v = 0; v < kTopVecs; ++v)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (v >= nv) {
        kw[v][k] = 0u;
        continue;
      }
      const u16x2 w2 = __builtin_bit_cast(u16x2, kw[v][k]);
      const u16x2 sg = __builtin_bit_cast(u16x2, (s16x2)(__builtin_bit_cast(s16x2, w2) >> (short)15));
      const u16x2 k2 = w2 ^ (sg | top2);
      kw[v][k] = __builtin_bit_cast(uint32_t, k2);
      hi2 = __builtin_elementwise_max(hi2, k2);
      lo2 = __builtin_elementwise_min(lo2, k2);
    }
  uint32_t kmax = max((uint32_t)hi2.x, (uint32_t)hi2.y);
  if (kmax > 0xff80u || min((uint32_t)lo2.x, (uint32_t)lo2.y) < 0x7fu) {
    const bool greedy = a.temps[b] <= 1e-5f;
    kmax = 0;
#pragma unroll
    for (int v = 0; v < kTopVecs; ++v)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t k0 = kw[v][k] & 0xffffu, k1 = kw[v][k] >> 16;
        const int id0 = beg + (v * kSegThreads + t) * 8 + 2 * k;
        if (k0 > 0xff80u || k0 < 0x7fu) k0 = greedy && v < nv && id0 < end ? 0xffffu : 0u;
        if (k1 > 0xff80u || k1 < 0x7fu) k1 = greedy && v < nv && id0 + 1 < end ? 0xffffu : 0u;
        kw[v][k] = k0 | k1 << 16;
        kmax = max(kmax, max(k0, k1));
      }
  }
  auto key_at = [&](int v, int k) { return (kw[v][k >> 1] >> (16 * (k & 1))) & 0xffffu; };
  kmax = wave_max_u(kmax);
  // count of this wave's keys >= x (wave uniform)
  auto count_ge = [&](uint32_t x) {
    int c = 0;
#pragma unroll
    for (int v = 0; v < kTopVecs; ++v)
      if (v < nv)
#pragma unroll
        for (int k = 0; k < 8; ++k) c += __popcll(__ballot(key_at(v, k) >= x));
    return c;
  };
  uint32_t T = 1;    // threshold key: every key > T is taken, and need_eq keys == T
  int need_eq = kTopList, n_eq = 0;
  if (kmax == 0) {
    T = 0xffffffffu;  // nothing but NaN: an empty list
    need_eq = 0;
  } else {
    // histogram of keys kmax - j, j = 0..255, in this wave's LDS row
    const uint32_t lo = kmax > 256u ? kmax - 255u : 1u;  // key 0 (NaN, padding) never counts
#pragma unroll
    for (int j = 0; j < 4; ++j) hist[w][lane + 64 * j] = 0u;
    // distances below kmax two at a time (no wrap: no key exceeds kmax), and
    // their byte offsets (which wrap only for distances past the range)
    const uint32_t span = kmax - lo;
    const u16x2 kmax2 = {(unsigned short)kmax, (unsigned short)kmax};
    char* const hrow = reinterpret_cast<char*>(&hist[w][0]);
#pragma unroll
    for (int v = 0; v < kTopVecs; ++v)
      if (v < nv)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u16x2 d2 = kmax2 - __builtin_bit_cast(u16x2, kw[v][j]);
          const u16x2 o2 = d2 << (unsigned short)2;
          if (d2.x <= span) atomicAdd(reinterpret_cast<uint32_t*>(hrow + o2.x), 1u);
          if (d2.y <= span) atomicAdd(reinterpret_cast<uint32_t*>(hrow + o2.y), 1u);
        }
    // lane l holds bins 4l .. 4l + 3 (keys kmax - 4l downwards)
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = hist[w][4 * lane + j];
    const int mine = (int)(h[0] + h[1] + h[2] + h[3]);
    const int incl = wave_incl_scan_i(mine);
    const int total = __shfl(incl, 63);
    if (total >= kTopList) {
      const int l = (int)wave_first(incl >= kTopList, 63);
      int above = __shfl(incl - mine, l);
      const uint32_t h0 = __shfl(h[0], l), h1 = __shfl(h[1], l), h2 = __shfl(h[2], l), h3 = __shfl(h[3], l);
      const uint32_t hh[4] = {h0, h1, h2, h3};
      int j = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (j == q && above + (int)hh[q] < kTopList) { above += (int)hh[q]; j = q + 1; }
      T = kmax - (uint32_t)(4 * l + j);
      n_eq = (int)(j == 0 ? h0 : j == 1 ? h1 : j == 2 ? h2 : h3);
      need_eq = kTopList - above;
    } else {
      // fewer than kTopList keys within 256 of the largest: the largest x
      // with count(keys >= x) >= kTopList, bit by bit (or every key)
      const int all = count_ge(1u);
      if (all <= kTopList) {  // every key: key > 0 selects them, no ranking
        T = 0;
        need_eq = 0;
      } else {
        uint32_t x = 0;
        for (int bit = 15; bit >= 0; --bit) {
          const uint32_t y = x | (1u << bit);
          if (count_ge(y) >= kTopList) x = y;
        }
        T = x;
        const int gt = count_ge(x + 1);
        need_eq = kTopList - gt;
        n_eq = count_ge(x) - gt;
      }
    }
  }
  // Compaction: keys > T, and keys == T in id order up to need_eq of them.
  // Each lane marks what it takes in a 32-bit mask (bit 4v + j: key 2j of
  // vector v, bit 16 + 4v + j: key 2j + 1), two keys per packed 16-bit
  // compare; one wave scan of the counts gives each lane its slots, and a
  // lane writes only its own candidates, reading their keys back from LDS.
  const bool rank_eq = n_eq > need_eq;
  const u16x2 one2 = {(unsigned short)1u, (unsigned short)1u};
  uint32_t take = 0;
  if (T != 0xffffffffu) {
    // without ranking every key >= T is taken (keys > 0 when T is 0)
    const uint32_t tg = rank_eq ? T : (T ? T - 1u : 0u);
    const u16x2 tg2 = {(unsigned short)tg, (unsigned short)tg};
    const u16x2 t2 = {(unsigned short)T, (unsigned short)T};
    uint32_t ne = 0, valid = 0;  // ne: keys != T
#pragma unroll
    for (int v = 0; v < kTopVecs; ++v) {
      if (v >= nv) break;
      valid |= 0x000f000fu << (4 * v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u16x2 k2 = __builtin_bit_cast(u16x2, kw[v][j]);
        take |= __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_elementwise_sub_sat(k2, tg2), one2))
                << (4 * v + j);
        if (rank_eq) ne |= __builtin_bit_cast(uint32_t, __builtin_elementwise_min(k2 ^ t2, one2)) << (4 * v + j);
      }
    }
    if (rank_eq) {
      // keys == T (T > 0 here, so never padding), ranked in id order: vector,
      // then lane, then key.  Per-vector counts in 16-bit fields of one word
      // (a wave holds at most 512 per vector), one scan for all four.
      const uint32_t eq = ~ne & valid;
      uint64_t pc = 0;
#pragma unroll
      for (int v = 0; v < kTopVecs; ++v) pc |= (uint64_t)__popc(eq & (0x000f000fu << (4 * v))) << (16 * v);
      const uint64_t inc = (uint64_t)wave_incl_scan_l((int64_t)pc);
      const uint64_t tot = (uint64_t)__shfl((long long)inc, 63);
      // first rank of each vector's keys in this lane: the wave's counts in
      // earlier vectors plus the lower lanes' in this one
      uint64_t first = inc - pc, run = 0;
#pragma unroll
      for (int v = 0; v < kTopVecs; ++v) {
        first += run << (16 * v);
        run += (tot >> (16 * v)) & 0xffffu;
      }
      for (uint32_t m = eq; m; m &= m - 1) {
        const int bit = __builtin_ctz(m), v = (bit & 15) >> 2, j = bit & 3;
        // this lane's keys == T of vector v at lower ids: pairs j' < j, and key 2j if this is 2j + 1
        const uint32_t lower = ((((1u << j) - 1u) * 0x00010001u) << (4 * v)) | ((bit >> 4) ? 1u << (bit & 15) : 0u);
        const int rank = (int)((first >> (16 * v)) & 0xffffu) + __popc(eq & lower);
        if (rank < need_eq) take |= 1u << bit;
      }
    }
  }
  // this lane's keys, for reading back by position
#pragma unroll
  for (int v = 0; v < kTopVecs; ++v)
    if (v < nv) kst[v][t] = make_uint4(kw[v][0], kw[v][1], kw[v][2], kw[v][3]);
  const int mine = __popc(take);
  const int incl = wave_incl_scan_i(mine);
  const int filled = __shfl(incl, 63);
  int slot = incl - mine;
  for (uint32_t m = take; m; m &= m - 1, ++slot) {
    const int bit = __builtin_ctz(m), v = (bit & 15) >> 2, k = 2 * (bit & 3) + (bit >> 4);
    const uint32_t key = reinterpret_cast<const unsigned short*>(&kst[v][t])[k];
    wl[w][slot] = key << 13 | (8191u - (uint32_t)((v * kSegThreads + t) * 8 + k));
  }
  uint32_t c = lane < filled ? wl[w][lane] : 0u;
  c = wave_sort_desc32(c);
  wl[w][lane] = c;
  __syncthreads();
  if (w == 0) {
    const uint32_t m = merge_top64_32(merge_top64_32(c, wl[1][lane]), merge_top64_32(wl[2][lane], wl[3][lane]));
    // back to the row's candidate word (key << 32 | ~id); 0 stays padding
    const uint32_t id = (uint32_t)beg + (8191u - (m & 8191u));
    a.cand[(int64_t)b * a.cand_stride + (int64_t)r * kTopList + lane] =
        m ? ((unsigned long long)(m >> 13) << 32) | (unsigned long long)(0xffffffffu - id) : 0ull;
  }
}

__global__ __launch_bounds__(kThreads) void row_topk_kernel(SegArgs a) {
  static_assert(kMaxSegs <= 2 * kWaves, "one merge per wave on the first level");
  __shared__ Shared s;
  __shared__ FastShared fs;
  const int b = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const RowParams p = row_params(a, b);
  if (!p.greedy && !(p.use_k && p.top_k <= kTopList)) {  // outside the bound: the one-workgroup path
    sample_row(s, fs, b, a.logits, a.stride, a.V, a.temps, a.top_ps, a.top_ks, a.min_ps, a.uniforms,
               a.flags & ~XV_SAMPLE_ALL_GREEDY, a.out_ids);
    return;
  }
  const unsigned long long* list = a.cand + (int64_t)b * a.cand_stride;
  // The merges run on 32-bit words key << 16 | (0xffff - i), i the entry's
  // index r * kTopList + j in the row's lists (entry j of segment r's list):
  // lists are sorted and segments ascend in id, so for equal keys a lower i
  // is a lower id, and the words order as the candidates do.  The lists are
  // staged in fs.cand to map the merged words back.  Level 0: wave w merges
  // segment lists 2w and 2w + 1 (missing lists are empty); later levels
  // alternate between two halves of a word buffer, one barrier each.
  static_assert(kMaxSegs * kTopList <= 0x10000 && 2 * kWaves * kTopList <= kWaves * kBuckets, "word layout");
  uint32_t* ml = &fs.wcnt[0][0];
  auto word = [&](unsigned long long c, int i) { return c ? cand_key(c) << 16 | (0xffffu - (uint32_t)i) : 0u; };
  {
    const int i0 = (2 * w) * kTopList + lane, i1 = i0 + kTopList;
    const unsigned long long x = 2 * w < a.R ? list[i0] : 0ull;
    const unsigned long long y = 2 * w + 1 < a.R ? list[i1] : 0ull;
    fs.cand[i0] = x;
    fs.cand[i1] = y;
    ml[w * kTopList + lane] = merge_top64_32(word(x, i0), word(y, i1));
  }
  __syncthreads();
  int src = 0;
  for (int half = kWaves / 2; half >= 1; half >>= 1) {
    const int dst = src ^ (kWaves * kTopList);
    if (w < half)
      ml[dst + w * kTopList + lane] =
          merge_top64_32(ml[src + (2 * w) * kTopList + lane], ml[src + (2 * w + 1) * kTopList + lane]);
    src = dst;
    __syncthreads();
  }
  if (t >= 64) return;
  const uint32_t mw = ml[src + lane];
  const unsigned long long c = mw ? fs.cand[0xffffu - (mw & 0xffffu)] : 0ull;
  const int n = __popcll(__ballot(c != 0ull));
  const unsigned long long top = __shfl(c, 0);
  if (p.greedy || n == 0) {  // argmax (NaN first for greedy rows); a sampled row of NaN only: 0
    if (t == 0) a.out_ids[b] = n ? cand_id(top) : 0;
    return;
  }
  RowPlan pl;
  pl.use_k = 1;
  pl.inv_t = 1.0f / p.temp;
  pl.zmax = bf16_to_f32(key_to_bits(cand_key(top))) * pl.inv_t;
  uint32_t kminp = 0xffffffffu;
  if (p.use_m && t < n) {
    const uint32_t key = cand_key(c);
    if (sampler_exp2(log2_ratio(key_to_bits(key), pl.inv_t, pl.zmax)) >= p.min_p) kminp = key;
  }
  pl.kminp = wave_min_u(kminp);
  row_cut_wave_list(a, pl, p, b, n, c, nullptr, true);  // top-k: drawn from the list, no per-segment masses
}


// ---------------------------------------------------------------------------
// Per row, after seg_stats and seg_hist, in one launch (row_finish_kernel):
// the plan (the bucket or buckets holding the cut-offs, from the summed
// segment histograms), the candidates of those buckets gathered from the row
// by this workgroup, the cut, and the draw.

constexpr uint32_t kInfKey = 0xff80u;  // +inf: the keys of non-NaN values are [1, kInfKey]

// Smallest key in [1, kInfKey] at which pred holds (pred is false below some
// key and true from it on), kInfKey + 1 if it holds at none.  Each round
// probes 64 keys at once, so three or four rounds cover the key range; every
// lane of the calling wave returns the result.
template <typename P>
XV_INLINE uint32_t wave_first_key(P&& pred) {
  const uint32_t lane = threadIdx.x & 63;
  uint32_t l = 1, h = kInfKey + 1;  // the result is in [l, h]: pred holds at h, or h is past the keys
  while (l < h) {
    const uint32_t span = h - l, step = (span + 63) / 64;
    const uint32_t k = l + lane * step;
    const unsigned long long m = __ballot(k < h && pred(k));
    if (m) {
      const uint32_t i = (uint32_t)__builtin_ctzll(m);
      h = l + i * step;
      if (i) l = h - step + 1;  // the probe before it failed
    } else {
      l += ((span + step - 1) / step - 1) * step + 1;  // past the last probe below h
    }
  }
  return l;
}

// Append every id of the row whose key lies in [klo, khi] (klo >= 1) to
// fs.cand as (key << 32) | ~id; fs.ncand counts them, also past kMaxCand.
// The key transform and the range test run on two logits per 32-bit word (the
// key of raw bits b is b ^ 0xffff for a negative b, else b ^ 0x8000; a
// saturating subtract leaves 0 exactly for the keys in range), so a vector
// without a hit costs a few instructions.  Ids with a hit are checked exactly
// (a NaN's key is 0 there).  The loads of a step go out together: every lane
// loads whole vectors (vectors past the row's last whole one reload it and
// are masked), and the ids past the last whole vector are taken one by one at
// the end.
constexpr int kGatherChunk = 10;  // 16-byte loads in flight per thread (more spill registers)
constexpr int kGatherRec = 4;     // vectors with a hit a lane records for later
XV_INLINE void gather_key_range(FastShared& fs, const bf16_t* row, int V, bool vec_ok, uint32_t klo,
                                uint32_t khi) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  auto append = [&](uint32_t bits, int id) {
    const uint32_t key = order_key(bits);
    if (key >= klo && key <= khi) {
      const int slot = atomicAdd(&fs.ncand, 1);
      if (slot < kMaxCand)
        fs.cand[slot] = ((unsigned long long)key << 32) | (unsigned long long)(0xffffffffu - (uint32_t)id);
    }
  };
  const int t = threadIdx.x;
  const int nfull = vec_ok ? V / 8 : 0;  // a row not 16-byte aligned goes id by id
  const u16x2 lo2 = {(unsigned short)klo, (unsigned short)klo};
  const u16x2 sp2 = {(unsigned short)(khi - klo), (unsigned short)(khi - klo)};
  const u16x2 top2 = {(unsigned short)0x8000u, (unsigned short)0x8000u};
  auto test = [&](const uint32_t (&wd)[4], uint32_t (&z)[4]) {  // true if some id may be in range
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u16x2 w2 = __builtin_bit_cast(u16x2, wd[k]);
      const u16x2 sg = __builtin_bit_cast(u16x2, (s16x2)(__builtin_bit_cast(s16x2, w2) >> (short)15));
      z[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat((u16x2)((w2 ^ (sg | top2)) - lo2), sp2));
    }
    const u16x2 m2 = __builtin_elementwise_min(
        __builtin_elementwise_min(__builtin_bit_cast(u16x2, z[0]), __builtin_bit_cast(u16x2, z[1])),
        __builtin_elementwise_min(__builtin_bit_cast(u16x2, z[2]), __builtin_bit_cast(u16x2, z[3])));
    return m2.x == 0 || m2.y == 0;
  };
  auto hits = [&](const uint32_t (&wd)[4], const uint32_t (&z)[4], int vi) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (((z[k >> 1] >> (16 * (k & 1))) & 0xffffu) == 0u) append((wd[k >> 1] >> (16 * (k & 1))) & 0xffffu, vi * 8 + k);
  };
  // Vectors with a hit are recorded (up to kGatherRec per lane, 16-bit indices)
  // and their ids handled after the scan, so a wave runs the per-id work a few
  // times instead of in most steps when hits are spread over the row.
  const bool defer = nfull <= 65536;
  unsigned long long rec = 0;
  int nrec = 0;
  for (int c0 = 0; c0 < nfull; c0 += kGatherChunk * kThreads) {
    uint32_t wv[kGatherChunk][4];
#pragma unroll
    for (int v = 0; v < kGatherChunk; ++v) {
      const int vi = c0 + v * kThreads + t;
      const Vec8 x = load_vec8(row + 8u * (uint32_t)min(vi, nfull - 1));
#pragma unroll
      for (int k = 0; k < 4; ++k) wv[v][k] = x.w[k];
    }
#pragma unroll
    for (int v = 0; v < kGatherChunk; ++v) {
      const int vi = c0 + v * kThreads + t;
      uint32_t z[4];
      if (test(wv[v], z) && vi < nfull) {
        if (defer && nrec < kGatherRec) {
          rec |= (unsigned long long)(uint32_t)vi << (16 * nrec);
          ++nrec;
        } else {
          hits(wv[v], z, vi);
        }
      }
    }
  }
  for (int r = 0; __ballot(nrec > r); ++r) {
    if (nrec > r) {
      const int vi = (int)((rec >> (16 * r)) & 0xffffu);
      const Vec8 x = load_vec8(row + 8u * (uint32_t)vi);
      const uint32_t wd[4] = {x.w[0], x.w[1], x.w[2], x.w[3]};
      uint32_t z[4];
      test(wd, z);
      hits(wd, z, vi);
    }
  }
  for (int id = nfull * 8 + t; id < V; id += kThreads) append((uint32_t)row[id], id);
}

XV_INLINE int64_t kept_mass_of(uint32_t bits, int id, uint32_t key_cut, int64_t id_cut, float inv_t, float zmax) {
  const uint32_t key = order_key(bits);
  const bool kept = key && (key > key_cut || (key == key_cut && (int64_t)id <= id_cut));
  return kept ? mass_of(exp_of(bits, inv_t, zmax)) : 0;
}

// The draw of a row whose cut is made: the segment holding floor(u * M) by
// the segments' kept masses, then in that segment, in id order, the first kept
// id whose inclusive mass exceeds the rest of the draw point.  Each thread
// takes a run of consecutive ids of the segment.
constexpr int kDrawRegs = 16;  // ids per thread whose masses the draw keeps in registers
XV_INLINE void row_draw(const SegArgs& a, Shared& s, const RowPlan& lp, const unsigned long long* segk, int b) {
  const int t = threadIdx.x, lane = t & 63;
  const float u = a.uniforms ? a.uniforms[b] : 0.5f;
  const int64_t rdraw = draw_point(u, lp.M);
  // every wave finds the segment itself: R <= 64, one segment per lane
  const int64_t sm = lane < a.R ? (int64_t)segk[lane] : 0;
  const int64_t incl = wave_incl_scan_l(sm);
  const int r = (int)wave_first(lane < a.R && rdraw < incl, kMaxSegs);
  if (r >= a.R) {  // no kept mass (cannot happen for a row with a finite logit)
    if (t == 0) a.out_ids[b] = 0;
    return;
  }
  const int64_t rr = rdraw - (__shfl(incl, r) - (int64_t)segk[r]);
  const uint32_t key_cut = lp.key_cut;
  const int64_t id_cut = lp.id_cut;
  const float inv_t = lp.inv_t, zmax = lp.zmax;
  const bf16_t* row = a.logits + (int64_t)b * a.stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int beg = r * a.seg_len, end = min(a.V, beg + a.seg_len);
  const int C = ((end - beg + kThreads - 1) / kThreads + 7) / 8 * 8;
  const int i0 = min(end, beg + t * C), i1 = min(end, i0 + C);
  if (C <= kDrawRegs) {
    // the thread's masses stay in registers for the second step
    int64_t q[kDrawRegs];
#pragma unroll
    for (int v = 0; v < kDrawRegs / 8; ++v) {
      uint32_t bits[8];
      const int base = i0 + 8 * v;
      if (base < i1) load8(row, i1, base, vec_ok, bits);  // i0 and C are multiples of 8
#pragma unroll
      for (int k = 0; k < 8; ++k)
        q[8 * v + k] = base + k < i1 ? kept_mass_of(bits[k], base + k, key_cut, id_cut, inv_t, zmax) : 0;
    }
    int64_t mine = 0;
#pragma unroll
    for (int k = 0; k < kDrawRegs; ++k) mine += q[k];
    int64_t seg_total;
    int64_t cum = block_excl_scan(s, mine, &seg_total);
    __syncthreads();
    if (t == 0) s.b_id = -1;
    __syncthreads();
    if (cum <= rr && rr < cum + mine) {
      int found = -1;
#pragma unroll
      for (int k = 0; k < kDrawRegs; ++k) {
        cum += q[k];
        if (found < 0 && cum > rr) found = i0 + k;
      }
      s.b_id = found;
    }
  } else {
    auto scan_range = [&](auto&& f) {
      for (int i = i0; i < i1; i += 8 * kSegChunk) {
        uint32_t bits[kSegChunk][8];
#pragma unroll
        for (int v = 0; v < kSegChunk; ++v)
          if (i + 8 * v < i1) load8(row, i1, i + 8 * v, vec_ok, bits[v]);
#pragma unroll
        for (int v = 0; v < kSegChunk; ++v)
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (i + 8 * v + k < i1) f(bits[v][k], i + 8 * v + k);
      }
    };
    int64_t mine = 0;
    scan_range([&](uint32_t bits, int id) { mine += kept_mass_of(bits, id, key_cut, id_cut, inv_t, zmax); });
    int64_t seg_total;
    int64_t cum = block_excl_scan(s, mine, &seg_total);
    __syncthreads();
    if (t == 0) s.b_id = -1;
    __syncthreads();
    if (cum <= rr && rr < cum + mine) {
      int64_t found = -1;
      scan_range([&](uint32_t bits, int id) {
        if (found >= 0) return;
        cum += kept_mass_of(bits, id, key_cut, id_cut, inv_t, zmax);
        if (cum > rr) found = id;
      });
      s.b_id = found;
    }
  }
  __syncthreads();
  if (t == 0) a.out_ids[b] = s.b_id >= 0 ? s.b_id : 0;
}

__global__ __launch_bounds__(kThreads) void row_finish_kernel(SegArgs a) {
  __shared__ Shared s;
  __shared__ FastShared fs;
  __shared__ RowPlan lp;
  __shared__ unsigned long long segk[kMaxSegs];
  __shared__ __attribute__((aligned(16))) uint32_t tie_ids[kTieRank];
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const RowParams p = row_params(a, b);
  if (p.greedy) {  // the best of the segments' best words (torch.argmax order)
    if (w == 0) {
      const unsigned long long best = wave_max_ull(lane < a.R ? a.seg_best[b * a.R + lane] : 0ull);
      if (lane == 0) a.out_ids[b] = best ? (int64_t)(0xffffffffu - (uint32_t)best) : 0;
    }
    return;
  }
  // Every load the plan needs goes out before any is used: the row's segment
  // statistics, and of bucket t % kBuckets the histogram entries of segments
  // t / kBuckets + kGroups * j.  Segment indices past R reload segment R - 1
  // (no branch between the loads) and are masked below.
  constexpr int kGroups = kThreads / kBuckets, kSegPerGroup = kMaxSegs / kGroups;
  static_assert(kGroups * kBuckets == kThreads && kSegPerGroup * kGroups == kMaxSegs, "bucket x segment layout");
  const int bt = t & (kBuckets - 1), g = t / kBuckets;
  uint32_t hc[kSegPerGroup];
  unsigned long long hm[kSegPerGroup];
#pragma unroll
  for (int j = 0; j < kSegPerGroup; ++j) {
    const int64_t o = ((int64_t)b * a.R + min(g + kGroups * j, a.R - 1)) * kBuckets + bt;
    hc[j] = a.seg_cnt[o];
    hm[j] = p.use_k ? 0ull : a.seg_mass[o];  // top-k rows take their masses from the list
  }
  const int sl = min(lane, a.R - 1);
  const uint32_t kmax_l = a.seg_kmax[b * a.R + sl], kmin_l = a.seg_kmin[b * a.R + sl];
  const uint32_t minp_l = a.seg_minp[b * a.R + sl];
  const RowConsts rc = row_consts_of(lane < a.R ? kmax_l : 0u, lane < a.R ? kmin_l : 0xffffffffu, p.temp);
  if (rc.kmax == 0) {  // every logit NaN: nothing has mass
    if (t == 0) a.out_ids[b] = 0;
    return;
  }
  if (!__builtin_isfinite(rc.zmax)) {  // no mass anywhere: the lowest id of the largest key
    const bf16_t* row = a.logits + (int64_t)b * a.stride;
    const int64_t id = lowest_id_of_key(s, row, a.V, ((reinterpret_cast<uintptr_t>(row) & 15u) == 0), rc.kmax);
    if (t == 0) a.out_ids[b] = id;
    return;
  }
  const uint32_t kminp = wave_min_u(lane < a.R ? minp_l : 0xffffffffu);
  if (t < kMaxSegs) segk[t] = 0ull;  // (ordered before its atomics by the scan's barriers)
  {  // each group's partial sums of the buckets, then thread t < kBuckets adds the groups'
    uint32_t c = 0;
    unsigned long long m = 0;
#pragma unroll
    for (int j = 0; j < kSegPerGroup; ++j)
      if (g + kGroups * j < a.R) {
        c += hc[j];
        m += hm[j];
      }
    fs.wcnt[g][bt] = c;
    fs.wmass[g][bt] = m;
  }
  __syncthreads();
  int64_t cnt = 0, mass = 0;
  if (t < kBuckets) {
#pragma unroll
    for (int gg = 0; gg < kGroups; ++gg) {
      cnt += fs.wcnt[gg][t];
      mass += p.use_k ? 0 : (int64_t)fs.wmass[gg][t];
    }
  }
  int64_t cnt_excl, mass_excl, cnt_all, total;
  block_excl_scan2(s, cnt, mass, &cnt_excl, &mass_excl, &cnt_all, &total);
  const int64_t cnt_incl = cnt_excl + cnt, mass_incl = mass_excl + mass;
  int status = kPlanDraw, lo = 0, hi = 0, cut_p = 0, cut_m = 0;
  int64_t thr = 0, m_before = 0;
  if (p.use_k) {
    // rank k-1 lies in the first bucket whose inclusive count reaches k
    const int bk = (int)block_min_l(s, (t < kBuckets && cnt_incl >= p.top_k) ? t : kBuckets);
    __syncthreads();
    if (t == bk) s.b_long[0] = cnt_incl;  // candidates in buckets 0..bk
    __syncthreads();
    const int64_t upto = bk < kBuckets ? s.b_long[0] : 0;
    status = (bk >= kBuckets - 1 || upto > kMaxCand) ? kPlanFallback : kPlanGather;
    hi = bk;
  } else if (p.use_p || p.use_m) {
    int bp = kBuckets;
    if (p.use_p) {
      thr = (int64_t)floor((double)p.top_p * (double)total);
      bp = (int)block_min_l(s, (t < kBuckets && mass_incl > thr) ? t : kBuckets);
    }
    int bm = kBuckets;
    if (p.use_m && kminp != 0xffffffffu) bm = bucket_of(log2_ratio(key_to_bits(kminp), rc.inv_t, rc.zmax), rc.bs);
    const int bf = min(bp, bm);
    if (bf < kBuckets) {
      __syncthreads();
      if (t == bf) {
        s.b_long[0] = cnt;
        s.b_long[1] = mass_incl - mass;  // mass of the buckets before bf
      }
      __syncthreads();
      m_before = s.b_long[1];
      status = s.b_long[0] > kMaxCand ? kPlanFallback : kPlanGather;
      lo = hi = bf;
      cut_p = bp == bf;
      cut_m = bm == bf;
    }
  }
  bool fallback = status == kPlanFallback;  // the boundary does not fit in LDS
  if (t == 0) {
    lp.status = status;
    lp.use_k = p.use_k;
    lp.cut_p = cut_p;
    lp.cut_m = cut_m;
    lp.kminp = kminp;
    lp.zmax = rc.zmax;
    lp.inv_t = rc.inv_t;
    lp.thr = thr;
    lp.mp_before = m_before;
    lp.m_before = m_before;
    lp.key_cut = 1u;  // no cut: every candidate kept
    lp.id_cut = kTieAll;
    lp.M = total;
    fs.ncand = 0;
  }
  if (fallback) {
  } else if (status == kPlanDraw) {  // no cut: the segments' total masses are their kept masses
    if (t < a.R) segk[t] = (unsigned long long)a.seg_kept[b * a.R + t];
  } else {
    // Buckets fall as keys rise over the keys of non-NaN values, so buckets
    // lo..hi hold exactly the keys of an interval: its ends by the same bucket
    // function.
    auto bkt = [&](uint32_t k) { return bucket_of(log2_ratio(key_to_bits(k), rc.inv_t, rc.zmax), rc.bs); };
    if (w == 0) {
      const uint32_t klo = wave_first_key([&](uint32_t k) { return bkt(k) <= hi; });
      if (lane == 0) lp.klo = klo;
    } else if (w == 1) {
      const uint32_t kend = wave_first_key([&](uint32_t k) { return bkt(k) < lo; });
      if (lane == 0) lp.khi = kend - 1;
    }
    // rows without top-k: each segment's mass of the buckets before lo (all
    // of whose candidates are kept; the list's part is added by the cut)
    if (!p.use_k) {
#pragma unroll
      for (int j = 0; j < kSegPerGroup; ++j) {
        const int r = g + kGroups * j;
        const int64_t v = wave_sum_l((r < a.R && bt < lo) ? (int64_t)hm[j] : 0);
        if (lane == 0 && r < a.R) atomicAdd(&segk[r], (unsigned long long)v);
      }
    }
  }
  __syncthreads();
  if (status == kPlanGather) {
    const bf16_t* row = a.logits + (int64_t)b * a.stride;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
    const uint32_t klo = lp.klo, khi = lp.khi;
    if (klo <= khi) gather_key_range(fs, row, a.V, vec_ok, klo, khi);
    __syncthreads();
    const int n = fs.ncand;
    // the cut's bucket holds its own boundary candidate, and the histograms
    // counted the list; should either fail, the one-workgroup path takes the row
    const float inv_t = rc.inv_t, zmax = rc.zmax;
    if (n == 0 || n > kMaxCand) {
      fallback = true;
    } else if (n <= 64) {
      if (t < 64) row_cut_wave_list(a, lp, p, b, n, lane < n ? fs.cand[lane] : 0ull, segk);
    } else if (p.use_k || !row_cut_by_keys(a, lp, s, fs, n, tie_ids, segk)) {
      sort_cand_desc(fs, n);
      int64_t jcut;
      if (p.use_k) {
        // the list is every candidate down to rank k-1 (as topk_boundary)
        const int64_t total_k = list_mass_prefix(s, fs, n, p.top_k, inv_t, zmax);
        jcut = (int64_t)p.top_k - 1;
        if (p.use_p) {
          const int64_t thr_k = (int64_t)floor((double)p.top_p * (double)total_k);
          jcut = min(jcut, list_first_exceed(s, fs, n, 0, thr_k, inv_t, zmax));
        }
        if (p.use_m && kminp != 0xffffffffu && kminp >= cand_key(fs.cand[n - 1]))
          jcut = min(jcut, list_count_ge(s, fs, n, kminp) - 1);
      } else {
        // the list is the bucket of the earliest cut (as fast_boundary)
        jcut = kTieAll;
        if (cut_p) jcut = min(jcut, list_first_exceed(s, fs, n, m_before, thr, inv_t, zmax));
        if (cut_m) jcut = min(jcut, list_count_ge(s, fs, n, kminp) - 1);
      }
      if (jcut >= n) jcut = n - 1;
      if (jcut < 0) jcut = 0;
      const unsigned long long edge = fs.cand[jcut];
      if (p.use_k) {
        const int64_t M = list_mass_prefix(s, fs, n, jcut + 1, inv_t, zmax);
        const float u = a.uniforms ? a.uniforms[b] : 0.5f;
        const int64_t found = list_draw(s, fs, (int)jcut + 1, inv_t, zmax, draw_point(u, M));
        if (t == 0) {
          a.out_ids[b] = found == kTieAll ? 0 : found;
          lp.status = kPlanDone;
        }
      } else {
        const int64_t M = m_before + list_mass_prefix(s, fs, n, jcut + 1, inv_t, zmax);
        for (int i = t; i <= jcut; i += kThreads)
          atomicAdd(&segk[cand_id(fs.cand[i]) / a.seg_len], (unsigned long long)cand_mass(fs.cand[i], inv_t, zmax));
        if (t == 0) {
          lp.key_cut = cand_key(edge);
          lp.id_cut = cand_id(edge);
          lp.M = M;
          lp.status = kPlanDraw;
        }
      }
    }
    __syncthreads();
  }
  if (fallback) {
    sample_row(s, fs, b, a.logits, a.stride, a.V, a.temps, a.top_ps, a.top_ks, a.min_ps, a.uniforms,
               a.flags & ~XV_SAMPLE_ALL_GREEDY, a.out_ids);
    return;
  }
  if (lp.status == kPlanDraw) row_draw(a, s, lp, segk, b);
}
}  // namespace

// Workspace: one 128-byte line per row (a 64-bit slot and a 32-bit arrival
// counter) for the multi-workgroup greedy path, then the per-segment
// statistics and histograms of the multi-workgroup sampled path, and room for
// kMaxCand candidates per row, which the top-k path's lists use (it sets how
// many rows that path takes; the sampled path keeps its candidates in LDS).
namespace {
struct SegLayout {
  int R, seg_len;
  size_t kmax, kmin, minp, best, kept, cnt, mass, cand, total;
};
size_t align256(size_t x) { return (x + 255) / 256 * 256; }
SegLayout seg_layout(int batch, int vocab) {
  SegLayout L;
  // about 2048 segment workgroups in all, at least 2048 ids per segment
  int segs = max(1, min(kMaxSegs, XV_SEG_TARGET / max(batch, 1)));
  segs = max(1, min(segs, vocab / 2048));
  L.seg_len = ((vocab + segs - 1) / segs + 7) / 8 * 8;
  L.R = (vocab + L.seg_len - 1) / L.seg_len;
  const size_t B = (size_t)max(batch, 0), BR = B * L.R;
  size_t o = 0;  // offsets within the sampled path's region
  L.kmax = o;  o = align256(o + BR * 4);
  L.kmin = o;  o = align256(o + BR * 4);
  L.minp = o;  o = align256(o + BR * 4);
  L.best = o;  o = align256(o + BR * 8);
  L.kept = o;  o = align256(o + BR * 8);
  L.cnt = o;   o = align256(o + BR * kBuckets * 4);
  L.mass = o;  o = align256(o + BR * kBuckets * 8);
  L.cand = o;  o = align256(o + B * kMaxCand * 8);
  L.total = o;
  return L;
}

// The greedy path's per-row lines, which must be zero before a call.
size_t greedy_bytes(int batch) { return align256((size_t)max(batch, 0) * kGreedyLine * 8); }
// The largest sampled-path region of any batch up to `batch`.
size_t seg_reserve(int batch, int vocab) {
  size_t r = 0;
  for (int b = 1; b <= min(batch, kSegMaxBatch); ++b) r = max(r, seg_layout(b, vocab).total);
  return r;
}
}  // namespace

// Workspace: the greedy lines at the bottom, the sampled path's region at the
// top (it ends at workspace_bytes).  A workspace of this size for B rows
// serves every call of up to B rows, greedy or sampled, in any order: the
// greedy lines [0, Bg * 128) of a call and the region a sampled call of Bs
// rows wrote at the top never overlap, since the size reserves both the lines
// of Bg rows and the largest region of any Bs <= B.
extern "C" size_t xv_sampler_workspace_size(int batch, int vocab) {
  if (batch <= 0 || vocab <= 0) return 256;
  return greedy_bytes(batch) + seg_reserve(batch, vocab);
}

extern "C" int xv_sample(const void* logits, int64_t logits_stride, int batch, int vocab,
                         const float* temperatures, const float* top_ps, const int32_t* top_ks,
                         const float* min_ps, const float* uniforms, int flags,
                         int64_t* out_ids, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (batch < 0 || vocab <= 0 || logits_stride < vocab) return (int)hipErrorInvalidValue;
  if (!(flags & XV_SAMPLE_ALL_GREEDY) && temperatures == nullptr) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  // All-greedy batches: several workgroups per row, about 2048 in all (1024
  // and 4096 measured slower).
  if ((flags & XV_SAMPLE_ALL_GREEDY) && workspace != nullptr &&
      workspace_bytes >= xv_sampler_workspace_size(batch, vocab) && batch <= 65535) {
    // segments of whole 8-id vectors
    const int segs = max(1, min(32, 2048 / batch));
    const int seg_len = ((vocab + segs - 1) / segs + 7) / 8 * 8;
    // one 128-byte line per row: atomics on one line serialise, so rows do not share
    unsigned long long* slots = (unsigned long long*)workspace;
    unsigned int* arrivals = (unsigned int*)(slots + 1);
    greedy_segment_kernel<<<dim3((unsigned)((vocab + seg_len - 1) / seg_len), (unsigned)batch),
                            kGreedyThreads, 0, stream>>>((const bf16_t*)logits, logits_stride, vocab, seg_len, slots,
                                                         arrivals, out_ids);
    XV_CHECK_LAUNCH();
    return 0;
  }
  // Calls whose every top_k is at most kTopList (the caller's max_top_k): the
  // two-launch top-k path, on its own segments (about 1024 workgroups, none
  // longer than the keys a thread holds) and a compact list region of
  // B * R * kTopList candidates at the top of the workspace.  It stays inside
  // the sampled region the size query reserves, so it never reaches the
  // greedy lines; batches whose lists do not fit take the paths below.
  if ((flags & XV_SAMPLE_TOP_K_LE_64) && workspace != nullptr && temperatures != nullptr &&
      workspace_bytes >= xv_sampler_workspace_size(batch, vocab)) {
    const int seg_cap = kTopVecs * 8 * kSegThreads;
    // about 1024 workgroups: one residency round (2048, as the chain, took 1.3 rounds and
    // 28.5 us at B 64 against 24.9 us)
    const int rt = max((vocab + seg_cap - 1) / seg_cap, min(kMaxSegs, max(1, 1024 / batch)));
    const int seg_len = min(seg_cap, ((vocab + rt - 1) / rt + 7) / 8 * 8);
    const int R = (vocab + seg_len - 1) / seg_len;
    const size_t region = align256((size_t)batch * R * kTopList * 8);
    if (R <= kMaxSegs && batch <= 65535 && region <= seg_reserve(batch, vocab)) {
      SegArgs a = {};
      a.logits = (const bf16_t*)logits; a.stride = logits_stride;
      a.V = vocab; a.R = R; a.seg_len = seg_len; a.flags = flags & ~XV_SAMPLE_ALL_GREEDY;
      a.temps = temperatures; a.top_ps = top_ps; a.top_ks = top_ks; a.min_ps = min_ps; a.uniforms = uniforms;
      a.out_ids = out_ids;
      a.cand = (unsigned long long*)((char*)workspace + ((workspace_bytes - region) & ~(size_t)255));
      a.cand_stride = (int64_t)R * kTopList;
      seg_topk_kernel<<<dim3((unsigned)R, (unsigned)batch), kSegThreads, 0, stream>>>(a);
      XV_CHECK_LAUNCH();
      row_topk_kernel<<<dim3((unsigned)batch), kThreads, 0, stream>>>(a);
      XV_CHECK_LAUNCH();
      return 0;
    }
  }
  // Sampled (or mixed) batches of up to kSegMaxBatch rows: several workgroups
  // per row.  Larger batches take one workgroup per row.
  if (workspace != nullptr && batch <= kSegMaxBatch && workspace_bytes >= xv_sampler_workspace_size(batch, vocab)) {
    const SegLayout L = seg_layout(batch, vocab);
    char* w = (char*)workspace + ((workspace_bytes - L.total) & ~(size_t)255);  // region at the top
    SegArgs a;
    a.logits = (const bf16_t*)logits; a.stride = logits_stride;
    a.V = vocab; a.R = L.R; a.seg_len = L.seg_len; a.flags = flags & ~XV_SAMPLE_ALL_GREEDY;
    a.temps = temperatures; a.top_ps = top_ps; a.top_ks = top_ks; a.min_ps = min_ps; a.uniforms = uniforms;
    a.out_ids = out_ids;
    a.seg_kmax = (uint32_t*)(w + L.kmax);
    a.seg_kmin = (uint32_t*)(w + L.kmin);
    a.seg_minp = (uint32_t*)(w + L.minp);
    a.seg_best = (unsigned long long*)(w + L.best);
    a.seg_kept = (int64_t*)(w + L.kept);
    a.seg_cnt = (uint32_t*)(w + L.cnt);
    a.seg_mass = (unsigned long long*)(w + L.mass);
    const dim3 segs((unsigned)L.R, (unsigned)batch), rows((unsigned)batch);
    seg_stats_kernel<<<segs, kSegThreads, 0, stream>>>(a);
    XV_CHECK_LAUNCH();
    seg_hist_kernel<<<segs, kSegThreads, 0, stream>>>(a);
    XV_CHECK_LAUNCH();
    row_finish_kernel<<<rows, kThreads, 0, stream>>>(a);
    XV_CHECK_LAUNCH();
    return 0;
  }
  sample_kernel<<<dim3((unsigned)batch), dim3(kThreads), 0, stream>>>(
      (const bf16_t*)logits, logits_stride, vocab, temperatures, top_ps, top_ks, min_ps, uniforms, flags, out_ids);
  XV_CHECK_LAUNCH();
  return 0;
}
