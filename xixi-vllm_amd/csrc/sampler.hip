// Vocab-wide sampler for gfx950: greedy argmax, temperature / top-k / top-p /
// min-p with an explicit uniform per row, one 1024-thread workgroup per row.
//
// Candidates are ordered by descending logit, ties by ascending id.  Every
// candidate's probability mass is an exact int64
//   q = trunc(2^40 * 2^d),  d = (l * (1/T) - x_max) * log2 e  (<= 0)
// with a fixed Taylor exp2 (explicit FMAs) shared with the C restatement of the
// oracle, so kept sets, masses and token ids are bit-identical to it.
//
// Fast path (every row whose boundary fits in LDS):
//   1. one pass: max key;
//   2. one pass: q of every candidate, binned by distance below the max,
//      bucket = min(255, floor(-16 d)) (1/16 of a binary order per bucket;
//      per-wave LDS histograms of counts and masses, the far bucket in registers);
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

// Phase timestamps for out-of-tree timing builds; compiled out here.
#ifndef XV_SAMPLER_TIMESTAMP
#define XV_SAMPLER_TIMESTAMP(slot)
#endif

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = kThreads * 8;
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
XV_INLINE int64_t mass_of(float e) { return (int64_t)(e * 1099511627776.0f); }
// Bucket of a candidate d below the max: floor(-d * bs), the last bucket
// holding everything further.  bs is per row (bucket_scale); any bs > 0 keeps
// the buckets monotone in the key, which is all the boundary search needs.
XV_INLINE int bucket_of(float d, float bs) {
  const float u = -d * bs;
  return u < 255.0f ? (int)u : 255;
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

XV_INLINE uint32_t wave_max_u(uint32_t x) {
  for (int o = 32; o > 0; o >>= 1) x = max(x, (uint32_t)__shfl_xor((int)x, o));
  return x;
}
XV_INLINE uint32_t wave_min_u(uint32_t x) {
  for (int o = 32; o > 0; o >>= 1) x = min(x, (uint32_t)__shfl_xor((int)x, o));
  return x;
}
XV_INLINE float wave_maxf(float x) {
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
XV_INLINE int64_t wave_sum_l(int64_t x) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
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
  int64_t inc = x;
  for (int o = 1; o < 64; o <<= 1) {
    int64_t y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
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
  for (int o = 32; o > 0; o >>= 1) {
    const int64_t y = __shfl_xor(x, o);
    x = y < x ? y : x;
  }
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
XV_INLINE int gather_bucket(FastShared& fs, const bf16_t* row, int V, bool vec_ok, int ntiles, float inv_t,
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
XV_INLINE uint32_t minp_key(Shared& s, const bf16_t* row, int V, bool vec_ok, int ntiles, float inv_t, float zmax,
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
XV_INLINE bool topk_boundary(Shared& s, FastShared& fs, const bf16_t* row, int V, bool vec_ok, int ntiles,
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
  XV_SAMPLER_TIMESTAMP(5);
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
  const uint32_t kminp = use_m ? minp_key(s, row, V, vec_ok, ntiles, inv_t, zmax, min_p) : 0xffffffffu;
  const int n = gather_bucket(fs, row, V, vec_ok, ntiles, inv_t, zmax, bs, bk, 0);
  XV_SAMPLER_TIMESTAMP(6);
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
XV_INLINE bool fast_boundary(Shared& s, FastShared& fs, const bf16_t* row, int V, bool vec_ok, int ntiles,
                             float inv_t, float zmax, float bs, int top_k, float top_p, float min_p, bool use_k, bool use_p,
                             bool use_m, uint32_t& key_cut, int64_t& id_cut, int64_t& M, int& list_kept) {
  const int t = threadIdx.x, w = t >> 6;
  if (use_k) return topk_boundary(s, fs, row, V, vec_ok, ntiles, inv_t, zmax, bs, top_k, top_p, min_p, use_p, use_m,
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
  XV_SAMPLER_TIMESTAMP(5);
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
    nk = gather_bucket(fs, row, V, vec_ok, ntiles, inv_t, zmax, bs, bk);
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
    n = gather_bucket(fs, row, V, vec_ok, ntiles, inv_t, zmax, bs, bf);
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

__global__ __launch_bounds__(kThreads) void sample_kernel(const bf16_t* __restrict__ logits, int64_t stride, int V,
                                                          const float* __restrict__ temps,
                                                          const float* __restrict__ top_ps,
                                                          const int32_t* __restrict__ top_ks,
                                                          const float* __restrict__ min_ps,
                                                          const float* __restrict__ uniforms, int flags,
                                                          int64_t* __restrict__ out_ids) {
  __shared__ Shared s;
  __shared__ FastShared fs;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const bf16_t* row = logits + (int64_t)b * stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int ntiles = (V + kTile - 1) / kTile;
  const float temp = temps ? temps[b] : 1.0f;
  const bool greedy = (flags & XV_SAMPLE_ALL_GREEDY) || temp <= 1e-5f;

  // ---- greedy: max value, then the lowest index holding it ----
  if (greedy) {
    // one pass: the lane's max and its lowest id, then the block's
    float fm = -INFINITY;
    uint32_t best = 0xffffffffu;
    for_each_strided(row, V, vec_ok, [&](uint32_t bits, int id) {
      if (!order_key(bits)) return;
      const float v = bf16_to_f32(bits);
      if (v > fm) { fm = v; best = (uint32_t)id; }  // ids ascend within a lane: keeps the lowest
    });
    const float gm = block_maxf(s, fm);
    best = block_min_u(s, fm == gm ? best : 0xffffffffu);
    if (t == 0) out_ids[b] = best == 0xffffffffu ? 0 : (int64_t)best;
    return;
  }

  XV_SAMPLER_TIMESTAMP(0);
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
  const float bs = kmax ? bucket_scale(log2_ratio(key_to_bits(kmin), inv_t, zmax)) : 16.0f;

  const int top_k = ((flags & XV_SAMPLE_USE_TOP_K) && top_ks) ? top_ks[b] : V;
  const float top_p = ((flags & XV_SAMPLE_USE_TOP_P) && top_ps) ? top_ps[b] : 1.0f;
  const float min_p = ((flags & XV_SAMPLE_USE_MIN_P) && min_ps) ? min_ps[b] : 0.0f;
  const bool use_k = top_k > 0 && top_k < V;
  const bool use_p = top_p < 1.0f;
  const bool use_m = min_p > 0.0f;
  XV_SAMPLER_TIMESTAMP(1);

  uint32_t key_cut;
  int64_t id_cut, M;
  int list_kept = 0;  // > 0: the kept set is the sorted list prefix fs.cand[0, list_kept)
  if (!fast_boundary(s, fs, row, V, vec_ok, ntiles, inv_t, zmax, bs, top_k, top_p, min_p, use_k, use_p, use_m,
                     key_cut, id_cut, M, list_kept)) {
    list_kept = 0;
    Boundary bd;
    general_boundary(s, row, V, vec_ok, inv_t, zmax, top_k, top_p, min_p, use_k, use_p, use_m, bd, id_cut,
                     M);
    key_cut = bd.key;
    XV_SAMPLER_TIMESTAMP(3);
  }
  XV_SAMPLER_TIMESTAMP(2);

  // ---- last pass: inverse-CDF draw in ascending id order (exp for kept ids only) ----
  // Thread t owns the contiguous ids [t*C, t*C + C), C a multiple of 8, so one
  // block scan orders the whole row.
  const float u = uniforms ? uniforms[b] : 0.5f;
  int64_t rdraw = (int64_t)((double)u * (double)M);
  if (rdraw >= M) rdraw = M - 1;
  if (rdraw < 0) rdraw = 0;
  if (list_kept > 0) {
    // The kept set is in LDS: re-key it as (~id << 32 | key), so the
    // descending sort puts ids in ascending order, then scan its masses.
    const int n = list_kept;
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
    found = block_min_l(s, found);
    if (t == 0) out_ids[b] = found == kTieAll ? 0 : found;
    XV_SAMPLER_TIMESTAMP(4);
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
  XV_SAMPLER_TIMESTAMP(4);
}

// ---------------------------------------------------------------------------
// All-greedy batches over several workgroups per row (a small batch would
// leave most CUs idle with one workgroup per row).  A lane keeps the largest
// logit of its ids and the lowest id holding it (float compares: -0 equals
// +0, NaN never wins), as the one-workgroup path does.  Each workgroup then
// folds its best into the row's 64-bit slot with one atomic max of
//   order key << 32 | (2^32 - 1 - id)
// (the largest logit wins, among equal logits the lowest id) and counts
// itself in the row's arrival counter; the last workgroup of the row writes the id
// and clears both words for the next call.  Every atomic is awaited before
// the next one is issued, so the count is only bumped after the workgroup's
// max has been performed.  Atomics on one cache line serialise, so each row
// has its own line and is cut into at most 32 segments.
constexpr int kGreedyThreads = 256;
constexpr int kGreedyUnroll = 8;
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
  float fm = -INFINITY;
  int bid = -1;
  constexpr int step = kGreedyThreads * 8;
  for (int i0 = beg + threadIdx.x * 8; i0 < end; i0 += kGreedyUnroll * step) {
    uint32_t bits[kGreedyUnroll][8];
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u)
      if (i0 + u * step < end) load8(row, V, i0 + u * step, vec_ok, bits[u]);
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u) {
      const int i = i0 + u * step;
      if (i >= end) break;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float v = bf16_to_f32(bits[u][k]);
        const bool better = v > fm && i + k < end;  // ids ascend within a lane: keeps the lowest
        fm = better ? v : fm;
        bid = better ? i + k : bid;
      }
    }
  }
  unsigned long long best = 0;
  if (bid >= 0) {
    const uint32_t fb = __float_as_uint(fm) >> 16;
    best = ((unsigned long long)order_key(fb == 0x8000u ? 0u : fb) << 32) | (0xffffffffu - (uint32_t)bid);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long y = __shfl_xor(best, o);
    best = y > best ? y : best;
  }
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
      out_ids[b] = c ? (int64_t)(0xffffffffu - (uint32_t)c) : 0;  // all-NaN row: 0, as the one-workgroup path
      __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(arrival, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

// Workspace: one 128-byte line per row (a 64-bit slot and a 32-bit arrival
// counter) for the multi-workgroup greedy path; the other paths keep their
// scratch in LDS.
extern "C" size_t xv_sampler_workspace_size(int batch, int vocab) {
  (void)vocab;
  return ((size_t)(batch > 0 ? batch : 0) * kGreedyLine * 8 + 255) / 256 * 256;
}

extern "C" int xv_sample(const void* logits, int64_t logits_stride, int batch, int vocab,
                         const float* temperatures, const float* top_ps, const int32_t* top_ks,
                         const float* min_ps, const float* uniforms, int flags,
                         int64_t* out_ids, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (batch < 0 || vocab <= 0 || logits_stride < vocab) return (int)hipErrorInvalidValue;
  if (!(flags & XV_SAMPLE_ALL_GREEDY) && temperatures == nullptr) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  // All-greedy batches: several workgroups per row, about 1024 in all.
  if ((flags & XV_SAMPLE_ALL_GREEDY) && workspace != nullptr &&
      workspace_bytes >= xv_sampler_workspace_size(batch, vocab) && batch <= 65535) {
    // segments of whole 8-id vectors
    const int segs = max(1, min(32, 1024 / batch));
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
  sample_kernel<<<dim3((unsigned)batch), dim3(kThreads), 0, stream>>>(
      (const bf16_t*)logits, logits_stride, vocab, temperatures, top_ps, top_ks, min_ps, uniforms, flags, out_ids);
  XV_CHECK_LAUNCH();
  return 0;
}
