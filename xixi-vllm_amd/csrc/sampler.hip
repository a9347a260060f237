// Vocab-wide sampler for gfx950: greedy argmax, temperature / top-k / top-p /
// min-p with an explicit uniform per row, one 1024-thread workgroup per row.
//
// The candidates are ordered by descending logit, ties by ascending id.  Since
// x = logit / T is monotone in the bf16 logit, the order key is the 16-bit
// order-preserving image of the bf16 bits, so every cut-off is found by a
// two-level (high byte, low byte) radix select over key histograms of counts
// and fixed-point masses held in LDS, instead of a sort:
//   q(key) = trunc(2^40 * 2^((x - x_max) * log2 e)), an exact int64 per candidate
//   top-k : rank k-1 found by count;   top-p : first rank whose inclusive mass
//   exceeds floor(top_p * mass(top-k));  min-p : smallest key with p >= min_p.
// The kept set is the shortest of the three prefixes (boundary = key + tie
// index); the token is the first kept id (ascending) whose inclusive mass
// exceeds floor(u * M_kept), found by a block-wide int64 prefix scan.
// exp2 is a fixed Taylor polynomial with explicit FMAs so that the masses,
// hence the token ids, are bit-identical to the C restatement of the oracle.
#include "xv_common.h"
#include "xv_kernels.h"
#include <math.h>

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = kThreads * 8;
constexpr int64_t kTieAll = 0x7fffffffffffffffll;

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

XV_INLINE float exp_of(uint32_t bits, float temp, float zmax) {
  float z = bf16_to_f32(bits) / temp;
  float d = z - zmax;
  d = d * 1.44269502162933349609375f;
  return sampler_exp2(d);
}
XV_INLINE int64_t mass_of(float e) { return (int64_t)(e * 1099511627776.0f); }

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

__global__ __launch_bounds__(kThreads) void sample_kernel(const bf16_t* __restrict__ logits, int64_t stride, int V,
                                                          const float* __restrict__ temps,
                                                          const float* __restrict__ top_ps,
                                                          const int32_t* __restrict__ top_ks,
                                                          const float* __restrict__ min_ps,
                                                          const float* __restrict__ uniforms, int flags,
                                                          int64_t* __restrict__ out_ids) {
  __shared__ Shared s;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const bf16_t* row = logits + (int64_t)b * stride;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
  const int ntiles = (V + kTile - 1) / kTile;
  const float temp = temps ? temps[b] : 1.0f;
  const bool greedy = (flags & XV_SAMPLE_ALL_GREEDY) || temp <= 1e-5f;

  // ---- pass 1: max (greedy: max value then lowest index holding it) ----
  if (greedy) {
    float fm = -INFINITY;
    for (int j = 0; j < ntiles; ++j) {
      uint32_t bits[8];
      load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (order_key(bits[k])) fm = fmaxf(fm, bf16_to_f32(bits[k]));
    }
    fm = block_maxf(s, fm);
    uint32_t best = 0xffffffffu;
    for (int j = 0; j < ntiles; ++j) {
      uint32_t bits[8];
      const int base = j * kTile + t * 8;
      load8(row, V, base, vec_ok, bits);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (order_key(bits[k]) && bf16_to_f32(bits[k]) == fm) best = min(best, (uint32_t)(base + k));
    }
    best = block_min_u(s, best);
    if (t == 0) out_ids[b] = best == 0xffffffffu ? 0 : (int64_t)best;
    return;
  }

  uint32_t kmax = 0;
  for (int j = 0; j < ntiles; ++j) {
    uint32_t bits[8];
    load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
    for (int k = 0; k < 8; ++k) kmax = max(kmax, order_key(bits[k]));
  }
  kmax = block_max_u(s, kmax);
  const float zmax = bf16_to_f32(key_to_bits(kmax)) / temp;

  const int top_k = ((flags & XV_SAMPLE_USE_TOP_K) && top_ks) ? top_ks[b] : V;
  const float top_p = ((flags & XV_SAMPLE_USE_TOP_P) && top_ps) ? top_ps[b] : 1.0f;
  const float min_p = ((flags & XV_SAMPLE_USE_MIN_P) && min_ps) ? min_ps[b] : 0.0f;
  const bool use_k = top_k > 0 && top_k < V;
  const bool use_p = top_p < 1.0f;
  const bool use_m = min_p > 0.0f;

  Boundary bd = {1u, kTieAll};  // everything kept

  if (use_k || use_p || use_m) {
    // ---- pass 2: high-byte histogram of counts and masses; min-p key ----
    for (int i = t; i < 256; i += kThreads) { s.cnt[i] = 0; s.mass[i] = 0; }
    __syncthreads();
    uint32_t kmin_p = 0xffffffffu;
    for (int j = 0; j < ntiles; ++j) {
      uint32_t bits[8];
      load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t key = order_key(bits[k]);
        if (!key) continue;
        const float e = exp_of(bits[k], temp, zmax);
        if (use_m && e >= min_p) kmin_p = min(kmin_p, key);
        atomicAdd(&s.cnt[key >> 8], 1u);
        atomicAdd(&s.mass[key >> 8], (unsigned long long)mass_of(e));
      }
    }
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
      __syncthreads();
      for (int i = t; i < 256; i += kThreads) { s.cnt[i] = 0; s.mass[i] = 0; }
      __syncthreads();
      for (int j = 0; j < ntiles; ++j) {
        uint32_t bits[8];
        load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t key = order_key(bits[k]);
          if (!key || (int)(key >> 8) != hb) continue;
          atomicAdd(&s.cnt[key & 255], 1u);
        }
      }
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
      for (int j = 0; j < ntiles; ++j) {
        uint32_t bits[8];
        load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t key = order_key(bits[k]);
          if (key > bk.key) above += mass_of(exp_of(bits[k], temp, zmax));
        }
      }
      above = block_sum_l(s, above);
      total_k = above + (bk.tie + 1) * mass_of(exp_of(key_to_bits(bk.key), temp, zmax));
    } else {
      total_k = s.b_total;
    }

    Boundary bp = {1u, kTieAll};
    if (use_p) {
      // ---- pass 4: first rank whose inclusive mass exceeds floor(top_p * total_k) ----
      const int64_t thr = (int64_t)floor((double)top_p * (double)total_k);
      // high-byte masses are still in s.mass only when top-k did not reuse them: rebuild
      __syncthreads();
      for (int i = t; i < 256; i += kThreads) { s.cnt[i] = 0; s.mass[i] = 0; }
      __syncthreads();
      for (int j = 0; j < ntiles; ++j) {
        uint32_t bits[8];
        load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t key = order_key(bits[k]);
          if (!key) continue;
          atomicAdd(&s.mass[key >> 8], (unsigned long long)mass_of(exp_of(bits[k], temp, zmax)));
        }
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
        __syncthreads();
        for (int i = t; i < 256; i += kThreads) { s.cnt[i] = 0; s.mass[i] = 0; }
        __syncthreads();
        for (int j = 0; j < ntiles; ++j) {
          uint32_t bits[8];
          load8(row, V, j * kTile + t * 8, vec_ok, bits);
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t key = order_key(bits[k]);
            if (!key || (int)(key >> 8) != hb) continue;
            atomicAdd(&s.mass[key & 255], (unsigned long long)mass_of(exp_of(bits[k], temp, zmax)));
          }
        }
        __syncthreads();
        if (t == 0) {
          int64_t m = m_above;
          int lb = 255;
          for (; lb > 0; --lb) {
            if (m + (int64_t)s.mass[lb] > thr) break;
            m += (int64_t)s.mass[lb];
          }
          const uint32_t key = ((uint32_t)hb << 8) | (uint32_t)lb;
          const int64_t q = mass_of(exp_of(key_to_bits(key), temp, zmax));
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

  // ---- pass 5: id of the boundary tie (when only part of the ties is kept) and kept mass ----
  int64_t id_cut = kTieAll;  // kept: key > bd.key, or key == bd.key and id <= id_cut
  int64_t M = 0;
  {
    int64_t carry = 0;  // ties of bd.key seen in earlier tiles
    if (t == 0) s.b_id = kTieAll;
    for (int j = 0; j < ntiles; ++j) {
      uint32_t bits[8];
      const int base = j * kTile + t * 8;
      load8(row, V, base, vec_ok, bits);
      int64_t nt = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) nt += order_key(bits[k]) == bd.key;
      int64_t tile_ties;
      int64_t r = carry + block_excl_scan(s, nt, &tile_ties);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t key = order_key(bits[k]);
        if (!key) continue;
        bool kept = key > bd.key;
        if (key == bd.key) {
          kept = r <= bd.tie;
          if (r == bd.tie) s.b_id = base + k;
          ++r;
        }
        if (kept) M += mass_of(exp_of(bits[k], temp, zmax));
      }
      carry += tile_ties;
    }
    M = block_sum_l(s, M);
    id_cut = s.b_id;
    __syncthreads();  // every thread has read b_id before it is reset below
  }

  // ---- pass 6: inverse-CDF draw in ascending id order ----
  const float u = uniforms ? uniforms[b] : 0.5f;
  int64_t rdraw = (int64_t)((double)u * (double)M);
  if (rdraw >= M) rdraw = M - 1;
  if (rdraw < 0) rdraw = 0;
  if (t == 0) s.b_id = -1;
  int64_t carry = 0;
  for (int j = 0; j < ntiles; ++j) {
    uint32_t bits[8];
    const int base = j * kTile + t * 8;
    load8(row, V, base, vec_ok, bits);
    int64_t qk[8];
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t key = order_key(bits[k]);
      const bool kept = key && (key > bd.key || (key == bd.key && (int64_t)(base + k) <= id_cut));
      qk[k] = kept ? mass_of(exp_of(bits[k], temp, zmax)) : 0;
      sum += qk[k];
    }
    int64_t tile_sum;
    int64_t cum = carry + block_excl_scan(s, sum, &tile_sum);
    if (cum <= rdraw && rdraw < cum + sum) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        cum += qk[k];
        if (cum > rdraw) { s.b_id = base + k; break; }
      }
    }
    carry += tile_sum;
    __syncthreads();
    if (s.b_id >= 0) break;
  }
  if (t == 0) out_ids[b] = s.b_id >= 0 ? s.b_id : 0;
}

}  // namespace

extern "C" size_t xv_sampler_workspace_size(int batch, int vocab) {
  (void)batch; (void)vocab;
  return 0;  // all scratch lives in LDS
}

extern "C" int xv_sample(const void* logits, int64_t logits_stride, int batch, int vocab,
                         const float* temperatures, const float* top_ps, const int32_t* top_ks,
                         const float* min_ps, const float* uniforms, int flags,
                         int64_t* out_ids, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  (void)workspace; (void)workspace_bytes;
  if (batch < 0 || vocab <= 0 || logits_stride < vocab) return (int)hipErrorInvalidValue;
  if (!(flags & XV_SAMPLE_ALL_GREEDY) && temperatures == nullptr) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  sample_kernel<<<dim3((unsigned)batch), dim3(kThreads), 0, stream>>>(
      (const bf16_t*)logits, logits_stride, vocab, temperatures, top_ps, top_ks, min_ps, uniforms, flags, out_ids);
  XV_CHECK_LAUNCH();
  return 0;
}
