// Weight-streaming GEMMs of the decode step: out[M, N] = x[M, K] . w[N, K]^T
// for M <= 64 rows (the decode batch), bf16 operands, fp32 accumulate.
//
// The decoder's projections (reference src/compute/models/qwen3.py:62-64,115,
// src/compute/layers/linear.py:141,306) at decode batch sizes read every
// weight once and do 2 M flops per weight: at M 64 that is 64 flops per byte,
// far under gfx950's bf16 ridge (2.5 PFLOP/s / 8 TB/s = 312), so the kernel
// is an HBM stream of the weights with the MFMA work hidden under it.
//
// Weight layout (packed once, at model load): w's rows in 16-row tiles and its
// K in 64-element steps; tile (nb, step sg) is 2 KB contiguous in the order
// the kernel's lanes read it: element e (0..7) of lane l (row 16 nb + l % 16)
// at 8 l + e for K offset 64 sg + 8 (l / 16) + e, and at 512 + 8 l + e for K
// offset 64 sg + 32 + 8 (l / 16) + e.  Tiles of one row block are consecutive
// in sg.  Every weight load is then 1 KB of contiguous memory per wave
// instruction, and a wave streams each of its tiles front to back; read in
// place from [N, K] rows (16 rows x 128 bytes per step) the same kernel
// streamed at 3-4 TB/s, no faster than hipBLASLt.
//
// Layout of one workgroup: WAVES waves over the same K range (all of K, or
// the workgroup's slice of a K split), each wave its own NT tiles (16 NT
// output columns).  Per step the workgroup copies x's [16 MT, 64] block
// (MT = ceil(M / 16)) once into an LDS ring slot (loaded into registers,
// written to LDS two steps later), and each wave loads its tiles' step into
// registers; both feed v_mfma_f32_16x16x32_bf16 as 8-element operands in the
// K placement above.  The products are summed over K in another order than a
// K-ordered loop, the same 64 per step.  Three steps are in flight while one
// is multiplied.  Weights are read with non-temporal loads (each is read once
// per decode step; the Qwen3-8B step ran 8.31 ms against 8.42 with plain
// loads).  Sharing x through LDS keeps its L2 traffic at
// M / (16 NT WAVES) of the weight bytes: read from L2 by every wave, x cost
// more than the weights themselves at M 64.
// The epilogue writes each wave's tiles in one of three forms:
//   kModeBf16      bf16 out[M, N] (row stride out_stride)
//   kModeParts     fp32 partial sums out[P][M][N] of a K split over P
//                  workgroup columns (gridDim.y), the input of the residual
//                  add + RMSNorm that sums them (fused_add_rmsnorm_parts)
//   kModeSiluMul   the gate/up projection followed by SiLU-and-mul: w holds
//                  the gate rows [0, I) then the up rows [I, 2I) (reference
//                  qwen3.py:50-51); a workgroup takes 8 NT gate rows and the
//                  8 NT matching up rows and writes bf16 out[M, I] =
//                  silu(g) * u, g and u first rounded to bf16 as the
//                  unfused GEMM would have stored them (reference
//                  src/compute/layers/activation.py:6-8).
#include "xv_common.h"

namespace {

constexpr int kModeBf16 = 0, kModeParts = 1, kModeSiluMul = 2;
constexpr int kStepK = 64;  // K elements per row per step
constexpr int kDepth = 4;   // steps in flight (the one being multiplied included) = LDS ring slots

struct GemmArgs {
  const bf16_t* x;
  int64_t xs;  // x row stride (elements)
  const bf16_t* w;  // packed tiles
  int64_t ksteps;   // K / 64: tiles per row block
  void* out;
  int64_t os;           // out row stride (elements of the output type)
  int64_t part_stride;  // kModeParts: elements between the P slices
  int m, kslice, inter;
};

struct Frag {
  bf16x8_t lo, hi;  // the lane's 8 elements in the first and in the last 32 of a step
};

// x's [16 MT, 64] block of one step in LDS: 16-byte piece c (0..7) of row r
// at piece index 8 r + (c ^ (r & 7)), so the 16 rows of one fragment read
// spread over the banks.
XV_INLINE int xpiece(int r, int c) { return 8 * r + (c ^ (r & 7)); }

XV_INLINE float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <int MT, int NT, int WAVES, int MODE>
__global__ __launch_bounds__(WAVES * 64) void dense_gemm_kernel(GemmArgs a) {
  constexpr int kSlot = MT * 16 * 128;                          // bytes of x per step
  constexpr int kXOps = (MT * 128 + WAVES * 64 - 1) / (WAVES * 64);  // x loads per wave per step
  __shared__ __attribute__((aligned(16))) char ring[kDepth * kSlot];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r16 = lane & 15, grp = lane >> 4;

  const int64_t kbase = (int64_t)blockIdx.y * a.kslice;
  // this lane's first element in each of its NT row blocks' packed tiles, at the K slice's first step
  const bf16_t* wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int64_t nb;  // row block
    if constexpr (MODE == kModeSiluMul) {
      constexpr int H = NT / 2;  // tiles t < H: gate rows; t >= H: the matching up rows
      nb = (t < H ? 0 : a.inter / 16) + ((int64_t)blockIdx.x * WAVES + wave) * H + t % H;
    } else {
      nb = ((int64_t)blockIdx.x * WAVES + wave) * NT + t;
    }
    wp[t] = a.w + (nb * a.ksteps + kbase / kStepK) * 1024 + lane * 8;
  }
  const int steps = a.kslice / kStepK;

  // x staging: piece index p = (op * WAVES + wave) * 64 + lane of the step
  // block, loaded into registers and written to its LDS slot two steps later;
  // rows past M read row M - 1 (their products are never stored)
  const bf16_t* xsrc[kXOps];
  bool xon[kXOps];
#pragma unroll
  for (int o = 0; o < kXOps; ++o) {
    const int p = (o * WAVES + wave) * 64 + lane;
    const int r = p >> 3, c = (p & 7) ^ (r & 7);
    xon[o] = p < MT * 128;
    xsrc[o] = a.x + (int64_t)min(r, a.m - 1) * a.xs + kbase + c * 8;
  }

  Frag wreg[kDepth][NT];
  bf16x8_t xreg[kDepth][kXOps];
  auto issue = [&](int u, int s) {  // step s (clamped: past the end, reload the last) into register slot u
    const int sc = min(s, steps - 1);
    const int64_t k = (int64_t)sc * kStepK;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bf16x8_t* q = reinterpret_cast<const bf16x8_t*>(wp[t] + (int64_t)sc * 1024);
      wreg[u][t] = Frag{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 64)};  // read once per step
    }
#pragma unroll
    for (int o = 0; o < kXOps; ++o)
      if (xon[o]) xreg[u][o] = *reinterpret_cast<const bf16x8_t*>(xsrc[o] + k);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads here, ahead of the MFMAs that follow
  };
  auto stage = [&](int u) {  // x of register slot u into LDS slot u
#pragma unroll
    for (int o = 0; o < kXOps; ++o)
      if (xon[o]) *reinterpret_cast<bf16x8_t*>(ring + u * kSlot + ((o * WAVES + wave) * 64 + lane) * 16) = xreg[u][o];
  };

  floatx4_t acc[NT][MT];
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int u = 0; u < kDepth - 1; ++u) issue(u, u);
  stage(0);
  for (int s0 = 0; s0 < steps; s0 += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      // step s = s0 + u: its x block was staged by every wave before this
      // barrier, and every wave is done with step s - 1's slot, reused next
      __syncthreads();
      issue((u + kDepth - 1) % kDepth, s0 + u + kDepth - 1);
      stage((u + 1) % kDepth);  // step s + 1, loaded two steps ago, into the slot step s - 3 used
      const char* slot = ring + u * kSlot;
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int r = j * 16 + r16;
        Frag xf;
        xf.lo = *reinterpret_cast<const bf16x8_t*>(slot + 16 * xpiece(r, grp));
        xf.hi = *reinterpret_cast<const bf16x8_t*>(slot + 16 * xpiece(r, 4 + grp));
#pragma unroll
        for (int i = 0; i < NT; ++i) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wreg[u][i].lo, xf.lo, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wreg[u][i].hi, xf.hi, acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // acc[i][j] lane l: rows 4 (l / 16) + 0..3 of weight tile i (output
  // columns), column l % 16 of x tile j (output row)
  if constexpr (MODE == kModeSiluMul) {
    constexpr int H = NT / 2;
#pragma unroll
    for (int i = 0; i < H; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int m = j * 16 + r16;
        if (m >= a.m) continue;
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gv = round_bf16(acc[i][j][e]), uv = round_bf16(acc[i + H][j][e]);
          r[e] = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * uv;
        }
        const int64_t col = ((int64_t)blockIdx.x * WAVES + wave) * (H * 16) + i * 16 + grp * 4;
        *reinterpret_cast<uint2*>(static_cast<bf16_t*>(a.out) + m * a.os + col) =
            make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
      }
  } else {
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int m = j * 16 + r16;
        if (m >= a.m) continue;
        const floatx4_t v = acc[i][j];
        const int64_t col = ((int64_t)blockIdx.x * WAVES + wave) * (NT * 16) + i * 16 + grp * 4;
        if constexpr (MODE == kModeBf16) {
          *reinterpret_cast<uint2*>(static_cast<bf16_t*>(a.out) + m * a.os + col) =
              make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        } else {
          *reinterpret_cast<floatx4_t*>(static_cast<float*>(a.out) + blockIdx.y * a.part_stride + m * a.os + col) = v;
        }
      }
  }
}

template <int NT, int WAVES, int MODE>
void launch_mt(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  switch ((a.m + 15) / 16) {
    case 1: dense_gemm_kernel<1, NT, WAVES, MODE><<<grid, WAVES * 64, 0, stream>>>(a); break;
    case 2: dense_gemm_kernel<2, NT, WAVES, MODE><<<grid, WAVES * 64, 0, stream>>>(a); break;
    case 3: dense_gemm_kernel<3, NT, WAVES, MODE><<<grid, WAVES * 64, 0, stream>>>(a); break;
    default: dense_gemm_kernel<4, NT, WAVES, MODE><<<grid, WAVES * 64, 0, stream>>>(a); break;
  }
}

template <int MODE>
void launch_shape(const GemmArgs& a, int col_tiles, int waves, dim3 grid, hipStream_t stream) {
  if constexpr (MODE != kModeSiluMul) {
    if (col_tiles == 1) {
      if (waves == 4) launch_mt<1, 4, MODE>(a, grid, stream);
      else launch_mt<1, 8, MODE>(a, grid, stream);
      return;
    }
  }
  if (col_tiles == 2) {
    if (waves == 4) launch_mt<2, 4, MODE>(a, grid, stream);
    else launch_mt<2, 8, MODE>(a, grid, stream);
  } else {
    if (waves == 4) launch_mt<4, 4, MODE>(a, grid, stream);
    else launch_mt<4, 8, MODE>(a, grid, stream);
  }
}

}  // namespace

extern "C" int xv_dense_gemm(const void* x, int64_t x_stride, const void* w_packed, void* out,
                             int64_t out_stride, int64_t part_stride, int m, int n, int k, int mode, int col_tiles,
                             int waves, int parts, hipStream_t stream) {
  if (m < 0 || m > 64 || n <= 0 || k <= 0 || mode < kModeBf16 || mode > kModeSiluMul || parts < 1)
    return (int)hipErrorInvalidValue;
  // tiles per wave 1, 2 or 4 (even for the gate/up pairs of kModeSiluMul), 4 or 8 waves
  if (!(col_tiles == 1 || col_tiles == 2 || col_tiles == 4) || !(waves == 4 || waves == 8) ||
      (mode == kModeSiluMul && col_tiles == 1))
    return (int)hipErrorInvalidValue;
  // whole workgroups of columns; every K slice a whole number of kDepth-step rounds
  if (n % (16 * col_tiles * waves) || k % ((int64_t)parts * kDepth * kStepK)) return (int)hipErrorInvalidValue;
  if (mode != kModeParts && parts != 1) return (int)hipErrorInvalidValue;
  if (!xv_al16(x) || !xv_al16(w_packed) || !xv_st8(x_stride) || x_stride < k)
    return (int)hipErrorInvalidValue;
  if (mode == kModeParts) {
    if (!xv_al16(out) || (out_stride & 3) || out_stride < n || (part_stride & 3) ||
        part_stride < (int64_t)m * out_stride)
      return (int)hipErrorInvalidValue;
  } else {
    const int64_t cols = mode == kModeSiluMul ? n / 2 : n;
    if (((uintptr_t)out & 7u) || (out_stride & 3) || out_stride < cols) return (int)hipErrorInvalidValue;
  }
  if (m == 0) return 0;
  GemmArgs a{(const bf16_t*)x, x_stride, (const bf16_t*)w_packed, k / kStepK, out, out_stride, part_stride,
             m, k / parts, mode == kModeSiluMul ? n / 2 : 0};
  const dim3 grid((unsigned)(n / (16 * col_tiles * waves)), (unsigned)parts);
  if (mode == kModeBf16) launch_shape<kModeBf16>(a, col_tiles, waves, grid, stream);
  else if (mode == kModeParts) launch_shape<kModeParts>(a, col_tiles, waves, grid, stream);
  else launch_shape<kModeSiluMul>(a, col_tiles, waves, grid, stream);
  XV_CHECK_LAUNCH();
  return 0;
}
