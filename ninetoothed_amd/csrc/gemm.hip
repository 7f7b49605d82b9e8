// GEMM with the addmm epilogue:  out = cast_out(beta * c + alpha * round(sum_k a*b)).
//
// fp16 / bf16 (MFMA-bound; 2*M*N*K flops per launch):
//   workgroup tile 256 x 256 x 64, 256 lanes = 4 waves in a 2 x 2 grid, each wave
//   owning a 128 x 128 sub-tile as 4 x 4 v_mfma_f32_32x32x16_{f16,bf16} blocks
//   (256 fp32 accumulators per lane).  Both operands sit in LDS k-contiguous
//   ([m][k] for a, [n][k] for b) so that each lane fetches its 8 k-values for an MFMA
//   with one ds_read_b128.  b arrives n-contiguous from HBM: each lane loads an
//   8(k) x 8(n) block with eight 16-byte loads and transposes it in registers
//   before a 16-byte LDS store.  LDS rows are 128 bytes; the 16-byte chunk index is
//   XOR-swizzled with (row ^ row >> 3) & 7 so that both the row-wise reads of the
//   MFMA fetch and the transposed b stores hit 8 distinct chunks per 8 lanes.
//   The next k-tile is fetched from HBM into registers while the current one is
//   multiplied out of LDS.  Workgroups are remapped so that the 8 XCDs (which the
//   dispatcher fills round-robin) each receive a compact block of output tiles.
// fp32 (config 1, 512^3): 32 x 32 workgroup tiles, four waves each computing a
//   16 x 16 block with v_mfma_f32_16x16x4f32, k-tiles of 32 staged through LDS.
#include "mfma_core.h"

namespace nt {

constexpr int GB_M = 256, GB_N = 256, GB_K = TILE_K;
constexpr int G_THREADS = 256;

struct GemmArgs {
  const void* a;
  const void* b;
  const void* c;
  void* out;
  int64_t sa_m, sa_k, sb_k, sb_n, sc_m, sc_n, so_m, so_n;
  int64_t M, N, K;
  float alpha, beta;
  int out_dtype, round_dtype;
  int tiles_m, tiles_n;
};

// Map a linear workgroup id to an output tile so that consecutive ids on one XCD
// (ids congruent mod 8) cover a compact group of tiles.
__device__ __forceinline__ void tile_of(int wg, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int lin = wg;
  if (total % 8 == 0) {
    const int per_xcd = total / 8;
    lin = (wg % 8) * per_xcd + wg / 8;
  }
  // Group rows of tiles in bands of 4 along m so neighbours share b panels.
  const int band = 4;
  const int band_tiles = band * tiles_n;
  const int b_id = lin / band_tiles;
  const int in_band = lin % band_tiles;
  const int rows_here = min(band, tiles_m - b_id * band);
  tm = b_id * band + in_band % rows_here;
  tn = in_band / rows_here;
}

template <typename T, bool FAST>
__global__ __launch_bounds__(G_THREADS) void gemm_mfma_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[(GB_M + GB_N) * GB_K];
  uint16_t* sA = smem;
  uint16_t* sB = smem + GB_M * GB_K;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * GB_M, n0 = (int64_t)tn * GB_N;
  const uint16_t* A = (const uint16_t*)g.a;
  const uint16_t* B = (const uint16_t*)g.b;

  floatx16 acc[4][4];
  zero_acc(acc);

  u32x4 ra[8], rb[8];
  // FAST loader geometry.
  const int a_row = tid >> 3, a_chunk = tid & 7;  // + i*32 rows
  const int b_nb = tid & 31, b_kb = tid >> 5;     // 8x8 block
  const int64_t nk = cdiv(g.K, GB_K);

  auto load_fast = [&](int64_t kt) {
    const int64_t k0 = kt * GB_K;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t row = m0 + i * 32 + a_row;
      ra[i] = *(const u32x4*)(A + row * g.sa_m + k0 + a_chunk * 8);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t k = k0 + b_kb * 8 + r;
      rb[r] = *(const u32x4*)(B + k * g.sb_k + n0 + b_nb * 8);
    }
  };
  auto store_fast = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = i * 32 + a_row;
      *(u32x4*)(sA + row * GB_K + swz(row, a_chunk) * 8) = ra[i];
    }
    u32x4 tb[8];
    transpose8x8(rb, tb);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = b_nb * 8 + j;
      *(u32x4*)(sB + row * GB_K + swz(row, b_kb) * 8) = tb[j];
    }
  };
  // Generic loader: element-wise, any strides, bounds-checked, zero fill.
  auto load_store_generic = [&](int64_t kt) {
    const int64_t k0 = kt * GB_K;
    for (int e = tid; e < GB_M * GB_K; e += G_THREADS) {
      const int row = e / GB_K, kk = e % GB_K;
      const int64_t m = m0 + row, k = k0 + kk;
      uint16_t v = 0;
      if (m < g.M && k < g.K) v = A[m * g.sa_m + k * g.sa_k];
      sA[lds_index(row, kk)] = v;
    }
    for (int e = tid; e < GB_N * GB_K; e += G_THREADS) {
      const int kk = e / GB_N, col = e % GB_N;
      const int64_t n = n0 + col, k = k0 + kk;
      uint16_t v = 0;
      if (n < g.N && k < g.K) v = B[k * g.sb_k + n * g.sb_n];
      sB[lds_index(col, kk)] = v;
    }
  };

  auto compute = [&]() { mma_ktile<T, 4, 4>(sA, sB, wm * 128, wn * 128, lane, acc); };

  if (FAST) {
    load_fast(0);
    store_fast();
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) load_fast(kt + 1);
      compute();
      __syncthreads();
      if (kt + 1 < nk) {
        store_fast();
        __syncthreads();
      }
    }
  } else {
    for (int64_t kt = 0; kt < nk; ++kt) {
      load_store_generic(kt);
      __syncthreads();
      compute();
      __syncthreads();
    }
  }

  // Epilogue: out = cast(beta * c + alpha * round(acc)), one 32-row slab per pass,
  // staged through LDS (16 KiB per wave) so that lanes then walk whole rows.
  __syncthreads();
  float* stage = (float*)smem + wave * (32 * 128);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    stage_slab<4>(stage, acc[i], lane);
    __syncthreads();
    const int64_t row0 = m0 + wm * 128 + i * 32, col0 = n0 + wn * 128;
    for (int e = lane; e < 32 * 32; e += 64) {  // 32 rows x 32 groups of 4 columns
      const int rr = e >> 5, cg = (e & 31) * 4;
      const int64_t row = row0 + rr;
      if (row >= g.M) continue;
      const float4 v4 = *(const float4*)(stage + rr * 128 + cg);
      const float vals[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t col = col0 + cg + u;
        if (col < g.N) {
          float v = g.alpha * round_through(vals[u], g.round_dtype);
          if (g.c) v += g.beta * load_as_float(g.c, row * g.sc_m + col * g.sc_n, g.out_dtype);
          store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
        }
      }
    }
    __syncthreads();
  }
}

// ----------------------------------------------------------------------------- fp32
constexpr int F32_TM = 32, F32_TN = 32, F32_TK = 32;

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs g) {
  __shared__ float sA[F32_TM][F32_TK + 1];
  __shared__ float sB[F32_TK][F32_TN + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tm = blockIdx.x / g.tiles_n, tn = blockIdx.x % g.tiles_n;
  const int64_t m0 = (int64_t)tm * F32_TM, n0 = (int64_t)tn * F32_TN;
  const int wm = wave >> 1, wn = wave & 1;  // 16x16 sub-block of the 32x32 tile
  const float* A = (const float*)g.a;
  const float* B = (const float*)g.b;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = 0; k0 < g.K; k0 += F32_TK) {
    for (int e = tid; e < F32_TM * F32_TK; e += 256) {
      const int r = e / F32_TK, kk = e % F32_TK;
      const int64_t m = m0 + r, k = k0 + kk;
      sA[r][kk] = (m < g.M && k < g.K) ? A[m * g.sa_m + k * g.sa_k] : 0.f;
    }
    for (int e = tid; e < F32_TK * F32_TN; e += 256) {
      const int kk = e / F32_TN, cidx = e % F32_TN;
      const int64_t n = n0 + cidx, k = k0 + kk;
      sB[kk][cidx] = (n < g.N && k < g.K) ? B[k * g.sb_k + n * g.sb_n] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < F32_TK; kk += 4) {
      const float av = sA[wm * 16 + (lane & 15)][kk + (lane >> 4)];
      const float bv = sB[kk + (lane >> 4)][wn * 16 + (lane & 15)];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = m0 + wm * 16 + (lane >> 4) * 4 + r;
    const int64_t col = n0 + wn * 16 + (lane & 15);
    if (row < g.M && col < g.N) {
      float v = g.alpha * round_through(acc[r], g.round_dtype);
      if (g.c) v += g.beta * load_as_float(g.c, row * g.sc_m + col * g.sc_n, g.out_dtype);
      store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
    }
  }
}

static int gemm_check(const GemmArgs& g) {
  if (g.M < 0 || g.N < 0 || g.K < 0) return NT_ERR_INVALID;
  if (!valid_dtype(g.out_dtype) || !valid_round(g.round_dtype)) return NT_ERR_INVALID;
  return 0;
}

// K == 0: out = cast(beta * c + alpha * round(0)).
__global__ void gemm_k0_kernel(GemmArgs g) {
  const int64_t total = g.M * g.N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / g.N, col = e % g.N;
    float v = 0.f;
    if (g.c) v += g.beta * load_as_float(g.c, row * g.sc_m + col * g.sc_n, g.out_dtype);
    store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
  }
}

template <typename T>
static int gemm16_launch(GemmArgs g, hipStream_t stream) {
  if (int e = gemm_check(g)) return e;
  if (g.M == 0 || g.N == 0) return 0;
  if (!g.a || !g.b || !g.out) return NT_ERR_INVALID;
  if (g.K == 0) {
    hipLaunchKernelGGL(gemm_k0_kernel, dim3(1024), dim3(256), 0, stream, g);
    return launch_status();
  }
  const int64_t tiles_m = cdiv(g.M, GB_M), tiles_n = cdiv(g.N, GB_N);
  if (tiles_m * tiles_n > 0x7fffffffLL) return NT_ERR_INVALID;
  g.tiles_m = (int)tiles_m;
  g.tiles_n = (int)tiles_n;
  const bool fast = g.sa_k == 1 && g.sb_n == 1 && g.M % GB_M == 0 && g.N % GB_N == 0 && g.K % GB_K == 0 &&
                    (uintptr_t)g.a % 16 == 0 && (uintptr_t)g.b % 16 == 0 && (g.sa_m * 2) % 16 == 0 &&
                    (g.sb_k * 2) % 16 == 0;
  const dim3 grid((unsigned)(tiles_m * tiles_n)), blk(G_THREADS);
  if (fast)
    hipLaunchKernelGGL((gemm_mfma_kernel<T, true>), grid, blk, 0, stream, g);
  else
    hipLaunchKernelGGL((gemm_mfma_kernel<T, false>), grid, blk, 0, stream, g);
  return launch_status();
}

static int gemm32_launch(GemmArgs g, hipStream_t stream) {
  if (int e = gemm_check(g)) return e;
  if (g.M == 0 || g.N == 0) return 0;
  if (!g.a || !g.b || !g.out) return NT_ERR_INVALID;
  if (g.K == 0) {
    hipLaunchKernelGGL(gemm_k0_kernel, dim3(1024), dim3(256), 0, stream, g);
    return launch_status();
  }
  const int64_t tiles_m = cdiv(g.M, F32_TM), tiles_n = cdiv(g.N, F32_TN);
  if (tiles_m * tiles_n > 0x7fffffffLL) return NT_ERR_INVALID;
  g.tiles_m = (int)tiles_m;
  g.tiles_n = (int)tiles_n;
  hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, stream, g);
  return launch_status();
}

static GemmArgs make_args(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                          const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                          int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta, int round_dtype) {
  GemmArgs g{};
  g.a = a; g.b = b; g.c = c; g.out = out;
  g.sa_m = sa_m; g.sa_k = sa_k; g.sb_k = sb_k; g.sb_n = sb_n;
  g.sc_m = sc_m; g.sc_n = sc_n; g.so_m = so_m; g.so_n = so_n;
  g.M = M; g.N = N; g.K = K;
  g.alpha = alpha; g.beta = beta;
  g.out_dtype = out_dtype; g.round_dtype = round_dtype;
  return g;
}

}  // namespace nt

#define NT_GEMM_PARAMS                                                                                           \
  const void *a, int64_t sa_m, int64_t sa_k, const void *b, int64_t sb_k, int64_t sb_n, const void *c,          \
      int64_t sc_m, int64_t sc_n, void *out, int64_t so_m, int64_t so_n, int out_dtype, int64_t M, int64_t N,   \
      int64_t K, float alpha, float beta, int round_dtype, hipStream_t stream
#define NT_GEMM_ARGS a, sa_m, sa_k, b, sb_k, sb_n, c, sc_m, sc_n, out, so_m, so_n, out_dtype, M, N, K, alpha, beta, round_dtype

extern "C" int nt_gemm_f16(NT_GEMM_PARAMS) { return nt::gemm16_launch<nt::f16_t>(nt::make_args(NT_GEMM_ARGS), stream); }
extern "C" int nt_gemm_bf16(NT_GEMM_PARAMS) {
  return nt::gemm16_launch<nt::bf16_t>(nt::make_args(NT_GEMM_ARGS), stream);
}
extern "C" int nt_gemm_f32(NT_GEMM_PARAMS) { return nt::gemm32_launch(nt::make_args(NT_GEMM_ARGS), stream); }
