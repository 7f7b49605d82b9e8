// 2-D convolution as an implicit GEMM on the MFMA tile core.
//
// GEMM view (as the conv2d arrangement builds it): rows m = (n, p, q) of the output
// positions, columns = output channels k, reduction over kk = (c, r, s).  The
// kernel computes the transposed product out^T[k][m] = sum_kk w[k][kk] * x_col[m][kk]
// so that lanes of a wave run along m, i.e. along q, which is the unit-stride
// direction of both the N-C-H-W input rows it gathers and the output it stores.
//
// Per 64-deep k-tile each lane of the 256-lane workgroup owns one m-row of the
// im2col tile: it walks (c, r, s) incrementally, gathers the 64 input values of its
// window positions (zero outside the input) and writes them to LDS as eight
// 16-byte chunks.  The filter tile is read as rows w[k][c*R*S + kk], with 16-byte
// loads when the filter is dense over (c, r, s).
// MFMA-bound in principle (2 * N*P*Q * K * C*R*S flops per launch).
#include "mfma_core.h"

namespace nt {

constexpr int CB_K = 256;  // output channels per workgroup
constexpr int CB_M = 256;  // output positions per workgroup
constexpr int C_THREADS = 256;

struct ConvArgs {
  const void* x;
  const void* w;
  void* y;
  int64_t xs[4], ws[4], ys[4];
  int64_t N, C, H, W, K, R, S, P, Q, ph, pw, sh, sw, dh, dw;
  int64_t M, KG;  // N*P*Q, C*R*S
  int y_dtype, round_dtype;
  int tiles_k, tiles_m;
};

template <typename T, bool DENSE_W>
__global__ __launch_bounds__(C_THREADS) void conv_direct_kernel(ConvArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[(CB_K + CB_M) * TILE_K];
  uint16_t* sW = smem;
  uint16_t* sX = smem + CB_K * TILE_K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wk = wave >> 1, wm = wave & 1;
  const int tk = blockIdx.x % g.tiles_k, tmi = blockIdx.x / g.tiles_k;
  const int64_t k0t = (int64_t)tk * CB_K, m0t = (int64_t)tmi * CB_M;
  const uint16_t* X = (const uint16_t*)g.x;
  const uint16_t* Wt = (const uint16_t*)g.w;

  // This lane's im2col row.
  const int64_t m = m0t + tid;
  const bool m_ok = m < g.M;
  int64_t hb = 0, wb = 0, xrow = 0;
  if (m_ok) {
    const int64_t q = m % g.Q, t = m / g.Q;
    const int64_t p = t % g.P, n = t / g.P;
    hb = p * g.sh - g.ph;
    wb = q * g.sw - g.pw;
    xrow = n * g.xs[0];
  }

  floatx16 acc[4][4];
  zero_acc(acc);
  const int64_t nk = cdiv(g.KG, TILE_K);
  const int f_row = tid >> 3, f_chunk = tid & 7;

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int64_t kk0 = kt * TILE_K;
    // Filter tile: rows = output channels, 64 reduction values each.
    if (DENSE_W) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = i * 32 + f_row;
        const int64_t k = k0t + row;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (k < g.K) v = *(const u32x4*)(Wt + k * g.ws[0] + kk0 + f_chunk * 8);
        *(u32x4*)(sW + row * TILE_K + swz(row, f_chunk) * 8) = v;
      }
    } else {
      for (int e = tid; e < CB_K * TILE_K; e += C_THREADS) {
        const int row = e / TILE_K, kk = e % TILE_K;
        const int64_t k = k0t + row, kg = kk0 + kk;
        uint16_t v = 0;
        if (k < g.K && kg < g.KG) {
          const int64_t s = kg % g.S, t = kg / g.S;
          const int64_t r = t % g.R, c = t / g.R;
          v = Wt[k * g.ws[0] + c * g.ws[1] + r * g.ws[2] + s * g.ws[3]];
        }
        sW[lds_index(row, kk)] = v;
      }
    }
    // im2col tile: this lane's row, 64 consecutive (c, r, s).
    {
      int64_t s = kk0 % g.S, t = kk0 / g.S;
      int64_t r = t % g.R, c = t / g.R;
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) {
        uint32_t packed[4];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t kg = kk0 + ch * 8 + u;
          uint16_t v = 0;
          const int64_t h = hb + r * g.dh, wv = wb + s * g.dw;
          if (m_ok && kg < g.KG && h >= 0 && h < g.H && wv >= 0 && wv < g.W)
            v = X[xrow + c * g.xs[1] + h * g.xs[2] + wv * g.xs[3]];
          if (u & 1)
            packed[u >> 1] |= (uint32_t)v << 16;
          else
            packed[u >> 1] = v;
          if (++s == g.S) {
            s = 0;
            if (++r == g.R) {
              r = 0;
              ++c;
            }
          }
        }
        *(u32x4*)(sX + tid * TILE_K + swz(tid, ch) * 8) = u32x4{packed[0], packed[1], packed[2], packed[3]};
      }
    }
    __syncthreads();
    mma_ktile<T, 4, 4>(sW, sX, wk * 128, wm * 128, lane, acc);
    __syncthreads();
  }

  // Epilogue: y[n, k, p, q] = cast(round(acc)); slabs of 32 channels staged in LDS,
  // then each lane stores runs of consecutive output positions m.
  __syncthreads();
  float* stage = (float*)smem + wave * (32 * 128);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    stage_slab<4>(stage, acc[i], lane);
    __syncthreads();
    const int64_t k_0 = k0t + wk * 128 + i * 32, m_0 = m0t + wm * 128;
    for (int e = lane; e < 32 * 128; e += 64) {
      const int kr = e >> 7, mc = e & 127;
      const int64_t k = k_0 + kr, mm = m_0 + mc;
      if (k >= g.K || mm >= g.M) continue;
      const int64_t q = mm % g.Q, t = mm / g.Q;
      const int64_t p = t % g.P, n = t / g.P;
      store_from_float(g.y, n * g.ys[0] + k * g.ys[1] + p * g.ys[2] + q * g.ys[3], g.y_dtype,
                       round_through(stage[kr * 128 + mc], g.round_dtype));
    }
    __syncthreads();
  }
}

template <typename T>
static int conv_launch(const void* x, const int64_t* xs, const void* w, const int64_t* ws, void* y, const int64_t* ys,
                       int y_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                       int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw, int64_t dh, int64_t dw,
                       int round_dtype, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (N < 0 || C < 0 || H < 0 || W < 0 || K < 0 || R < 0 || S < 0 || P < 0 || Q < 0 || ph < 0 || pw < 0 || sh <= 0 ||
      sw <= 0 || dh <= 0 || dw <= 0)
    return NT_ERR_INVALID;
  if (!valid_dtype(y_dtype) || !valid_round(round_dtype)) return NT_ERR_INVALID;
  if (N * P * Q == 0 || K == 0) return 0;
  if (!x || !w || !y || !xs || !ws || !ys) return NT_ERR_INVALID;
  ConvArgs g{};
  g.x = x; g.w = w; g.y = y;
  for (int i = 0; i < 4; ++i) {
    g.xs[i] = xs[i];
    g.ws[i] = ws[i];
    g.ys[i] = ys[i];
  }
  g.N = N; g.C = C; g.H = H; g.W = W; g.K = K; g.R = R; g.S = S; g.P = P; g.Q = Q;
  g.ph = ph; g.pw = pw; g.sh = sh; g.sw = sw; g.dh = dh; g.dw = dw;
  g.M = N * P * Q;
  g.KG = C * R * S;
  g.y_dtype = y_dtype;
  g.round_dtype = round_dtype;
  const int64_t tiles_k = cdiv(K, CB_K), tiles_m = cdiv(g.M, CB_M);
  if (tiles_k * tiles_m > 0x7fffffffLL) return NT_ERR_INVALID;
  g.tiles_k = (int)tiles_k;
  g.tiles_m = (int)tiles_m;
  const bool dense_w = ws[3] == 1 && ws[2] == S && ws[1] == R * S && g.KG % TILE_K == 0 && (ws[0] * 2) % 16 == 0 &&
                       (uintptr_t)w % 16 == 0;
  const dim3 grid((unsigned)(tiles_k * tiles_m)), blk(C_THREADS);
  if (dense_w)
    hipLaunchKernelGGL((conv_direct_kernel<T, true>), grid, blk, 0, stream, g);
  else
    hipLaunchKernelGGL((conv_direct_kernel<T, false>), grid, blk, 0, stream, g);
  return launch_status();
}

}  // namespace nt

extern "C" int64_t nt_conv2d_workspace_size(int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R,
                                            int64_t S, int64_t ph, int64_t pw, int dtype) {
  (void)N; (void)C; (void)H; (void)W; (void)K; (void)R; (void)S; (void)ph; (void)pw; (void)dtype;
  return 0;
}

#define NT_CONV_ENTRY(NAME, T)                                                                                       \
  extern "C" int NAME(const void* x, const int64_t* xs, const void* w, const int64_t* ws, void* y, const int64_t* ys, \
                      int y_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,       \
                      int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw, int64_t dh, int64_t dw,   \
                      int round_dtype, void* workspace, int64_t workspace_bytes, hipStream_t stream) {               \
    return nt::conv_launch<T>(x, xs, w, ws, y, ys, y_dtype, N, C, H, W, K, R, S, P, Q, ph, pw, sh, sw, dh, dw,       \
                              round_dtype, workspace, workspace_bytes, stream);                                      \
  }
NT_CONV_ENTRY(nt_conv2d_f16, nt::f16_t)
NT_CONV_ENTRY(nt_conv2d_bf16, nt::bf16_t)
