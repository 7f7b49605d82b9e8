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

#include <atomic>
#include <mutex>
#include <type_traits>

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
  int64_t Cr;     // channels of x and w; C is the re-laid layout's (Cr rounded up, zero-filled)
  // conv_dma_kernel split along the reduction: `splits` workgroups per output tile, each
  // `kt_per` 32-deep k-tiles, fp32 partial tiles to part[split][K][M] (splits 1: none).
  int splits, kt_per;
  float* part;
  int64_t Mp;  // rows of the partials: M rounded up to 8
  int qvec;    // Q % 8 == 0 and y's q stride 1: 8 consecutive positions are one 16-byte run
  int y_dtype, round_dtype;
  int tiles_k, tiles_m;
  // Reduction order of the re-laid filter (and of the k-tiles that walk it): 1 for the DMA
  // kernels, (c / 32, r, s, c % 32), so that the nine taps of one 32-channel block come in
  // consecutive k-tiles and a workgroup's input rows for that block stay in L2 while they
  // are re-read; 0 for conv_nhwc_kernel, (r, s, c).
  int cb_order;
};

// Workgroups are dispatched to the eight XCDs round-robin (b to XCD b % 8), each XCD with
// its own L2.  This order hands XCD x the consecutive indices [x q + min(x, r), ...) of
// `total` = 8 q + r, so neighbouring image rows of the re-layout, which share the cache
// lines where one row of a channel plane runs into the next, meet in one L2.
__device__ __forceinline__ int64_t xcd_order(int64_t b, int64_t total) {
  const int64_t x = b % 8, q = total / 8, r = total % 8;
  return x * q + (x < r ? x : r) + b / 8;
}

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


// ----------------------------------------------------------------------------- N-H-W-C path
// With a workspace the input is re-laid as zero-padded N-Hp-Wp-C (Hp = H + 2ph, Wp = W + 2pw)
// and the filter as K-R-S-C (for the DMA kernels K-(C/32)-R-S-32: ConvArgs::cb_order).
// Reduction index kk = (r*S + s)*C + c then walks channels contiguously, so for a 64-deep k-tile inside one (r, s) every im2col row and every
// filter row is 128 contiguous bytes: both operands load with 16-byte loads straight
// into the k-contiguous LDS layout of the MFMA core, no gathers, no transposes, no
// padding tests.  Needs C % 64 == 0.  Cost of the re-layout: one read and one write of
// the input (plus the small filter).

// x (N-C-H-W indexed, any strides) -> xp [N][Hp][Wp][C].  One workgroup per (n, hp, 64
// channels): the 64 x W slab goes through LDS so that reads run along w and writes
// along c (16 bytes per lane).
template <typename T>
__global__ __launch_bounds__(256) void nchw_to_nhwc_pad_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xp,
                                                               ConvArgs g, int64_t Hp, int64_t Wp) {
  __shared__ uint16_t tile[64][64 + 2];
  const int64_t cblocks = cdiv(g.C, 64);  // the last block may hold 32 channels
  const int64_t b = blockIdx.x;
  const int64_t cb = b % cblocks, row = b / cblocks;
  const int64_t hp = row % Hp, n = row / Hp;
  const int64_t h = hp - g.ph;
  const int64_t c0 = cb * 64;
  uint16_t* out_row = xp + ((n * Hp + hp) * Wp) * g.C + c0;
  const int tid = threadIdx.x;
  if (h < 0 || h >= g.H) {
    for (int64_t e = tid; e < Wp * 8; e += 256) {
      const int64_t wp = e / 8, ch = e % 8;
      if (c0 + ch * 8 < g.C) *(u32x4*)(out_row + wp * g.C + ch * 8) = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const uint16_t* xb = x + n * g.xs[0] + c0 * g.xs[1] + h * g.xs[2];
  for (int64_t w0 = -g.pw; w0 < Wp - g.pw; w0 += 64) {
    // load 64 channels x 64 positions [w0, w0 + 64)
    for (int e = tid; e < 64 * 64; e += 256) {
      const int c = e / 64, wi = e % 64;
      const int64_t w = w0 + wi;
      tile[c][wi] = (w >= 0 && w < g.W && c0 + c < g.Cr) ? xb[c * g.xs[1] + w * g.xs[3]] : (uint16_t)0;
    }
    __syncthreads();
    for (int e = tid; e < 64 * 8; e += 256) {
      const int wi = e / 8, ch = e % 8;
      const int64_t wp = w0 + g.pw + wi;
      if (wp < Wp && c0 + ch * 8 < g.C) {
        uint16_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = tile[ch * 8 + u][wi];
        *(u32x4*)(out_row + wp * g.C + ch * 8) = *(const u32x4*)v;
      }
    }
    __syncthreads();
  }
}

// w (K-C-R-S indexed, any strides) -> wt [K][R][S][C].
template <typename T>
__global__ __launch_bounds__(256) void filter_krsc_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                          ConvArgs g) {
  // One (k, r, s) row of C channels per workgroup and step (index arithmetic once per row).
  const int64_t krs = g.K * g.R * g.S;
  for (int64_t row = blockIdx.x; row < krs; row += gridDim.x) {
    const int64_t s = row % g.S, t = row / g.S;
    const int64_t r = t % g.R, k = t / g.R;
    const uint16_t* src = w + k * g.ws[0] + r * g.ws[2] + s * g.ws[3];
    uint16_t* dst = g.cb_order ? wt + k * g.KG + (r * g.S + s) * 32 : wt + row * g.C;
    const int64_t cb_step = g.R * g.S * 32;
    for (int64_t c = threadIdx.x; c < g.C; c += blockDim.x)
      dst[g.cb_order ? (c >> 5) * cb_step + (c & 31) : c] = c < g.Cr ? src[c * g.ws[1]] : (uint16_t)0;
  }
}

// One launch for both re-layouts.  Workgroups [0, N * Hp): padded input row (n, hp) of
// xp; pad rows and pad columns are written as zeros; interior 8 (channel) x 8 (w) blocks
// go one per lane: eight 16-byte loads along w (one per channel), an 8 x 8 transpose of
// 16-bit values with v_perm_b32, eight 16-byte stores along c (one per position).  Needs
// unit w stride, 16-byte aligned input rows and W % 8 == 0.  Workgroups past N * Hp:
// the filter into K-R-S-C (or K-(C/32)-R-S-32), one (k, r, s) row of C channels at a time.
// STAGE (C * W * 2 <= RELAYOUT_STAGE_BYTES): lanes along w for the loads (each load
// instruction reads runs of one channel row), the transposed chunks into LDS in the output
// row's order, 16-byte chunk (pos, cb) at pos * C/8 + (cb ^ (pos / 8 & mask)) (mask < 8
// divides C/8, so the XOR stays inside the row; it spreads one store instruction's chunks,
// eight positions apart, over the banks), then consecutive lanes copy the W * C values of
// the row out (each store instruction one contiguous run).  Otherwise lanes along channel
// chunks, stored straight from registers.
constexpr int RELAYOUT_STAGE_BYTES = 32768;
template <typename T, bool STAGE>
__global__ __launch_bounds__(256) void conv_relayout_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xp,
                                                            const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                            ConvArgs g, int64_t Hp, int64_t Wp) {
  const int64_t rows = g.N * Hp;
  const int tid = threadIdx.x;
  if ((int64_t)blockIdx.x >= rows) {
    // Filter: one (k, r, s) row of C channels per workgroup and step, its index arithmetic
    // done once per row (workgroup-uniform), lanes along c (coalesced stores).
    const int64_t krs = g.K * g.R * g.S, nb = (int64_t)gridDim.x - rows;
    for (int64_t row = (int64_t)blockIdx.x - rows; row < krs; row += nb) {
      const int64_t s = row % g.S, t = row / g.S;
      const int64_t r = t % g.R, k = t / g.R;
      const uint16_t* src = w + k * g.ws[0] + r * g.ws[2] + s * g.ws[3];
      uint16_t* dst = g.cb_order ? wt + k * g.KG + (r * g.S + s) * 32 : wt + row * g.C;
      const int64_t cb_step = g.R * g.S * 32;
      for (int64_t c = tid; c < g.C; c += 256)
        dst[g.cb_order ? (c >> 5) * cb_step + (c & 31) : c] = c < g.Cr ? src[c * g.ws[1]] : (uint16_t)0;
    }
    return;
  }
  const int64_t rb = xcd_order(blockIdx.x, rows);
  const int64_t hp = rb % Hp, n = rb / Hp;
  const int64_t h = hp - g.ph;
  const int64_t C = g.C, W = g.W;
  uint16_t* out_row = xp + ((n * Hp + hp) * Wp) * C;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  const int64_t cchunks = C / 8;
  if (h < 0 || h >= g.H) {
    for (int64_t e = tid; e < Wp * cchunks; e += 256) *(u32x4*)(out_row + e * 8) = zero;
    return;
  }
  // pad columns
  for (int64_t e = tid; e < (Wp - W) * cchunks; e += 256) {
    const int64_t col = e / cchunks, ch = e % cchunks;
    const int64_t wp = col < g.pw ? col : col + W;
    *(u32x4*)(out_row + wp * C + ch * 8) = zero;
  }
  const uint16_t* xb = x + n * g.xs[0] + h * g.xs[2];
  const int64_t wblocks = W / 8;
  // eight channel rows at columns wb*8 .. +7 -> eight positions of channel chunk cb
  auto transpose = [&](int64_t cb, int64_t wb, u32x4 (&out)[8]) {
    u32x4 in[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      in[i] = cb * 8 + i < g.Cr ? *(const u32x4*)(xb + (cb * 8 + i) * g.xs[1] + wb * 8) : zero;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = j >> 1;
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      out[j] = u32x4{__builtin_amdgcn_perm(in[1][d], in[0][d], sel), __builtin_amdgcn_perm(in[3][d], in[2][d], sel),
                     __builtin_amdgcn_perm(in[5][d], in[4][d], sel), __builtin_amdgcn_perm(in[7][d], in[6][d], sel)};
    }
  };
  if constexpr (STAGE) {
    __shared__ __attribute__((aligned(16))) u32x4 stage[RELAYOUT_STAGE_BYTES / 16];
    const int cc = (int)cchunks, wbk = (int)wblocks;
    const int mask = cc % 8 == 0 ? 7 : cc % 4 == 0 ? 3 : cc % 2 == 0 ? 1 : 0;
    for (int e = tid; e < cc * wbk; e += 256) {
      const int cb = e / wbk, wb = e - cb * wbk;
      u32x4 out[8];
      transpose(cb, wb, out);
#pragma unroll
      for (int j = 0; j < 8; ++j) stage[(wb * 8 + j) * cc + (cb ^ (wb & mask))] = out[j];
    }
    __syncthreads();
    u32x4* dst = (u32x4*)(out_row + g.pw * C);  // positions pw .. pw + W - 1: W * C/8 chunks in a row
    for (int k = tid; k < (int)W * cc; k += 256) {
      const int pos = k / cc, cb = k - pos * cc;
      dst[k] = stage[pos * cc + (cb ^ ((pos >> 3) & mask))];
    }
  } else {
    for (int64_t e = tid; e < cchunks * wblocks; e += 256) {
      // lanes along channel chunks: each store instruction writes whole runs of a position's
      // channels (12.6-12.9 us against 13.5-13.8 with lanes along w, whose loads coalesced
      // instead, at [16,256,56,56])
      const int64_t wb = e / cchunks, cb = e % cchunks;
      u32x4 out[8];
      transpose(cb, wb, out);
#pragma unroll
      for (int j = 0; j < 8; ++j) *(u32x4*)(out_row + (g.pw + wb * 8 + j) * C + cb * 8) = out[j];
    }
  }
}

// The filter into K-R-S-C, or K-(C/32)-R-S-32 (cb_order), for conv_relayout_pipe_kernel:
// one output channel k per workgroup and step, lanes along the destination row (coalesced
// stores), loads gathered from any strides.
__device__ __forceinline__ void relayout_filter_rows(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                     const ConvArgs& g, int64_t first, int64_t step) {
  const int RS = (int)(g.R * g.S), S = (int)g.S, C = (int)g.C, KG = (int)g.KG, Cr = (int)g.Cr;
  for (int64_t k = first; k < g.K; k += step) {
    const uint16_t* src = w + k * g.ws[0];
    uint16_t* dst = wt + k * g.KG;
    for (int d = threadIdx.x; d < KG; d += blockDim.x) {
      int c, rs;
      if (g.cb_order) {
        const int cb = d / (RS * 32), rem = d - cb * RS * 32;
        rs = rem >> 5;
        c = cb * 32 + (rem & 31);
      } else {
        rs = d / C;
        c = d - rs * C;
      }
      const int r = rs / S, s = rs - r * S;
      dst[d] = c < Cr ? src[c * g.ws[1] + r * g.ws[2] + s * g.ws[3]] : (uint16_t)0;
    }
  }
}

// conv_relayout_kernel's STAGE form for rows of at most 256 8 x 8 blocks (one per lane),
// with fewer workgroups than rows: workgroup b takes rows b, b + row_blocks, ... (in
// xcd_order) and issues the loads of its next row before it transposes, stages and stores
// the current one, so each CU reads and writes at once.  With one workgroup per row, all of
// them resident, the GPU read every row before it wrote any: 10.9 us for the rows of
// [16,256,56,56] against 53.6 MB moved.  Workgroups from row_blocks on re-lay the filter,
// one output channel at a time (one workgroup per filter row (k, r, s) took 5.3 us alone).
template <typename T>
__global__ __launch_bounds__(256) void conv_relayout_pipe_kernel(const uint16_t* __restrict__ x,
                                                                 uint16_t* __restrict__ xp,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ wt, ConvArgs g, int64_t Hp,
                                                                 int64_t Wp, int row_blocks) {
  const int tid = threadIdx.x;
  if ((int)blockIdx.x >= row_blocks) {
    relayout_filter_rows(w, wt, g, (int)blockIdx.x - row_blocks, (int)gridDim.x - row_blocks);
    return;
  }
  __shared__ __attribute__((aligned(16))) u32x4 stage[RELAYOUT_STAGE_BYTES / 16];
  const int64_t rows = g.N * Hp;
  const int64_t C = g.C, W = g.W;
  const int cc = (int)(C / 8), wbk = (int)(W / 8);
  const int mask = cc % 8 == 0 ? 7 : cc % 4 == 0 ? 3 : cc % 2 == 0 ? 1 : 0;
  const bool active = tid < cc * wbk;
  const int cb = active ? tid / wbk : 0, wb = active ? tid - cb * wbk : 0;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  // Loads of row `it` (xcd_order) into `in`: this lane's 8 (channel) x 8 (w) block.
  auto load = [&](int64_t it, u32x4 (&in)[8]) {
    const int64_t rb = xcd_order(it, rows);
    const int64_t hp = rb % Hp, n = rb / Hp, h = hp - g.ph;
    if (!active || h < 0 || h >= g.H) return;
    const uint16_t* xb = x + n * g.xs[0] + h * g.xs[2] + wb * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) in[i] = cb * 8 + i < g.Cr ? *(const u32x4*)(xb + (cb * 8 + i) * g.xs[1]) : zero;
  };
  // Row `it` from `cur`, after issuing the loads of row it + row_blocks into `nxt`.
  auto step = [&](int64_t it, u32x4 (&cur)[8], u32x4 (&nxt)[8]) {
    if (it + row_blocks < rows) load(it + row_blocks, nxt);
    const int64_t rb = xcd_order(it, rows);
    const int64_t hp = rb % Hp, n = rb / Hp, h = hp - g.ph;
    uint16_t* out_row = xp + ((n * Hp + hp) * Wp) * C;
    if (h < 0 || h >= g.H) {  // a pad row (workgroup-uniform)
      for (int64_t e = tid; e < Wp * cc; e += 256) *(u32x4*)(out_row + e * 8) = zero;
      return;
    }
    for (int64_t e = tid; e < (Wp - W) * cc; e += 256) {  // pad columns
      const int64_t col = e / cc, ch = e % cc;
      const int64_t wp = col < g.pw ? col : col + W;
      *(u32x4*)(out_row + wp * C + ch * 8) = zero;
    }
    if (active) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = j >> 1;
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        stage[(wb * 8 + j) * cc + (cb ^ (wb & mask))] =
            u32x4{__builtin_amdgcn_perm(cur[1][d], cur[0][d], sel), __builtin_amdgcn_perm(cur[3][d], cur[2][d], sel),
                  __builtin_amdgcn_perm(cur[5][d], cur[4][d], sel), __builtin_amdgcn_perm(cur[7][d], cur[6][d], sel)};
      }
    }
    __syncthreads();
    u32x4* dst = (u32x4*)(out_row + g.pw * C);  // positions pw .. pw + W - 1: W * C/8 chunks in a row
    for (int k = tid; k < (int)W * cc; k += 256) {
      const int pos = k / cc, c8 = k - pos * cc;
      dst[k] = stage[pos * cc + (c8 ^ ((pos >> 3) & mask))];
    }
    __syncthreads();  // the stage is rewritten by the next row
  };
  u32x4 a[8], b[8];
  int64_t it = blockIdx.x;
  if (it < rows) load(it, a);
  for (; it < rows; it += 2 * (int64_t)row_blocks) {
    step(it, a, b);
    if (it + row_blocks < rows) step(it + row_blocks, b, a);
  }
}

// Implicit GEMM over the re-laid operands: out^T[k][m] = sum_kk wt[k][kk] * xcol[m][kk].
// 512 lanes, waves 4 (k) x 2 (m), 256 x 256 tile, two 64 KiB LDS buffers, tile kt+2
// fetched while kt is multiplied (as the GEMM fast path).
template <typename T>
__global__ __launch_bounds__(512) void conv_nhwc_kernel(const uint16_t* __restrict__ xp, const uint16_t* __restrict__ wt,
                                                        ConvArgs g, int64_t Hp, int64_t Wp) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (CB_K + CB_M) * TILE_K];
  constexpr int BUF = (CB_K + CB_M) * TILE_K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wk = wave >> 1, wm = wave & 1;
  const int tk = blockIdx.x % g.tiles_k, tmi = blockIdx.x / g.tiles_k;
  const int64_t k0t = (int64_t)tk * CB_K, m0t = (int64_t)tmi * CB_M;
  const int row_in = tid >> 3, chunk = tid & 7;  // rows row_in + 64*i, 16-byte chunk
  const int64_t KG = g.KG;

  // Per-lane row bases: filter rows k and im2col rows m.
  const uint16_t* wrow[4];
  int64_t xrow[4];
  bool wok[4], xok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = k0t + row_in + 64 * i;
    wok[i] = k < g.K;
    wrow[i] = wt + (wok[i] ? k : 0) * KG + chunk * 8;
    const int64_t m = m0t + row_in + 64 * i;
    xok[i] = m < g.M;
    const int64_t mm = xok[i] ? m : 0;
    const int64_t q = mm % g.Q, t = mm / g.Q;
    const int64_t p = t % g.P, n = t / g.P;
    xrow[i] = ((n * Hp + p * g.sh) * Wp + q * g.sw) * g.C + chunk * 8;
  }
  int st[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = row_in + 64 * i;
    st[i] = r * TILE_K + swz(r, chunk) * 8;
  }
  const int nk = (int)(KG / TILE_K);
  u32x4 ra[4], rb[4];
  auto load = [&](int kt) {
    const int64_t kk0 = (int64_t)kt * TILE_K;
    const int64_t rs = kk0 / g.C, c0 = kk0 % g.C;
    const int64_t r = rs / g.S, s = rs % g.S;
    const int64_t xoff = (r * g.dh * Wp + s * g.dw) * g.C + c0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = wok[i] ? *(const u32x4*)(wrow[i] + kk0) : u32x4{0u, 0u, 0u, 0u};
      rb[i] = xok[i] ? *(const u32x4*)(xp + xrow[i] + xoff) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](uint16_t* buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(u32x4*)(buf + st[i]) = ra[i];
      *(u32x4*)(buf + CB_K * TILE_K + st[i]) = rb[i];
    }
  };

  floatx16 acc[2][4];
  zero_acc(acc);
  load(0);
  store(smem);
  if (nk > 1) load(1);
  __syncthreads();
  typedef typename mfma_traits<T>::frag frag;
  auto step = [&](auto has1_c, auto has2_c, int kt) {
    constexpr bool HAS1 = decltype(has1_c)::value, HAS2 = decltype(has2_c)::value;
    const uint16_t* sW = smem + (kt & 1) * BUF;
    const uint16_t* sX = sW + CB_K * TILE_K;
    if constexpr (HAS1) {
      store(smem + ((kt & 1) ^ 1) * BUF);
      if constexpr (HAS2) load(kt + 2);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < TILE_K / 16; ++kk) {
      const int ch = kk * 2 + (lane >> 5);
      frag fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wk * 64 + i * 32 + (lane & 31);
        fa[i] = *(const frag*)(sW + row * TILE_K + swz(row, ch) * 8);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = wm * 128 + j * 32 + (lane & 31);
        fb[j] = *(const frag*)(sX + row * TILE_K + swz(row, ch) * 8);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_traits<T>::mma(fa[i], fb[j], acc[i][j]);
    }
    __syncthreads();
  };
  using T1 = std::integral_constant<bool, true>;
  using F1 = std::integral_constant<bool, false>;
  int kt = 0;
  for (; kt + 2 < nk; ++kt) step(T1{}, T1{}, kt);
  if (kt + 1 < nk) step(T1{}, F1{}, kt++);
  step(F1{}, F1{}, kt);

  // Epilogue: slabs of 32 channels x 128 positions staged in LDS; 8 consecutive output
  // positions per lane, one 16-byte store when they share an output row.
  float* stage = (float*)smem + wave * (32 * 128);
  const bool vec = g.y_dtype != NT_DTYPE_F32 && g.ys[3] == 1 && g.Q % 8 == 0 && ((uintptr_t)g.y % 16) == 0 &&
                   (g.ys[0] % 8) == 0 && (g.ys[1] % 8) == 0 && (g.ys[2] % 8) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    stage_slab<4>(stage, acc[i], lane);
    __syncthreads();
    const int64_t k_0 = k0t + wk * 64 + i * 32, m_0 = m0t + wm * 128;
    for (int e = lane; e < 32 * 16; e += 64) {
      const int kr = e >> 4, mg = (e & 15) * 8;
      const int64_t k = k_0 + kr, mm = m_0 + mg;
      if (k >= g.K || mm >= g.M) continue;
      const int64_t q = mm % g.Q, t = mm / g.Q;
      const int64_t p = t % g.P, n = t / g.P;
      const float* sv = stage + kr * 128 + mg;
      if (vec && mm + 8 <= g.M) {
        u32x4 raw;
        uint16_t* h = (uint16_t*)&raw;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float v = round_through(sv[u], g.round_dtype);
          h[u] = g.y_dtype == NT_DTYPE_F16 ? float_to_f16_bits(v) : float_to_bf16_bits(v);
        }
        *(u32x4*)((uint16_t*)g.y + n * g.ys[0] + k * g.ys[1] + p * g.ys[2] + q) = raw;
      } else {
        for (int u = 0; u < 8 && mm + u < g.M; ++u) {
          const int64_t m2 = mm + u;
          const int64_t q2 = m2 % g.Q, t2 = m2 / g.Q;
          const int64_t p2 = t2 % g.P, n2 = t2 / g.P;
          store_from_float(g.y, n2 * g.ys[0] + k * g.ys[1] + p2 * g.ys[2] + q2 * g.ys[3], g.y_dtype,
                           round_through(sv[u], g.round_dtype));
        }
      }
    }
    __syncthreads();
  }
}

// DMA form of the implicit GEMM (the GEMM's gemm_dma_kernel pipeline on two k-contiguous
// operands): 512 lanes, two waves per SIMD in a 2 (output channels) x 4 (positions) grid,
// each owning 128 x 64 of the 256 x 256 tile; k-tiles of 32 in a four-stage LDS ring
// filled by buffer_load ... lds from inline assembly (tile kt+3 into the stage of tile
// kt-1, one barrier per k-tile, no register staging).  Both operands are stored [row][k]
// in 64-byte rows whose 16-byte chunks are XOR-swizzled by (row / 4) % 4 and read with
// ds_read_b128: a = filter rows (K-(C/32)-R-S-32), b = im2col rows of the padded N-H-W-C
// input, addressed by a per-lane base offset plus one scalar (channel block, r, s) offset
// per k-tile (C % 32 == 0: a k-tile is one tap of one 32-channel block); rows past M point
// past the end of the resource and read zeros.  Epilogue: 16-row halves of each wave's
// accumulators staged in its own 4 KiB of LDS, each lane storing 8 consecutive
// positions of one channel (their (n, p, q) computed once).
namespace cdma {
constexpr int STAGE = 16384, B0 = 65536, EPI = 131072;
__device__ __forceinline__ int asw(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }
__device__ __forceinline__ u32x4 rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, bytes, 0x00020000u};
}
__device__ __forceinline__ void load_lds16(u32x4 rs, uint32_t lds_addr, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rs), "s"(soffset)
               : "memory", "m0");
}
}  // namespace cdma

template <typename T, int TW = 256>
__global__ __launch_bounds__(TW * 2) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_dma_kernel(
    const uint16_t* __restrict__ xp, const uint16_t* __restrict__ wt, ConvArgs g, int64_t Hp, int64_t Wp) {
  // TW: the tile, TW channels x TW positions (256: eight waves of 128 x 64; 128: four waves
  // of 64 x 64, 80 KiB of LDS, two workgroups per CU, for outputs of few 256 x 256 tiles).
  static_assert(TW == 256 || TW == 128, "256 or 128 wide tiles");
  constexpr int NW = TW / 32, NI = TW / 64;  // waves; 32-row filter blocks per wave
  constexpr int STAGE = TW * 64, B0 = 4 * STAGE, EPI = 8 * STAGE;
  __shared__ __attribute__((aligned(1024))) char lds[EPI + NW * 4096];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wk = wave / (NW / 2), wm = wave % (NW / 2);
  const int ntile = g.tiles_k * g.tiles_m;
  const int split = (int)blockIdx.x / ntile, tile = (int)blockIdx.x - split * ntile;
  const int tk = tile % g.tiles_k, tmi = tile / g.tiles_k;
  const int k0t = tk * TW, m0t = tmi * TW;
  const int KG = (int)g.KG, C = (int)g.C;
  // This workgroup's k-tiles [kt0, kt1): all of them, or one split's (at least 3).
  const int kt0 = split * g.kt_per, kt1 = min(KG / 32, kt0 + g.kt_per);

  // Load q (0, 1) of this wave per k-tile: rows 32 wave + 16 q + lane / 4 of each operand,
  // LDS chunk lane % 4.  Filter rows past K lie past the resource's end (zeros).
  const u32x4 rsW = cdma::rsrc(wt + (int64_t)k0t * KG, (uint32_t)((g.K - k0t) * KG * 2));
  const uint32_t x_bytes = (uint32_t)(g.N * Hp * Wp * g.C * 2);
  const u32x4 rsX = cdma::rsrc(xp, x_bytes);
  int vw[2], vx[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 32 * wave + 16 * q + (lane >> 2);
    const int ch = cdma::asw(row, lane & 3);
    vw[q] = (row * KG + ch * 8) * 2;
    const int m = m0t + row;
    if (m < g.M) {
      const int qq = m % (int)g.Q, t = m / (int)g.Q;
      const int p = t % (int)g.P, n = t / (int)g.P;
      vx[q] = (((n * (int)Hp + p * (int)g.sh) * (int)Wp + qq * (int)g.sw) * C + ch * 8) * 2;
    } else {
      vx[q] = (int)x_bytes;
    }
  }
  // Scalar byte offset of k-tile kt inside an im2col row: channel block cb, tap (r, s).
  auto x_off = [&](int kt) {
    const int taps = (int)(g.R * g.S);
    const int cb = kt / taps, rs = kt - cb * taps;
    const int r = rs / (int)g.S, s = rs - r * (int)g.S;
    return ((r * (int)g.dh * (int)Wp + s * (int)g.dw) * C + cb * 32) * 2;
  };
  // Load u (0..3) of tile kt into its stage: filter q0, im2col q0, filter q1, im2col q1.
  auto load_unit = [&](int u, int kt, int xo) {
    const int st = (kt & 3) * STAGE, q = u >> 1;
    if ((u & 1) == 0)
      cdma::load_lds16(rsW, lds0 + st + 2048 * wave + 1024 * q, vw[q], kt * 64);
    else
      cdma::load_lds16(rsX, lds0 + B0 + st + 2048 * wave + 1024 * q, vx[q], xo);
  };

  // Fragment reads: filter rows 32 NI wk + 32 i + lane % 32, im2col rows 64 wm + 32 j + lane % 32,
  // chunk 2 s + lane / 32 (the swizzle depends on lane % 32 only).
  int a_rd[2], b_rd[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const int ra = wk * 32 * NI + (lane & 31), rb = wm * 64 + (lane & 31);
    a_rd[s2] = ra * 64 + cdma::asw(ra, 2 * s2 + (lane >> 5)) * 16;
    b_rd[s2] = B0 + rb * 64 + cdma::asw(rb, 2 * s2 + (lane >> 5)) * 16;
  }
  typedef typename mfma_traits<T>::frag frag;
  frag fa[2][NI], fb[2][2];
  // Read unit x (0..NI+1) of slice s2 of the tile at stage byte offset st: a0, b0, b1, a1, ..
  auto read_unit = [&](int x, int s2, int st) {
    if (x == 0 || x >= 3) {
      const int i = x == 0 ? 0 : x - 2;
      fa[s2][i] = *(const frag*)(lds + a_rd[s2] + st + i * 2048);
    } else {
      const int j = x - 1;
      fb[s2][j] = *(const frag*)(lds + b_rd[s2] + st + j * 2048);
    }
  };

  floatx16 acc[NI][2];
  zero_acc(acc);

  // kt1 - kt0 >= 3 (the launcher checks): tiles kt0..kt0+2 in flight, wait for kt0.
  for (int kt = kt0; kt < kt0 + 3; ++kt) {
    const int xo = x_off(kt);
    for (int u = 0; u < 4; ++u) load_unit(u, kt, xo);
  }
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int x = 0; x < NI + 2; ++x) read_unit(x, 0, (kt0 & 3) * STAGE);

#define NT_CFENCE() __builtin_amdgcn_sched_barrier(0)
  // One k-tile, as gemm_dma_kernel's: HAS1 reads slice 0 of tile kt+1 during slice 1, LOAD
  // fetches tile kt+3, VM is the number of loads allowed outstanding once tile kt+1 has
  // landed (-1: the last tile, no wait and no barrier).
  auto step = [&](auto has1_c, auto load_c, auto vm_c, int kt) {
    constexpr bool HAS1 = decltype(has1_c)::value, LOAD = decltype(load_c)::value;
    constexpr int VM = decltype(vm_c)::value;
    const int st = (kt & 3) * STAGE, st1 = ((kt + 1) & 3) * STAGE;
    const int xo3 = LOAD ? x_off(kt + 3) : 0;
    static_for<0, 4 * NI>([&](auto m_c) {
      constexpr int m = decltype(m_c)::value;
      constexpr int s2 = m / (2 * NI), x = m % (2 * NI);
      if constexpr (m == 2 * NI && VM >= 0) {
        NT_CFENCE();
        if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        NT_CFENCE();
      }
      acc[x >> 1][x & 1] = mfma_traits<T>::mma(fa[s2][x >> 1], fb[s2][x & 1], acc[x >> 1][x & 1]);
      NT_CFENCE();
      if constexpr (x < NI + 2) {
        if constexpr (s2 == 0)
          read_unit(x, 1, st);
        else if constexpr (HAS1)
          read_unit(x, 0, st1);
      }
      if constexpr (s2 == 1 && LOAD && x < 4) load_unit(x, kt + 3, xo3);
      NT_CFENCE();
    });
  };
#undef NT_CFENCE
  using T1 = std::integral_constant<bool, true>;
  using F1 = std::integral_constant<bool, false>;
  using V4 = std::integral_constant<int, 4>;
  using V0 = std::integral_constant<int, 0>;
  using VN = std::integral_constant<int, -1>;
  int kt = kt0;
  for (; kt + 3 < kt1; ++kt) step(T1{}, T1{}, V4{}, kt);
  step(T1{}, F1{}, V4{}, kt);
  step(T1{}, F1{}, V0{}, kt + 1);
  step(F1{}, F1{}, VN{}, kt + 2);

  // Epilogue: this lane's 8 output positions (columns (lane % 8) * 8 .. + 7 of the wave's 64)
  // and their (n, p, q); channels rows t * 8 + lane / 8 of each 16-row half.
  float* stage = (float*)(lds + EPI + wave * 4096);
  const int cg = (lane & 7) * 8;
  const int mpos = m0t + wm * 64 + cg;
  const bool m_ok = mpos < g.M;
  // qvec: the 8 positions share one output row (one 16-byte store per channel); otherwise
  // each position's own offset (they may run across rows), stored element by element.
  int64_t ybase = 0;
  int64_t yoff[8];
  uint32_t yvalid = 0;  // bit u: position mpos + u < M (an offset may be negative for flipped views)
  if (m_ok) {
    const int q = mpos % (int)g.Q, t = mpos / (int)g.Q;
    const int p = t % (int)g.P, n = t / (int)g.P;
    ybase = n * g.ys[0] + p * g.ys[2] + q;
  }
  if (!g.qvec) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t m = mpos + u;
      const int64_t q = m % g.Q, t = m / g.Q;
      yoff[u] = (t / g.P) * g.ys[0] + (t % g.P) * g.ys[2] + q * g.ys[3];
      yvalid |= (m < g.M ? 1u : 0u) << u;
    }
  }
  uint16_t* Y = (uint16_t*)g.y;
  if (g.splits > 1) {
    // A split's partial tile, fp32, unrounded: conv_splitk_reduce_kernel sums the splits.
    float* P = g.part + (int64_t)split * g.K * g.Mp;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        wave_lds_order();
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 8 * h; r < 8 * h + 8; ++r)
            stage[(acc_row(r, lane) - 16 * h) * 64 + j * 32 + (lane & 31)] = acc[i][j][r];
        wave_lds_order();
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int rr = t * 8 + (lane >> 3);
          const int k = k0t + wk * 32 * NI + i * 32 + h * 16 + rr;
          if (m_ok && k < g.K) {
            float* dst = P + (int64_t)k * g.Mp + mpos;
            *(float4*)dst = *(const float4*)(stage + rr * 64 + cg);
            *(float4*)(dst + 4) = *(const float4*)(stage + rr * 64 + cg + 4);
          }
        }
      }
    return;
  }
  auto finish = [&](auto round_c) {
    constexpr int ROUND = decltype(round_c)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        wave_lds_order();  // the previous half's reads come first
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 8 * h; r < 8 * h + 8; ++r)
            stage[(acc_row(r, lane) - 16 * h) * 64 + j * 32 + (lane & 31)] = acc[i][j][r];
        wave_lds_order();  // every lane's writes before any lane reads
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int rr = t * 8 + (lane >> 3);
          const int k = k0t + wk * 32 * NI + i * 32 + h * 16 + rr;
          const float4 v0 = *(const float4*)(stage + rr * 64 + cg);
          const float4 v1 = *(const float4*)(stage + rr * 64 + cg + 4);
          const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
          u32x4 ow;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            float a = v[2 * d], b = v[2 * d + 1];
            if constexpr (ROUND == NT_DTYPE_F16) {
              a = f16_bits_to_float(float_to_f16_bits(a));
              b = f16_bits_to_float(float_to_f16_bits(b));
            }
            if constexpr (ROUND == NT_DTYPE_BF16) {
              a = bf16_bits_to_float(float_to_bf16_bits(a));
              b = bf16_bits_to_float(float_to_bf16_bits(b));
            }
            ow[d] = (uint32_t)elem<T>::from_float(a) | ((uint32_t)elem<T>::from_float(b) << 16);
          }
          if (m_ok && k < g.K) {
            if (g.qvec) {
              __builtin_nontemporal_store(ow, (u32x4*)(Y + ybase + (int64_t)k * g.ys[1]));
            } else {
#pragma unroll
              for (int u = 0; u < 8; ++u)
                if ((yvalid >> u) & 1u) Y[yoff[u] + (int64_t)k * g.ys[1]] = (uint16_t)(ow[u >> 1] >> (16 * (u & 1)));
            }
          }
        }
      }
  };
  if (g.round_dtype == NT_DTYPE_F16)
    finish(std::integral_constant<int, NT_DTYPE_F16>{});
  else if (g.round_dtype == NT_DTYPE_BF16)
    finish(std::integral_constant<int, NT_DTYPE_BF16>{});
  else
    finish(std::integral_constant<int, NT_DTYPE_NONE>{});
}

// Epilogue of the 224-position kernels (conv_dma224_kernel, conv_strip224_kernel): wave `wave`
// holds channels 64 (wave % 4) .. + 63 by positions 128 (wave / 4) .. + 32 NB - 1 of the tile
// whose first output channel is k0t and first position m0t.
template <typename T, int NB>
__device__ __forceinline__ void conv224_store(char* lds, floatx16 (&acc)[2][NB], const ConvArgs& g, int wave, int lane,
                                              int m0t, int k0t) {
  const int wk = wave & 3, wm = wave >> 2;
  uint16_t* Y = (uint16_t*)g.y;
  // Once every wave has left the k-loop the LDS ring and the staging area are
  // free: each wave owns 20 KiB of them and stages one 32-channel block of its tile at a
  // time (32 rows of its PW positions in fp32; a row stride of PW + 8 floats keeps the two
  // lane halves, four rows apart, on different banks), then each lane stores 16-byte runs
  // of 8 positions: positions 8 (lane % 16) .. + 7 of rows lane / 16 + 4 t.  One LDS round
  // trip per 32 channels, and eight stores per lane issued back to back.
  __syncthreads();
  constexpr int PW = NB * 32, SW = PW + 8;
  float* stage = (float*)(lds + wave * 20480);
  const int cp = (lane & 15) * 8;
  const int mpos = m0t + wm * 128 + cp;
  const bool m_ok = cp < PW && mpos < g.M;
  int64_t ybase = 0;
  int64_t yoff[8];
  uint32_t yvalid = 0;  // bit u: position mpos + u < M (an offset may be negative for flipped views)
  if (m_ok) {
    const int q = mpos % (int)g.Q, t = mpos / (int)g.Q;
    const int p = t % (int)g.P, n = t / (int)g.P;
    ybase = n * g.ys[0] + p * g.ys[2] + q;
  }
  if (!g.qvec) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t m = mpos + u;
      const int64_t q = m % g.Q, t = m / g.Q;
      yoff[u] = (t / g.P) * g.ys[0] + (t % g.P) * g.ys[2] + q * g.ys[3];
      yvalid |= (m < g.M ? 1u : 0u) << u;
    }
  }
  auto finish = [&](auto round_c) {
    constexpr int ROUND = decltype(round_c)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      wave_lds_order();  // the previous block's reads come first
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) stage[acc_row(r, lane) * SW + j * 32 + (lane & 31)] = acc[i][j][r];
      wave_lds_order();  // every lane's writes before any lane reads
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int rr = (lane >> 4) + 4 * t;
        const int k = k0t + wk * 64 + i * 32 + rr;
        const float4 v0 = *(const float4*)(stage + rr * SW + cp);
        const float4 v1 = *(const float4*)(stage + rr * SW + cp + 4);
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        u32x4 ow;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          float a = v[2 * d], b = v[2 * d + 1];
          if constexpr (ROUND == NT_DTYPE_F16) {
            a = f16_bits_to_float(float_to_f16_bits(a));
            b = f16_bits_to_float(float_to_f16_bits(b));
          }
          if constexpr (ROUND == NT_DTYPE_BF16) {
            a = bf16_bits_to_float(float_to_bf16_bits(a));
            b = bf16_bits_to_float(float_to_bf16_bits(b));
          }
          ow[d] = (uint32_t)elem<T>::from_float(a) | ((uint32_t)elem<T>::from_float(b) << 16);
        }
        if (m_ok && k < g.K) {
          if (g.qvec) {
            __builtin_nontemporal_store(ow, (u32x4*)(Y + ybase + (int64_t)k * g.ys[1]));
          } else {
#pragma unroll
            for (int u = 0; u < 8; ++u)
              if ((yvalid >> u) & 1u) Y[yoff[u] + (int64_t)k * g.ys[1]] = (uint16_t)(ow[u >> 1] >> (16 * (u & 1)));
          }
        }
      }
    }
  };
  if (g.round_dtype == NT_DTYPE_F16)
    finish(std::integral_constant<int, NT_DTYPE_F16>{});
  else if (g.round_dtype == NT_DTYPE_BF16)
    finish(std::integral_constant<int, NT_DTYPE_BF16>{});
  else
    finish(std::integral_constant<int, NT_DTYPE_NONE>{});
}

// conv_dma_kernel with tiles of 224 positions (seven 32-position blocks) by 256 channels,
// for outputs whose 256 x 256 tiles leave CUs idle: [16,256,56,56] has 196 such tiles for
// 256 CUs, and 224 of these.  Waves w and w + 4 of a workgroup run on one SIMD; wave w
// (0..3) takes channels 64 w .. 64 w + 63 and positions 0..127 of the tile, wave w + 4
// the same channels and positions 128..223, so each SIMD issues 8 + 6 MFMAs per 16-deep
// slice where a 256 x 256 tile takes 16: the workgroup's time scales with its 224
// positions.  Loads, ring, waits and barriers are conv_dma_kernel's (rows 224..255 of the
// position operand read zeros); each wave's body is compiled for its own block count, so
// neither carries a branch per MFMA.  No split reduction.
constexpr int CB_M224 = 224;
template <typename T>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_dma224_kernel(
    const uint16_t* __restrict__ xp, const uint16_t* __restrict__ wt, ConvArgs g, int64_t Hp, int64_t Wp) {
  __shared__ __attribute__((aligned(1024))) char lds[cdma::EPI + 8 * 4096];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = (int)blockIdx.x;
  const int tk = tile % g.tiles_k, tmi = tile / g.tiles_k;
  const int k0t = tk * CB_K, m0t = tmi * CB_M224;
  const int KG = (int)g.KG, C = (int)g.C;
  const int nkt = KG / 32;

  const u32x4 rsW = cdma::rsrc(wt + (int64_t)k0t * KG, (uint32_t)((g.K - k0t) * KG * 2));
  const uint32_t x_bytes = (uint32_t)(g.N * Hp * Wp * g.C * 2);
  const u32x4 rsX = cdma::rsrc(xp, x_bytes);
  int vw[2], vx[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 32 * wave + 16 * q + (lane >> 2);
    const int ch = cdma::asw(row, lane & 3);
    vw[q] = (row * KG + ch * 8) * 2;
    const int m = m0t + row;
    if (row < CB_M224 && m < g.M) {
      const int qq = m % (int)g.Q, t = m / (int)g.Q;
      const int p = t % (int)g.P, n = t / (int)g.P;
      vx[q] = (((n * (int)Hp + p * (int)g.sh) * (int)Wp + qq * (int)g.sw) * C + ch * 8) * 2;
    } else {
      vx[q] = (int)x_bytes;
    }
  }
  auto x_off = [&](int kt) {
    const int taps = (int)(g.R * g.S);
    const int cb = kt / taps, rs = kt - cb * taps;
    const int r = rs / (int)g.S, s = rs - r * (int)g.S;
    return ((r * (int)g.dh * (int)Wp + s * (int)g.dw) * C + cb * 32) * 2;
  };
  auto load_unit = [&](int u, int kt, int xo) {
    const int st = (kt & 3) * cdma::STAGE, q = u >> 1;
    if ((u & 1) == 0)
      cdma::load_lds16(rsW, lds0 + st + 2048 * wave + 1024 * q, vw[q], kt * 64);
    else
      cdma::load_lds16(rsX, lds0 + cdma::B0 + st + 2048 * wave + 1024 * q, vx[q], xo);
  };
  const int wk = wave & 3, wm = wave >> 2;

  auto body = [&](auto nb_c) {
    constexpr int NB = decltype(nb_c)::value;  // 32-position blocks of this wave
    // Fragment rows: channels 64 wk + 32 i + lane % 32, positions 128 wm + 32 j + lane % 32.
    int a_rd[2], b_rd[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int ra = wk * 64 + (lane & 31), rb = wm * 128 + (lane & 31);
      a_rd[s2] = ra * 64 + cdma::asw(ra, 2 * s2 + (lane >> 5)) * 16;
      b_rd[s2] = cdma::B0 + rb * 64 + cdma::asw(rb, 2 * s2 + (lane >> 5)) * 16;
    }
    typedef typename mfma_traits<T>::frag frag;
    frag fa[2][2], fb[2][NB];
    // Unit u (0..NB+1) of slice s2 at stage offset st, in the order the slice's MFMAs
    // (channel block x / NB, position block x % NB) consume them: a0, b0 .. b(NB-1), a1.
    auto read_unit = [&](int u, int s2, int st) {
      if (u == 0)
        fa[s2][0] = *(const frag*)(lds + a_rd[s2] + st);
      else if (u == NB + 1)
        fa[s2][1] = *(const frag*)(lds + a_rd[s2] + st + 2048);
      else
        fb[s2][u - 1] = *(const frag*)(lds + b_rd[s2] + st + (u - 1) * 2048);
    };
    floatx16 acc[2][NB];
    zero_acc(acc);
    for (int kt = 0; kt < 3; ++kt) {
      const int xo = x_off(kt);
      for (int u = 0; u < 4; ++u) load_unit(u, kt, xo);
    }
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int u = 0; u < NB + 2; ++u) read_unit(u, 0, 0);

#define NT_CFENCE() __builtin_amdgcn_sched_barrier(0)
    auto step = [&](auto has1_c, auto load_c, auto vm_c, int kt) {
      constexpr bool HAS1 = decltype(has1_c)::value, LOAD = decltype(load_c)::value;
      constexpr int VM = decltype(vm_c)::value;
      const int st = (kt & 3) * cdma::STAGE, st1 = ((kt + 1) & 3) * cdma::STAGE;
      const int xo3 = LOAD ? x_off(kt + 3) : 0;
      static_for<0, 4 * NB>([&](auto m_c) {
        constexpr int m = decltype(m_c)::value;
        constexpr int s2 = m / (2 * NB), x = m % (2 * NB);
        if constexpr (m == 2 * NB && VM >= 0) {
          NT_CFENCE();
          if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
          if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
          NT_CFENCE();
        }
        acc[x / NB][x % NB] = mfma_traits<T>::mma(fa[s2][x / NB], fb[s2][x % NB], acc[x / NB][x % NB]);
        NT_CFENCE();
        if constexpr (x < NB + 2) {
          if constexpr (s2 == 0)
            read_unit(x, 1, st);
          else if constexpr (HAS1)
            read_unit(x, 0, st1);
        }
        if constexpr (s2 == 1 && LOAD && x < 4) load_unit(x, kt + 3, xo3);
        NT_CFENCE();
      });
    };
#undef NT_CFENCE
    using T1 = std::integral_constant<bool, true>;
    using F1 = std::integral_constant<bool, false>;
    using V4 = std::integral_constant<int, 4>;
    using V0 = std::integral_constant<int, 0>;
    using VN = std::integral_constant<int, -1>;
    int kt = 0;
    for (; kt + 3 < nkt; ++kt) step(T1{}, T1{}, V4{}, kt);
    step(T1{}, F1{}, V4{}, kt);
    step(T1{}, F1{}, V0{}, kt + 1);
    step(F1{}, F1{}, VN{}, kt + 2);

    conv224_store<T, NB>(lds, acc, g, wave, lane, m0t, k0t);
  };
  if (wm == 0)
    body(std::integral_constant<int, 4>{});
  else
    body(std::integral_constant<int, 3>{});
}

// conv_dma224_kernel for 3 x 3 filters reading the N-C-H-W input itself, with no re-laid copy
// of it.  A tile is TR = 224 / Q whole output rows of one image (stride 1, dilation 1), so
// for one 32-channel block every tap (r, s) reads a window of the same srows = TR + 2 input
// rows.  The workgroup keeps that block's rows in LDS as a strip [srows][pitch][32 channels],
// zero outside the input (input column c at strip column c + pw), and reads the position
// operand of tap (r, s) for output (t, w) at strip position (t + r) * pitch + w + s.  A strip
// position takes 80 bytes (64 of data, 16 of padding) so that the 16 consecutive positions
// of one ds_read_b128 pass land on distinct banks; pitch = Q + 16 keeps that so across a row
// change.  Strips are double-buffered: during the nine k-tiles (taps) of block cb, block
// cb + 1's rows arrive by DMA as NP raw pieces (512 lanes x 16 bytes of channel rows, w
// fastest, so a wave reads runs of whole rows) on taps 0 .. NP - 1, and tap NP + 1 transposes
// them into the other strip (per lane 8 positions x 2 channels: two ds_read_b128, eight
// v_perm, eight ds_write_b32).  The filter operand (K-(C/32)-R-S-32, re-laid by
// filter_cb_kernel before this kernel) runs through conv_dma224_kernel's four-stage DMA ring,
// with its waits and barriers.  The nine taps of a block are unrolled, so tap offsets, piece
// and transposition steps and the vmcnt budget of each barrier (2 filter loads per k-tile,
// plus 1 after a k-tile that issued a piece) are constants: no division and no branch inside
// a block.  LDS: filter ring [0, 64 KiB), two strips, NP raw pieces; the epilogue
// (conv224_store) reuses all of it.
namespace cstrip {
constexpr int RING = 65536;   // the filter ring: four 16 KiB stages
constexpr int SPOS = 80;      // bytes per strip position
constexpr int PIECE = 8192;   // one raw piece: 512 lanes x 16 bytes
constexpr int MAX_PIECES = 3;
constexpr int LDS_BYTES = cdma::EPI + 8 * 4096;
}  // namespace cstrip

template <typename T, int NP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_strip224_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wt, ConvArgs g, int pitch, int srows) {
  constexpr int TAPS = 9;
  __shared__ __attribute__((aligned(1024))) char lds[cstrip::LDS_BYTES];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = (int)xcd_order(blockIdx.x, (int64_t)g.tiles_k * g.tiles_m);
  const int tk = tile % g.tiles_k, tmi = tile / g.tiles_k;
  const int k0t = tk * CB_K, m0t = tmi * CB_M224;
  const int Q = (int)g.Q, PQ = (int)(g.P * g.Q);
  const int n_img = m0t / PQ, p0 = (m0t - n_img * PQ) / Q;
  const int KG = (int)g.KG, ncb = (int)g.C / 32;
  const int wch = (int)g.W / 8, ntask = srows * 32 * wch;
  const int row_bytes = pitch * cstrip::SPOS;
  const int strip_bytes = srows * row_bytes;
  const int strip0 = cstrip::RING, raw0 = cstrip::RING + 2 * strip_bytes;
  // Byte offset of tap j's window inside a strip.
  auto tap = [&](int j) { return (j / 3) * row_bytes + (j % 3) * cstrip::SPOS; };

  // Filter ring loads, as conv_dma224_kernel's: rows 32 wave + 16 q + lane / 4, chunk lane % 4.
  const u32x4 rsW = cdma::rsrc(wt + (int64_t)k0t * KG, (uint32_t)((g.K - k0t) * KG * 2));
  int vw[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 32 * wave + 16 * q + (lane >> 2);
    vw[q] = (row * KG + cdma::asw(row, lane & 3) * 8) * 2;
  }
  auto load_filter = [&](int q, int kt) {
    cdma::load_lds16(rsW, lds0 + (kt & 3) * cdma::STAGE + 2048 * wave + 1024 * q, vw[q], kt * 64);
  };
  // Raw pieces: lane tid of piece j fetches chunk e = 512 j + tid, e = ((row * 32 + c) * wch + wc),
  // input row p0 - ph + row, channel 32 cb + c (cb in the scalar offset), w 8 wc .. 8 wc + 7;
  // rows outside the input (and e past the strip) point at the resource's end and read zeros.
  const uint32_t img_bytes = (uint32_t)(((g.C - 1) * g.xs[1] + (g.H - 1) * g.xs[2] + g.W) * 2);
  const u32x4 rsX = cdma::rsrc(x + (int64_t)n_img * g.xs[0], img_bytes);
  const int cb_bytes = (int)(32 * g.xs[1] * 2);
  int vp[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int e = j * 512 + tid;
    vp[j] = (int)img_bytes;
    if (e < ntask) {
      const int wc = e % wch, rc = e / wch;
      const int c = rc & 31, in_row = p0 - (int)g.ph + (rc >> 5);
      if (in_row >= 0 && in_row < (int)g.H) vp[j] = (int)((c * g.xs[1] + in_row * g.xs[2] + wc * 8) * 2);
    }
  }
  auto load_piece = [&](int j, int cb) {
    cdma::load_lds16(rsX, lds0 + raw0 + j * cstrip::PIECE + 1024 * wave, vp[j], cb * cb_bytes);
  };
  // Transposition: task u = tid + 512 h (h = 0, 1) of ntask / 2 takes channels 2 cp, 2 cp + 1 of
  // strip row `row`, w 8 wc .. 8 wc + 7 (cp fastest, so 16 lanes fill one position's 64 bytes).
  int tr_raw[2], tr_dst[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int u = tid + 512 * h;
    tr_raw[h] = tr_dst[h] = -1;
    if (u < ntask / 2) {
      const int cp = u & 15, rw = u >> 4;
      const int wc = rw % wch, row = rw / wch;
      tr_raw[h] = raw0 + ((row * 32 + 2 * cp) * wch + wc) * 16;
      tr_dst[h] = (row * pitch + (int)g.pw + wc * 8) * cstrip::SPOS + cp * 4;
    }
  }
  auto tr_read = [&](int h, u32x4& a, u32x4& b) {
    if (tr_raw[h] >= 0) {
      a = *(const u32x4*)(lds + tr_raw[h]);
      b = *(const u32x4*)(lds + tr_raw[h] + wch * 16);
    }
  };
  auto tr_write = [&](int h, const u32x4& a, const u32x4& b, int strip) {
    if (tr_dst[h] >= 0) {
      char* d = lds + strip + tr_dst[h];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *(uint32_t*)(d + i * cstrip::SPOS) =
            __builtin_amdgcn_perm(b[i >> 1], a[i >> 1], (i & 1) ? 0x07060302u : 0x05040100u);
    }
  };

  // Prologue: strip 0's pieces, filter tiles 0..2; pieces and tile 0 landed (vmcnt 4: tiles 1
  // and 2 may still fly); strip 0 transposed, the pad columns of both strips zeroed.
#pragma unroll
  for (int j = 0; j < NP; ++j) load_piece(j, 0);
  for (int kt = 0; kt < 3; ++kt) {
    load_filter(0, kt);
    load_filter(1, kt);
  }
  asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  {
    u32x4 a = {0u, 0u, 0u, 0u}, b = a;
    tr_read(0, a, b);
    tr_write(0, a, b, strip0);
    tr_read(1, a, b);
    tr_write(1, a, b, strip0);
  }
  {
    const int padc = pitch - (int)g.W, chunks = 2 * srows * padc * 4;
    for (int e = tid; e < chunks; e += 512) {
      const int ch = e & 3, rest = e >> 2;
      const int col = rest % padc, rb = rest / padc;  // rb = strip buffer * srows + row
      const int c = col < (int)g.pw ? col : col + (int)g.W;
      const int buf = rb / srows, row = rb - buf * srows;
      *(u32x4*)(lds + strip0 + buf * strip_bytes + (row * pitch + c) * cstrip::SPOS + ch * 16) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  __syncthreads();

  const int wk = wave & 3, wm = wave >> 2;
  auto body = [&](auto nb_c) {
    constexpr int NB = decltype(nb_c)::value;  // 32-position blocks of this wave
    // Fragment reads: filter rows 64 wk + 32 i + lane % 32 of the ring; positions 128 wm +
    // 32 j + lane % 32 = output (t, w) of the strip, channels 16 s2 + 8 (lane / 32) .. + 7.
    int a_rd[2], pb[NB];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int ra = wk * 64 + (lane & 31);
      a_rd[s2] = ra * 64 + cdma::asw(ra, 2 * s2 + (lane >> 5)) * 16;
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int m = wm * 128 + 32 * j + (lane & 31);
      const int t = m / Q, w = m - t * Q;
      pb[j] = (t * pitch + w) * cstrip::SPOS + (lane >> 5) * 16;
    }
    typedef typename mfma_traits<T>::frag frag;
    frag fa[2][2], fb[2][NB];
    // Unit u (0..NB+1) of slice s2 of the k-tile at ring stage st and position offset po:
    // a0, b0 .. b(NB-1), a1.
    auto read_unit = [&](int u, int s2, int st, int po) {
      if (u == 0)
        fa[s2][0] = *(const frag*)(lds + a_rd[s2] + st);
      else if (u == NB + 1)
        fa[s2][1] = *(const frag*)(lds + a_rd[s2] + st + 2048);
      else
        fb[s2][u - 1] = *(const frag*)(lds + pb[u - 1] + po + s2 * 32);
    };
    floatx16 acc[2][NB];
    zero_acc(acc);
#pragma unroll
    for (int u = 0; u < NB + 2; ++u) read_unit(u, 0, 0, strip0);

#define NT_CFENCE() __builtin_amdgcn_sched_barrier(0)
    // Tap J of channel block cb (k-tile kt = 9 cb + J).  HAS1 reads slice 0 of the next k-tile
    // during slice 1, LOAD fetches filter tile kt + 3, VM is the number of loads allowed in
    // flight at the barrier (-1: the last k-tile, no wait and no barrier), NEXT: a block
    // follows whose strip this block fetches and transposes.
    auto step = [&](auto j_c, auto has1_c, auto load_c, auto vm_c, auto next_c, int cb) {
      constexpr int J = decltype(j_c)::value, VM = decltype(vm_c)::value;
      constexpr bool HAS1 = decltype(has1_c)::value, LOAD = decltype(load_c)::value;
      constexpr bool NEXT = decltype(next_c)::value;
      constexpr bool PIECE = NEXT && J < NP, TRANS = NEXT && J == NP + 1;
      const int kt = cb * TAPS + J;
      const int st = (kt & 3) * cdma::STAGE, st1 = ((kt + 1) & 3) * cdma::STAGE;
      const int sb = strip0 + (cb & 1) * strip_bytes, sbn = strip0 + ((cb + 1) & 1) * strip_bytes;
      const int po = sb + tap(J), po1 = J + 1 < TAPS ? sb + tap(J + 1) : sbn;
      u32x4 ta = {0u, 0u, 0u, 0u}, tb = ta;
      static_for<0, 4 * NB>([&](auto m_c) {
        constexpr int m = decltype(m_c)::value;
        constexpr int s2 = m / (2 * NB), x = m % (2 * NB);
        if constexpr (m == 2 * NB && VM >= 0) {
          NT_CFENCE();
          if constexpr (VM == 3) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
          if constexpr (VM == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
          if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
          NT_CFENCE();
        }
        acc[x / NB][x % NB] = mfma_traits<T>::mma(fa[s2][x / NB], fb[s2][x % NB], acc[x / NB][x % NB]);
        NT_CFENCE();
        if constexpr (x < NB + 2) {
          if constexpr (s2 == 0)
            read_unit(x, 1, st, po);
          else if constexpr (HAS1)
            read_unit(x, 0, st1, po1);
        }
        if constexpr (s2 == 1 && LOAD && x < 2) load_filter(x, kt + 3);
        if constexpr (s2 == 1 && PIECE && x == 2) load_piece(J, cb + 1);
        if constexpr (s2 == 1 && TRANS && (x == 0 || x == 3)) tr_read(x == 0 ? 0 : 1, ta, tb);
        if constexpr (s2 == 1 && TRANS && x == 2) tr_write(0, ta, tb, sbn);
        if constexpr (s2 == 1 && TRANS && x == 5) {
          tr_write(1, ta, tb, sbn);
          // The next barrier can come before any LDS read issued after these writes has
          // been waited for, and a barrier alone does not wait for LDS operations.
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        NT_CFENCE();
      });
    };
#undef NT_CFENCE
    using T1 = std::integral_constant<bool, true>;
    using F1 = std::integral_constant<bool, false>;
    using V3 = std::integral_constant<int, 3>;
    using V2 = std::integral_constant<int, 2>;
    using V0 = std::integral_constant<int, 0>;
    using VN = std::integral_constant<int, -1>;
    int cb = 0;
    for (; cb + 1 < ncb; ++cb) {
      static_for<0, TAPS>([&](auto j_c) {
        constexpr int J = decltype(j_c)::value;
        // taps 1 .. NP follow a tap that issued a piece
        using VM = std::conditional_t<(J >= 1 && J <= NP), V3, V2>;
        step(j_c, T1{}, T1{}, VM{}, T1{}, cb);
      });
    }
    static_for<0, TAPS - 3>([&](auto j_c) { step(j_c, T1{}, T1{}, V2{}, F1{}, cb); });
    step(std::integral_constant<int, TAPS - 3>{}, T1{}, F1{}, V2{}, F1{}, cb);
    step(std::integral_constant<int, TAPS - 2>{}, T1{}, F1{}, V0{}, F1{}, cb);
    step(std::integral_constant<int, TAPS - 1>{}, F1{}, F1{}, VN{}, F1{}, cb);
    conv224_store<T, NB>(lds, acc, g, wave, lane, m0t, k0t);
  };
  if (wm == 0)
    body(std::integral_constant<int, 4>{});
  else
    body(std::integral_constant<int, 3>{});
}

// The filter w (K-C-R-S, any strides) into K-(C/32)-R-S-32 for the strip kernel (C % 32 == 0):
// one lane per 8 consecutive values of the destination (one output channel k, channel block
// cb, tap rs, channels 8 (e % 4) .. + 7 of the block), gathered with eight loads and stored
// as one 16-byte vector.  One round of loads per lane: the kernel is as short as its latency.
template <typename T>
__global__ __launch_bounds__(256) void filter_cb_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                        ConvArgs g) {
  const int KG8 = (int)(g.KG / 8), RS = (int)(g.R * g.S), S = (int)g.S;
  const int64_t chunks = g.K * KG8;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < chunks; e += (int64_t)gridDim.x * 256) {
    const int64_t k = e / KG8;
    const int ce = (int)(e - k * KG8), cbrs = ce >> 2;
    const int cb = cbrs / RS, rs = cbrs - cb * RS;
    const int c = cb * 32 + (ce & 3) * 8, r = rs / S, s = rs - r * S;
    const uint16_t* src = w + k * g.ws[0] + c * g.ws[1] + r * g.ws[2] + s * g.ws[3];
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = src[i * g.ws[1]];
    *(u32x4*)(wt + e * 8) = *(const u32x4*)v;
  }
}

// The same re-layout for a contiguous 3x3 filter (strides C*9, 9, 3, 1; 16-byte aligned), where
// unit u = k * (C / 32) + cb is the 32 x 9 block w[k][32 cb .. 32 cb + 31][.][.] at elements
// [288 u, 288 u + 288) of both w and wt, transposed to 9 x 32.  A 144-lane workgroup takes four
// units: one 16-byte load per lane into LDS, then one 16-byte store per lane of 8 consecutive
// channels of one tap.  Against filter_cb_kernel's eight 2-byte gathers per lane this saves
// about 0.8 us per call at [256, 256, 3, 3], where the step costs about 3 us in all (1.7 us of
// it the kernel boundary itself, measured with an empty kernel in its place).
__global__ __launch_bounds__(144) void filter_cb9_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ wt,
                                                         int units) {
  constexpr int U = 4, CH = 36;  // units per workgroup, 16-byte chunks per unit
  __shared__ __attribute__((aligned(16))) uint16_t sm[U * 288];
  const int t = threadIdx.x, u0 = blockIdx.x * U;
  const int n = (units - u0 < U ? units - u0 : U) * CH;
  if (t < n) *(u32x4*)(sm + t * 8) = *(const u32x4*)(w + (int64_t)u0 * 288 + t * 8);
  __syncthreads();
  if (t < n) {
    const int un = t / CH, q = t - un * CH, rs = q >> 2, c8 = (q & 3) * 8;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = sm[un * 288 + (c8 + i) * 9 + rs];
    *(u32x4*)(wt + (int64_t)u0 * 288 + t * 8) = *(const u32x4*)v;
  }
}

// conv2d's 1 x 1 path when H W is no multiple of 8: each input image's rows [C][H W] copied
// into [N][C][HWp] (HWp = H W rounded up to 8, zeros past H W), so that the batch of products
// reads 16-byte aligned rows; one lane per 8 destination elements, one 16-byte store.
__global__ __launch_bounds__(256) void rows_pad8_kernel(const uint16_t* __restrict__ x, int64_t xs0, int64_t xs1,
                                                        uint16_t* __restrict__ dst, int64_t N, int64_t C, int64_t HW,
                                                        int64_t HWp) {
  const int64_t per_row = HWp / 8, total = N * C * per_row;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / per_row, j0 = (e - row * per_row) * 8;
    const int64_t n = row / C, c = row - n * C;
    const uint16_t* src = x + n * xs0 + c * xs1;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = j0 + i < HW ? src[j0 + i] : (uint16_t)0;
    *(u32x4*)(dst + row * HWp + j0) = *(const u32x4*)v;
  }
}

// ... and the products' [N][K][HWp] back into y's images: y[n][k][j] for j < H W.
__global__ __launch_bounds__(256) void rows_unpad_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ y,
                                                         int64_t ys0, int64_t ys1, int64_t N, int64_t K, int64_t HW,
                                                         int64_t HWp) {
  const int64_t total = N * K * HW;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / HW, j = e - row * HW;
    const int64_t n = row / K, k = row - n * K;
    y[n * ys0 + k * ys1 + j] = src[row * HWp + j];
  }
}

// Sum of conv_dma_kernel's split partials: one lane per 8 consecutive output positions of
// one channel, rounded and stored as one 16-byte vector when they share an output row
// (qvec), else element by element.
template <typename T>
__global__ __launch_bounds__(256) void conv_splitk_reduce_kernel(ConvArgs g) {
  const int64_t mv = g.Mp / 8, total = g.K * mv;
  uint16_t* Y = (uint16_t*)g.y;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t k = e / mv, m = (e - k * mv) * 8;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < g.splits; ++sp) {
      const float* src = g.part + ((int64_t)sp * g.K + k) * g.Mp + m;
      const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
      v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
      v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
    }
    u32x4 ow;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = round_through(v[2 * d], g.round_dtype), b = round_through(v[2 * d + 1], g.round_dtype);
      ow[d] = (uint32_t)elem<T>::from_float(a) | ((uint32_t)elem<T>::from_float(b) << 16);
    }
    if (g.qvec) {
      const int64_t q = m % g.Q, t = m / g.Q;
      const int64_t p = t % g.P, n = t / g.P;
      __builtin_nontemporal_store(ow, (u32x4*)(Y + n * g.ys[0] + k * g.ys[1] + p * g.ys[2] + q));
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t mu = m + u;
        if (mu < g.M) {
          const int64_t q = mu % g.Q, t = mu / g.Q;
          Y[(t / g.P) * g.ys[0] + k * g.ys[1] + (t % g.P) * g.ys[2] + q * g.ys[3]] =
              (uint16_t)(ow[u >> 1] >> (16 * (u & 1)));
        }
      }
    }
  }
}

static int64_t nhwc_bytes(int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S, int64_t ph,
                          int64_t pw) {
  const int64_t xp = N * (H + 2 * ph) * (W + 2 * pw) * C * 2;
  const int64_t wt = K * R * S * C * 2;
  return ((xp + 255) / 256) * 256 + wt;
}

// Channels of the DMA kernel's re-laid layout: C rounded up to 32, and far enough that the
// reduction C*R*S holds the three 32-deep k-tiles its pipeline keeps in flight (a 1 x 1
// filter over 64 channels runs as 96, the last 32 zero).
static int64_t dma_channels(int64_t C, int64_t R, int64_t S) {
  int64_t c = cdiv(C, 32) * 32;
  if (R * S > 0 && c * R * S < 96) c = cdiv(cdiv(96, R * S), 32) * 32;
  return c;
}

// Splits of conv_dma_kernel's reduction for an output of `tiles` 256 x 256 tiles and nk
// 32-deep k-tiles: none when the tiles alone fill the GPU (128 or more), else enough to
// give about 256 workgroups, at most 16, each with at least 4 k-tiles (the last at least
// 3), and no more than `room` bytes of fp32 partials (K x M each).  Returns the number of
// splits and sets *per to the k-tiles of each.
// The re-laid DMA path takes 128 x 128 tiles by default below this many 256 x 256 tiles:
// measured fp16 3 x 3, it wins up to 98 such tiles ([32,128,28,28] x 128 36.7 against 64.3 us
// on the 256-wide kernel; [4,256,56,56] x 256 36.6 against 45.6 on the strip kernel) and
// loses at 196 (the headline, 103.8 against the strip kernel's 60.8).
constexpr int64_t CONV128_BELOW = 136;

static int64_t conv_splits(int64_t tiles, int64_t nk, int64_t K, int64_t M, int64_t room, int64_t* per) {
  *per = nk;
  if (tiles >= 128) return 1;
  int64_t sp = cdiv(256, tiles);
  if (sp > 16) sp = 16;
  if (sp > nk / 4) sp = nk / 4;
  for (; sp > 1; --sp) {
    const int64_t p = cdiv(nk, sp), used = cdiv(nk, p);
    if (nk - (used - 1) * p >= 3 && used * K * M * 4 <= room && used * tiles <= 0x7fffffffLL) {
      *per = p;
      return used;
    }
  }
  return 1;
}

template <typename T>
static int conv_launch(const void* x, const int64_t* xs, const void* w, const int64_t* ws, void* y, const int64_t* ys,
                       int y_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                       int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw, int64_t dh, int64_t dw,
                       int round_dtype, void* workspace, int64_t workspace_bytes, hipStream_t stream,
                       int config = 0) {
  // config: 0 = the fastest path whose conditions hold; 1 = re-laid input through the DMA
  // kernel, 2 = re-laid input through conv_nhwc_kernel, 3 = the direct kernel (no
  // workspace), 4 = re-laid input through the DMA kernel of 224-position tiles, 5 = the
  // input read in place by conv_strip224_kernel (only the filter re-laid), 6 = 1 x 1 filters
  // as a batch of products on gemm_dma128_kernel, 7 = re-laid input through the DMA kernel
  // of 128 x 128 tiles.  A forced path whose conditions do not hold is rejected before
  // launching.
  if (config < 0 || config > 7) return NT_ERR_INVALID;
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
  g.N = N; g.C = C; g.Cr = C; g.H = H; g.W = W; g.K = K; g.R = R; g.S = S; g.P = P; g.Q = Q;
  g.splits = 1;
  g.kt_per = (int)((C * R * S) / 32);
  g.part = nullptr;
  g.ph = ph; g.pw = pw; g.sh = sh; g.sw = sw; g.dh = dh; g.dw = dw;
  g.M = N * P * Q;
  g.KG = C * R * S;
  g.y_dtype = y_dtype;
  g.round_dtype = round_dtype;
  const int64_t tiles_k = cdiv(K, CB_K), tiles_m = cdiv(g.M, CB_M);
  if (tiles_k * tiles_m > 0x7fffffffLL) return NT_ERR_INVALID;
  g.tiles_k = (int)tiles_k;
  g.tiles_m = (int)tiles_m;
  // 1 x 1 filters at stride 1 without padding, over images whose H W positions are back to
  // back (unit w stride, rows adjacent) into an output laid out alike: output image n
  // [K, P Q] is the filter [K, C] times input image n [C, H W], so the N products run as one
  // batch on gemm_dma128_kernel, the input read in place (gemm16_batch128 checks alignment,
  // strides and sizes and declines, launching nothing, what it does not take).
  // When H W is no multiple of 8, the images go through the workspace with rows padded to
  // a multiple of 8 (zeros past H W, whose products are dropped on the way back), if it
  // holds them: nt_conv2d_workspace_size asks for no more than the re-laid path needs, which
  // covers the padded images wherever that path splits the reduction (small outputs, where
  // this one pays); elsewhere the call goes on to the re-laid path.
  if (config == 0 || config == 6) {
    const bool one_by_one = R == 1 && S == 1 && ph == 0 && pw == 0 && sh == 1 && sw == 1 && dh == 1 && dw == 1 &&
                            xs[3] == 1 && xs[2] == W && ys[3] == 1 && ys[2] == Q && ws[1] == 1 && N <= 65535;
    int e = one_by_one ? gemm16_batch128(elem<T>::code, w, ws[0], 0, x, xs[1], xs[0], y, ys[1], ys[0], y_dtype, K,
                                         P * Q, C, N, round_dtype, stream)
                       : NT_ERR_INVALID;
    const int64_t HW = H * W, HWp = cdiv(HW, 8) * 8;
    const int64_t xb = cdiv(N * C * HWp * 2, 256) * 256, yb = N * K * HWp * 2;
    if (e == NT_ERR_INVALID && one_by_one && HW % 8 != 0 && workspace && (uintptr_t)workspace % 256 == 0 &&
        workspace_bytes >= xb + yb) {
      uint16_t* xp = (uint16_t*)workspace;
      uint16_t* yp = (uint16_t*)((char*)workspace + xb);
      if (gemm16_batch128(elem<T>::code, w, ws[0], 0, xp, HWp, C * HWp, yp, HWp, K * HWp, y_dtype, K, HWp, C, N,
                          round_dtype, stream, true) == 0) {
        const int64_t pad_blocks = cdiv(N * C * (HWp / 8), 256), back_blocks = cdiv(N * K * HW, 256);
        hipLaunchKernelGGL(rows_pad8_kernel, dim3((unsigned)(pad_blocks < 16384 ? pad_blocks : 16384)), dim3(256), 0,
                           stream, (const uint16_t*)x, xs[0], xs[1], xp, N, C, HW, HWp);
        e = gemm16_batch128(elem<T>::code, w, ws[0], 0, xp, HWp, C * HWp, yp, HWp, K * HWp, y_dtype, K, HWp, C, N,
                            round_dtype, stream);
        if (e) return e;
        hipLaunchKernelGGL(rows_unpad_kernel, dim3((unsigned)(back_blocks < 16384 ? back_blocks : 16384)), dim3(256),
                           0, stream, (const uint16_t*)yp, (uint16_t*)y, ys[0], ys[1], N, K, HW, HWp);
        return launch_status();
      }
    }
    if (e != NT_ERR_INVALID || config == 6) return e;
  }
  const int64_t Hp = H + 2 * ph, Wp = W + 2 * pw;
  // The re-laid input and filter carry Cl channels: C rounded up to 32 for the DMA kernel
  // (its 32-deep k-tiles stay inside one filter tap), to 64 for conv_nhwc_kernel (64-deep
  // ones); the channels past C are zeros, so they add nothing to any sum.
  // DMA kernel: at least three 32-deep k-tiles, 32-bit operand offsets, output written as
  // 16-byte runs of 8 positions of one channel (Q % 8 == 0, y of the input type with unit
  // q stride and 16-byte aligned rows).
  auto dma_fits = [&](int64_t Cl) {
    const int64_t KGl = Cl * R * S;
    return KGl >= 3 * 32 && N * Hp * Wp * Cl * 2 < 0x7fffffffLL && K * KGl * 2 < 0x7fffffffLL && g.M < 0x7fffffffLL &&
           y_dtype == elem<T>::code;
  };
  // Its output as 16-byte runs of 8 positions of one channel, or else element by element.
  g.qvec = Q % 8 == 0 && ys[3] == 1 && ys[0] % 8 == 0 && ys[1] % 8 == 0 && ys[2] % 8 == 0 && (uintptr_t)y % 16 == 0;
  g.Mp = cdiv(g.M, 8) * 8;
  // conv_strip224_kernel: a 3 x 3 filter, whole output rows per 224-position tile (Q divides
  // 224, the tile's TR rows divide P), stride and dilation 1, 32-channel blocks, input rows of
  // unit w stride in 16-byte chunks (W % 8 == 0, 16-byte aligned), a strip row of Q + 16
  // positions that holds the padded input row, two or three raw pieces per strip, strips and
  // pieces inside LDS beside the filter ring, 32-bit offsets; the re-laid filter in the
  // workspace.
  // Config 0 takes the re-laid input on 128 x 128 tiles for outputs of fewer than
  // CONV128_BELOW tiles of 256 x 256, where the strip kernel's one 224-position tile per CU
  // leaves most of the chip idle, when that path can run here.
  const bool prefer128 = config == 0 && tiles_k * tiles_m < CONV128_BELOW && R * S > 0 &&
                         dma_fits(dma_channels(C, R, S)) && workspace != nullptr && (uintptr_t)workspace % 256 == 0 &&
                         workspace_bytes >= nhwc_bytes(N, dma_channels(C, R, S), H, W, K, R, S, ph, pw) &&
                         (P - 1) * sh + (R - 1) * dh < Hp && (Q - 1) * sw + (S - 1) * dw < Wp;
  const int64_t strip_pitch = Q + 16;
  const int64_t strip_rows = Q > 0 && 224 % Q == 0 ? 224 / Q + R - 1 : 0;
  int64_t strip_np = 0;
  const bool strip = [&] {
    if (R != 3 || S != 3 || strip_rows == 0 || P % (224 / Q) != 0 || sh != 1 || sw != 1 || dh != 1 || dw != 1)
      return false;
    if (C % 32 != 0 || y_dtype != elem<T>::code) return false;
    if (xs[3] != 1 || W % 8 != 0 || (uintptr_t)x % 16 != 0 || xs[0] < 0 || xs[1] < 0 || xs[2] < 0 || xs[0] % 8 != 0 ||
        xs[1] % 8 != 0 || xs[2] % 8 != 0)
      return false;
    if (Q + S - 1 > strip_pitch || pw + W > strip_pitch) return false;
    strip_np = cdiv(strip_rows * 32 * (W / 8), 512);
    if (strip_np < 2 || strip_np > cstrip::MAX_PIECES) return false;
    if (cstrip::RING + 2 * strip_rows * strip_pitch * cstrip::SPOS + strip_np * cstrip::PIECE > cstrip::LDS_BYTES)
      return false;
    if (((C - 1) * xs[1] + (H - 1) * xs[2] + W) * 2 >= 0x7fffffffLL || K * C * R * S * 2 >= 0x7fffffffLL ||
        g.M >= 0x7fffffffLL || tiles_k * (g.M / 224) > 0x7fffffffLL)
      return false;
    return workspace != nullptr && (uintptr_t)workspace % 256 == 0 && workspace_bytes >= K * C * R * S * 2;
  }();
  if (config == 5 && !strip) return NT_ERR_INVALID;
  if (strip && (config == 5 || (config == 0 && !prefer128))) {
    g.cb_order = 1;
    g.tiles_m = (int)(g.M / 224);
    uint16_t* wt = (uint16_t*)workspace;
    const int64_t units = K * C / 32;
    if (ws[3] == 1 && ws[2] == 3 && ws[1] == 9 && ws[0] == C * 9 && (uintptr_t)w % 16 == 0 && units <= 0x7fffffffLL) {
      hipLaunchKernelGGL(filter_cb9_kernel, dim3((unsigned)cdiv(units, 4)), dim3(144), 0, stream, (const uint16_t*)w,
                         wt, (int)units);
    } else {
      const int64_t fchunks = K * (g.KG / 8), fblocks = cdiv(fchunks, 256) < 16384 ? cdiv(fchunks, 256) : 16384;
      hipLaunchKernelGGL(filter_cb_kernel<T>, dim3((unsigned)fblocks), dim3(256), 0, stream, (const uint16_t*)w, wt, g);
    }
    const dim3 grid((unsigned)(tiles_k * g.tiles_m));
    if (strip_np == 2)
      hipLaunchKernelGGL((conv_strip224_kernel<T, 2>), grid, dim3(512), 0, stream, (const uint16_t*)x,
                         (const uint16_t*)wt, g, (int)strip_pitch, (int)strip_rows);
    else
      hipLaunchKernelGGL((conv_strip224_kernel<T, 3>), grid, dim3(512), 0, stream, (const uint16_t*)x,
                         (const uint16_t*)wt, g, (int)strip_pitch, (int)strip_rows);
    return launch_status();
  }
  const int64_t C32 = dma_channels(C, R, S), C64 = cdiv(C, 64) * 64;
  const bool dma = config != 2 && dma_fits(C32);
  const int64_t Cl = dma ? C32 : C64;
  const int64_t need = nhwc_bytes(N, Cl, H, W, K, R, S, ph, pw);
  // (an empty filter, R or S zero, sums nothing: the direct kernel writes the zeros)
  const bool nhwc = config != 3 && R * S > 0 && workspace != nullptr && workspace_bytes >= need && (uintptr_t)workspace % 256 == 0 &&
                    (P - 1) * sh + (R - 1) * dh < Hp && (Q - 1) * sw + (S - 1) * dw < Wp;
  if (((config == 1 || config == 4 || config == 7) && !(nhwc && dma)) || (config == 2 && !nhwc)) return NT_ERR_INVALID;
  if (nhwc) {
    g.C = Cl;
    g.KG = Cl * R * S;
    g.cb_order = dma ? 1 : 0;
    // Few output tiles: the DMA kernel splits the reduction, partials after the re-layout.
    const int64_t part_at = cdiv(need, 256) * 256;
    // 128 x 128 tiles (conv_dma_kernel<T, 128>) for outputs of few 256 x 256 tiles: four
    // times as many workgroups, two per CU, and fewer splits.
    const bool t128 = dma && (config == 7 || (config == 0 && tiles_k * tiles_m < CONV128_BELOW));
    const int64_t tk = t128 ? cdiv(K, 128) : tiles_k, tm = t128 ? cdiv(g.M, 128) : tiles_m;
    int64_t per = g.KG / 32;
    const int64_t sp = dma && config != 4 ? conv_splits(tk * tm, g.KG / 32, K, g.Mp, workspace_bytes - part_at, &per) : 1;
    // 224-position tiles when, without a split, they leave fewer CUs idle: per CU and round
    // of 256 workgroups, a workgroup's time goes with its positions (224 or 256).
    const int64_t tiles_m224 = cdiv(g.M, CB_M224);
    const bool m224 = dma && !t128 && sp == 1 && tiles_k * tiles_m224 <= 0x7fffffffLL &&
                      (config == 4 || (config == 0 && cdiv(tiles_k * tiles_m224, 256) * 224 * 100 <
                                                          cdiv(tiles_k * tiles_m, 256) * 256 * 97));
    g.splits = (int)sp;
    g.kt_per = (int)per;
    g.part = sp > 1 ? (float*)((char*)workspace + part_at) : nullptr;
    uint16_t* xp = (uint16_t*)workspace;
    uint16_t* wt = (uint16_t*)((char*)workspace + ((N * Hp * Wp * Cl * 2 + 255) / 256) * 256);
    int64_t fblocks = K * R * S;  // filter rows of the fast re-layout (at most 4096 workgroups)
    if (fblocks > 4096) fblocks = 4096;
    const bool fast_relayout = xs[3] == 1 && W % 8 == 0 && (uintptr_t)x % 16 == 0 && (xs[0] * 2) % 16 == 0 &&
                               (xs[1] * 2) % 16 == 0 && (xs[2] * 2) % 16 == 0;
    if (fast_relayout && Cl * W * 2 <= RELAYOUT_STAGE_BYTES && (Cl / 8) * (W / 8) <= 256) {
      // rows in workgroups that each take several, two per CU; the filter one channel k at a time
      const int64_t row_blocks = N * Hp < 512 ? N * Hp : 512, kblocks = K < 256 ? K : 256;
      hipLaunchKernelGGL(conv_relayout_pipe_kernel<T>, dim3((unsigned)(row_blocks + kblocks)), dim3(256), 0, stream,
                         (const uint16_t*)x, xp, (const uint16_t*)w, wt, g, Hp, Wp, (int)row_blocks);
    } else if (fast_relayout) {
      if (N * Hp + fblocks > 0x7fffffffLL) return NT_ERR_INVALID;
      if (Cl * W * 2 <= RELAYOUT_STAGE_BYTES)
        hipLaunchKernelGGL((conv_relayout_kernel<T, true>), dim3((unsigned)(N * Hp + fblocks)), dim3(256), 0, stream,
                           (const uint16_t*)x, xp, (const uint16_t*)w, wt, g, Hp, Wp);
      else
        hipLaunchKernelGGL((conv_relayout_kernel<T, false>), dim3((unsigned)(N * Hp + fblocks)), dim3(256), 0, stream,
                           (const uint16_t*)x, xp, (const uint16_t*)w, wt, g, Hp, Wp);
    } else {
      const int64_t relayout_blocks = N * Hp * cdiv(Cl, 64);
      if (relayout_blocks > 0x7fffffffLL) return NT_ERR_INVALID;
      hipLaunchKernelGGL(nchw_to_nhwc_pad_kernel<T>, dim3((unsigned)relayout_blocks), dim3(256), 0, stream,
                         (const uint16_t*)x, xp, g, Hp, Wp);
      hipLaunchKernelGGL(filter_krsc_kernel<T>, dim3((unsigned)fblocks), dim3(256), 0, stream, (const uint16_t*)w, wt,
                         g);
    }
    if (m224) {
      g.tiles_m = (int)tiles_m224;
      hipLaunchKernelGGL(conv_dma224_kernel<T>, dim3((unsigned)(tiles_k * tiles_m224)), dim3(512), 0, stream,
                         (const uint16_t*)xp, (const uint16_t*)wt, g, Hp, Wp);
    } else if (dma) {
      g.tiles_k = (int)tk;
      g.tiles_m = (int)tm;
      if (sp * tk * tm > 0x7fffffffLL) return NT_ERR_INVALID;
      if (t128)
        hipLaunchKernelGGL((conv_dma_kernel<T, 128>), dim3((unsigned)(sp * tk * tm)), dim3(256), 0, stream,
                           (const uint16_t*)xp, (const uint16_t*)wt, g, Hp, Wp);
      else
        hipLaunchKernelGGL(conv_dma_kernel<T>, dim3((unsigned)(sp * tk * tm)), dim3(512), 0, stream,
                           (const uint16_t*)xp, (const uint16_t*)wt, g, Hp, Wp);
      if (sp > 1) {
        const int64_t vecs = K * (g.Mp / 8);
        hipLaunchKernelGGL(conv_splitk_reduce_kernel<T>, dim3((unsigned)(cdiv(vecs, 256) < 4096 ? cdiv(vecs, 256) : 4096)),
                           dim3(256), 0, stream, g);
      }
    } else
      hipLaunchKernelGGL(conv_nhwc_kernel<T>, dim3((unsigned)(tiles_k * tiles_m)), dim3(512), 0, stream,
                         (const uint16_t*)xp, (const uint16_t*)wt, g, Hp, Wp);
    return launch_status();
  }
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
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0 || K <= 0 || R <= 0 || S <= 0 || ph < 0 || pw < 0) return 0;
  if (dtype != NT_DTYPE_F16 && dtype != NT_DTYPE_BF16) return 0;
  // Enough for either layout's channels (rounded up to 64, or the DMA kernel's), plus the
  // split partials of the largest output the shape can have (stride and dilation 1).
  const int64_t c64 = nt::cdiv(C, 64) * 64, cd = nt::dma_channels(C, R, S);
  const int64_t base = nt::cdiv(nt::nhwc_bytes(N, c64 > cd ? c64 : cd, H, W, K, R, S, ph, pw), 256) * 256;
  const int64_t P = H + 2 * ph - R + 1, Q = W + 2 * pw - S + 1;
  if (P <= 0 || Q <= 0) return base;
  const int64_t M = nt::cdiv(N * P * Q, 8) * 8;
  int64_t per = 0;
  const int64_t sp = nt::conv_splits(nt::cdiv(K, nt::CB_K) * nt::cdiv(M, nt::CB_M), cd * R * S / 32, K, M, INT64_MAX,
                                     &per);
  return base + (sp > 1 ? sp * K * M * 4 : 0);
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

#define NT_CONV_CONFIG_ENTRY(NAME, T)                                                                                \
  extern "C" int NAME(const void* x, const int64_t* xs, const void* w, const int64_t* ws, void* y, const int64_t* ys, \
                      int y_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,       \
                      int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw, int64_t dh, int64_t dw,   \
                      int round_dtype, void* workspace, int64_t workspace_bytes, int config, hipStream_t stream) {   \
    return nt::conv_launch<T>(x, xs, w, ws, y, ys, y_dtype, N, C, H, W, K, R, S, P, Q, ph, pw, sh, sw, dh, dw,       \
                              round_dtype, workspace, workspace_bytes, stream, config);                              \
  }
NT_CONV_CONFIG_ENTRY(nt_conv2d_config_f16, nt::f16_t)
NT_CONV_CONFIG_ENTRY(nt_conv2d_config_bf16, nt::bf16_t)

// ----------------------------------------------------------------------------- allocation-free entry
// The re-layout workspace of nt_conv2d_* as a file-scope device array (one per GPU the library
// runs on).  In host code `scratch` names a host-side stand-in, not device memory: its device
// address comes from hipGetSymbolAddress, looked up once per device on the first call with
// that device current and kept in scratch_ptr.
static __device__ __align__(256) char scratch[NT_CONV2D_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_ptr[kMaxDevices];
std::mutex scratch_mutex;

// The current device's scratch address, or a nonzero status.
int current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return NT_ERR_INVALID;
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(scratch_mutex);
    p = scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (p == nullptr || (uintptr_t)p % 256 != 0) return NT_ERR_INVALID;
      scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}
}  // namespace

#define NT_CONV_NOALLOC_ENTRY(NAME, T, CODE)                                                                         \
  extern "C" int NAME(const void* x, const int64_t* xs, const void* w, const int64_t* ws, void* y, const int64_t* ys, \
                      int y_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,       \
                      int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw, int64_t dh, int64_t dw,   \
                      int round_dtype, hipStream_t stream) {                                                          \
    if (nt_conv2d_workspace_size(N, C, H, W, K, R, S, ph, pw, CODE) > NT_CONV2D_SCRATCH_BYTES) return NT_ERR_SCRATCH; \
    void* ws_ptr = nullptr;                                                                                          \
    if (int e = current_scratch(&ws_ptr)) return e;                                                                  \
    return nt::conv_launch<T>(x, xs, w, ws, y, ys, y_dtype, N, C, H, W, K, R, S, P, Q, ph, pw, sh, sw, dh, dw,       \
                              round_dtype, ws_ptr, NT_CONV2D_SCRATCH_BYTES, stream);                                 \
  }
NT_CONV_NOALLOC_ENTRY(nt_conv2d_noalloc_f16, nt::f16_t, NT_DTYPE_F16)
NT_CONV_NOALLOC_ENTRY(nt_conv2d_noalloc_bf16, nt::bf16_t, NT_DTYPE_BF16)
