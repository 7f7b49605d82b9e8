// Row softmax over segments of `block` columns (the application's BLOCK_SIZE).
//
// One 256-lane workgroup per segment.  HBM-bound: each element is read once and
// written once (2 * rows * cols * sizeof(T) bytes).  The segment is held in
// registers between the three phases (max, sum of exp, scale), so nothing is
// re-read; reductions are wave64 butterflies plus one LDS exchange across the four
// waves.  exp(x) is computed as exp2(x * log2 e) on the hardware v_exp_f32.
// Segments longer than the register path holds use a two-sweep kernel: an online
// (max, sum) sweep, then a scaling sweep.
#include "nt_common.h"

namespace nt {

constexpr int SM_THREADS = 256;
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * LOG2E); }

template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += red[i];
  __syncthreads();
  return r;
}

// Register path: NT lanes per workgroup, each owning VPT vectors of V elements.
template <typename T, int VPT, bool VEC, int NT = SM_THREADS>
__global__ __launch_bounds__(NT) void softmax_reg_kernel(const typename elem<T>::storage* __restrict__ x,
                                                                 int64_t xs, typename elem<T>::storage* __restrict__ y,
                                                                 int64_t ys, int64_t cols, int64_t block,
                                                                 int64_t segs_per_row) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S);
  __shared__ float red[NT / 64];
  const int64_t seg = blockIdx.x;
  const int64_t row = seg / segs_per_row;
  const int64_t c0 = (seg % segs_per_row) * block;
  const int64_t len = (cols - c0 < block) ? (cols - c0) : block;
  const S* xr = x + row * xs + c0;
  S* yr = y + row * ys + c0;

  float v[VPT][V];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t e0 = ((int64_t)j * NT + threadIdx.x) * V;
    if (VEC && e0 + V <= len) {
      u32x4 raw = *(const u32x4*)(xr + e0);  // plain load: nontemporal loads cost ~8% here
      const S* p = (const S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) v[j][u] = elem<T>::to_float(p[u]);
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u) v[j][u] = (e0 + u < len) ? elem<T>::to_float(xr[e0 + u]) : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < V; ++u) mx = fmaxf(mx, v[j][u]);
  }
  mx = block_max<NT / 64>(mx, red);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
#pragma unroll
    for (int u = 0; u < V; ++u) {
      v[j][u] = fast_exp(v[j][u] - mx);
      sum += v[j][u];
    }
  }
  sum = block_sum<NT / 64>(sum, red);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t e0 = ((int64_t)j * NT + threadIdx.x) * V;
    if (VEC && e0 + V <= len) {
      u32x4 raw;
      S* p = (S*)&raw;
#pragma unroll
      for (int u = 0; u < V; ++u) p[u] = elem<T>::from_float(v[j][u] * inv);
      __builtin_nontemporal_store(raw, (u32x4*)(yr + e0));
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u)
        if (e0 + u < len) yr[e0 + u] = elem<T>::from_float(v[j][u] * inv);
    }
  }
}

// Long segments: online (max, sum) sweep, then a scaling sweep.
template <typename T>
__global__ __launch_bounds__(SM_THREADS) void softmax_long_kernel(const typename elem<T>::storage* __restrict__ x,
                                                                  int64_t xs, typename elem<T>::storage* __restrict__ y,
                                                                  int64_t ys, int64_t cols, int64_t block,
                                                                  int64_t segs_per_row) {
  typedef typename elem<T>::storage S;
  __shared__ float red[SM_THREADS / 64];
  const int64_t seg = blockIdx.x;
  const int64_t row = seg / segs_per_row;
  const int64_t c0 = (seg % segs_per_row) * block;
  const int64_t len = (cols - c0 < block) ? (cols - c0) : block;
  const S* xr = x + row * xs + c0;
  S* yr = y + row * ys + c0;
  float m = -INFINITY, s = 0.f;
  for (int64_t e = threadIdx.x; e < len; e += SM_THREADS) {
    const float xv = elem<T>::to_float(xr[e]);
    const float nm = fmaxf(m, xv);
    if (nm != -INFINITY) {  // an all -inf prefix contributes nothing yet
      s = s * fast_exp(m - nm) + fast_exp(xv - nm);
      m = nm;
    }
  }
  // Combine per-lane (m, s) pairs: rescale every partial sum to the block max.
  const float gm = block_max<SM_THREADS / 64>(m, red);
  const float part = (m == -INFINITY) ? 0.f : s * fast_exp(m - gm);
  const float gs = block_sum<SM_THREADS / 64>(part, red);
  const float inv = 1.0f / gs;
  for (int64_t e = threadIdx.x; e < len; e += SM_THREADS)
    yr[e] = elem<T>::from_float(fast_exp(elem<T>::to_float(xr[e]) - gm) * inv);
}

// config: 0 = the four-wave register path when the segment fits it (16 vectors of 16 bytes
// per lane at most), else the two-sweep kernel; 1 = four-wave register path; 2 = eight-wave
// register path; 3 = one-wave register path; 4 = two-sweep kernel (the reference's
// auto-tuner times num_warps 4, 8, 1: src/ninetoothed/backends/triton.py:151-155).  A
// forced register path whose segment does not fit returns NT_ERR_INVALID unlaunched.
template <typename T>
static int softmax_launch(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                          int64_t cols, int64_t block, hipStream_t stream, int config = 0) {
  typedef typename elem<T>::storage S;
  constexpr int V = 16 / sizeof(S);
  if (config < 0 || config > 4) return NT_ERR_INVALID;
  if (rows < 0 || cols < 0 || block <= 0) return NT_ERR_INVALID;
  if (rows == 0 || cols == 0) return 0;
  if (!x || !y) return NT_ERR_INVALID;
  if (cols > 1 && (xcs != 1 || ycs != 1)) return NT_ERR_INVALID;
  const int64_t segs_per_row = cdiv(cols, block);
  const int64_t segs = rows * segs_per_row;
  if (segs > 0x7fffffffLL) return NT_ERR_INVALID;
  const int64_t len = block < cols ? block : cols;
  const bool vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && ((xs * (int64_t)sizeof(S)) % 16 == 0 || rows == 1) &&
                   ((ys * (int64_t)sizeof(S)) % 16 == 0 || rows == 1) &&
                   ((block * (int64_t)sizeof(S)) % 16 == 0 || segs_per_row == 1);
  const dim3 grid((unsigned)segs);
  const S* xp = (const S*)x;
  S* yp = (S*)y;
  // Launch the register path with NT lanes and the smallest VPT that holds the segment (up
  // to 16 with 16-byte accesses, 8 with element-wise ones, whose per-element bounds checks
  // would spill beyond); false when none does.
  auto reg = [&](auto nt_c) {
    constexpr int NT = decltype(nt_c)::value;
    bool done = false;
    static_for<0, 5>([&](auto e_c) {
      constexpr int VPT = 1 << decltype(e_c)::value;
      if (done || len > (int64_t)NT * V * VPT) return;
      if (vec) {
        hipLaunchKernelGGL((softmax_reg_kernel<T, VPT, true, NT>), grid, dim3(NT), 0, stream, xp, xs, yp, ys, cols,
                           block, segs_per_row);
        done = true;
      } else if constexpr (VPT <= 8) {
        hipLaunchKernelGGL((softmax_reg_kernel<T, VPT, false, NT>), grid, dim3(NT), 0, stream, xp, xs, yp, ys, cols,
                           block, segs_per_row);
        done = true;
      }
    });
    return done;
  };
  using W4 = std::integral_constant<int, 256>;
  using W8 = std::integral_constant<int, 512>;
  using W1 = std::integral_constant<int, 64>;
  if (config == 4 || (config == 0 && !reg(W4{}))) {
    hipLaunchKernelGGL(softmax_long_kernel<T>, grid, dim3(SM_THREADS), 0, stream, xp, xs, yp, ys, cols, block,
                       segs_per_row);
  } else if ((config == 1 && !reg(W4{})) || (config == 2 && !reg(W8{})) || (config == 3 && !reg(W1{}))) {
    return NT_ERR_INVALID;
  }
  return launch_status();
}

}  // namespace nt

extern "C" int nt_softmax_f32(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                              int64_t cols, int64_t block, hipStream_t stream) {
  return nt::softmax_launch<float>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
}
extern "C" int nt_softmax_f16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                              int64_t cols, int64_t block, hipStream_t stream) {
  return nt::softmax_launch<nt::f16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
}
extern "C" int nt_softmax_bf16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs, int64_t rows,
                               int64_t cols, int64_t block, hipStream_t stream) {
  return nt::softmax_launch<nt::bf16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream);
}
extern "C" int nt_softmax_config_f32(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs,
                                     int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config) {
  return nt::softmax_launch<float>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream, config);
}
extern "C" int nt_softmax_config_f16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs,
                                     int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config) {
  return nt::softmax_launch<nt::f16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream, config);
}
extern "C" int nt_softmax_config_bf16(const void* x, int64_t xs, int64_t xcs, void* y, int64_t ys, int64_t ycs,
                                      int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config) {
  return nt::softmax_launch<nt::bf16_t>(x, xs, xcs, y, ys, ycs, rows, cols, block, stream, config);
}
