// 2-D max pooling.
//
// HBM-bound: every input element of a window grid is read once and every output
// written once.  Max involves no rounding, so the result is bit-exact for any
// evaluation order; fp16/bf16 values are compared after an exact widening to fp32.
//
// Fast paths (the common non-overlapping 2-wide window on 16-bit data, unit inner
// strides, no padding or dilation).  2-high windows: a lane takes 8 consecutive inputs of a
// window's first row and the same columns of its second row (4 outputs), consecutive lanes
// consecutive units over all planes in one flat order, eight per lane per step with all
// their loads issued first (pool_w2_pair_kernel).  Taller windows: one workgroup per (n, c)
// plane, a lane producing 8 consecutive outputs from kh input rows of 16 elements
// (pool_w2_plane_kernel).  Other windows take strips of input rows through LDS
// (pool_lds_kernel); what does not fit runs the generic kernel, one lane per output.
#include "nt_common.h"

#include <algorithm>
#include <type_traits>

namespace nt {

struct PoolShape {
  int64_t N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw;
  int64_t xs[4], ys[4];
};

// One lane per output, any strides; the output may be of another element type than the
// input (the reference's store casts): the max of widened values, rounded once on store,
// equals the rounded max, since rounding is monotone.
template <typename T, typename To = T>
__global__ __launch_bounds__(256) void pool_generic_kernel(const typename elem<T>::storage* __restrict__ x,
                                                           typename elem<To>::storage* __restrict__ y, PoolShape s) {
  const int64_t total = s.N * s.C * s.P * s.Q;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
    int64_t q = o % s.Q, t = o / s.Q;
    int64_t p = t % s.P;
    t /= s.P;
    int64_t c = t % s.C, n = t / s.C;
    float m = -INFINITY;
    const typename elem<T>::storage* xb = x + n * s.xs[0] + c * s.xs[1];
    for (int64_t r = 0; r < s.kh; ++r) {
      const int64_t h = p * s.sh - s.ph + r * s.dh;
      if (h < 0 || h >= s.H) continue;
      for (int64_t u = 0; u < s.kw; ++u) {
        const int64_t w = q * s.sw - s.pw + u * s.dw;
        if (w < 0 || w >= s.W) continue;
        m = fmaxf(m, elem<T>::to_float(xb[h * s.xs[2] + w * s.xs[3]]));
      }
    }
    y[n * s.ys[0] + c * s.ys[1] + p * s.ys[2] + q * s.ys[3]] = elem<To>::from_float(m);
  }
}

// kw == sw == 2, dw == 1, no padding, 16-bit, x/y inner stride 1, Q % 8 == 0,
// all rows 16-byte aligned, every window inside the input.  One workgroup per (n, c)
// plane: in-plane indices are 32-bit, and consecutive lanes walk consecutive 16-byte
// output vectors, so a wave reads one contiguous stretch of input rows.
template <typename T>
__global__ __launch_bounds__(256) void pool_w2_plane_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                            PoolShape s) {
  const int64_t plane = blockIdx.x;
  const int64_t c = plane % s.C, n = plane / s.C;
  const uint16_t* xb = x + n * s.xs[0] + c * s.xs[1];
  uint16_t* yb = y + n * s.ys[0] + c * s.ys[1];
  const int qv_per_row = (int)(s.Q / 8);
  const int total = (int)s.P * qv_per_row;
  const int xh = (int)s.xs[2], yh = (int)s.ys[2], kh = (int)s.kh, sh = (int)s.sh, dh = (int)s.dh;
  for (int v = threadIdx.x; v < total; v += 256) {
    const int p = v / qv_per_row, qv = v - p * qv_per_row;
    const uint16_t* row = xb + (p * sh) * xh + qv * 16;
    float m[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = -INFINITY;
    for (int r = 0; r < kh; ++r) {
      const u32x4 a = *(const u32x4*)(row + r * dh * xh);
      const u32x4 b = *(const u32x4*)(row + r * dh * xh + 8);
      const uint16_t* pa = (const uint16_t*)&a;
      const uint16_t* pb = (const uint16_t*)&b;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m[j] = fmaxf(m[j], fmaxf(elem<T>::to_float(pa[2 * j]), elem<T>::to_float(pa[2 * j + 1])));
        m[4 + j] = fmaxf(m[4 + j], fmaxf(elem<T>::to_float(pb[2 * j]), elem<T>::to_float(pb[2 * j + 1])));
      }
    }
    u32x4 out;
    uint16_t* po = (uint16_t*)&out;
#pragma unroll
    for (int j = 0; j < 8; ++j) po[j] = elem<T>::from_float(m[j]);
    *(u32x4*)(yb + p * yh + qv * 8) = out;
  }
}

// Any window, stride, padding and dilation, through LDS.  A workgroup takes G whole (n, c)
// planes (G > 1 where planes are small and x and y both plane-contiguous), or one strip of
// PR output rows of one plane.  It copies the input rows its windows reach into LDS once,
// then every output takes its window's max out of LDS, consecutive lanes on consecutive
// outputs.  So each input element is read from HBM once per workgroup (overlapping windows,
// as 3 x 3 with stride 2, re-read only LDS) instead of once per window covering it.
// Rows outside the input are not copied and count as padding.
//   MODE 0: the copied rows are one contiguous range of x (rows of W elements back to back,
//           and for G > 1 planes back to back): a scalar head up to x's first 16-byte
//           boundary, 16-byte vectors, a scalar tail.  The tile starts at the range's
//           address modulo 16 in LDS, so LDS and global addresses share their alignment.
//   MODE 1: rows strided but each row whole 16-byte vectors (G == 1).
//   MODE 2: any strides, element by element (G == 1).
// U loads per lane are issued before their LDS stores.  KH, KW > 0 fix the window at
// compile time; 0 reads it from the shape.
// Division by a divisor fixed for the launch, for 0 <= n < 2^31: with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, m) + n) >> l (the round-up
// multiplier method of Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994); a few instructions where a runtime 32-bit division takes dozens.
struct PoolDiv {
  uint32_t m, l;
};
static PoolDiv pool_div(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  return PoolDiv{(uint32_t)((((1ull << l) - d) << 32) / d + 1), l};
}
__device__ __forceinline__ int pool_divide(int n, PoolDiv f) {
  const uint32_t t = __umulhi((uint32_t)n, f.m);
  return (int)((t + (uint32_t)n) >> f.l);  // t <= n < 2^31: the sum fits 32 bits
}

#ifndef NT_POOL_LDS_BYTES
#define NT_POOL_LDS_BYTES 16384
#endif
constexpr int POOL_LDS_BYTES = NT_POOL_LDS_BYTES;
template <typename T, int MODE, int KH, int KW>
__global__ __launch_bounds__(256) void pool_lds_kernel(const typename elem<T>::storage* __restrict__ x,
                                                       typename elem<T>::storage* __restrict__ y, PoolShape s, int G,
                                                       int PR, int strips, PoolDiv div_q, PoolDiv div_pq) {
  typedef typename elem<T>::storage S;
  constexpr int V = MODE == 2 ? 1 : 16 / sizeof(S), U = 4;
  typedef typename std::conditional<MODE == 2, S, u32x4>::type L;
  extern __shared__ __attribute__((aligned(16))) unsigned char pool_lds[];
  const int64_t b = blockIdx.x;
  const int strip = (int)(b % strips);
  const int64_t g0 = (b / strips) * G;
  const int gn = (int)(s.N * s.C - g0 < G ? s.N * s.C - g0 : G);
  const int W = (int)s.W, H = (int)s.H, P = (int)s.P, Q = (int)s.Q;
  const int kh = KH > 0 ? KH : (int)s.kh, kw = KW > 0 ? KW : (int)s.kw;
  const int sh = (int)s.sh, sw = (int)s.sw, ph = (int)s.ph, pw = (int)s.pw, dh = (int)s.dh, dw = (int)s.dw;
  const int p0 = strip * PR, p1 = p0 + PR < P ? p0 + PR : P;
  // input rows [hv0, hv1) of each plane are in the tile, row h at (h - hv0) * W; a plane
  // spans ts elements of the tile
  int hv0 = 0, hv1 = H;
  if (G == 1) {
    const int hs = p0 * sh - ph, he = (p1 - 1) * sh - ph + (kh - 1) * dh + 1;
    hv0 = hs > 0 ? hs : 0;
    hv1 = he < H ? he : H;
  }
  const int nrows = hv1 > hv0 ? hv1 - hv0 : 0, ts = H * W;
  const int64_t c0 = g0 % s.C, n0 = g0 / s.C;
  const S* xb = x + n0 * s.xs[0] + c0 * s.xs[1];
  const int tid = threadIdx.x;
  S* tile;
  if (MODE == 0) {
    const S* src = xb + (int64_t)hv0 * W;
    const int len = (gn - 1) * ts + nrows * W;
    const int shift = (int)((uintptr_t)src & 15);
    tile = (S*)(pool_lds + shift);
    int head = ((16 - shift) & 15) / (int)sizeof(S);
    head = head < len ? head : len;
    const int nv = (len - head) / V, tail0 = head + nv * V;
    const int nscalar = head + len - tail0;
    for (int e = tid; e < nscalar; e += 256) {
      const int t = e < head ? e : tail0 + e - head;
      tile[t] = src[t];
    }
    const u32x4* vs = (const u32x4*)(src + head);
    u32x4* vt = (u32x4*)(tile + head);
    for (int e0 = tid; e0 < nv; e0 += 256 * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (e0 + u * 256 < nv) v[u] = vs[e0 + u * 256];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (e0 + u * 256 < nv) vt[e0 + u * 256] = v[u];
    }
  } else {
    tile = (S*)pool_lds;
    const int vpr = W / V, n_units = nrows * vpr, xh = (int)s.xs[2], xw = (int)s.xs[3];
    for (int e0 = tid; e0 < n_units; e0 += 256 * U) {
      L v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * 256;
        if (e < n_units) {
          const int r = e / vpr, k = e - r * vpr;
          v[u] = *(const L*)(xb + (hv0 + r) * xh + k * V * xw);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * 256;
        if (e < n_units) {
          const int r = e / vpr, k = e - r * vpr;
          *(L*)(tile + r * W + k * V) = v[u];
        }
      }
    }
  }
  __syncthreads();
  const int np = p1 - p0, per_plane = np * Q;
  S* yb = y + n0 * s.ys[0] + c0 * s.ys[1];  // for G > 1, y is plane-contiguous: plane g at g * P * Q
  const int64_t ys2 = s.ys[2], ys3 = s.ys[3];
  for (int o = tid; o < gn * per_plane; o += 256) {
    const int g = G > 1 ? pool_divide(o, div_pq) : 0, rem = o - g * per_plane;  // G > 1: per_plane = P * Q
    const int pp = pool_divide(rem, div_q), q = rem - pp * Q;
    const int tb = g * ts - hv0 * W;  // tile offset of row 0 of plane g (rows below hv0 are never read)
    const int hb = (p0 + pp) * sh - ph, wb = q * sw - pw;
    // every tap reads LDS (a tap outside the input reads an address inside the plane's tile
    // and its value is dropped), so the window's reads issue back to back
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < (KH > 0 ? KH : 1); ++r) {
      for (int rr = r; rr < (KH > 0 ? r + 1 : kh); ++rr) {
        const int h = hb + rr * dh;
        const bool hok = h >= hv0 && h < hv1;
        const int row = tb + (hok ? h : hv0) * W;
#pragma unroll
        for (int u = 0; u < (KW > 0 ? KW : 1); ++u) {
          for (int uu = u; uu < (KW > 0 ? u + 1 : kw); ++uu) {
            const int w = wb + uu * dw;
            const bool ok = hok && w >= 0 && w < W;
            const float v = elem<T>::to_float(tile[row + (ok ? w : 0)]);
            m = ok ? fmaxf(m, v) : m;
          }
        }
      }
    }
    if (G > 1)
      yb[o] = elem<T>::from_float(m);
    else
      yb[(int64_t)(p0 + pp) * ys2 + (int64_t)q * ys3] = elem<T>::from_float(m);
  }
}

// config: 0 = the pair kernel for 2-high windows, else the plane kernel, where their
// conditions hold, else the LDS strip kernel where a strip of one output row fits its LDS,
// else the element-wise kernel; 1 = those vector kernels only; 2 = element-wise kernel;
// 3 = the flat kernel below; 4 = the LDS strip kernel.  A forced kernel whose conditions do
// not hold returns NT_ERR_INVALID unlaunched.
// Flat kernel (kh == 2 form of the plane kernel): output vector g of the flattened (plane, row, vector)
// order, U = 4 per lane per grid-stride step, the 16 loads of a step issued before any max
// (one workgroup per plane left a ragged last pass per plane and only four loads in flight
// per lane).  Indices fit 32 bits (the launcher checks).
template <typename T>
__global__ __launch_bounds__(256) void pool_w2_flat_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                           PoolShape s, int vpp, int qvpr, int total) {
  constexpr int U = 4;
  const int stride = (int)gridDim.x * 256;
  const int64_t xh = s.xs[2], yh = s.ys[2], sh = s.sh, dh = s.dh, C = s.C;
  auto locate = [&](int g, const uint16_t*& row, uint16_t*& out) {
    const int plane = g / vpp, within = g - plane * vpp;
    const int p = within / qvpr, qv = within - p * qvpr;
    const int64_t n = plane / C, c = plane - n * C;
    row = x + n * s.xs[0] + c * s.xs[1] + p * sh * xh + qv * 16;
    out = y + n * s.ys[0] + c * s.ys[1] + p * yh + qv * 8;
  };
  auto finish = [&](const u32x4 (&v)[2][2], uint16_t* out) {
    u32x4 o;
    uint16_t* po = (uint16_t*)&o;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t* p0 = (const uint16_t*)&v[0][h];
      const uint16_t* p1 = (const uint16_t*)&v[1][h];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        po[4 * h + j] = elem<T>::from_float(fmaxf(fmaxf(elem<T>::to_float(p0[2 * j]), elem<T>::to_float(p0[2 * j + 1])),
                                                  fmaxf(elem<T>::to_float(p1[2 * j]), elem<T>::to_float(p1[2 * j + 1]))));
    }
    __builtin_nontemporal_store(o, (u32x4*)out);
  };
  int g = (int)blockIdx.x * 256 + (int)threadIdx.x;
  for (; g + (U - 1) * stride < total; g += U * stride) {
    const uint16_t* row[U];
    uint16_t* out[U];
    u32x4 v[U][2][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      locate(g + u * stride, row[u], out[u]);
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) v[u][r][h] = *(const u32x4*)(row[u] + r * dh * xh + h * 8);  // plain loads: a lane's two halves share lines
    }
#pragma unroll
    for (int u = 0; u < U; ++u) finish(v[u], out[u]);
  }
  for (; g < total; g += stride) {
    const uint16_t* row;
    uint16_t* out;
    locate(g, row, out);
    u32x4 v[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h) v[r][h] = *(const u32x4*)(row + r * dh * xh + h * 8);
    finish(v, out);
  }
}

// 2-wide windows of stride 2 (2-high, any vertical stride and dilation) on 16-bit data: a
// unit is 8 consecutive inputs of a window's first row and the same columns of its second
// row, giving 4 outputs.  Consecutive lanes take consecutive units, so each 16-byte load
// instruction reads contiguous chunks of one row (whole cache lines, where two half-rows
// per instruction would leave each line half used) and each 8-byte store continues the
// previous lane's.  U units per lane per step, all loads issued first.
template <typename T>
__global__ __launch_bounds__(256) void pool_w2_pair_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                           PoolShape s, int upp, int upr, int total) {
  constexpr int U = 8;
  const int stride = (int)gridDim.x * 256;
  const int64_t xh = s.xs[2], yh = s.ys[2], sh = s.sh, dh = s.dh, C = s.C;
  auto locate = [&](int g, const uint16_t*& row, uint16_t*& out) {
    const int plane = g / upp, within = g - plane * upp;
    const int p = within / upr, j = within - p * upr;
    const int64_t n = plane / C, c = plane - n * C;
    row = x + n * s.xs[0] + c * s.xs[1] + p * sh * xh + j * 8;
    out = y + n * s.ys[0] + c * s.ys[1] + p * yh + j * 4;
  };
  auto finish = [&](const u32x4& a, const u32x4& b, uint16_t* out) {
    u32x2 o;
    uint16_t* po = (uint16_t*)&o;
    const uint16_t* pa = (const uint16_t*)&a;
    const uint16_t* pb = (const uint16_t*)&b;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      po[j] = elem<T>::from_float(fmaxf(fmaxf(elem<T>::to_float(pa[2 * j]), elem<T>::to_float(pa[2 * j + 1])),
                                        fmaxf(elem<T>::to_float(pb[2 * j]), elem<T>::to_float(pb[2 * j + 1]))));
    __builtin_nontemporal_store(o, (u32x2*)out);
  };
  int g = (int)blockIdx.x * 256 + (int)threadIdx.x;
  for (; g + (U - 1) * stride < total; g += U * stride) {  // the launcher keeps total + U * stride within int
    const uint16_t* row[U];
    uint16_t* out[U];
    u32x4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      locate(g + u * stride, row[u], out[u]);
      a[u] = *(const u32x4*)row[u];
      b[u] = *(const u32x4*)(row[u] + dh * xh);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) finish(a[u], b[u], out[u]);
  }
  for (; g < total; g += stride) {
    const uint16_t* row;
    uint16_t* out;
    locate(g, row, out);
    finish(*(const u32x4*)row, *(const u32x4*)(row + dh * xh), out);
  }
}

template <typename T>
static int pool_launch(const void* x, const int64_t* xs, void* y, const int64_t* ys, int64_t N, int64_t C, int64_t H,
                       int64_t W, int64_t P, int64_t Q, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                       int64_t pw, int64_t dh, int64_t dw, hipStream_t stream, int config = 0) {
  typedef typename elem<T>::storage S;
  if (config < 0 || config > 4) return NT_ERR_INVALID;
  if (N < 0 || C < 0 || H < 0 || W < 0 || P < 0 || Q < 0 || kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 || dh <= 0 ||
      dw <= 0 || ph < 0 || pw < 0)
    return NT_ERR_INVALID;
  if (N * C * P * Q == 0) return 0;
  if (!x || !y || !xs || !ys) return NT_ERR_INVALID;
  PoolShape s{N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, {xs[0], xs[1], xs[2], xs[3]}, {ys[0], ys[1], ys[2], ys[3]}};
  const bool windows_inside = (P - 1) * sh + (kh - 1) * dh < H && (Q - 1) * sw + (kw - 1) * dw < W;
  const bool fast = sizeof(S) == 2 && kw == 2 && sw == 2 && dw == 1 && ph == 0 && pw == 0 && xs[3] == 1 &&
                    ys[3] == 1 && Q % 8 == 0 && windows_inside && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 &&
                    (xs[0] * 2) % 16 == 0 && (xs[1] * 2) % 16 == 0 && (xs[2] * 2) % 16 == 0 &&
                    (ys[0] * 2) % 16 == 0 && (ys[1] * 2) % 16 == 0 && (ys[2] * 2) % 16 == 0 && N * C <= 0x7fffffffLL &&
                    H * xs[2] <= 0x7fffffffLL && P * ys[2] <= 0x7fffffffLL;
  // the pair kernel: as `fast`, with 4 outputs (8 bytes) per unit instead of 8
  const bool pair = sizeof(S) == 2 && kh == 2 && kw == 2 && sw == 2 && dw == 1 && ph == 0 && pw == 0 && xs[3] == 1 &&
                    ys[3] == 1 && Q % 4 == 0 && windows_inside && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 8 == 0 &&
                    (xs[0] * 2) % 16 == 0 && (xs[1] * 2) % 16 == 0 && (xs[2] * 2) % 16 == 0 &&
                    (ys[0] * 2) % 8 == 0 && (ys[1] * 2) % 8 == 0 && (ys[2] * 2) % 8 == 0 && N * C <= 0x7fffffffLL &&
                    H * xs[2] <= 0x7fffffffLL && P * ys[2] <= 0x7fffffffLL;
  // unit counts stay below 2^31 - 2^24, so a lane's next unit index (at most 8 grid strides of
  // at most 2^19 lanes further) still fits an int
  constexpr int64_t MAX_UNITS = 0x7fffffffLL - (1LL << 24);
  const int64_t upp = P * (Q / 4), total_units = N * C * upp;
  // The LDS kernel.  Small planes: G whole planes per workgroup, as many as fit its LDS but
  // no more than leave the chip 8 workgroups per CU, when x and y are plane-contiguous.
  // Otherwise one strip of PR output rows of one plane: at most as many as the LDS holds the
  // input rows of, and fewer where that leaves the chip under 8 workgroups per CU.  In-plane
  // and in-tile indices are 32-bit; the grid stays under 2^24 workgroups of 256 lanes.
  constexpr int64_t LDS_TARGET = 256 * 8, LDS_ROOM = POOL_LDS_BYTES - 16;
  const int64_t per_row = W * (int64_t)sizeof(S), span = (kh - 1) * dh + 1, NC = N * C;
  const bool rows_flat = xs[3] == 1 && xs[2] == W;
  const bool planes_flat = rows_flat && xs[1] == H * W && xs[0] == C * H * W && ys[3] == 1 && ys[2] == Q &&
                           ys[1] == P * Q && ys[0] == C * P * Q;
  int64_t G = 1, PR = 0;
  if (H > 0 && W > 0 && W * H <= 0x7fffffffLL && P * Q <= 0x7fffffffLL && P * ys[2] + Q * ys[3] <= 0x7fffffffLL &&
      H * xs[2] + W * xs[3] <= 0x7fffffffLL) {
    if (planes_flat && H * per_row <= LDS_ROOM / 2) {
      G = std::min<int64_t>(LDS_ROOM / (H * per_row), cdiv(NC, LDS_TARGET));
      G = std::max<int64_t>(G, 1);
      if (G * P * Q > 0x7fffffffLL) G = 1;  // a group's output index stays a 32-bit int
    }
    if (G > 1) {
      PR = P;
    } else if (span * per_row <= LDS_ROOM) {
      PR = std::min<int64_t>(P, 1 + (LDS_ROOM / per_row - span) / sh);
      PR = std::max<int64_t>(1, std::min<int64_t>(PR, cdiv(P * NC, LDS_TARGET)));
      PR = cdiv(P, cdiv(P, PR));  // strips of equal height
    }
  }
  const int64_t strips = PR > 0 ? cdiv(P, PR) : 0, lds_blocks = strips * cdiv(NC, G);
  const bool lds = PR > 0 && lds_blocks < (1LL << 24) && G * H * W <= 0x7fffffffLL;
  const int64_t lds_bytes = G > 1 ? G * H * per_row + 16 : ((PR - 1) * sh + span) * per_row + 16;
  const int lds_mode = rows_flat ? 0
                       : (xs[3] == 1 && per_row % 16 == 0 && (uintptr_t)x % 16 == 0 &&
                          (xs[0] * (int64_t)sizeof(S)) % 16 == 0 && (xs[1] * (int64_t)sizeof(S)) % 16 == 0 &&
                          (xs[2] * (int64_t)sizeof(S)) % 16 == 0)
                           ? 1
                           : 2;
  if ((config == 1 && !fast && !pair) || (config == 3 && !(fast && kh == 2)) || (config == 4 && !lds))
    return NT_ERR_INVALID;
  const int64_t vpp = P * (Q / 8), total_vec = N * C * vpp;
  if (config == 4 || (config == 0 && !fast && !pair && lds && lds_mode != 2)) {
    const dim3 grid((unsigned)lds_blocks);
    const unsigned shm = (unsigned)lds_bytes;
    const PoolDiv div_q = pool_div((uint32_t)Q), div_pq = pool_div((uint32_t)(G > 1 ? P * Q : 1));
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(256), shm, stream, (const S*)x, (S*)y, s, (int)G, (int)PR, (int)strips,
                         div_q, div_pq);
    };
    auto pick = [&](auto mode) {
      constexpr int M = decltype(mode)::value;
      if (kh == 3 && kw == 3)
        go(pool_lds_kernel<T, M, 3, 3>);
      else if (kh == 2 && kw == 2)
        go(pool_lds_kernel<T, M, 2, 2>);
      else
        go(pool_lds_kernel<T, M, 0, 0>);
    };
    if (lds_mode == 0)
      pick(std::integral_constant<int, 0>());
    else if (lds_mode == 1)
      pick(std::integral_constant<int, 1>());
    else
      pick(std::integral_constant<int, 2>());
  } else if (pair && (config == 0 || config == 1) && total_units <= MAX_UNITS) {
    const int64_t blocks = std::min<int64_t>(cdiv(total_units, 256 * 8), 256 * 8);
    hipLaunchKernelGGL(pool_w2_pair_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, (const uint16_t*)x,
                       (uint16_t*)y, s, (int)upp, (int)(Q / 4), (int)total_units);
  } else if (fast && config != 2 && kh == 2 && total_vec <= MAX_UNITS) {
    const int64_t blocks = std::min<int64_t>(cdiv(total_vec, 256 * 4), 256 * 8);
    hipLaunchKernelGGL(pool_w2_flat_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, (const uint16_t*)x,
                       (uint16_t*)y, s, (int)vpp, (int)(Q / 8), (int)total_vec);
  } else if (fast && config != 2 && config != 3) {
    hipLaunchKernelGGL(pool_w2_plane_kernel<T>, dim3((unsigned)(N * C)), dim3(256), 0, stream, (const uint16_t*)x,
                       (uint16_t*)y, s);
  } else {
    int64_t blocks = cdiv(N * C * P * Q, 256);
    if (blocks > 256 * 32) blocks = 256 * 32;
    hipLaunchKernelGGL(pool_generic_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, (const S*)x, (S*)y, s);
  }
  return launch_status();
}

// Input and output of any two element types: same types take pool_launch's kernels, others
// the element-wise kernel.
template <typename T>
static int pool_cast_to(const void* x, const int64_t* xs, void* y, int y_dtype, const int64_t* ys, int64_t N,
                        int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q, int64_t kh, int64_t kw, int64_t sh,
                        int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, hipStream_t stream) {
  if (y_dtype == elem<T>::code)
    return pool_launch<T>(x, xs, y, ys, N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, stream);
  if (!valid_dtype(y_dtype)) return NT_ERR_INVALID;
  if (N < 0 || C < 0 || H < 0 || W < 0 || P < 0 || Q < 0 || kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 || dh <= 0 ||
      dw <= 0 || ph < 0 || pw < 0)
    return NT_ERR_INVALID;
  if (N * C * P * Q == 0) return 0;
  if (!x || !y || !xs || !ys) return NT_ERR_INVALID;
  PoolShape s{N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, {xs[0], xs[1], xs[2], xs[3]}, {ys[0], ys[1], ys[2], ys[3]}};
  const dim3 grid((unsigned)std::min<int64_t>(cdiv(N * C * P * Q, 256), 256 * 32));
  typedef typename elem<T>::storage S;
  if (y_dtype == NT_DTYPE_F32)
    hipLaunchKernelGGL((pool_generic_kernel<T, float>), grid, dim3(256), 0, stream, (const S*)x, (float*)y, s);
  else if (y_dtype == NT_DTYPE_F16)
    hipLaunchKernelGGL((pool_generic_kernel<T, f16_t>), grid, dim3(256), 0, stream, (const S*)x, (uint16_t*)y, s);
  else
    hipLaunchKernelGGL((pool_generic_kernel<T, bf16_t>), grid, dim3(256), 0, stream, (const S*)x, (uint16_t*)y, s);
  return launch_status();
}

}  // namespace nt

extern "C" int nt_max_pool2d_cast(const void* x, int x_dtype, const int64_t* xs, void* y, int y_dtype,
                                  const int64_t* ys, int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                                  int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh,
                                  int64_t dw, hipStream_t stream) {
  if (x_dtype == NT_DTYPE_F32)
    return nt::pool_cast_to<float>(x, xs, y, y_dtype, ys, N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, stream);
  if (x_dtype == NT_DTYPE_F16)
    return nt::pool_cast_to<nt::f16_t>(x, xs, y, y_dtype, ys, N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, stream);
  if (x_dtype == NT_DTYPE_BF16)
    return nt::pool_cast_to<nt::bf16_t>(x, xs, y, y_dtype, ys, N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, stream);
  return NT_ERR_INVALID;
}

#define NT_POOL_ENTRY(NAME, T)                                                                                      \
  extern "C" int NAME(const void* x, const int64_t* xs, void* y, const int64_t* ys, int64_t N, int64_t C, int64_t H, \
                      int64_t W, int64_t P, int64_t Q, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,   \
                      int64_t pw, int64_t dh, int64_t dw, hipStream_t stream) {                                      \
    return nt::pool_launch<T>(x, xs, y, ys, N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, stream);              \
  }
NT_POOL_ENTRY(nt_max_pool2d_f32, float)
NT_POOL_ENTRY(nt_max_pool2d_f16, nt::f16_t)
NT_POOL_ENTRY(nt_max_pool2d_bf16, nt::bf16_t)
#define NT_POOL_CONFIG_ENTRY(NAME, T)                                                                               \
  extern "C" int NAME(const void* x, const int64_t* xs, void* y, const int64_t* ys, int64_t N, int64_t C, int64_t H, \
                      int64_t W, int64_t P, int64_t Q, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,   \
                      int64_t pw, int64_t dh, int64_t dw, hipStream_t stream, int config) {                          \
    return nt::pool_launch<T>(x, xs, y, ys, N, C, H, W, P, Q, kh, kw, sh, sw, ph, pw, dh, dw, stream, config);      \
  }
NT_POOL_CONFIG_ENTRY(nt_max_pool2d_config_f32, float)
NT_POOL_CONFIG_ENTRY(nt_max_pool2d_config_f16, nt::f16_t)
NT_POOL_CONFIG_ENTRY(nt_max_pool2d_config_bf16, nt::bf16_t)
