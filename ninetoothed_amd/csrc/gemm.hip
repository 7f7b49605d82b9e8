// GEMM with the addmm epilogue:  out = cast_out(beta * c + alpha * round(sum_k a*b)).
//
// fp16 / bf16 (MFMA-bound; 2*M*N*K flops per launch): workgroup tile 256 x 256 x 64 on
// v_mfma_f32_32x32x16_{f16,bf16}.  Kernels, fastest first:
//   gemm_dma_kernel    a k-contiguous, b n-contiguous, M, N multiples of 256, K of 64 and at
//                      least 128: 8 waves of 128 x 64, both operands DMA'd from HBM into a
//                      four-stage LDS ring (k-tiles of 32), b read with transposing LDS reads;
//   gemm_fast8_kernel  same layouts, other K multiples of 64: 8 waves of 64 x 128;
//   gemm_mfma_kernel   anything else (any strides, ragged edges, zero fill).
// Both operands sit in LDS k-contiguous ([m][k] for a, [n][k] for b) so that each lane
// fetches its 8 k-values for an MFMA with one ds_read_b128.  b arrives n-contiguous
// from HBM: each lane loads an 8(k) x 8(n) block (or 4(k) x 8(n)) with 16-byte loads
// and transposes it in registers before storing it.  LDS rows are 128 bytes; the
// 16-byte chunk index is XOR-swizzled with (row ^ row >> 3) & 7 so that both the
// row-wise fragment reads and the transposed b stores hit 8 distinct chunks per 8
// lanes.  The next k-tile is fetched from HBM into registers while the current one is
// multiplied out of LDS (two LDS buffers).  Workgroups are remapped so that the 8 XCDs
// (which the dispatcher fills round-robin) each receive a compact block of tiles.
// fp32 (512^3 reference case): 32 x 32 workgroup tiles, four waves each computing a
//   16 x 16 block with v_mfma_f32_16x16x4f32, K staged through LDS 256 at a time.
#include "mfma_core.h"

#include <cstring>
#include <type_traits>

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
  int c_dtype;  // c's element type: out's, or an fp8 format (widened exactly)
  int tiles_m, tiles_n;
  int c_pre;  // gemm_dma_kernel's fast epilogue: 16-bit out (and c) with unit column stride,
              // 16-byte aligned rows, out and c panel offsets within 32 bits
  // gemm_dma128_kernel only: product blockIdx.y of a batch, its a, b and out at these element
  // strides from the first's (0 outside a batch).
  int64_t sa_b, sb_b, so_b;
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

// Operand storage of gemm_mfma_kernel's element-wise loader.  16-bit operands are used as
// they are; fp8 operands are widened exactly to fp16 (every e5m2 and e4m3fn value is an
// fp16 value) and multiplied on the fp16 matrix core, so the products are exact in fp32
// as on an fp8 matrix core.
struct src16 {
  typedef uint16_t storage;
  __device__ __forceinline__ static uint16_t widen(uint16_t v) { return v; }
};
struct src_e5m2 {  // OCP E5M2: sign, 5 exponent bits (bias 15), 2 mantissa bits = the top byte of an fp16
  typedef uint8_t storage;
  __device__ __forceinline__ static uint16_t widen(uint8_t v) { return (uint16_t)((uint16_t)v << 8); }
};
struct src_e4m3 {  // OCP E4M3FN: sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities, S.1111.111 = NaN
  typedef uint8_t storage;
  __device__ __forceinline__ static uint16_t widen(uint8_t v) {
    const uint16_t s = (uint16_t)(v & 0x80) << 8;
    const int e = (v >> 3) & 0xf, m = v & 7;
    if (e == 0xf && m == 7) return s | 0x7e00;
    if (e == 0) {  // m * 2^-9: normalised in fp16 with the leading one of m as the implicit bit
      if (m == 0) return s;
      const int lead = m >= 4 ? 2 : (m >= 2 ? 1 : 0);
      return s | (uint16_t)((lead + 6) << 10) | (uint16_t)((m - (1 << lead)) << (10 - lead));
    }
    return s | (uint16_t)((e + 8) << 10) | (uint16_t)(m << 7);
  }
};

// One element of c as fp32: f32/f16/bf16, or (C8: kernels of fp8 operands, whose c may be
// fp8 too) an fp8 value widened exactly through fp16.  The 16- and 32-bit launchers reject
// an fp8 c, so their kernels carry no fp8 code.
template <bool C8>
__device__ __forceinline__ float load_c(const GemmArgs& g, int64_t i) {
  if constexpr (C8) {
    if (g.c_dtype == NT_DTYPE_E5M2) return f16_bits_to_float(src_e5m2::widen(((const uint8_t*)g.c)[i]));
    if (g.c_dtype == NT_DTYPE_E4M3) return f16_bits_to_float(src_e4m3::widen(((const uint8_t*)g.c)[i]));
  }
  return load_as_float(g.c, i, g.c_dtype);
}

// Epilogue shared by the GEMM kernels: out = cast(beta * c + alpha * round(acc)), one
// 32-row slab per pass staged through LDS (32 x WJ*32 fp32 per wave), then each lane
// handles 8 consecutive columns.
//
// Fast path (the wave's whole tile in bounds, c and out 16-bit, unit column stride,
// 16-byte aligned rows): all of a slab's c vectors are loaded at once, the next slab's
// while the current one is stored, so the epilogue pays the HBM latency about once
// instead of once per vector; 16-byte loads and stores.  A wave only reads back what it
// staged itself, so the slabs need no workgroup barrier.  Otherwise element-wise with
// bounds checks and any strides.
template <int WI, int WJ, bool C8 = false>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, const floatx16 (&acc)[WI][WJ], uint16_t* smem,
                                              int wave, int lane, int64_t row_base, int64_t col_base) {
  constexpr int COLS = WJ * 32;
  constexpr int VPR = COLS / 8;          // 16-byte vectors per row
  constexpr int VPL = 32 * VPR / 64;     // per lane per slab
  float* stage = (float*)smem + wave * (32 * COLS);
  const bool vec16 = g.out_dtype != NT_DTYPE_F32 && g.so_n == 1 && (g.so_m % 8) == 0 && ((uintptr_t)g.out % 16) == 0 &&
                     (!g.c || (g.c_dtype == g.out_dtype && g.sc_n == 1 && (g.sc_m % 8) == 0 &&
                               ((uintptr_t)g.c % 16) == 0));
  const bool full = vec16 && row_base + WI * 32 <= g.M && col_base + COLS <= g.N;
  __syncthreads();  // the LDS still holds operand tiles other waves may be reading
  if (full) {
    const bool f16 = g.out_dtype == NT_DTYPE_F16;
    const uint16_t* C = (const uint16_t*)g.c;
    uint16_t* O = (uint16_t*)g.out;
    u32x4 cv[2][VPL];
    auto load_c = [&](int i, int buf) {
#pragma unroll
      for (int t = 0; t < VPL; ++t) {
        const int e = t * 64 + lane, rr = e / VPR, cg = (e % VPR) * 8;
        cv[buf][t] = *(const u32x4*)(C + (row_base + i * 32 + rr) * g.sc_m + col_base + cg);
      }
    };
    if (g.c) load_c(0, 0);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      if (g.c && i + 1 < WI) load_c(i + 1, (i + 1) & 1);
      stage_slab<WJ>(stage, acc[i], lane);
#pragma unroll
      for (int t = 0; t < VPL; ++t) {
        const int e = t * 64 + lane, rr = e / VPR, cg = (e % VPR) * 8;
        const float4 v0 = *(const float4*)(stage + rr * COLS + cg);
        const float4 v1 = *(const float4*)(stage + rr * COLS + cg + 4);
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const uint16_t* ch = (const uint16_t*)&cv[i & 1][t];
        u32x4 oraw;
        uint16_t* oh = (uint16_t*)&oraw;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          float r = g.alpha * round_through(v[u], g.round_dtype);
          if (g.c) r += g.beta * (f16 ? f16_bits_to_float(ch[u]) : bf16_bits_to_float(ch[u]));
          oh[u] = f16 ? float_to_f16_bits(r) : float_to_bf16_bits(r);
        }
        *(u32x4*)(O + (row_base + i * 32 + rr) * g.so_m + col_base + cg) = oraw;
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    stage_slab<WJ>(stage, acc[i], lane);
    const int64_t row0 = row_base + i * 32;
    for (int e = lane; e < 32 * VPR; e += 64) {
      const int rr = e / VPR, cg = (e % VPR) * 8;
      const int64_t row = row0 + rr, col = col_base + cg;
      if (row >= g.M) continue;
      const float4 v0 = *(const float4*)(stage + rr * COLS + cg);
      const float4 v1 = *(const float4*)(stage + rr * COLS + cg + 4);
      const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int u = 0; u < 8; ++u) {  // unrolled, so v stays in registers
        if (col + u < g.N) {
          float r = g.alpha * round_through(v[u], g.round_dtype);
          if (g.c) r += g.beta * load_c<C8>(g, row * g.sc_m + (col + u) * g.sc_n);
          store_from_float(g.out, row * g.so_m + (col + u) * g.so_n, g.out_dtype, r);
        }
      }
    }
  }
}

template <typename T, bool FAST, typename S = src16>
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
  const typename S::storage* As = (const typename S::storage*)g.a;
  const typename S::storage* Bs = (const typename S::storage*)g.b;
  auto load_store_generic = [&](int64_t kt) {
    const int64_t k0 = kt * GB_K;
    for (int e = tid; e < GB_M * GB_K; e += G_THREADS) {
      const int row = e / GB_K, kk = e % GB_K;
      const int64_t m = m0 + row, k = k0 + kk;
      uint16_t v = 0;
      if (m < g.M && k < g.K) v = S::widen(As[m * g.sa_m + k * g.sa_k]);
      sA[lds_index(row, kk)] = v;
    }
    for (int e = tid; e < GB_N * GB_K; e += G_THREADS) {
      const int kk = e / GB_N, col = e % GB_N;
      const int64_t n = n0 + col, k = k0 + kk;
      uint16_t v = 0;
      if (n < g.N && k < g.K) v = S::widen(Bs[k * g.sb_k + n * g.sb_n]);
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

  gemm_epilogue<4, 4, !std::is_same<S, src16>::value>(g, acc, smem, wave, lane, m0 + wm * 128, n0 + wn * 128);
}

// Fast path (M, N multiples of 256, K of 64, a k-contiguous, b n-contiguous, 16-byte
// aligned rows): 512 lanes, waves in a 4 (m) x 2 (n) grid, each owning 64 x 128 of the
// 256 x 256 tile (128 accumulators), so two waves share each SIMD and one's matrix work
// covers the other's waits.  Two 64 KiB LDS buffers: while tile kt is multiplied out of
// one, tile kt+1 (already in registers) is stored into the other and tile kt+2 is
// fetched from HBM, one barrier per k-tile.  a: 4 chunks of 16 bytes per lane; b: a 4(k) x
// 8(n) block per lane, transposed in registers and stored as eight 8-byte rows.
__device__ __forceinline__ void transpose4x8(const u32x4 (&in)[4], u32x2 (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int d = j >> 1;
    const bool hi = j & 1;
    uint32_t w[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t x0 = in[2 * r][d], x1 = in[2 * r + 1][d];
      w[r] = hi ? ((x0 >> 16) | (x1 & 0xffff0000u)) : ((x0 & 0xffffu) | (x1 << 16));
    }
    out[j] = u32x2{w[0], w[1]};
  }
}

template <typename T>
__global__ __launch_bounds__(512) void gemm_fast8_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (GB_M + GB_N) * GB_K];
  constexpr int BUF = (GB_M + GB_N) * GB_K;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 4 x 2
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * GB_M, n0 = (int64_t)tn * GB_N;
  const int a_row = tid >> 3, a_chunk = tid & 7;  // rows a_row + 64*i
  const int b_nb = tid & 31, b_kq = tid >> 5;     // 4(k) x 8(n) block: k = 4*b_kq .. +3
  const uint16_t* A = (const uint16_t*)g.a + (m0 + a_row) * g.sa_m + a_chunk * 8;
  const uint16_t* B = (const uint16_t*)g.b + (int64_t)(b_kq * 4) * g.sb_k + n0 + b_nb * 8;
  const int64_t a_step = 64 * g.sa_m;
  const int nk = (int)(g.K / GB_K);

  floatx16 acc[2][4];
  zero_acc(acc);
  u32x4 ra[4], rb[4];
  u32x2 tb[8];
  int a_st[4], b_st[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = i * 64 + a_row;
    a_st[i] = row * GB_K + swz(row, a_chunk) * 8;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int nrow = b_nb * 8 + j;
    b_st[j] = GB_M * GB_K + nrow * GB_K + swz(nrow, b_kq >> 1) * 8 + (b_kq & 1) * 4;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) ra[i] = *(const u32x4*)(A + i * a_step);
#pragma unroll
  for (int r = 0; r < 4; ++r) rb[r] = *(const u32x4*)(B + r * g.sb_k);
  transpose4x8(rb, tb);
#pragma unroll
  for (int i = 0; i < 4; ++i) *(u32x4*)(smem + a_st[i]) = ra[i];
#pragma unroll
  for (int j = 0; j < 8; ++j) *(u32x2*)(smem + b_st[j]) = tb[j];
  if (nk > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = *(const u32x4*)(A + i * a_step + GB_K);
#pragma unroll
    for (int r = 0; r < 4; ++r) rb[r] = *(const u32x4*)(B + (GB_K + r) * g.sb_k);
  }
  __syncthreads();

  typedef typename mfma_traits<T>::frag frag;
  // One k-tile.  First the staged tile kt+1 (loaded one iteration ago) goes to the other
  // LDS buffer and the loads of tile kt+2 are issued; the scheduling barrier keeps those
  // loads here, a whole k-tile of matrix work ahead of their use.
  auto step = [&](auto has1_c, auto has2_c, int kt) {
    constexpr bool HAS1 = decltype(has1_c)::value, HAS2 = decltype(has2_c)::value;
    const uint16_t* sA = smem + (kt & 1) * BUF;
    const uint16_t* sB = sA + GB_M * GB_K;
    uint16_t* nxt = smem + ((kt & 1) ^ 1) * BUF;
    const int64_t k2 = (int64_t)(kt + 2) * GB_K;
    if constexpr (HAS1) {
      transpose4x8(rb, tb);
#pragma unroll
      for (int i = 0; i < 4; ++i) *(u32x4*)(nxt + a_st[i]) = ra[i];
#pragma unroll
      for (int j = 0; j < 8; ++j) *(u32x2*)(nxt + b_st[j]) = tb[j];
      if constexpr (HAS2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = *(const u32x4*)(A + i * a_step + k2);
#pragma unroll
        for (int r = 0; r < 4; ++r) rb[r] = *(const u32x4*)(B + (k2 + r) * g.sb_k);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < GB_K / 16; ++kk) {
      const int chunk = kk * 2 + (lane >> 5);
      frag fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + i * 32 + (lane & 31);
        fa[i] = *(const frag*)(sA + row * GB_K + swz(row, chunk) * 8);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = wn * 128 + j * 32 + (lane & 31);
        fb[j] = *(const frag*)(sB + row * GB_K + swz(row, chunk) * 8);
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

  gemm_epilogue<2, 4>(g, acc, smem, wave, lane, m0 + wm * 64, n0 + wn * 128);
}

// DMA form: 512 lanes, two waves per SIMD in a 2 (m) x 4 (n) grid, each owning 128 x 64 of
// the 256 x 256 tile (128 accumulators), k-tiles of 32.  Both operands go from HBM straight
// into LDS (buffer_load ... lds: lane l of a load writes bytes 16 l .. 16 l + 15 past the
// LDS address in M0), so the k loop holds no staging registers and issues no LDS stores.
//   a: [m][k] rows of 64 bytes whose four 16-byte chunks are XOR-swizzled by (row / 4) % 4;
//      each lane fetches the global chunk that belongs at its LDS position; fragments are
//      ds_read_b128 (16 lanes of one pass hit 16 distinct bank groups).
//   b: [k][n] as in HBM, rows of 512 bytes whose 64-byte chunks (32 n) are XOR-swizzled by
//      bsw(k); fragments come from two ds_read_b64_tr_b16 each.  That instruction works on
//      groups of 16 lanes: lane 4 r + q reads 4 consecutive 16-bit values, and lane j of
//      the group receives value j % 4 of lanes j / 4, 4 + j / 4, 8 + j / 4, 12 + j / 4.  So if
//      lane 4 r + q reads row k0 + r at columns 4 q .. 4 q + 3, lane j receives column j at
//      rows k0 .. k0 + 3: the MFMA's b operand (8 consecutive k of one n) in two reads.
// Four LDS stages of 32 KiB (a at 16 Ki * stage, b at 64 Ki + 16 Ki * stage) and 32 KiB of
// epilogue staging at 128 Ki.  Tile kt+3 is fetched during tile kt into the stage of tile
// kt-1: every read of that stage has completed by then, since LDS operations complete in
// order and the wave has already waited for a later read of tile kt.  So the one barrier
// per k-tile (which also publishes tile kt+1, each wave having waited for its own loads)
// needs no wait for outstanding reads, and a load has two k-tiles to land.
// The loads are issued from inline assembly: the compiler would otherwise make every LDS
// read wait for them.  The waves of a SIMD take turns on the matrix core, so one's LDS
// waits hide behind the other's MFMAs.  Per 32-deep k-tile a wave issues 16 MFMAs, 8
// ds_read_b128, 8 transposing reads and 4 loads.
namespace dma {
constexpr int STAGES = 4, STAGE = 16384, B0 = 65536, EPI = 131072;
__device__ __forceinline__ int bsw(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }
__device__ __forceinline__ int asw(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }
typedef short v4i16 __attribute__((ext_vector_type(4)));
// Buffer resource: base, no stride, `bytes` records (offsets at or past it read zero).
__device__ __forceinline__ u32x4 rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, bytes, 0x00020000u};
}
// 16 bytes per lane from buffer `rs` at voffset + soffset into LDS at lds_addr + 16 * lane.
__device__ __forceinline__ void load_lds16(u32x4 rs, uint32_t lds_addr, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rs), "s"(soffset)
               : "memory", "m0");
}
}  // namespace dma

// The DMA kernels' fast epilogue (16-bit out, c absent or of out's type, unit column
// stride, 16-byte aligned rows; the launcher's c_pre).  acc holds a wave's 128 x (32 WJ)
// block as 4 x WJ tiles of 32 x 32 (the 32x32 MFMA accumulator layout); lds + EPI +
// 2 KiB * WJ * wave is the wave's staging.  NI: the wave's 32-row slabs (4: 128 rows; 2 in
// gemm_dma128_kernel, whose staging starts at EPI_AT).
template <int WJ = 2, bool BOUNDED = false, int NI = 4, int EPI_AT = dma::EPI>
__device__ __forceinline__ void dma_fast_epilogue(const GemmArgs& g, const floatx16 (&acc)[NI][WJ], char* lds, int wave,
                                                  int lane, int64_t row_base, int64_t col_base) {
  // Fast epilogue: the accumulators go through this wave's staging (never touched by the k
  // loop: no barrier) 16 rows at a time; a lane finishes rows t * (64 / CPR) + lane / CPR
  // (CPR = 4 WJ lanes per row, t < WJ) at columns (lane % CPR) * 8 .. + 7.  c is read
  // through a buffer resource (the host checks its offsets fit 32 bits); c of slab i + 2 is
  // fetched while slab i is finished.  Without c the resource has no records: the loads
  // return zeros.
  static_assert(WJ == 2 || WJ == 4, "two or four 32-wide column blocks");
  constexpr int COLS = 32 * WJ, CPR = COLS / 8, RPP = 64 / CPR;  // lanes per row, rows per pass
  constexpr int CPR_LOG2 = WJ == 2 ? 3 : 4;
  const int lrow = lane >> CPR_LOG2, lcol = lane & (CPR - 1);
  // BOUNDED: rows and columns of this wave's block inside out (ragged M and N; N is a
  // multiple of 8, so each lane's 8 columns are all inside or all outside).  Otherwise the
  // launcher has checked that every tile is whole.
  constexpr int ROWS = 32 * NI;
  int rows_v = ROWS, cols_v = COLS;
  if constexpr (BOUNDED) {
    rows_v = (int)(g.M - row_base < ROWS ? g.M - row_base : ROWS);
    cols_v = (int)(g.N - col_base < COLS ? g.N - col_base : COLS);
    if (rows_v <= 0 || cols_v <= 0) return;
  }
  const bool col_ok = !BOUNDED || lcol * 8 < cols_v;
  const bool has_c = g.c != nullptr;
  // c through a buffer resource ending at the block's last valid element: rows past M read
  // zeros instead of memory past the tensor.
  const __amdgpu_buffer_rsrc_t rsC = __builtin_amdgcn_make_buffer_rsrc(
      has_c ? (void*)((const uint16_t*)g.c + row_base * g.sc_m + col_base) : (void*)g.a, (short)0,
      has_c ? (int)(((rows_v - 1) * g.sc_m + cols_v) * 2) : 0, 0x00020000);
  const int vc = has_c ? (int)((lrow * g.sc_m + lcol * 8) * 2) : 0;
  const int c_row = has_c ? (int)(g.sc_m * 2) : 0;
  // out through plain global stores: a buffer store whose data registers a VALU instruction
  // rewrote a few instructions later has been seen to store the new values on this target.
  char* o_lane = (char*)((uint16_t*)g.out + (row_base + lrow) * g.so_m + col_base + lcol * 8);
  const int64_t o_row = g.so_m * 2;
  u32x4 cv[2][2][WJ];
  auto load_c = [&](int i) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int t = 0; t < WJ; ++t)
        cv[i & 1][h][t] = __builtin_amdgcn_raw_buffer_load_b128(rsC, vc, (i * 32 + h * 16 + t * RPP) * c_row, 0);
  };
  float* stage = (float*)(lds + EPI_AT + wave * (2048 * WJ));
  auto finish = [&](auto out_f16_c, auto round_c, int i, int h) {
    constexpr bool OUT_F16 = decltype(out_f16_c)::value;
    constexpr int ROUND = decltype(round_c)::value;
    wave_lds_order();  // the previous half's reads come first
#pragma unroll
    for (int j = 0; j < WJ; ++j)
#pragma unroll
      for (int r = 8 * h; r < 8 * h + 8; ++r)
        stage[(acc_row(r, lane) - 16 * h) * COLS + j * 32 + (lane & 31)] = acc[i][j][r];
    wave_lds_order();  // every lane's writes before any lane reads
#pragma unroll
    for (int t = 0; t < WJ; ++t) {
      const int rr = t * RPP + lrow, cg = lcol * 8;
      const float4 v0 = *(const float4*)(stage + rr * COLS + cg);
      const float4 v1 = *(const float4*)(stage + rr * COLS + cg + 4);
      const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      const u32x4 cw = cv[i & 1][h][t];
      u32x4 ow;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float r2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float x = v[2 * d + e];
          if constexpr (ROUND == NT_DTYPE_F16) x = f16_bits_to_float(float_to_f16_bits(x));
          if constexpr (ROUND == NT_DTYPE_BF16) x = bf16_bits_to_float(float_to_bf16_bits(x));
          r2[e] = g.alpha * x;
          if (has_c) {
            const uint16_t cb = (uint16_t)(cw[d] >> (16 * e));
            r2[e] += g.beta * (OUT_F16 ? f16_bits_to_float(cb) : bf16_bits_to_float(cb));
          }
        }
        ow[d] = OUT_F16 ? ((uint32_t)float_to_f16_bits(r2[0]) | ((uint32_t)float_to_f16_bits(r2[1]) << 16))
                        : ((uint32_t)float_to_bf16_bits(r2[0]) | ((uint32_t)float_to_bf16_bits(r2[1]) << 16));
      }
      if (!BOUNDED || (col_ok && i * 32 + h * 16 + t * RPP + lrow < rows_v))
        __builtin_nontemporal_store(ow, (u32x4*)(o_lane + (i * 32 + h * 16 + t * RPP) * o_row));  // not re-read: no L2 allocation
    }
  };
  using OutF16 = std::integral_constant<bool, true>;
  using OutBF16 = std::integral_constant<bool, false>;
  using RNone = std::integral_constant<int, NT_DTYPE_NONE>;
  using RF16 = std::integral_constant<int, NT_DTYPE_F16>;
  using RBF16 = std::integral_constant<int, NT_DTYPE_BF16>;
  auto all = [&](auto out_f16_c, auto round_c) {
    load_c(0);
    load_c(1);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
#pragma unroll
      for (int h = 0; h < 2; ++h) finish(out_f16_c, round_c, i, h);
      if (i + 2 < NI) load_c(i + 2);
    }
  };
  const bool out_f16 = g.out_dtype == NT_DTYPE_F16;
  if (g.round_dtype == NT_DTYPE_F16) {
    if (out_f16) all(OutF16{}, RF16{}); else all(OutBF16{}, RF16{});
  } else if (g.round_dtype == NT_DTYPE_BF16) {
    if (out_f16) all(OutF16{}, RBF16{}); else all(OutBF16{}, RBF16{});
  } else {
    if (out_f16) all(OutF16{}, RNone{}); else all(OutBF16{}, RNone{});
  }
}

// The DMA kernels' element-wise epilogue (any out type, any c type, any strides).  After a
// barrier the operand ring is free: each wave stages two of its four 32-row slabs there at
// once (16 KiB per wave), finishes them one element per lane per step (consecutive lanes on
// consecutive columns, nothing unrolled), then does the same with the other two, so that
// at most half of the accumulators are live while elements are stored.
template <int WJ = 2, bool C8 = false>
__device__ __forceinline__ void dma_any_epilogue(const GemmArgs& g, const floatx16 (&acc)[4][WJ], char* lds, int wave,
                                                 int lane, int64_t row_base, int64_t col_base) {
  constexpr int COLS = 32 * WJ;
  float* stage = (float*)(lds + wave * (2 * 32 * COLS * 4));
  __syncthreads();  // other waves may still read the last operand stage
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    wave_lds_order();  // the previous pair's reads come first
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < WJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          stage[(i * 32 + acc_row(r, lane)) * COLS + j * 32 + (lane & 31)] = acc[2 * p + i][j][r];
    wave_lds_order();  // every lane's writes before any lane reads
    const int64_t row0 = row_base + p * 64;
#pragma unroll 1
    for (int e = lane; e < 64 * COLS; e += 64) {
      const int rr = e / COLS, cc = e % COLS;
      const int64_t row = row0 + rr, col = col_base + cc;
      if (row < g.M && col < g.N) {
        float r = g.alpha * round_through(stage[rr * COLS + cc], g.round_dtype);
        if (g.c) r += g.beta * load_c<C8>(g, row * g.sc_m + col * g.sc_n);
        store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, r);
      }
    }
  }
}

// FAST_EPI: the launcher's c_pre condition holds (16-bit out and c of one type, unit column
// stride, aligned rows); the other instance finishes through the element-wise epilogue.  Two
// instances so that the fast one holds no code of the other (whose registers would spill).
// BT: b is k-contiguous (column-major [K, N], i.e. rows of b^T, the layout of x @ w.t());
// its tiles then go to LDS exactly as a's do (rows of 64 bytes, XOR chunk swizzle) and its
// fragments are single ds_read_b128, with no transposing reads.
template <typename T, bool FAST_EPI, bool BT = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_dma_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char lds[dma::EPI + 8 * 4096];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * GB_M, n0 = (int64_t)tn * GB_N;
  const int nk = (int)((g.K + 31) / 32);

  // Global side (byte offsets within each operand's panel fit in 32 bits; checked on the host).
  // Each resource ends at the panel's last valid element, so rows of a past M and rows of b
  // past K read zeros; columns of b past N read the next row's values, which reach only
  // outputs past N (never stored).  With K not a multiple of 32, the chunks of a past K in
  // the last k-tile are fetched from offset a_end (zeros): an a value past K would otherwise
  // be the next row's, and an infinity there times a zero of b is not zero.
  const int rows_a = (int)(g.M - m0 < GB_M ? g.M - m0 : GB_M), cols_b = (int)(g.N - n0 < GB_N ? g.N - n0 : GB_N);
  const uint32_t a_end = (uint32_t)(((rows_a - 1) * g.sa_m + g.K) * 2);
  const u32x4 rsA = dma::rsrc((const uint16_t*)g.a + m0 * g.sa_m, a_end);
  // b^T (BT) ends at its last valid row (column of b) like a; its chunks past K in the last
  // k-tile read zeros the same way.
  const uint32_t b_end = BT ? (uint32_t)(((cols_b - 1) * g.sb_n + g.K) * 2) : (uint32_t)(((g.K - 1) * g.sb_k + cols_b) * 2);
  const u32x4 rsB = dma::rsrc((const uint16_t*)g.b + (BT ? n0 * g.sb_n : n0), b_end);
  // Load q (0, 1) of this wave per k-tile: a rows 32 wave + 16 q + lane / 4, LDS chunk
  // lane % 4; b rows 4 wave + 2 q + lane / 32, LDS bytes (lane % 32) * 16 of the row (BT:
  // b^T rows as a's).
  int va[2], vb[2], va_last[2], vb_last[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int ra = 32 * wave + 16 * q + (lane >> 2);
    va[q] = (int)(ra * g.sa_m * 2) + dma::asw(ra, lane & 3) * 16;
    va_last[q] = (nk - 1) * 32 + dma::asw(ra, lane & 3) * 8 < g.K ? va[q] : (int)a_end;
    if constexpr (BT) {
      vb[q] = (int)(ra * g.sb_n * 2) + dma::asw(ra, lane & 3) * 16;
      vb_last[q] = (nk - 1) * 32 + dma::asw(ra, lane & 3) * 8 < g.K ? vb[q] : (int)b_end;
    } else {
      const int kb = 4 * wave + 2 * q + (lane >> 5);
      const int nb = 32 * (((lane & 31) >> 2) ^ dma::bsw(kb)) + 8 * (lane & 3);
      vb[q] = (int)(kb * g.sb_k * 2) + nb * 2;
      vb_last[q] = vb[q];
    }
  }
  const int b_kstep = BT ? 64 : (int)(32 * g.sb_k * 2);
  // Load u (0..3) of tile kt into its stage: a q0, b q0, a q1, b q1.
  auto load_unit = [&](int u, int kt) {
    const int st = (kt % dma::STAGES) * dma::STAGE, q = u >> 1;
    if ((u & 1) == 0)
      dma::load_lds16(rsA, lds0 + st + 2048 * wave + 1024 * q, kt == nk - 1 ? va_last[q] : va[q], kt * 64);
    else
      dma::load_lds16(rsB, lds0 + dma::B0 + st + 2048 * wave + 1024 * q, kt == nk - 1 ? vb_last[q] : vb[q],
                      kt * b_kstep);
  };

  // Fragment reads.  a: row 128 wm + 32 i + lane % 32, chunk 2 s + lane / 32 (the swizzle
  // depends on lane % 32 only).  b (two reads per fragment): lane (group g = lane / 16, r, q)
  // reads row 16 s + 8 (g / 2) + 4 half + r at columns 64 wn + 32 j + 16 (g % 2) + 4 q .. + 3.
  int a_rd[2], b_rd[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const int row = wm * 128 + (lane & 31);
    a_rd[s2] = row * 64 + dma::asw(row, 2 * s2 + (lane >> 5)) * 16;
  }
  if constexpr (BT) {  // b^T: row 64 wn + 32 j + lane % 32 (j at + 2048 j), as a; indexed by slice
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int row = wn * 64 + (lane & 31);
      b_rd[s2] = dma::B0 + row * 64 + dma::asw(row, 2 * s2 + (lane >> 5)) * 16;
    }
  } else {
    const int gq = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
    const int f = r | ((gq >> 1) << 2);  // bsw of every row this lane reads
#pragma unroll
    for (int j = 0; j < 2; ++j)
      b_rd[j] = dma::B0 + (8 * (gq >> 1) + r) * 512 + (((2 * wn + j) ^ f) * 64) + (16 * (gq & 1) + 4 * q) * 2;
  }
  typedef typename mfma_traits<T>::frag frag;
  frag fa[2][4], fb[2][2];
  // Read unit x (0..5) of slice s2 of the tile in stage byte offset `st`, into slot s2:
  // a0, b0, b1, a1, a2, a3, the order the slice's MFMAs consume them.
  auto read_unit = [&](int x, int s2, int st) {
    if (x == 0 || x >= 3) {
      const int i = x == 0 ? 0 : x - 2;
      fa[s2][i] = *(const frag*)(lds + a_rd[s2] + st + i * 2048);
    } else if constexpr (BT) {
      const int j = x - 1;
      fb[s2][j] = *(const frag*)(lds + b_rd[s2] + st + j * 2048);
    } else {
      const int j = x - 1;
      const char* p = lds + b_rd[j] + st + s2 * 8192;
      const dma::v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) dma::v4i16*)p);
      const dma::v4i16 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) dma::v4i16*)(p + 2048));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      fb[s2][j] = __builtin_bit_cast(frag, u32x4{l2[0], l2[1], h2[0], h2[1]});
    }
  };

  floatx16 acc[4][2];
  zero_acc(acc);

  // nk >= 3 (the launcher checks): tiles 0..2 in flight, wait for tile 0.
  for (int kt = 0; kt < 3; ++kt)
    for (int u = 0; u < 4; ++u) load_unit(u, kt);
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int x = 0; x < 6; ++x) read_unit(x, 0, 0);

#define NT_FENCE() __builtin_amdgcn_sched_barrier(0)
  // One k-tile.  HAS1: a tile kt+1 exists (read its slice 0 during slice 1); LOAD: fetch
  // tile kt+3; VM: loads allowed outstanding once tile kt+1 has landed (-1: no wait and no
  // barrier, the last tile).
  auto step = [&](auto has1_c, auto load_c, auto vm_c, int kt) {
    constexpr bool HAS1 = decltype(has1_c)::value, LOAD = decltype(load_c)::value;
    constexpr int VM = decltype(vm_c)::value;
    const int st = (kt % dma::STAGES) * dma::STAGE, st1 = ((kt + 1) % dma::STAGES) * dma::STAGE;
    static_for<0, 16>([&](auto m_c) {
      constexpr int m = decltype(m_c)::value;
      constexpr int s2 = m >> 3, x = m & 7;
      if constexpr (m == 8 && VM >= 0) {
        NT_FENCE();
        if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        NT_FENCE();
      }
      acc[x >> 1][x & 1] = mfma_traits<T>::mma(fa[s2][x >> 1], fb[s2][x & 1], acc[x >> 1][x & 1]);
      NT_FENCE();
      if constexpr (x < 6) {
        if constexpr (s2 == 0)
          read_unit(x, 1, st);
        else if constexpr (HAS1)
          read_unit(x, 0, st1);
      }
      if constexpr (s2 == 1 && LOAD && x < 4) load_unit(x, kt + 3);
      NT_FENCE();
    });
  };
#undef NT_FENCE
  using T1 = std::integral_constant<bool, true>;
  using F1 = std::integral_constant<bool, false>;
  using V4 = std::integral_constant<int, 4>;
  using V0 = std::integral_constant<int, 0>;
  using VN = std::integral_constant<int, -1>;
  int kt = 0;
  for (; kt + 3 < nk; ++kt) step(T1{}, T1{}, V4{}, kt);
  step(T1{}, F1{}, V4{}, kt);
  step(T1{}, F1{}, V0{}, kt + 1);
  step(F1{}, F1{}, VN{}, kt + 2);

  const int64_t row_base = m0 + wm * 128, col_base = n0 + wn * 64;
  if constexpr (!FAST_EPI) {
    dma_any_epilogue<2>(g, acc, lds, wave, lane, row_base, col_base);
    return;
  }
  dma_fast_epilogue<2, true>(g, acc, lds, wave, lane, row_base, col_base);
}

// gemm_dma_kernel's pipeline on 128 x 128 tiles, for outputs with too few 256 x 256 tiles to
// fill the chip (2048^2 has 64 of those for 256 CUs, 256 of these).  Four waves of 64 x 64
// (2 x 2 blocks of 32 x 32) per workgroup and 80 KiB of LDS (ring 64 KiB, staging 16 KiB),
// so two workgroups share a CU.  The ring holds four 32-deep k-tiles of 8 KiB of a and 8 KiB
// of b, filled by DMA with each wave's two loads of each operand per k-tile as in the
// 256-wide kernel: a rows 32 wave + 16 q + lane / 4 (64-byte rows, XOR chunk swizzle); b
// rows 8 wave + 4 q + lane / 16 (256-byte rows of 128 columns; 32-column group g of row k
// stored at group g ^ (k % 4), so the transposing reads of 32 lanes, rows r = 0..3 of one
// group each, hit 4 x 16 distinct banks), or b^T rows as a's (BT).  Per k-tile a wave issues
// eight MFMAs (its 2 x 2 blocks, two 16-deep slices) with the next slice's four fragment
// reads between them, one barrier per k-tile, and the fast epilogue on 2 slabs of 32 rows.
// Only for calls whose epilogue is the fast one (the launcher's c_pre).
namespace dma128 {
constexpr int STAGE = 8192, B0 = 32768, EPI = 65536, LDS = EPI + 4 * 4096;
__device__ __forceinline__ int bsw(int k) { return k & 3; }
}  // namespace dma128

template <typename T, bool BT = false>
__global__ __launch_bounds__(256) void gemm_dma128_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char lds[dma128::LDS];
  if (blockIdx.y) {  // product blockIdx.y of a batch (no c)
    g.a = (const uint16_t*)g.a + blockIdx.y * g.sa_b;
    g.b = (const uint16_t*)g.b + blockIdx.y * g.sb_b;
    g.out = (uint16_t*)g.out + blockIdx.y * g.so_b;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  constexpr int TM = 128, TN = 128;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * TM, n0 = (int64_t)tn * TN;
  const int nk = (int)((g.K + 31) / 32);

  // Buffer resources end at each panel's last valid element, as in gemm_dma_kernel: rows of a
  // past M and rows of b past K read zeros; the chunks of a (and b^T) past K in the last
  // k-tile are fetched from the resource's end.
  const int rows_a = (int)(g.M - m0 < TM ? g.M - m0 : TM), cols_b = (int)(g.N - n0 < TN ? g.N - n0 : TN);
  const uint32_t a_end = (uint32_t)(((rows_a - 1) * g.sa_m + g.K) * 2);
  const u32x4 rsA = dma::rsrc((const uint16_t*)g.a + m0 * g.sa_m, a_end);
  const uint32_t b_end = BT ? (uint32_t)(((cols_b - 1) * g.sb_n + g.K) * 2) : (uint32_t)(((g.K - 1) * g.sb_k + cols_b) * 2);
  const u32x4 rsB = dma::rsrc((const uint16_t*)g.b + (BT ? n0 * g.sb_n : n0), b_end);
  int va[2], vb[2], va_last[2], vb_last[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int ra = 32 * wave + 16 * q + (lane >> 2);
    va[q] = (int)(ra * g.sa_m * 2) + dma::asw(ra, lane & 3) * 16;
    va_last[q] = (nk - 1) * 32 + dma::asw(ra, lane & 3) * 8 < g.K ? va[q] : (int)a_end;
    if constexpr (BT) {
      vb[q] = (int)(ra * g.sb_n * 2) + dma::asw(ra, lane & 3) * 16;
      vb_last[q] = (nk - 1) * 32 + dma::asw(ra, lane & 3) * 8 < g.K ? vb[q] : (int)b_end;
    } else {
      const int kb = 8 * wave + 4 * q + (lane >> 4);
      const int nb = 32 * (((lane & 15) >> 2) ^ dma128::bsw(kb)) + 8 * (lane & 3);
      vb[q] = (int)(kb * g.sb_k * 2) + nb * 2;
      vb_last[q] = vb[q];
    }
  }
  const int b_kstep = BT ? 64 : (int)(32 * g.sb_k * 2);
  // Load u (0..3) of tile kt into its stage: a q0, b q0, a q1, b q1 (1 KiB each).
  auto load_unit = [&](int u, int kt) {
    const int st = (kt % dma::STAGES) * dma128::STAGE, q = u >> 1;
    if ((u & 1) == 0)
      dma::load_lds16(rsA, lds0 + st + 2048 * wave + 1024 * q, kt == nk - 1 ? va_last[q] : va[q], kt * 64);
    else
      dma::load_lds16(rsB, lds0 + dma128::B0 + st + 2048 * wave + 1024 * q, kt == nk - 1 ? vb_last[q] : vb[q],
                      kt * b_kstep);
  };

  // Fragment reads.  a: row 64 wm + 32 i + lane % 32 (i at + 2048 i), chunk 2 s + lane / 32.
  // b: lane (group gq = lane / 16, r, q) reads row 16 s + 8 (gq / 2) + 4 half + r at columns
  // 64 wn + 32 j + 16 (gq % 2) + 4 q .. + 3 (rows 16 s at + 4096 s, the half at + 1024).
  int a_rd[2], b_rd[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const int row = wm * 64 + (lane & 31);
    a_rd[s2] = row * 64 + dma::asw(row, 2 * s2 + (lane >> 5)) * 16;
  }
  if constexpr (BT) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int row = wn * 64 + (lane & 31);
      b_rd[s2] = dma128::B0 + row * 64 + dma::asw(row, 2 * s2 + (lane >> 5)) * 16;
    }
  } else {
    const int gq = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      b_rd[j] = dma128::B0 + (8 * (gq >> 1) + r) * 256 + (((2 * wn + j) ^ r) * 64) + (16 * (gq & 1) + 4 * q) * 2;
  }
  typedef typename mfma_traits<T>::frag frag;
  frag fa[2][2], fb[2][2];
  // Unit x (0..3) of slice s2 of the tile at stage offset st, in the order the slice's MFMAs
  // consume them: a0, b0, b1, a1.
  auto read_unit = [&](int x, int s2, int st) {
    if (x == 0 || x == 3) {
      const int i = x == 0 ? 0 : 1;
      fa[s2][i] = *(const frag*)(lds + a_rd[s2] + st + i * 2048);
    } else if constexpr (BT) {
      const int j = x - 1;
      fb[s2][j] = *(const frag*)(lds + b_rd[s2] + st + j * 2048);
    } else {
      const int j = x - 1;
      const char* p = lds + b_rd[j] + st + s2 * 4096;
      const dma::v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) dma::v4i16*)p);
      const dma::v4i16 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) dma::v4i16*)(p + 1024));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      fb[s2][j] = __builtin_bit_cast(frag, u32x4{l2[0], l2[1], h2[0], h2[1]});
    }
  };

  floatx16 acc[2][2];
  zero_acc(acc);

  // nk >= 3 (the launcher checks): tiles 0..2 in flight, wait for tile 0.
  for (int kt = 0; kt < 3; ++kt)
    for (int u = 0; u < 4; ++u) load_unit(u, kt);
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int x = 0; x < 4; ++x) read_unit(x, 0, 0);

#define NT_FENCE() __builtin_amdgcn_sched_barrier(0)
  // One k-tile, as gemm_dma_kernel's: HAS1 reads the next tile's slice 0 during slice 1, LOAD
  // fetches tile kt + 3 into the stage of tile kt - 1, VM the loads left in flight at the
  // barrier (-1: the last tile, no wait and no barrier).
  auto step = [&](auto has1_c, auto load_c, auto vm_c, int kt) {
    constexpr bool HAS1 = decltype(has1_c)::value, LOAD = decltype(load_c)::value;
    constexpr int VM = decltype(vm_c)::value;
    const int st = (kt % dma::STAGES) * dma128::STAGE, st1 = ((kt + 1) % dma::STAGES) * dma128::STAGE;
    static_for<0, 8>([&](auto m_c) {
      constexpr int m = decltype(m_c)::value;
      constexpr int s2 = m >> 2, x = m & 3;
      if constexpr (m == 4 && VM >= 0) {
        NT_FENCE();
        if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        NT_FENCE();
      }
      acc[x >> 1][x & 1] = mfma_traits<T>::mma(fa[s2][x >> 1], fb[s2][x & 1], acc[x >> 1][x & 1]);
      NT_FENCE();
      if constexpr (s2 == 0)
        read_unit(x, 1, st);
      else if constexpr (HAS1)
        read_unit(x, 0, st1);
      if constexpr (s2 == 1 && LOAD) load_unit(x, kt + 3);
      NT_FENCE();
    });
  };
#undef NT_FENCE
  using T1 = std::integral_constant<bool, true>;
  using F1 = std::integral_constant<bool, false>;
  using V4 = std::integral_constant<int, 4>;
  using V0 = std::integral_constant<int, 0>;
  using VN = std::integral_constant<int, -1>;
  int kt = 0;
  for (; kt + 3 < nk; ++kt) step(T1{}, T1{}, V4{}, kt);
  step(T1{}, F1{}, V4{}, kt);
  step(T1{}, F1{}, V0{}, kt + 1);
  step(F1{}, F1{}, VN{}, kt + 2);

  dma_fast_epilogue<2, true, 2, dma128::EPI>(g, acc, lds, wave, lane, m0 + wm * 64, n0 + wn * 64);
}

// Few rows (M <= 64) against k-contiguous b (b^T rows, x @ w.t(): a linear layer on a few
// tokens).  The product reads b once and is bound by streaming it, which the 128-wide tiles
// spread over too few workgroups (N / 128).  Here a workgroup owns 32 columns (32 rows of
// b^T) and one 32-row block of a (blockIdx.y); its eight waves take contiguous eighths of K
// and load their MFMA fragments straight from memory (a lane's row of a, or column of b, at
// k 8 (lane / 32) .. + 7 of each 16-deep step: 16 bytes per operand), four steps in flight.
// The eight partial 32 x 32 tiles are then summed through LDS and finished element by
// element (alpha, round, beta c, any out type).  One row block per workgroup rather than
// both in one: 64 x 4096 x 4096 fp16 18.8 against 26.9 us (more workgroups, half the work
// each).
namespace skinny {
constexpr int NW = 8, STEPS = 4;
}  // namespace skinny

template <typename T>
__global__ __launch_bounds__(64 * skinny::NW) void gemm_skinny_kernel(GemmArgs g) {
  constexpr int MB = 1;  // 32-row blocks of a per workgroup
  __shared__ float part[skinny::NW * MB * 16 * 64];
  const int64_t m0 = 32 * (int64_t)blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = (int64_t)blockIdx.x * 32;
  const int nsteps = (int)((g.K + 15) / 16);
  const int per = (nsteps + skinny::NW - 1) / skinny::NW;
  const int s0 = wave * per, s1 = min(nsteps, s0 + per);
  const int kl = 8 * (lane >> 5);
  const int64_t n = n0 + (lane & 31);
  const bool n_ok = n < g.N;
  const uint16_t* brow = (const uint16_t*)g.b + (n_ok ? n : 0) * g.sb_n + kl;
  const uint16_t* arow[MB];
  bool m_ok[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int64_t m = m0 + 32 * i + (lane & 31);
    m_ok[i] = m < g.M;
    arow[i] = (const uint16_t*)g.a + (m_ok[i] ? m : 0) * g.sa_m + kl;
  }
  typedef typename mfma_traits<T>::frag frag;
  // Step s: this lane's 8 k of a row of each a block and of a column of b (zeros past M, N, K;
  // K is a multiple of 8, so a lane's 8 k are all inside or all outside).
  auto load = [&](int st, frag (&fa)[MB], frag& fb) {
    const int64_t k = (int64_t)st * 16;
    const bool k_ok = k + kl < g.K;
    const u32x4 z = {0u, 0u, 0u, 0u};
    fb = __builtin_bit_cast(frag, n_ok && k_ok ? *(const u32x4*)(brow + k) : z);
#pragma unroll
    for (int i = 0; i < MB; ++i) fa[i] = __builtin_bit_cast(frag, m_ok[i] && k_ok ? *(const u32x4*)(arow[i] + k) : z);
  };
  floatx16 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  frag fa[skinny::STEPS][MB], fb[skinny::STEPS];
#pragma unroll
  for (int j = 0; j < skinny::STEPS; ++j)
    if (s0 + j < s1) load(s0 + j, fa[j], fb[j]);
  for (int st = s0; st < s1; st += skinny::STEPS) {
#pragma unroll
    for (int j = 0; j < skinny::STEPS; ++j) {
      if (st + j < s1) {
#pragma unroll
        for (int i = 0; i < MB; ++i) acc[i] = mfma_traits<T>::mma(fa[j][i], fb[j], acc[i]);
        if (st + j + skinny::STEPS < s1) load(st + j + skinny::STEPS, fa[j], fb[j]);
      }
    }
  }
  // Sum the eight waves' partial tiles: acc[i][r] of lane l is C[32 i + acc_row(r, l)][n0 + l % 32].
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) part[((wave * MB + i) * 16 + r) * 64 + lane] = acc[i][r];
  __syncthreads();
  for (int e = tid; e < MB * 16 * 64; e += 64 * skinny::NW) {
    const int l = e & 63, ir = e >> 6, i = ir >> 4, r = ir & 15;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < skinny::NW; ++w) v += part[((w * MB + i) * 16 + r) * 64 + l];
    const int64_t row = m0 + 32 * i + acc_row(r, l), col = n0 + (l & 31);
    if (row < g.M && col < g.N) {
      float out = g.alpha * round_through(v, g.round_dtype);
      if (g.c) out += g.beta * load_c<false>(g, row * g.sc_m + col * g.sc_n);
      store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, out);
    }
  }
}

// ----------------------------------------------------------------------------- fp32
constexpr int F32_TM = 32, F32_TN = 32, F32_KC = 256;
constexpr int F32_AS = F32_KC + 4;  // a chunk row stride (floats): 16-byte aligned rows
constexpr int F32_BS = F32_TN + 16;  // b chunk row stride: 32 lanes of one read hit 32 banks

// fp32: 32 x 32 output tile per workgroup, four waves of 16 x 16 on
// v_mfma_f32_16x16x4f32.  K is staged through LDS in chunks of 256 with 16-byte loads
// (a 512-deep reduction takes two load phases instead of sixteen).
template <bool VEC>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float sA[F32_TM * F32_AS];
  __shared__ __attribute__((aligned(16))) float sB[F32_KC * F32_BS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tm = blockIdx.x / g.tiles_n, tn = blockIdx.x % g.tiles_n;
  const int64_t m0 = (int64_t)tm * F32_TM, n0 = (int64_t)tn * F32_TN;
  const int wm = wave >> 1, wn = wave & 1;
  const float* A = (const float*)g.a;
  const float* B = (const float*)g.b;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f}, acc1 = acc, acc2 = acc, acc3 = acc;
  for (int64_t k0 = 0; k0 < g.K; k0 += F32_KC) {
    if (VEC) {  // full tiles, unit inner strides, 16-byte aligned rows
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int e = it * 256 + tid;  // a: 32 rows x 64 float4
        const int r = e >> 6, c4 = e & 63;
        const int64_t k = k0 + c4 * 4;
        float4 v = {0.f, 0.f, 0.f, 0.f};
        if (k < g.K) v = *(const float4*)(A + (m0 + r) * g.sa_m + k);
        *(float4*)(sA + r * F32_AS + c4 * 4) = v;
      }
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int e = it * 256 + tid;  // b: 256 rows x 8 float4
        const int kk = e >> 3, c4 = e & 7;
        const int64_t k = k0 + kk;
        float4 v = {0.f, 0.f, 0.f, 0.f};
        if (k < g.K) v = *(const float4*)(B + k * g.sb_k + n0 + c4 * 4);
        *(float4*)(sB + kk * F32_BS + c4 * 4) = v;
      }
    } else {
      for (int e = tid; e < F32_TM * F32_KC; e += 256) {
        const int r = e / F32_KC, kk = e % F32_KC;
        const int64_t m = m0 + r, k = k0 + kk;
        sA[r * F32_AS + kk] = (m < g.M && k < g.K) ? A[m * g.sa_m + k * g.sa_k] : 0.f;
      }
      for (int e = tid; e < F32_KC * F32_TN; e += 256) {
        const int kk = e / F32_TN, c = e % F32_TN;
        const int64_t n = n0 + c, k = k0 + kk;
        sB[kk * F32_BS + c] = (n < g.N && k < g.K) ? B[k * g.sb_k + n * g.sb_n] : 0.f;
      }
    }
    __syncthreads();
    const int kmax = (int)((g.K - k0 < F32_KC) ? (g.K - k0) : F32_KC);
    const float* ap = sA + (wm * 16 + (lane & 15)) * F32_AS + (lane >> 4);
    const float* bp = sB + (lane >> 4) * F32_BS + wn * 16 + (lane & 15);
    int kk = 0;
    for (; kk + 16 <= kmax; kk += 16) {  // four independent accumulator chains
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ap[kk], bp[kk * F32_BS], acc, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ap[kk + 4], bp[(kk + 4) * F32_BS], acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(ap[kk + 8], bp[(kk + 8) * F32_BS], acc2, 0, 0, 0);
      acc3 = __builtin_amdgcn_mfma_f32_16x16x4f32(ap[kk + 12], bp[(kk + 12) * F32_BS], acc3, 0, 0, 0);
    }
    for (; kk < kmax; kk += 4) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ap[kk], bp[kk * F32_BS], acc, 0, 0, 0);
    __syncthreads();
  }
  acc = (acc + acc1) + (acc2 + acc3);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = m0 + wm * 16 + (lane >> 4) * 4 + r;
    const int64_t col = n0 + wn * 16 + (lane & 15);
    if (row < g.M && col < g.N) {
      float v = g.alpha * round_through(acc[r], g.round_dtype);
      if (g.c) v += g.beta * load_c<false>(g, row * g.sc_m + col * g.sc_n);
      store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
    }
  }
}

// fp32 GEMMs of at most a few hundred 32 x 32 tiles (e.g. 512^3): one tile per
// workgroup of eight waves, each wave multiplying an eighth of K with its operands
// loaded straight into registers, then the eight partial tiles summed through LDS, two
// outputs per lane.  (Sixteen waves of one 32-deep chunk each measured 10.4 us median at
// 512^3 against 9.9-10.0 for eight; four were no faster.)  MFMA step s of a 32-deep k chunk
// uses k = 8 t + s in lane group t (the sum is over all k, so any bijection will do), so a
// lane's a values for the chunk are eight consecutive floats of one row.
constexpr int F32S_WAVES = 8;
template <bool AVEC>
__global__ __launch_bounds__(64 * F32S_WAVES) void gemm_f32_splitk_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float part[F32S_WAVES * F32_TM * F32_TN];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tm = blockIdx.x / g.tiles_n, tn = blockIdx.x % g.tiles_n;
  const int64_t m0 = (int64_t)tm * F32_TM, n0 = (int64_t)tn * F32_TN;
  const float* A = (const float*)g.a;
  const float* B = (const float*)g.b;
  const int r16 = lane & 15, t = lane >> 4;
  const int64_t chunks = (g.K + 31) / 32;
  const int64_t per = (chunks + F32S_WAVES - 1) / F32S_WAVES;
  const int64_t c_lo = wave * per, c_hi = min(chunks, c_lo + per);
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Two chunks per step, all their loads issued before the first MFMA: the second chunk's
  // fetch latency hides behind the first's (512^3: one step per wave; 0.8 us less per call
  // than loading and multiplying one chunk at a time).  A chunk at or past c_hi reads zeros.
  for (int64_t ch0 = c_lo; ch0 < c_hi; ch0 += 2) {
    float a[2][2][8], b[2][2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool live = ch0 + h < c_hi;
      const int64_t kb = (ch0 + h) * 32 + 8 * t;  // this lane group's eight k values: kb .. kb + 7
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t row = m0 + i * 16 + r16;
        if (AVEC && live && row < g.M && kb + 8 <= g.K) {
          const float4 lo = *(const float4*)(A + row * g.sa_m + kb);
          const float4 hi = *(const float4*)(A + row * g.sa_m + kb + 4);
          a[h][i][0] = lo.x; a[h][i][1] = lo.y; a[h][i][2] = lo.z; a[h][i][3] = lo.w;
          a[h][i][4] = hi.x; a[h][i][5] = hi.y; a[h][i][6] = hi.z; a[h][i][7] = hi.w;
        } else {
#pragma unroll
          for (int s = 0; s < 8; ++s)
            a[h][i][s] = (live && row < g.M && kb + s < g.K) ? A[row * g.sa_m + (kb + s) * g.sa_k] : 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + j * 16 + r16;
#pragma unroll
        for (int s = 0; s < 8; ++s)
          b[h][j][s] = (live && col < g.N && kb + s < g.K) ? B[(kb + s) * g.sb_k + col * g.sb_n] : 0.f;
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[h][i][s], b[h][j][s], acc[i][j], 0, 0, 0);
  }
  // 16 x 16 blocks: lane l holds rows 4 (l / 16) + v, column l % 16.
  float* mine = part + wave * (F32_TM * F32_TN);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) mine[(i * 16 + 4 * t + v) * F32_TN + j * 16 + r16] = acc[i][j][v];
  __syncthreads();
  for (int e = tid; e < F32_TM * F32_TN; e += 64 * F32S_WAVES) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < F32S_WAVES; ++w) sum += part[w * (F32_TM * F32_TN) + e];
    const int64_t row = m0 + e / F32_TN, col = n0 + e % F32_TN;
    if (row < g.M && col < g.N) {
      float v = g.alpha * round_through(sum, g.round_dtype);
      if (g.c) v += g.beta * load_c<false>(g, row * g.sc_m + col * g.sc_n);
      store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
    }
  }
}

// gemm_f32_splitk_kernel for whole tiles: M, N multiples of 32, K of 512 (every wave takes
// an even number of 32-deep chunks), a and b with unit inner strides, 16-byte aligned a
// rows, byte offsets within 32 bits.  The tile is (blockIdx.y, blockIdx.x).  This kernel
// is latency-bound at 512^3 (a few microseconds, a third of it launch and drain), so it
// keeps to what shortens the path to the first load and from the last MFMA: no bounds
// checks, scalar address arithmetic, no division for the tile, and (PLAIN:
// alpha 1, no c, fp32 out without rounding, unit column stride) a bare store.  K512: K is
// exactly 512, two chunks per wave without a loop.
template <bool PLAIN, bool K512>
__global__ __launch_bounds__(64 * F32S_WAVES) void gemm_f32_splitk_full_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float part[F32S_WAVES * F32_TM * F32_TN];
  const int m0 = blockIdx.y * F32_TM, n0 = blockIdx.x * F32_TN;
  const int sa = (int)g.sa_m, sb = (int)g.sb_k;
  const int tid = threadIdx.x, lane = tid & 63, r16 = lane & 15, t = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int per = K512 ? 2 : (int)(g.K / (32 * F32S_WAVES));
  // Buffer loads: the per-lane part of each offset (voffset) is fixed, the part that
  // varies from load to load is wave-uniform and goes in soffset, so the scalar unit
  // computes every address and the vector unit only issues loads and MFMAs.
  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
      (void*)g.a, (short)0, (int)(((g.M - 1) * g.sa_m + g.K) * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(
      (void*)g.b, (short)0, (int)(((g.K - 1) * g.sb_k + g.N) * 4), 0x00020000);
  const int va = ((m0 + r16) * sa + 8 * t) * 4, vb = (8 * t * sb + n0 + r16) * 4;
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < per; c0 += 2) {
    float a[2][2][8], b[2][2][8];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int kb = (wave * per + c0 + c) * 32;  // wave-uniform
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int so = (i * 16 * sa + kb) * 4;
        const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(rsA, va, so, 0);
        const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(rsA, va + 16, so, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a[c][i][q] = __uint_as_float(lo[q]);
          a[c][i][4 + q] = __uint_as_float(hi[q]);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int s = 0; s < 8; ++s)
          b[c][j][s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsB, vb + j * 64, (kb + s) * sb * 4, 0));
      // the loads in issue order, first chunk then second, all ahead of the MFMAs: left
      // to itself the scheduler trades them for registers and waits on each in turn
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c][i][s], b[c][j][s], acc[i][j], 0, 0, 0);
  }
  float* mine = part + wave * (F32_TM * F32_TN);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) mine[(i * 16 + 4 * t + v) * F32_TN + j * 16 + r16] = acc[i][j][v];
  __syncthreads();
#pragma unroll
  for (int e = tid; e < F32_TM * F32_TN; e += 64 * F32S_WAVES) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < F32S_WAVES; ++w) sum += part[w * (F32_TM * F32_TN) + e];
    if (PLAIN) {
      ((float*)g.out)[(m0 + e / F32_TN) * (int)g.so_m + n0 + e % F32_TN] = sum;
    } else {
      const int64_t row = m0 + e / F32_TN, col = n0 + e % F32_TN;
      float v = g.alpha * round_through(sum, g.round_dtype);
      if (g.c) v += g.beta * load_c<false>(g, row * g.sc_m + col * g.sc_n);
      store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
    }
  }
}

// fp32 GEMMs of more tiles (1024^2 and up) on v_mfma_f32_32x32x2_f32: 256 lanes in a 2 x 2
// grid of waves, each owning (32 WI) x (32 WJ) of the (64 WI) x (64 WJ) tile.  K in
// 16-deep chunks, double-buffered in LDS and staged through registers (the next chunk's
// 16-byte loads are in flight while this one is multiplied; one barrier per chunk).  MFMA
// step s of a chunk takes k = 8 h + s in lane half h (the sum runs over all k, so any
// bijection will do): a lane's a values for the chunk are then 8 consecutive floats of one
// row (two ds_read_b128), its b values 8 floats of one column (ds_read_b32, consecutive
// lanes on consecutive banks).  a rows are padded to 20 floats (16 lanes of a 16-byte read
// on 16 distinct bank quads), b rows to BN + 4 floats (the two lane halves 8 rows apart
// on different banks).  M, N, K may be ragged; N and K multiples of 4 (16-byte loads).
constexpr int F32M_KC = 16, F32M_AS = F32M_KC + 4;
template <int WI, int WJ>
__global__ __launch_bounds__(256) void gemm_f32_mfma_kernel(GemmArgs g) {
  constexpr int BM = 64 * WI, BN = 64 * WJ, BS = BN + 4;
  constexpr int A_F4 = BM * F32M_KC / 4 / 256, B_F4 = F32M_KC * BN / 4 / 256;  // float4 per lane per chunk
  constexpr int A_ELEMS = BM * F32M_AS, B_ELEMS = F32M_KC * BS;
  constexpr int EPI_ELEMS = 4 * 32 * WJ * 32;  // gemm_epilogue's staging (fp32)
  constexpr int LDS_ELEMS = 2 * (A_ELEMS + B_ELEMS) > EPI_ELEMS ? 2 * (A_ELEMS + B_ELEMS) : EPI_ELEMS;
  __shared__ __attribute__((aligned(16))) float lds[LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const float* A = (const float*)g.a;
  const float* B = (const float*)g.b;
  const int nk = (int)((g.K + F32M_KC - 1) / F32M_KC);

  float4 ra[A_F4], rb[B_F4];
  auto load = [&](int kt) {
    const int64_t k0 = (int64_t)kt * F32M_KC;
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int e = i * 256 + tid, row = e >> 2, c4 = e & 3;
      const int64_t m = m0 + row, k = k0 + c4 * 4;
      ra[i] = (m < g.M && k < g.K) ? *(const float4*)(A + m * g.sa_m + k) : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int e = i * 256 + tid, kk = e / (BN / 4), c4 = e % (BN / 4);
      const int64_t k = k0 + kk, n = n0 + c4 * 4;
      rb[i] = (k < g.K && n < g.N) ? *(const float4*)(B + k * g.sb_k + n) : float4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store = [&](int buf) {
    float* sA = lds + buf * (A_ELEMS + B_ELEMS);
    float* sB = sA + A_ELEMS;
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int e = i * 256 + tid, row = e >> 2, c4 = e & 3;
      *(float4*)(sA + row * F32M_AS + c4 * 4) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int e = i * 256 + tid, kk = e / (BN / 4), c4 = e % (BN / 4);
      *(float4*)(sB + kk * BS + c4 * 4) = rb[i];
    }
  };
  floatx16 acc[WI][WJ];
  zero_acc(acc);
  const int r32 = lane & 31, hf = lane >> 5;
  auto compute = [&](int buf) {
    const float* sA = lds + buf * (A_ELEMS + B_ELEMS);
    const float* sB = sA + A_ELEMS;
    float a[WI][8], b[WJ][8];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const float* p = sA + (wm * WI * 32 + i * 32 + r32) * F32M_AS + 8 * hf;
      const float4 lo = *(const float4*)p, hi = *(const float4*)(p + 4);
      a[i][0] = lo.x; a[i][1] = lo.y; a[i][2] = lo.z; a[i][3] = lo.w;
      a[i][4] = hi.x; a[i][5] = hi.y; a[i][6] = hi.z; a[i][7] = hi.w;
    }
#pragma unroll
    for (int j = 0; j < WJ; ++j)
#pragma unroll
      for (int st = 0; st < 8; ++st) b[j][st] = sB[(8 * hf + st) * BS + wn * WJ * 32 + j * 32 + r32];
#pragma unroll
    for (int st = 0; st < 8; ++st)
#pragma unroll
      for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][st], b[j][st], acc[i][j], 0, 0, 0);
  };

  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load(kt + 1);
    compute(kt & 1);
    if (kt + 1 < nk) store((kt + 1) & 1);
    __syncthreads();
  }
  gemm_epilogue<WI, WJ>(g, acc, (uint16_t*)lds, wave, lane, m0 + wm * WI * 32, n0 + wn * WJ * 32);
}

static int gemm_check(const GemmArgs& g) {
  if (g.M < 0 || g.N < 0 || g.K < 0) return NT_ERR_INVALID;
  if (!valid_dtype(g.out_dtype) || !valid_round(g.round_dtype)) return NT_ERR_INVALID;
  if (!valid_dtype(g.c_dtype) && g.c_dtype != NT_DTYPE_E5M2 && g.c_dtype != NT_DTYPE_E4M3) return NT_ERR_INVALID;
  return 0;
}

// K == 0: out = cast(beta * c + alpha * round(0)).
__global__ void gemm_k0_kernel(GemmArgs g) {
  const int64_t total = g.M * g.N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / g.N, col = e % g.N;
    float v = 0.f;
    if (g.c) v += g.beta * load_c<true>(g, row * g.sc_m + col * g.sc_n);
    store_from_float(g.out, row * g.so_m + col * g.so_n, g.out_dtype, v);
  }
}

// config: 0 = the fastest kernel whose conditions hold; 1 = the DMA kernel, 2 = the
// register-staged eight-wave kernel, 3 = the element-wise loader kernel (any strides), 4 =
// the DMA kernel on 128 x 128 tiles, 5 = the few-rows kernel (M <= 64, b^T rows): a forced
// kernel whose conditions do not hold is rejected before anything is launched.  Config 0 takes the 128 x 128 tiles when they fit
// and the output has fewer than DMA128_BELOW tiles of 256 x 256: measured fp16, the
// 128-wide kernel wins up to 128 such tiles (2048^3 729 against 412 TFLOP/s, 8192 x 1024 x
// 8192 814 against 770) and loses from 144 (3072^3 681 against 849).
constexpr int64_t DMA128_BELOW = 136;
template <typename T>
static int gemm16_launch(GemmArgs g, hipStream_t stream, int config = 0) {
  if (config < 0 || config > 5) return NT_ERR_INVALID;
  if (int e = gemm_check(g)) return e;
  if (!valid_dtype(g.c_dtype)) return NT_ERR_INVALID;  // an fp8 c goes with fp8 operands
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
  // (row strides non-negative: the DMA kernels address panels with unsigned 32-bit offsets)
  const bool aligned = g.sa_k == 1 && g.sb_n == 1 && g.sa_m >= 0 && g.sb_k >= 0 && (uintptr_t)g.a % 16 == 0 &&
                       (uintptr_t)g.b % 16 == 0 &&
                       (g.sa_m * 2) % 16 == 0 && (g.sb_k * 2) % 16 == 0;
  const bool fast = aligned && g.M % GB_M == 0 && g.N % GB_N == 0 && g.K % GB_K == 0;
  const dim3 grid((unsigned)(tiles_m * tiles_n)), blk(G_THREADS);
  // DMA kernel: operand panel offsets fit its 32-bit buffer offsets and K holds at least the
  // three 32-deep k-tiles its pipeline keeps in flight.  M may be ragged; N and K must be
  // multiples of 8, so that every 16-byte operand chunk lies wholly inside or wholly past
  // the matrix (its buffer resources return zeros past the end, per chunk).
  const bool dma_nn = aligned && g.N % 8 == 0 && g.K % 8 == 0 && (GB_M - 1) * g.sa_m + g.K <= 0x3fffffffLL &&
                      (g.K - 1) * g.sb_k + GB_N <= 0x3fffffffLL && g.K >= 3 * 32;
  // ... or with b k-contiguous (b^T rows, as a's): any N.
  const bool dma_bt = g.sa_k == 1 && g.sb_k == 1 && g.sa_m >= 0 && (uintptr_t)g.a % 16 == 0 && (uintptr_t)g.b % 16 == 0 &&
                      (g.sa_m * 2) % 16 == 0 && (g.sb_n * 2) % 16 == 0 && g.sb_n > 0 && g.K % 8 == 0 &&
                      (GB_M - 1) * g.sa_m + g.K <= 0x3fffffffLL && (GB_N - 1) * g.sb_n + g.K <= 0x3fffffffLL &&
                      g.K >= 3 * 32 && !dma_nn;
  const bool dma_ok = dma_nn || dma_bt;
  // Its fast epilogue: 16-byte out vectors, and c (if any) fetched with 32-bit buffer offsets.
  const bool out_vec = g.out_dtype != NT_DTYPE_F32 && g.so_n == 1 && g.so_m >= 0 && g.so_m % 8 == 0 &&
                       (uintptr_t)g.out % 16 == 0;
  const bool c_vec = !g.c || (g.c_dtype == g.out_dtype && g.sc_n == 1 && g.sc_m >= 0 && g.sc_m % 8 == 0 && (uintptr_t)g.c % 16 == 0 &&
                              127 * g.sc_m + 128 <= 0x3fffffffLL);
  // gemm_dma128_kernel: the same conditions on 128 x 128 tiles, with the fast epilogue only.
  const bool dma128_nn = aligned && g.N % 8 == 0 && g.K % 8 == 0 && 127 * g.sa_m + g.K <= 0x3fffffffLL &&
                         (g.K - 1) * g.sb_k + 128 <= 0x3fffffffLL && g.K >= 3 * 32;
  const bool dma128_bt = g.sa_k == 1 && g.sb_k == 1 && g.sa_m >= 0 && (uintptr_t)g.a % 16 == 0 &&
                         (uintptr_t)g.b % 16 == 0 && (g.sa_m * 2) % 16 == 0 && (g.sb_n * 2) % 16 == 0 && g.sb_n > 0 &&
                         g.K % 8 == 0 && 127 * g.sa_m + g.K <= 0x3fffffffLL && 127 * g.sb_n + g.K <= 0x3fffffffLL &&
                         g.K >= 3 * 32 && !dma128_nn;
  const int64_t tiles128 = cdiv(g.M, 128) * cdiv(g.N, 128);
  const bool ok128 = (dma128_nn || dma128_bt) && out_vec && c_vec && g.N % 8 == 0 && tiles128 <= 0x7fffffffLL;
  // gemm_skinny_kernel: at most 64 rows, a and b^T rows k-contiguous with 16-byte aligned rows.
  const bool skinny = g.M <= 64 && g.sa_k == 1 && g.sb_k == 1 && g.sa_m >= 0 && g.sb_n > 0 && (uintptr_t)g.a % 16 == 0 &&
                      (uintptr_t)g.b % 16 == 0 && g.sa_m % 8 == 0 && g.sb_n % 8 == 0 && g.K % 8 == 0 &&
                      cdiv(g.N, 32) <= 0x7fffffffLL;
  if ((config == 1 && !dma_ok) || (config == 2 && !fast) || (config == 4 && !ok128) || (config == 5 && !skinny))
    return NT_ERR_INVALID;
  // Default: up to 32 rows, or up to 64 with N <= 4096; past 32 rows with wide N the 128-wide
  // tiles win (fp16, interleaved medians, few-rows / 128-wide / torch: 1 x 4096 x 4096
  // 11.6 / 29.4 / 21.4 us; 16 x 4096 x 4096 14.8 / 30.3 / 19.9; 8 x 11008 x 4096 26.9 / 32.1 /
  // 21.6; 64 x 4096 x 4096 18.8 / 32.6 / 21.4; 64 x 4096 x 11008 48.2 / 84.2 / 30.5; 33 x 11008 x
  // 4096 47.6 / 33.1 / 21.7).
  if (config == 5 || (config == 0 && skinny && (g.M <= 32 || g.N <= 4096))) {
    const dim3 gridS((unsigned)cdiv(g.N, 32), (unsigned)cdiv(g.M, 32));
    hipLaunchKernelGGL((gemm_skinny_kernel<T>), gridS, dim3(64 * skinny::NW), 0, stream, g);
    return launch_status();
  }
  if (config == 4 || (config == 0 && ok128 && tiles_m * tiles_n < DMA128_BELOW)) {
    g.tiles_m = (int)cdiv(g.M, 128);
    g.tiles_n = (int)cdiv(g.N, 128);
    g.c_pre = 1;
    const dim3 grid128((unsigned)tiles128);
    if (dma128_bt)
      hipLaunchKernelGGL((gemm_dma128_kernel<T, true>), grid128, dim3(256), 0, stream, g);
    else
      hipLaunchKernelGGL((gemm_dma128_kernel<T, false>), grid128, dim3(256), 0, stream, g);
    return launch_status();
  }
  const bool use_dma = config == 0 ? dma_ok : config == 1;
  const bool use_fast8 = config == 0 ? fast && !dma_ok : config == 2;
  g.c_pre = use_dma && out_vec && c_vec && g.N % 8 == 0;
  if (use_dma && dma_bt) {
    if (g.c_pre)
      hipLaunchKernelGGL((gemm_dma_kernel<T, true, true>), grid, dim3(512), 0, stream, g);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<T, false, true>), grid, dim3(512), 0, stream, g);
  } else if (use_dma && g.c_pre)
    hipLaunchKernelGGL((gemm_dma_kernel<T, true>), grid, dim3(512), 0, stream, g);
  else if (use_dma)
    hipLaunchKernelGGL((gemm_dma_kernel<T, false>), grid, dim3(512), 0, stream, g);
  else if (use_fast8)
    hipLaunchKernelGGL((gemm_fast8_kernel<T>), grid, dim3(512), 0, stream, g);
  else
    hipLaunchKernelGGL((gemm_mfma_kernel<T, false>), grid, blk, 0, stream, g);
  return launch_status();
}

// fp8 operands (any strides): the element-wise loader widens them to fp16.
// fp8 operands at the fp8 matrix rate: v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales
// (E8M0 127), FMT 0 = e4m3fn, 1 = e5m2 (the OCP formats the instruction takes).  a [m][k]
// and b^T [n][k] both k-contiguous (b column-major), M and N multiples of 256, K of 64 and
// at least 192.  The structure of gemm_dma_kernel with 64-byte k-tiles (64 elements): the
// same four-stage LDS ring filled by DMA, a and b^T rows alike with the XOR chunk swizzle.
// An MFMA operand lane holds row (column) lane % 32 at k = 32 (lane / 32) .. + 31 (checked
// on the device against an integer product), i.e. two ds_read_b128 of LDS chunks
// 2 (lane / 32) and 2 (lane / 32) + 1.  Per k-tile a wave issues eight MFMAs (its 4 x 2
// blocks of 32 x 32); the next tile's b fragments go to a second set, its a fragments
// replace each a fragment right after the tile's last MFMA that reads it.
// FAST_EPI as in gemm_dma_kernel (the 32 KiB past the operand stages are its staging).
template <int FMT, bool FAST_EPI>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_f8_dma_kernel(GemmArgs g) {
  typedef int v8i __attribute__((ext_vector_type(8)));
  __shared__ __attribute__((aligned(1024))) char lds[dma::EPI + (FAST_EPI ? 8 * 4096 : 0)];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  int tm, tn;
  tile_of(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * GB_M, n0 = (int64_t)tn * GB_N;
  const int nk = (int)(g.K / 64);

  // Global side: byte offsets within each operand's 256-row panel fit in 32 bits (checked on
  // the host).  Load q (0, 1) of this wave per k-tile: rows 32 wave + 16 q + lane / 4 of
  // each operand, LDS chunk lane % 4 holding global chunk asw(row, lane % 4).
  const u32x4 rsA = dma::rsrc((const uint8_t*)g.a + m0 * g.sa_m, (uint32_t)((GB_M - 1) * g.sa_m + g.K));
  const u32x4 rsB = dma::rsrc((const uint8_t*)g.b + n0 * g.sb_n, (uint32_t)((GB_N - 1) * g.sb_n + g.K));
  int va[2], vb[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r = 32 * wave + 16 * q + (lane >> 2);
    const int ch = dma::asw(r, lane & 3) * 16;
    va[q] = (int)(r * g.sa_m) + ch;
    vb[q] = (int)(r * g.sb_n) + ch;
  }
  // Load u (0..3) of tile kt into its stage: a q0, b q0, a q1, b q1.
  auto load_unit = [&](int u, int kt) {
    const int st = (kt % dma::STAGES) * dma::STAGE, q = u >> 1;
    if ((u & 1) == 0)
      dma::load_lds16(rsA, lds0 + st + 2048 * wave + 1024 * q, va[q], kt * 64);
    else
      dma::load_lds16(rsB, lds0 + dma::B0 + st + 2048 * wave + 1024 * q, vb[q], kt * 64);
  };

  // Fragment reads: a rows 128 wm + 32 i + lane % 32, b^T rows 64 wn + 32 j + lane % 32, the
  // lane's chunks 2 (lane / 32) + c (the swizzle depends on lane % 32 only, so block i or j
  // is 2048 bytes further).
  int a_rd[2], b_rd[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int ra = wm * 128 + (lane & 31), rb = wn * 64 + (lane & 31);
    a_rd[c] = ra * 64 + dma::asw(ra, 2 * (lane >> 5) + c) * 16;
    b_rd[c] = dma::B0 + rb * 64 + dma::asw(rb, 2 * (lane >> 5) + c) * 16;
  }
  auto frag = [&](const int (&rd)[2], int st, int blk) {
    const u32x4 lo = *(const u32x4*)(lds + rd[0] + st + blk * 2048);
    const u32x4 hi = *(const u32x4*)(lds + rd[1] + st + blk * 2048);
    return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  // The next tile's b fragments and its last-used a fragment (fa[3]) go into spare
  // registers, so that every read of the next tile is issued two MFMAs before this tile
  // ends (a read into fa[3] itself would have to follow this tile's last MFMA and leave its
  // latency exposed at the next tile's first wait).
  v8i fa[4], fb[2], fbn[2], fa3n;
  floatx16 acc[4][2];
  zero_acc(acc);

  // nk >= 3 (the launcher checks): tiles 0..2 in flight, wait for tile 0.
  for (int kt = 0; kt < 3; ++kt)
    for (int u = 0; u < 4; ++u) load_unit(u, kt);
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) fa[i] = frag(a_rd, 0, i);
#pragma unroll
  for (int j = 0; j < 2; ++j) fb[j] = frag(b_rd, 0, j);

#define NT_F8FENCE() __builtin_amdgcn_sched_barrier(0)
  // One k-tile.  HAS1: tile kt+1 exists (its fragments are read during this tile); LOAD:
  // fetch tile kt+3 (into the stage of tile kt-1, whose fragments were all read during
  // tile kt-2); VM: loads allowed outstanding once tile kt+1 has landed (-1: the last
  // tile, no wait and no barrier).
  auto step = [&](auto has1_c, auto load_c, auto vm_c, int kt) {
    constexpr bool HAS1 = decltype(has1_c)::value, LOAD = decltype(load_c)::value;
    constexpr int VM = decltype(vm_c)::value;
    const int st1 = ((kt + 1) % dma::STAGES) * dma::STAGE;
    static_for<0, 8>([&](auto m_c) {
      constexpr int m = decltype(m_c)::value;
      constexpr int i = m >> 1, j = m & 1;
      if constexpr (m == 0 && VM >= 0) {
        NT_F8FENCE();
        if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        NT_F8FENCE();
      }
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], FMT, FMT, 0, 127, 0, 127);
      NT_F8FENCE();
      if constexpr (HAS1) {
        if constexpr (m == 0) fbn[0] = frag(b_rd, st1, 0);
        if constexpr (m == 1) fbn[1] = frag(b_rd, st1, 1);
        if constexpr (m == 2) fa3n = frag(a_rd, st1, 3);
        if constexpr (j == 1 && i < 3) fa[i] = frag(a_rd, st1, i);
      }
      if constexpr (LOAD && m >= 1 && m <= 4) load_unit(m - 1, kt + 3);
      NT_F8FENCE();
    });
    if constexpr (HAS1) {
      fb[0] = fbn[0];
      fb[1] = fbn[1];
      fa[3] = fa3n;
    }
  };
#undef NT_F8FENCE
  using T1 = std::integral_constant<bool, true>;
  using F1 = std::integral_constant<bool, false>;
  using V4 = std::integral_constant<int, 4>;
  using V0 = std::integral_constant<int, 0>;
  using VN = std::integral_constant<int, -1>;
  int kt = 0;
  for (; kt + 3 < nk; ++kt) step(T1{}, T1{}, V4{}, kt);
  step(T1{}, F1{}, V4{}, kt);
  step(T1{}, F1{}, V0{}, kt + 1);
  step(F1{}, F1{}, VN{}, kt + 2);

  if constexpr (FAST_EPI)
    dma_fast_epilogue(g, acc, lds, wave, lane, m0 + wm * 128, n0 + wn * 64);
  else
    dma_any_epilogue<2, true>(g, acc, lds, wave, lane, m0 + wm * 128, n0 + wn * 64);
}

template <typename S>
static int gemm8_launch(GemmArgs g, hipStream_t stream) {
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
  // The fp8-rate kernel: a k-contiguous, b column-major (b^T k-contiguous), whole 256 x 256
  // tiles, 64-deep k-tiles (at least the three its pipeline keeps in flight), 16-byte
  // aligned rows and 32-bit panel offsets.
  const bool f8dma = g.sa_k == 1 && g.sb_k == 1 && g.M % GB_M == 0 && g.N % GB_N == 0 && g.K % 64 == 0 &&
                     g.K >= 3 * 64 && g.sa_m >= 0 && g.sb_n >= 0 && g.sa_m % 16 == 0 && g.sb_n % 16 == 0 &&
                     (uintptr_t)g.a % 16 == 0 && (uintptr_t)g.b % 16 == 0 &&
                     (GB_M - 1) * g.sa_m + g.K <= 0x3fffffffLL && (GB_N - 1) * g.sb_n + g.K <= 0x3fffffffLL;
  if (f8dma) {
    constexpr int fmt = std::is_same<S, src_e4m3>::value ? 0 : 1;
    // The fast epilogue: 16-bit out with unit column stride and aligned rows; c absent or of
    // out's type, fetched with 32-bit buffer offsets.
    const bool fast_epi = g.out_dtype != NT_DTYPE_F32 && g.so_n == 1 && g.so_m >= 0 && g.so_m % 8 == 0 &&
                          (uintptr_t)g.out % 16 == 0 &&
                          (!g.c || (g.c_dtype == g.out_dtype && g.sc_n == 1 && g.sc_m >= 0 && g.sc_m % 8 == 0 &&
                                    (uintptr_t)g.c % 16 == 0 && 127 * g.sc_m + 128 <= 0x3fffffffLL));
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    if (fast_epi)
      hipLaunchKernelGGL((gemm_f8_dma_kernel<fmt, true>), grid, dim3(512), 0, stream, g);
    else
      hipLaunchKernelGGL((gemm_f8_dma_kernel<fmt, false>), grid, dim3(512), 0, stream, g);
    return launch_status();
  }
  hipLaunchKernelGGL((gemm_mfma_kernel<f16_t, false, S>), dim3((unsigned)(tiles_m * tiles_n)), dim3(G_THREADS), 0,
                     stream, g);
  return launch_status();
}

static int gemm32_launch(GemmArgs g, hipStream_t stream) {
  if (int e = gemm_check(g)) return e;
  if (!valid_dtype(g.c_dtype)) return NT_ERR_INVALID;  // an fp8 c goes with fp8 operands
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
  // At most two tiles per CU: the split-k kernel (its LDS tile sum replaces a second load phase).
  if (tiles_m * tiles_n <= 512 && g.K >= 64) {
    const bool avec = g.sa_k == 1 && g.sa_m % 4 == 0 && (uintptr_t)g.a % 16 == 0;
    // whole-tile instance: byte offsets of a and b (buffer loads) within 32 bits
    const bool full = avec && g.sb_n == 1 && g.M % F32_TM == 0 && g.N % F32_TN == 0 && g.K % 512 == 0 &&
                      g.sa_m >= 0 && g.sb_k >= 0 && (g.M - 1) * g.sa_m + g.K < (1LL << 30) &&
                      (g.K - 1) * g.sb_k + g.N < (1LL << 30);
    if (full) {
      const bool plain = !g.c && g.alpha == 1.f && g.out_dtype == NT_DTYPE_F32 && g.round_dtype != NT_DTYPE_F16 &&
                         g.round_dtype != NT_DTYPE_BF16 &&
                         g.so_n == 1 && g.so_m >= 0 && (g.M - 1) * g.so_m + g.N < 0x7fffffffLL;
      const dim3 grid((unsigned)tiles_n, (unsigned)tiles_m), block(64 * F32S_WAVES);
      if (plain && g.K == 512)
        hipLaunchKernelGGL((gemm_f32_splitk_full_kernel<true, true>), grid, block, 0, stream, g);
      else if (plain)
        hipLaunchKernelGGL((gemm_f32_splitk_full_kernel<true, false>), grid, block, 0, stream, g);
      else if (g.K == 512)
        hipLaunchKernelGGL((gemm_f32_splitk_full_kernel<false, true>), grid, block, 0, stream, g);
      else
        hipLaunchKernelGGL((gemm_f32_splitk_full_kernel<false, false>), grid, block, 0, stream, g);
    } else if (avec)
      hipLaunchKernelGGL(gemm_f32_splitk_kernel<true>, dim3((unsigned)(tiles_m * tiles_n)), dim3(64 * F32S_WAVES), 0, stream, g);
    else
      hipLaunchKernelGGL(gemm_f32_splitk_kernel<false>, dim3((unsigned)(tiles_m * tiles_n)), dim3(64 * F32S_WAVES), 0, stream, g);
    return launch_status();
  }
  // More tiles: the MFMA kernel with 128 x 128 tiles when they alone fill the GPU, else 64 x 64.
  const bool mfma = g.sa_k == 1 && g.sb_n == 1 && g.N % 4 == 0 && g.K % 4 == 0 && g.sa_m % 4 == 0 && g.sb_k % 4 == 0 &&
                    (uintptr_t)g.a % 16 == 0 && (uintptr_t)g.b % 16 == 0;
  if (mfma) {
    const int64_t t128 = cdiv(g.M, 128) * cdiv(g.N, 128);
    if (t128 >= 256) {
      g.tiles_m = (int)cdiv(g.M, 128);
      g.tiles_n = (int)cdiv(g.N, 128);
      hipLaunchKernelGGL((gemm_f32_mfma_kernel<2, 2>), dim3((unsigned)t128), dim3(256), 0, stream, g);
    } else {
      g.tiles_m = (int)cdiv(g.M, 64);
      g.tiles_n = (int)cdiv(g.N, 64);
      hipLaunchKernelGGL((gemm_f32_mfma_kernel<1, 1>), dim3((unsigned)(g.tiles_m * g.tiles_n)), dim3(256), 0, stream, g);
    }
    return launch_status();
  }
  const bool vec = g.sa_k == 1 && g.sb_n == 1 && g.M % F32_TM == 0 && g.N % F32_TN == 0 && g.K % 4 == 0 &&
                   g.sa_m % 4 == 0 && g.sb_k % 4 == 0 && (uintptr_t)g.a % 16 == 0 && (uintptr_t)g.b % 16 == 0;
  if (vec)
    hipLaunchKernelGGL(gemm_f32_kernel<true>, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, stream, g);
  else
    hipLaunchKernelGGL(gemm_f32_kernel<false>, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, stream, g);
  return launch_status();
}

// A batch of 16-bit products out_i = round(a_i @ b_i) (a_i = a + i sa_b, and so on; no c,
// alpha 1) on gemm_dma128_kernel: conv2d's 1 x 1 filters over N-C-H-W images, a = the filter
// [K, C], b_i = image i [C, H W], out_i = output image i [K, P Q].  a k-contiguous, b and out
// row-major with 16-byte aligned rows, N and K multiples of 8, K at least 96, 16-bit out;
// NT_ERR_INVALID (nothing launched) otherwise.  check_only: 0 when it would launch, and no
// launch.
int gemm16_batch128(int dtype, const void* a, int64_t sa_m, int64_t sa_b, const void* b, int64_t sb_k, int64_t sb_b,
                    void* out, int64_t so_m, int64_t so_b, int out_dtype, int64_t M, int64_t N, int64_t K,
                    int64_t batch, int round_dtype, hipStream_t stream, bool check_only) {
  if (dtype != NT_DTYPE_F16 && dtype != NT_DTYPE_BF16) return NT_ERR_INVALID;
  if (out_dtype != NT_DTYPE_F16 && out_dtype != NT_DTYPE_BF16) return NT_ERR_INVALID;
  if (M <= 0 || N <= 0 || K < 3 * 32 || batch <= 0 || batch > 65535) return NT_ERR_INVALID;
  if (!a || !b || !out || N % 8 || K % 8 || sa_m < 0 || sb_k < 0 || so_m < 0 || sa_b < 0 || sb_b < 0 || so_b < 0)
    return NT_ERR_INVALID;
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16 || (uintptr_t)out % 16 || sa_m % 8 || sb_k % 8 || so_m % 8 ||
      sa_b % 8 || sb_b % 8 || so_b % 8)
    return NT_ERR_INVALID;
  if (127 * sa_m + K > 0x3fffffffLL || (K - 1) * sb_k + 128 > 0x3fffffffLL) return NT_ERR_INVALID;
  const int64_t tiles = cdiv(M, 128) * cdiv(N, 128);
  if (tiles > 0x7fffffffLL) return NT_ERR_INVALID;
  if (check_only) return 0;
  GemmArgs g{};
  g.a = a; g.b = b; g.out = out;
  g.sa_m = sa_m; g.sa_k = 1; g.sb_k = sb_k; g.sb_n = 1; g.so_m = so_m; g.so_n = 1;
  g.sa_b = sa_b; g.sb_b = sb_b; g.so_b = so_b;
  g.M = M; g.N = N; g.K = K;
  g.alpha = 1.0f; g.beta = 0.0f;
  g.out_dtype = out_dtype; g.c_dtype = out_dtype; g.round_dtype = round_dtype;
  g.tiles_m = (int)cdiv(M, 128);
  g.tiles_n = (int)cdiv(N, 128);
  g.c_pre = 1;
  const dim3 grid((unsigned)tiles, (unsigned)batch);
  if (dtype == NT_DTYPE_F16)
    hipLaunchKernelGGL((gemm_dma128_kernel<f16_t, false>), grid, dim3(256), 0, stream, g);
  else
    hipLaunchKernelGGL((gemm_dma128_kernel<bf16_t, false>), grid, dim3(256), 0, stream, g);
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
  // out_dtype: bits 0-7 out's type; bits 8-15 c's type + 1 (0: c has out's type).
  const int c_field = (out_dtype >> 8) & 0xff;
  g.out_dtype = (out_dtype < 0 || (out_dtype >> 16)) ? -2 : (out_dtype & 0xff);  // -2: rejected by gemm_check
  g.c_dtype = c_field ? c_field - 1 : g.out_dtype;
  g.round_dtype = round_dtype;
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
extern "C" int nt_gemm_config_f16(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k,
                                  int64_t sb_n, const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m,
                                  int64_t so_n, int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                                  int round_dtype, int config, hipStream_t stream) {
  return nt::gemm16_launch<nt::f16_t>(nt::make_args(NT_GEMM_ARGS), stream, config);
}
extern "C" int nt_gemm_config_bf16(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k,
                                   int64_t sb_n, const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m,
                                   int64_t so_n, int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                                   int round_dtype, int config, hipStream_t stream) {
  return nt::gemm16_launch<nt::bf16_t>(nt::make_args(NT_GEMM_ARGS), stream, config);
}
extern "C" int nt_gemm_f32(NT_GEMM_PARAMS) { return nt::gemm32_launch(nt::make_args(NT_GEMM_ARGS), stream); }
extern "C" int nt_gemm_e5m2(NT_GEMM_PARAMS) {
  return nt::gemm8_launch<nt::src_e5m2>(nt::make_args(NT_GEMM_ARGS), stream);
}
extern "C" int nt_gemm_e4m3(NT_GEMM_PARAMS) {
  return nt::gemm8_launch<nt::src_e4m3>(nt::make_args(NT_GEMM_ARGS), stream);
}

// The GEMM entry points with their arguments in one int64 array (see nt_mi355x.h).
extern "C" int nt_gemm_packed(const int64_t* v) {
  if (v == nullptr) return NT_ERR_INVALID;
  auto ptr = [&](int i) { return (void*)(intptr_t)v[i]; };
  auto flt = [&](int i) {
    const uint32_t bits = (uint32_t)(uint64_t)v[i];
    float x;
    std::memcpy(&x, &bits, sizeof(x));
    return x;
  };
  const void* a = ptr(1);
  const int64_t sa_m = v[2], sa_k = v[3];
  const void* b = ptr(4);
  const int64_t sb_k = v[5], sb_n = v[6];
  const void* c = ptr(7);
  const int64_t sc_m = v[8], sc_n = v[9];
  void* out = ptr(10);
  const int64_t so_m = v[11], so_n = v[12];
  const int out_dtype = (int)v[13];
  const int64_t M = v[14], N = v[15], K = v[16];
  const float alpha = flt(17), beta = flt(18);
  const int round_dtype = (int)v[19], config = (int)v[20];
  hipStream_t stream = (hipStream_t)ptr(21);
  if (config != 0 && v[0] > 1) return NT_ERR_INVALID;
  switch (v[0]) {
    case 0:
      return config ? nt_gemm_config_f16(NT_GEMM_ARGS, config, stream) : nt_gemm_f16(NT_GEMM_ARGS, stream);
    case 1:
      return config ? nt_gemm_config_bf16(NT_GEMM_ARGS, config, stream) : nt_gemm_bf16(NT_GEMM_ARGS, stream);
    case 2:
      return nt_gemm_f32(NT_GEMM_ARGS, stream);
    case 3:
      return nt_gemm_e5m2(NT_GEMM_ARGS, stream);
    case 4:
      return nt_gemm_e4m3(NT_GEMM_ARGS, stream);
    default:
      return NT_ERR_INVALID;
  }
}
