// LayerNorm (wave-per-row, f32 two-pass statistics; written row-major or in
// the panel order of the GEMM's X operand) and split-half RoPE.
#include <stdexcept>
#include <type_traits>

#include "common.h"

namespace hb {

const float* rope_table(uintptr_t ctx, int64_t L, int64_t D, double base);

// One wave per row; each lane keeps its 4-element groups in registers, so
// the row is read from HBM once and written once (2 x 2 x D bytes per row).
// x and y share the 16-bit type BF (f16 / bf16); the affine parameters are of
// type PK (0: none, 1: f16, 2: bf16, 3: f32) and are read 4 at a time.
template <int PK>
__device__ __forceinline__ void load4_param(const void* p, int c, float (&v)[4]) {
  if constexpr (PK == 3) {
    const float4v f = *(const float4v*)((const float*)p + c);
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = f[e];
  } else {
    const uint2v raw = *(const uint2v*)((const uint16_t*)p + c);
    const uint16_t h[4] = {(uint16_t)(raw.x & 0xffff), (uint16_t)(raw.x >> 16), (uint16_t)(raw.y & 0xffff),
                           (uint16_t)(raw.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = PK == 1 ? f16_bits_to_f32(h[e]) : bf16_to_f32(h[e]);
  }
}

// One row of the 16-bit path, held by a half-wave (32 lanes, `hl` = lane
// % 32): raw[g] holds columns (g * 32 + hl) * 8 + 0..7 of the row (one
// 16-byte load each); out[g] gets the normalised values at the same
// columns.  The sums reduce over the half-wave only, so the two halves of a
// wave normalise two rows side by side.  Both 16-bit kernels below call
// this, so their outputs agree bit for bit.
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int G, bool BF, int PK>
__device__ __forceinline__ void ln_row(const uint4v (&raw)[G], int hl, const void* __restrict__ w,
                                       const void* __restrict__ b, int D, float eps, uint4v (&out)[G]) {
  float v[G][8];
  float s = 0.0f;
#pragma unroll
  for (int g = 0; g < G; g++) {
    const uint32_t wd[4] = {raw[g].x, raw[g].y, raw[g].z, raw[g].w};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint16_t h = (uint16_t)(wd[e >> 1] >> (16 * (e & 1)));
      v[g][e] = BF ? bf16_to_f32(h) : f16_bits_to_f32(h);
      s += v[g][e];
    }
  }
  const float mean = half_wave_sum(s) / (float)D;
  float q = 0.0f;
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float d = v[g][e] - mean;
      q += d * d;
    }
  const float rstd = 1.0f / sqrtf(half_wave_sum(q) / (float)D + eps);
#pragma unroll
  for (int g = 0; g < G; g++) {
    const int c = (g * 32 + hl) * 8;
    float wv[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f}, bv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if constexpr (PK != 0) {
      if (w) {
        load4_param<PK>(w, c, *(float(*)[4])(wv));
        load4_param<PK>(w, c + 4, *(float(*)[4])(wv + 4));
      }
      if (b) {
        load4_param<PK>(b, c, *(float(*)[4])(bv));
        load4_param<PK>(b, c + 4, *(float(*)[4])(bv + 4));
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      uint16_t r2[2];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        float t = (v[g][e + k] - mean) * rstd;
        if constexpr (PK != 0) {
          if (w) t = pin_f32(t * wv[e + k]);
          if (b) t += bv[e + k];
        }
        r2[k] = BF ? f32_to_bf16(t) : f32_to_f16_bits(t);
      }
      o[e >> 1] = (uint32_t)r2[0] | ((uint32_t)r2[1] << 16);
    }
    out[g] = uint4v{o[0], o[1], o[2], o[3]};
  }
}

// Row-major output: 8 rows per block of 256 threads, one per half-wave.
template <int G, bool BF, int PK>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                            const void* __restrict__ w, const void* __restrict__ b,
                                                            uint16_t* __restrict__ y, int64_t rows, int D, float eps) {
  const int hl = threadIdx.x & 31;
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (row >= rows) return;  // a whole half-wave: its sums never read the other half
  const uint16_t* xr = x + row * ldx;
  uint4v raw[G], out[G];
#pragma unroll
  for (int g = 0; g < G; g++) raw[g] = *(const uint4v*)(xr + (g * 32 + hl) * 8);
  ln_row<G, BF, PK>(raw, hl, w, b, D, eps, out);
  uint16_t* yr = y + row * (int64_t)D;
#pragma unroll
  for (int g = 0; g < G; g++) *(uint4v*)(yr + (g * 32 + hl) * 8) = out[g];
}

// Panel-order output: a block of 256 threads normalises 8 consecutive rows,
// one per half-wave.  In panel order those rows' chunks of one (16-column
// block, half) pair form one 128-byte line, so the block stages its rows in
// LDS line by line -- chunk of row i in line l at slot (i + l) % 8, which
// spreads a half-wave's writes over the banks -- and writes each line whole
// with 8 consecutive 16-byte stores.  The grid covers the padding rows of the
// last 32-row block, which are written as zeros.
constexpr int kLnNT = 256;  // threads per block (8 rows)
template <int G, bool BF, int PK>
__global__ __launch_bounds__(kLnNT) void layernorm_panel_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                const void* __restrict__ w,
                                                                const void* __restrict__ b, uint16_t* __restrict__ y,
                                                                int64_t rows, int D, float eps) {
  extern __shared__ __attribute__((aligned(16))) uint16_t tile[];  // [D / 8 lines][8 slots][8]
  const int hl = threadIdx.x & 31, r = threadIdx.x >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * 8;
  const int64_t row = row0 + r;
  const uint16_t* xr = x + (row < rows ? row : rows - 1) * ldx;
  uint4v raw[G], out[G];
#pragma unroll
  for (int g = 0; g < G; g++) raw[g] = *(const uint4v*)(xr + (g * 32 + hl) * 8);
  if (row < rows) {
    ln_row<G, BF, PK>(raw, hl, w, b, D, eps, out);
  } else {
#pragma unroll
    for (int g = 0; g < G; g++) out[g] = uint4v{0, 0, 0, 0};
  }
#pragma unroll
  for (int g = 0; g < G; g++) {
    const int l = g * 32 + hl;  // the chunk's line: columns 8l .. 8l + 7
    *(uint4v*)(tile + l * 64 + ((r + l) & 7) * 8) = out[g];
  }
  __syncthreads();
  const int64_t kb = D >> 4;  // 16-column blocks per row
  uint16_t* yb = y + (row0 >> 5) * kb * 512;
  for (int q = threadIdx.x; q < D; q += kLnNT) {
    const int l = q >> 3, sl = q & 7, i = (sl - l) & 7;
    const int r32 = (int)(row0 & 31) + i;
    *(uint4v*)(yb + (int64_t)(l >> 1) * 512 + ((l & 1) * 32 + r32) * 8) = *(const uint4v*)(tile + q * 8);
  }
}

// Generic: any dtype and width; the row is re-read for each pass.
__global__ __launch_bounds__(256) void layernorm_kernel(int dt_x, const void* __restrict__ x, int64_t ldx, int dt_w,
                                                        const void* __restrict__ w, const void* __restrict__ b,
                                                        int dt_y, void* __restrict__ y, int64_t rows, int64_t D,
                                                        float eps) {
  int lane = threadIdx.x & 63;
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float s = 0.0f;
  for (int64_t i = lane; i < D; i += 64) s += load_f(x, row * ldx + i, dt_x);
  float mean = wave_sum(s) / (float)D;
  float q = 0.0f;
  for (int64_t i = lane; i < D; i += 64) {
    float d = load_f(x, row * ldx + i, dt_x) - mean;
    q += d * d;
  }
  float rstd = 1.0f / sqrtf(wave_sum(q) / (float)D + eps);
  for (int64_t i = lane; i < D; i += 64) {
    float t = (load_f(x, row * ldx + i, dt_x) - mean) * rstd;
    if (w) t *= load_f(w, i, dt_w);
    if (b) t += load_f(b, i, dt_w);
    store_f(y, row * D + i, dt_y, t);
  }
}

// One thread per rotation pair (j, j + D/2) of one (b, h, l) row.
__global__ void rope_kernel(int dt_x, const void* __restrict__ x, int64_t s0, int64_t s1, int64_t s2, int64_t s3,
                            int dt_y, void* __restrict__ y, int64_t B, int64_t H, int64_t L, int64_t D,
                            const float2* __restrict__ tab) {
  int64_t half = D / 2;
  int64_t n = B * H * L * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t j = i % half;
    int64_t r = i / half;
    int64_t l = r % L;
    int64_t bh = r / L;
    int64_t h = bh % H, bb = bh / H;
    int64_t src = bb * s0 + h * s1 + l * s2;
    float x0 = load_f(x, src + j * s3, dt_x);
    float x1 = load_f(x, src + (j + half) * s3, dt_x);
    float2 cs = tab[l * half + j];
    int64_t dst = r * D;
    store_f(y, dst + j, dt_y, fmaf(-x1, cs.y, x0 * cs.x));
    store_f(y, dst + j + half, dt_y, fmaf(x0, cs.y, x1 * cs.x));
  }
}

// Kind of the affine parameters for the 16-bit kernels: 0 none, 1 f16,
// 2 bf16, 3 f32, -1 other.
static int ln_param_kind(int dt_w, uintptr_t w, uintptr_t b) {
  return (w == 0 && b == 0) ? 0 : dt_w == HB_F16 ? 1 : dt_w == HB_BF16 ? 2 : dt_w == HB_F32 ? 3 : -1;
}

// The 16-bit kernels' conditions (besides the output's).
static bool ln_vec_ok(int dt_x, uintptr_t x, int64_t ldx, int pk, uintptr_t w, uintptr_t b, int64_t D) {
  const int64_t pal = pk == 3 ? 16 : 8;  // parameter alignment the 4-wide loads need
  return (dt_x == HB_F16 || dt_x == HB_BF16) && D % 256 == 0 && D <= 2048 && ldx % 8 == 0 && x % 16 == 0 &&
         pk >= 0 && w % pal == 0 && b % pal == 0;
}

static void launch_ln16(bool panel, hipStream_t st, bool bf, int pk, const uint16_t* x, int64_t ldx, uintptr_t w,
                        uintptr_t b, uint16_t* y, int64_t rows, int D, float eps) {
  const int G = D / 256;
  auto launch = [&](auto gc, auto pc) {
    constexpr int GG = decltype(gc)::value, PP = decltype(pc)::value;
    if (panel) {
      constexpr size_t lds = (size_t)8 * GG * 256 * sizeof(uint16_t);  // 8 rows
      static std::atomic<uint64_t> attr{0};
      once_per_device(attr, [&] {
        HB_CHECK_HIP(hipFuncSetAttribute((const void*)layernorm_panel_kernel<GG, true, PP>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        HB_CHECK_HIP(hipFuncSetAttribute((const void*)layernorm_panel_kernel<GG, false, PP>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
      });
      auto kern = bf ? layernorm_panel_kernel<GG, true, PP> : layernorm_panel_kernel<GG, false, PP>;
      kern<<<(unsigned)((rows + 31) / 32 * 4), kLnNT, lds, st>>>(x, ldx, (const void*)w, (const void*)b, y, rows, D,
                                                                  eps);
    } else {
      auto kern = bf ? layernorm_vec_kernel<GG, true, PP> : layernorm_vec_kernel<GG, false, PP>;
      kern<<<(unsigned)((rows + 7) / 8), 256, 0, st>>>(x, ldx, (const void*)w, (const void*)b, y, rows, D, eps);
    }
  };
  auto by_g = [&](auto pc) {
    switch (G) {
      case 1: launch(std::integral_constant<int, 1>{}, pc); break;
      case 2: launch(std::integral_constant<int, 2>{}, pc); break;
      case 3: launch(std::integral_constant<int, 3>{}, pc); break;
      case 4: launch(std::integral_constant<int, 4>{}, pc); break;
      case 5: launch(std::integral_constant<int, 5>{}, pc); break;
      case 6: launch(std::integral_constant<int, 6>{}, pc); break;
      case 7: launch(std::integral_constant<int, 7>{}, pc); break;
      default: launch(std::integral_constant<int, 8>{}, pc); break;
    }
  };
  switch (pk) {
    case 0: by_g(std::integral_constant<int, 0>{}); break;
    case 1: by_g(std::integral_constant<int, 1>{}); break;
    case 2: by_g(std::integral_constant<int, 2>{}); break;
    default: by_g(std::integral_constant<int, 3>{}); break;
  }
}

}  // namespace hb

using namespace hb;

extern "C" {

int hb_layernorm(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_w, uintptr_t w, uintptr_t b, int dt_y,
                 uintptr_t y, int64_t rows, int64_t D, float eps) {
  HB_API_BEGIN
  HB_REQUIRE(D > 0 && ldx >= D, "hb_layernorm: bad row width");
  if (rows == 0) return 0;
  hipStream_t st = stream_of(ctx);
  const int pk = ln_param_kind(dt_w, w, b);
  if (dt_y == dt_x && ln_vec_ok(dt_x, x, ldx, pk, w, b, D) && y % 16 == 0) {
    launch_ln16(false, st, dt_x == HB_BF16, pk, (const uint16_t*)x, ldx, w, b, (uint16_t*)y, rows, (int)D, eps);
  } else {
    layernorm_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(dt_x, (const void*)x, ldx, dt_w, (const void*)w,
                                                                 (const void*)b, dt_y, (void*)y, rows, D, eps);
  }
  check_launch("hb_layernorm");
  HB_API_END
}

int hb_layernorm_panel(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_w, uintptr_t w, uintptr_t b,
                       uintptr_t y, int64_t rows, int64_t D, float eps) {
  HB_API_BEGIN
  HB_REQUIRE(D > 0 && ldx >= D, "hb_layernorm_panel: bad row width");
  const int pk = ln_param_kind(dt_w, w, b);
  HB_REQUIRE(ln_vec_ok(dt_x, x, ldx, pk, w, b, D) && y % 16 == 0,
             "hb_layernorm_panel: needs f16/bf16, D % 256 == 0, D <= 2048, ldx % 8 == 0 and 16-byte aligned operands");
  if (rows == 0) return 0;
  launch_ln16(true, stream_of(ctx), dt_x == HB_BF16, pk, (const uint16_t*)x, ldx, w, b, (uint16_t*)y, rows, (int)D,
              eps);
  check_launch("hb_layernorm_panel");
  HB_API_END
}

int hb_rope(uintptr_t ctx, int dt_x, uintptr_t x, const int64_t* xs, int dt_y, uintptr_t y, int64_t B, int64_t H,
            int64_t L, int64_t D, double base) {
  HB_API_BEGIN
  HB_REQUIRE(D % 2 == 0, "hb_rope: head dim must be even");
  int64_t n = B * H * L * (D / 2);
  if (n == 0) return 0;
  const float2* tab = (const float2*)rope_table(ctx, L, D, base);
  rope_kernel<<<grid_for(n, 256), 256, 0, stream_of(ctx)>>>(dt_x, (const void*)x, xs[0], xs[1], xs[2], xs[3], dt_y,
                                                             (void*)y, B, H, L, D, tab);
  check_launch("hb_rope");
  HB_API_END
}

}  // extern "C"
