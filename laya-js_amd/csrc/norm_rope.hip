// LayerNorm (wave-per-row, f32 two-pass statistics) and split-half RoPE.
#include <stdexcept>

#include "common.h"

namespace hb {

const float* rope_table(uintptr_t ctx, int64_t L, int64_t D, double base);

// One wave per row; each lane keeps its 4-element groups in registers, so
// the row is read from HBM once and written once (2 x 2 x D bytes per row).
template <int G>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(int dt_x, const uint16_t* __restrict__ x, int64_t ldx,
                                                            int dt_w, const void* __restrict__ w,
                                                            const void* __restrict__ b, int dt_y,
                                                            uint16_t* __restrict__ y, int64_t rows, int D,
                                                            float eps) {
  int lane = threadIdx.x & 63;
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * ldx;
  float v[G][4];
  float s = 0.0f;
#pragma unroll
  for (int g = 0; g < G; g++) {
    int c = (g * 64 + lane) * 4;
    uint2v raw = *(const uint2v*)(xr + c);
    uint16_t h[4] = {(uint16_t)(raw.x & 0xffff), (uint16_t)(raw.x >> 16), (uint16_t)(raw.y & 0xffff),
                     (uint16_t)(raw.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[g][e] = dt_x == HB_F16 ? f16_bits_to_f32(h[e]) : bf16_to_f32(h[e]);
      s += v[g][e];
    }
  }
  float mean = wave_sum(s) / (float)D;
  float q = 0.0f;
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float d = v[g][e] - mean;
      q += d * d;
    }
  float rstd = 1.0f / sqrtf(wave_sum(q) / (float)D + eps);
  uint16_t* yr = y + row * (int64_t)D;
#pragma unroll
  for (int g = 0; g < G; g++) {
    int c = (g * 64 + lane) * 4;
    uint16_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float t = (v[g][e] - mean) * rstd;
      if (w) t *= load_f(w, c + e, dt_w);
      if (b) t += load_f(b, c + e, dt_w);
      o[e] = dt_y == HB_F16 ? f32_to_f16_bits(t) : f32_to_bf16(t);
    }
    uint2v out;
    out.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
    out.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
    *(uint2v*)(yr + c) = out;
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

}  // namespace hb

using namespace hb;

extern "C" {

int hb_layernorm(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_w, uintptr_t w, uintptr_t b, int dt_y,
                 uintptr_t y, int64_t rows, int64_t D, float eps) {
  HB_API_BEGIN
  HB_REQUIRE(D > 0 && ldx >= D, "hb_layernorm: bad row width");
  if (rows == 0) return 0;
  hipStream_t st = stream_of(ctx);
  unsigned grid = (unsigned)((rows + 3) / 4);
  bool vec = (dt_x == HB_F16 || dt_x == HB_BF16) && (dt_y == HB_F16 || dt_y == HB_BF16) && D % 256 == 0 &&
             D <= 2048 && ldx % 4 == 0 && x % 8 == 0 && y % 8 == 0;
  if (vec) {
    int G = (int)(D / 256);
#define LN_CASE(g)                                                                                                \
  case g:                                                                                                         \
    layernorm_vec_kernel<g><<<grid, 256, 0, st>>>(dt_x, (const uint16_t*)x, ldx, dt_w, (const void*)w,          \
                                                  (const void*)b, dt_y, (uint16_t*)y, rows, (int)D, eps);         \
    break;
    switch (G) {
      LN_CASE(1)
      LN_CASE(2)
      LN_CASE(3)
      LN_CASE(4)
      LN_CASE(5)
      LN_CASE(6)
      LN_CASE(7)
      LN_CASE(8)
      default: break;
    }
#undef LN_CASE
  } else {
    layernorm_kernel<<<grid, 256, 0, st>>>(dt_x, (const void*)x, ldx, dt_w, (const void*)w, (const void*)b, dt_y,
                                           (void*)y, rows, D, eps);
  }
  check_launch("hb_layernorm");
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
