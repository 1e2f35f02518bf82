// Bandwidth kernels: strided copy/cast and elementwise math, broadcasting
// binary ops, where, GeGLU, gathers, masked mean pooling, fills, and the
// row-major <-> panel-order repacking of 16-bit matrices.
#include <stdexcept>

#include "common.h"

namespace hb {

static Strided make_strided(const int64_t* shape, int rank, const int64_t* s0, const int64_t* s1,
                            const int64_t* s2) {
  HB_REQUIRE(rank >= 0 && rank <= kMaxRank, "rank must be <= 8");
  Strided s{};
  s.rank = rank;
  for (int d = 0; d < rank; d++) {
    HB_REQUIRE(shape[d] >= 0, "negative dimension");
    s.shape[d] = shape[d];
    s.st[0][d] = s0 ? s0[d] : 0;
    s.st[1][d] = s1 ? s1[d] : 0;
    s.st[2][d] = s2 ? s2[d] : 0;
  }
  return s;
}

__host__ __device__ static inline bool is_int_dt(int dt) { return dt != HB_F32 && dt != HB_F16 && dt != HB_BF16; }

__device__ __forceinline__ float unary_f(int op, float x, float alpha) {
  switch (op) {
    case HB_UN_COPY: return x;
    case HB_UN_SCALE: return x * alpha;
    case HB_UN_EXP: return expf(x);
    case HB_UN_LOG: return logf(x);
    case HB_UN_RELU: return x > 0.0f ? x : 0.0f;
    case HB_UN_GELU: return gelu_erf(x);
    case HB_UN_NEG: return -x;
    case HB_UN_ABS: return fabsf(x);
    case HB_UN_SQRT: return sqrtf(x);
    case HB_UN_RSQRT: return 1.0f / sqrtf(x);
    case HB_UN_TANH: return tanhf(x);
    case HB_UN_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case HB_UN_ERF: return erff(x);
    case HB_UN_NOT: return x == 0.0f ? 1.0f : 0.0f;
    default: return x;
  }
}

__global__ void unary_kernel(int op, int dt_x, const void* __restrict__ x, int dt_y, void* __restrict__ y,
                             Strided s, int64_t n, float alpha, int int_path, int y_strided) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t ox, oy, o2;
    strided_offsets(s, i, &ox, &oy, &o2);
    if (!y_strided) oy = i;
    if (int_path) {
      int32_t v = load_i(x, ox, dt_x);
      if (op == HB_UN_NEG) v = -v;
      else if (op == HB_UN_ABS) v = v < 0 ? -v : v;
      else if (op == HB_UN_NOT) v = v == 0;
      store_i(y, oy, dt_y, v);
    } else {
      store_f(y, oy, dt_y, unary_f(op, load_f(x, ox, dt_x), alpha));
    }
  }
}

// contiguous 16-bit -> 16-bit copy (the common reshape/transpose materialisation
// has a strided source; this handles the plain contiguous case fast)
__global__ void copy_bytes_kernel(const uint4v* __restrict__ x, uint4v* __restrict__ y, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = x[i];
}

// Panel order <-> row-major for a 16-bit [M, K] matrix: one thread per
// 16-byte panel chunk p = 64 * block + 32 * h + r of block (i, j) =
// divmod(block, K / 16), i.e. row 32 * i + r, columns 16 * j + 8 * h + 0..7.
__device__ __forceinline__ void panel_chunk_rc(int64_t p, int64_t K, int64_t& row, int64_t& col) {
  const int64_t blk = p >> 6, kb = K >> 4;
  const int c = (int)(p & 63);
  row = (blk / kb) * 32 + (c & 31);
  col = (blk % kb) * 16 + (c >> 5) * 8;
}

__global__ void panel_pack_kernel(const uint16_t* __restrict__ src, int64_t ld, uint4v* __restrict__ dst, int64_t M,
                                  int64_t K, int64_t chunks) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < chunks; p += (int64_t)gridDim.x * blockDim.x) {
    int64_t row, col;
    panel_chunk_rc(p, K, row, col);
    dst[p] = row < M ? *(const uint4v*)(src + row * ld + col) : uint4v{0, 0, 0, 0};
  }
}

__global__ void panel_unpack_kernel(const uint4v* __restrict__ src, uint16_t* __restrict__ dst, int64_t ld, int64_t M,
                                    int64_t K, int64_t chunks) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < chunks; p += (int64_t)gridDim.x * blockDim.x) {
    int64_t row, col;
    panel_chunk_rc(p, K, row, col);
    if (row < M) *(uint4v*)(dst + row * ld + col) = src[p];
  }
}

__global__ void fill_kernel(uint8_t* __restrict__ y, uint8_t v, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = v;
}

__device__ __forceinline__ float binary_f(int op, float a, float b) {
  switch (op) {
    case HB_BIN_ADD: return a + b;
    case HB_BIN_SUB: return a - b;
    case HB_BIN_MUL: return a * b;
    case HB_BIN_DIV: return a / b;
    case HB_BIN_MAX: return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
    case HB_BIN_MIN: return (a != a || b != b) ? __builtin_nanf("") : fminf(a, b);
    case HB_BIN_POW: return powf(a, b);
    case HB_BIN_EQ: return a == b;
    case HB_BIN_NE: return a != b;
    case HB_BIN_LT: return a < b;
    case HB_BIN_LE: return a <= b;
    case HB_BIN_GT: return a > b;
    case HB_BIN_GE: return a >= b;
    case HB_BIN_AND: return (a != 0.0f) && (b != 0.0f);
    case HB_BIN_OR: return (a != 0.0f) || (b != 0.0f);
    default: return 0.0f;
  }
}
__device__ __forceinline__ int32_t binary_i(int op, int32_t a, int32_t b) {
  switch (op) {
    case HB_BIN_ADD: return (int32_t)((uint32_t)a + (uint32_t)b);
    case HB_BIN_SUB: return (int32_t)((uint32_t)a - (uint32_t)b);
    case HB_BIN_MUL: return (int32_t)((uint32_t)a * (uint32_t)b);
    case HB_BIN_DIV: return b == 0 ? 0 : a / b;
    case HB_BIN_MAX: return a > b ? a : b;
    case HB_BIN_MIN: return a < b ? a : b;
    case HB_BIN_EQ: return a == b;
    case HB_BIN_NE: return a != b;
    case HB_BIN_LT: return a < b;
    case HB_BIN_LE: return a <= b;
    case HB_BIN_GT: return a > b;
    case HB_BIN_GE: return a >= b;
    case HB_BIN_AND: return a != 0 && b != 0;
    case HB_BIN_OR: return a != 0 || b != 0;
    default: return 0;
  }
}

__global__ void binary_kernel(int op, int dt_a, const void* __restrict__ a, int dt_b, const void* __restrict__ b,
                              int dt_y, void* __restrict__ y, Strided s, int64_t n, int int_path) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t oa, ob, oc;
    strided_offsets(s, i, &oa, &ob, &oc);
    if (int_path) store_i(y, i, dt_y, binary_i(op, load_i(a, oa, dt_a), load_i(b, ob, dt_b)));
    else store_f(y, i, dt_y, binary_f(op, load_f(a, oa, dt_a), load_f(b, ob, dt_b)));
  }
}

__global__ void where_kernel(const uint8_t* __restrict__ c, int dt_a, const void* __restrict__ a, int dt_b,
                             const void* __restrict__ b, int dt_y, void* __restrict__ y, Strided s, int64_t n,
                             int int_path) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t oc, oa, ob;
    strided_offsets(s, i, &oc, &oa, &ob);
    bool t = c[oc] != 0;
    if (int_path) store_i(y, i, dt_y, t ? load_i(a, oa, dt_a) : load_i(b, ob, dt_b));
    else store_f(y, i, dt_y, t ? load_f(a, oa, dt_a) : load_f(b, ob, dt_b));
  }
}

// y[r, j] = round(gelu(x[r, j]) * x[r, F + j]) in f32 with one rounding to dt_y.
// A 16-bit output takes gelu_fast, the GELU of the GEMMs' fused GeGLU
// epilogue, so the fused and unfused paths give the same bits; f32 keeps
// libm's erf.
__global__ void geglu_kernel(int dt_x, const void* __restrict__ x, int64_t ldx, int dt_y, void* __restrict__ y,
                             int64_t rows, int64_t F) {
  int64_t n = rows * F;
  const bool fast = dt_y == HB_F16 || dt_y == HB_BF16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i / F, j = i - r * F;
    float v = load_f(x, r * ldx + j, dt_x);
    float g = load_f(x, r * ldx + F + j, dt_x);
    store_f(y, i, dt_y, pin_f32((fast ? gelu_fast(v) : gelu_erf(v)) * g));
  }
}

__global__ void gather_kernel(int dt, const void* __restrict__ table, int64_t V, int64_t D,
                              const int32_t* __restrict__ ids, int64_t n, int64_t batch_rows, int dt_out,
                              void* __restrict__ out) {
  int64_t total = n * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i / D, d = i - r * D;
    int64_t id = ids[r];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    int64_t base = batch_rows > 0 ? (r / batch_rows) * V * D : 0;
    int64_t src = base + id * D + d;
    if (is_int_dt(dt) && is_int_dt(dt_out)) store_i(out, i, dt_out, load_i(table, src, dt));
    else store_f(out, i, dt_out, load_f(table, src, dt));
  }
}

// bytes of one element of a dtype code
static int dt_size(int dt) {
  return (dt == HB_F32 || dt == HB_I32 || dt == HB_U32) ? 4
         : (dt == HB_F16 || dt == HB_BF16 || dt == HB_U16 || dt == HB_I16) ? 2 : 1;
}

// Same-dtype gather of whole 16-byte chunks (rows of D * elem bytes, a
// multiple of 16): one thread per chunk, a bit copy.
__global__ void gather16_kernel(const uint8_t* __restrict__ table, int64_t V, int64_t row_bytes,
                                const int32_t* __restrict__ ids, int64_t n, int64_t batch_rows,
                                uint8_t* __restrict__ out) {
  const int64_t cpr = row_bytes >> 4, total = n * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cpr, c = i - r * cpr;
    int64_t id = ids[r];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    const int64_t base = batch_rows > 0 ? (r / batch_rows) * V : 0;
    ((uint4v*)out)[i] = *(const uint4v*)(table + (base + id) * row_bytes + c * 16);
  }
}

__global__ void meanpool_kernel(int dt_x, const void* __restrict__ x, const uint8_t* __restrict__ mask, int64_t B,
                                int64_t L, int64_t D, float* __restrict__ out) {
  int64_t total = B * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t b = i / D, d = i - b * D;
    float s = 0.0f, cnt = 0.0f;
    for (int64_t l = 0; l < L; l++) {
      if (mask[b * L + l]) {
        s += load_f(x, (b * L + l) * D + d, dt_x);
        cnt += 1.0f;
      }
    }
    out[i] = s / fmaxf(cnt, 1.0f);
  }
}

// 16-bit x, D % 8 == 0: two passes.  meanpool16_partial: block (column chunk
// of 512, row slice s of S, batch row b); thread t sums columns 8 (t % 64)
// .. + 7 of the chunk over the slice's rows l = l0 + t / 64 (mod 4), with
// 16-byte loads; the four row groups are added in LDS in a fixed order.
// meanpool16_final adds the S slice sums in order and divides by the
// count of visible rows.  Same result on every run (no atomics).
template <bool BF>
__global__ __launch_bounds__(256) void meanpool16_partial(const uint16_t* __restrict__ x,
                                                          const uint8_t* __restrict__ mask, int64_t B, int64_t L,
                                                          int64_t D, int S, float* __restrict__ part,
                                                          float* __restrict__ cnt) {
  __shared__ float red[4][512];
  __shared__ float redn[4];
  const int c = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t b = blockIdx.z, s = blockIdx.y, d = (int64_t)blockIdx.x * 512 + c * 8;
  const int64_t l0 = L * s / S, l1 = L * (s + 1) / S;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float n = 0.f;
  const bool dok = d < D;
  const uint16_t* xb = x + b * L * D + (dok ? d : 0);
  const uint8_t* mb = mask + b * L;
#pragma unroll 4
  for (int64_t l = l0 + g; l < l1; l += 4) {
    const uint4v v = *(const uint4v*)(xb + l * D);
    const bool vis = mb[l] != 0;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float lo = BF ? bf16_to_f32((uint16_t)(w[e] & 0xffff)) : f16_bits_to_f32((uint16_t)(w[e] & 0xffff));
      const float hi = BF ? bf16_to_f32((uint16_t)(w[e] >> 16)) : f16_bits_to_f32((uint16_t)(w[e] >> 16));
      acc[2 * e] += vis ? lo : 0.f;
      acc[2 * e + 1] += vis ? hi : 0.f;
    }
    n += vis ? 1.f : 0.f;
  }
#pragma unroll
  for (int e = 0; e < 8; e++) red[g][c * 8 + e] = acc[e];
  if (c == 0) redn[g] = n;
  __syncthreads();
  if (g == 0 && dok) {
    float* pp = part + (s * B + b) * D + d;
#pragma unroll
    for (int e = 0; e < 8; e++) pp[e] = ((red[0][c * 8 + e] + red[1][c * 8 + e]) + red[2][c * 8 + e]) + red[3][c * 8 + e];
  }
  if (threadIdx.x == 0 && blockIdx.x == 0) cnt[s * B + b] = ((redn[0] + redn[1]) + redn[2]) + redn[3];
}

__global__ void meanpool16_final(const float* __restrict__ part, const float* __restrict__ cnt, int64_t B, int64_t D,
                                 int S, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * D) return;
  const int64_t b = i / D;
  float sum = 0.f, n = 0.f;
  for (int s = 0; s < S; s++) {
    sum += part[s * B * D + i];
    n += cnt[s * B + b];
  }
  out[i] = sum / fmaxf(n, 1.0f);
}

// Index of the first maximum (minimum) of x[base + j * inner], j < n; a NaN
// counts as the extremum (numpy's rule).
__device__ __noinline__ int32_t argreduce(bool is_max, int dt_x, const void* __restrict__ x, int64_t base, int64_t n,
                                          int64_t inner) {
  int32_t best = 0;
  if (is_int_dt(dt_x)) {
    int32_t bv = load_i(x, base, dt_x);
    for (int64_t j = 1; j < n; j++) {
      int32_t v = load_i(x, base + j * inner, dt_x);
      if (is_max ? (v > bv) : (v < bv)) {
        bv = v;
        best = (int32_t)j;
      }
    }
    return best;
  }
  float bv = load_f(x, base, dt_x);
  if (__builtin_isnan(bv)) return 0;
  for (int64_t j = 1; j < n; j++) {
    float v = load_f(x, base + j * inner, dt_x);
    if (__builtin_isnan(v)) return (int32_t)j;
    if (is_max ? (v > bv) : (v < bv)) {
      bv = v;
      best = (int32_t)j;
    }
  }
  return best;
}

// One thread per (outer, inner) slice: the contract's reductions run on the
// decision head's small tensors, never on the encoder's hot path.
__global__ void reduce_kernel(int op, int dt_x, const void* __restrict__ x, int64_t outer, int64_t n, int64_t inner,
                              int dt_y, void* __restrict__ y) {
  int64_t total = outer * inner;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t o = i / inner, in = i - o * inner;
    int64_t base = o * n * inner + in;
    bool ints = is_int_dt(dt_x) && (op == HB_RED_SUM || op == HB_RED_MAX || op == HB_RED_MIN) && is_int_dt(dt_y);
    if (op == HB_RED_ARGMAX || op == HB_RED_ARGMIN) {
      store_i(y, i, dt_y, argreduce(op == HB_RED_ARGMAX, dt_x, x, base, n, inner));
    } else if (ints) {
      int32_t acc = op == HB_RED_SUM ? 0 : load_i(x, base, dt_x);
      for (int64_t j = op == HB_RED_SUM ? 0 : 1; j < n; j++) {
        int32_t v = load_i(x, base + j * inner, dt_x);
        if (op == HB_RED_SUM) acc = (int32_t)((uint32_t)acc + (uint32_t)v);
        else if (op == HB_RED_MAX) acc = v > acc ? v : acc;
        else acc = v < acc ? v : acc;
      }
      store_i(y, i, dt_y, acc);
    } else {
      float acc = (op == HB_RED_SUM || op == HB_RED_MEAN) ? 0.f : load_f(x, base, dt_x);
      for (int64_t j = (op == HB_RED_SUM || op == HB_RED_MEAN) ? 0 : 1; j < n; j++) {
        float v = load_f(x, base + j * inner, dt_x);
        if (op == HB_RED_SUM || op == HB_RED_MEAN) acc += v;
        else if (op == HB_RED_MAX) acc = (v > acc || v != v) ? v : acc;
        else acc = (v < acc || v != v) ? v : acc;
      }
      if (op == HB_RED_MEAN) acc /= (float)n;
      store_f(y, i, dt_y, acc);
    }
  }
}

__global__ void scan_kernel(int op, int dt_x, const void* __restrict__ x, int64_t outer, int64_t n, int64_t inner,
                            int dt_y, void* __restrict__ y) {
  int64_t total = outer * inner;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t o = i / inner, in = i - o * inner;
    int64_t base = o * n * inner + in;
    if (op == HB_SCAN_SOFTMAX) {
      float mx = -INFINITY;
      for (int64_t j = 0; j < n; j++) mx = fmaxf(mx, load_f(x, base + j * inner, dt_x));
      float s = 0.f;
      for (int64_t j = 0; j < n; j++) s += expf(load_f(x, base + j * inner, dt_x) - mx);
      float inv = 1.0f / s;
      for (int64_t j = 0; j < n; j++) store_f(y, base + j * inner, dt_y, expf(load_f(x, base + j * inner, dt_x) - mx) * inv);
    } else if (op == HB_SCAN_CUMSUM) {
      if (is_int_dt(dt_y)) {
        int32_t acc = 0;
        for (int64_t j = 0; j < n; j++) {
          acc = (int32_t)((uint32_t)acc + (uint32_t)load_i(x, base + j * inner, dt_x));
          store_i(y, base + j * inner, dt_y, acc);
          acc = load_i(y, base + j * inner, dt_y);  // wrap within the output dtype
        }
      } else {
        float acc = 0.f;
        for (int64_t j = 0; j < n; j++) {
          acc += load_f(x, base + j * inner, dt_x);
          store_f(y, base + j * inner, dt_y, acc);
        }
      }
    } else {  // insertion sort, ascending; NaN sorts last
      for (int64_t j = 0; j < n; j++) {
        if (is_int_dt(dt_x)) store_i(y, base + j * inner, dt_y, load_i(x, base + j * inner, dt_x));
        else store_f(y, base + j * inner, dt_y, load_f(x, base + j * inner, dt_x));
      }
      for (int64_t j = 1; j < n; j++) {
        if (is_int_dt(dt_y)) {
          int32_t v = load_i(y, base + j * inner, dt_y);
          int64_t k = j - 1;
          while (k >= 0 && load_i(y, base + k * inner, dt_y) > v) {
            store_i(y, base + (k + 1) * inner, dt_y, load_i(y, base + k * inner, dt_y));
            k--;
          }
          store_i(y, base + (k + 1) * inner, dt_y, v);
        } else {
          float v = load_f(y, base + j * inner, dt_y);
          int64_t k = j - 1;
          while (k >= 0) {
            float u = load_f(y, base + k * inner, dt_y);
            bool gt = (u != u) ? (v == v) : (v == v && u > v);
            if (!gt) break;
            store_f(y, base + (k + 1) * inner, dt_y, u);
            k--;
          }
          store_f(y, base + (k + 1) * inner, dt_y, v);
        }
      }
    }
  }
}

}  // namespace hb

using namespace hb;

extern "C" {

int hb_fill(uintptr_t ctx, uintptr_t dst, int value, size_t bytes) {
  HB_API_BEGIN
  if (!bytes) return 0;
  fill_kernel<<<grid_for((int64_t)bytes, 256), 256, 0, stream_of(ctx)>>>((uint8_t*)dst, (uint8_t)value,
                                                                          (int64_t)bytes);
  check_launch("hb_fill");
  HB_API_END
}

int hb_unary(uintptr_t ctx, int op, int dt_x, uintptr_t x, const int64_t* xs, int dt_y, uintptr_t y,
             const int64_t* ys, const int64_t* shape, int rank, double alpha) {
  HB_API_BEGIN
  Strided s = make_strided(shape, rank, xs, ys, nullptr);
  int64_t n = numel(shape, rank);
  if (n == 0) return 0;
  hipStream_t st = stream_of(ctx);
  // fast path: contiguous same-dtype copy of whole 16-byte vectors
  if (op == HB_UN_COPY && dt_x == dt_y && ys == nullptr) {
    bool contig = true;
    int64_t expect = 1;
    for (int d = rank - 1; d >= 0; d--) {
      if (shape[d] != 1 && xs[d] != expect) contig = false;
      expect *= shape[d];
    }
    int es = dt_size(dt_x);
    if (contig && ((n * es) % 16 == 0) && (x % 16 == 0) && (y % 16 == 0)) {
      int64_t n16 = n * es / 16;
      copy_bytes_kernel<<<grid_for(n16, 256), 256, 0, st>>>((const uint4v*)x, (uint4v*)y, n16);
      check_launch("hb_unary(copy)");
      return 0;
    }
  }
  int int_path = is_int_dt(dt_x) && is_int_dt(dt_y) &&
                 (op == HB_UN_COPY || op == HB_UN_NEG || op == HB_UN_ABS || op == HB_UN_NOT);
  unary_kernel<<<grid_for(n, 256), 256, 0, st>>>(op, dt_x, (const void*)x, dt_y, (void*)y, s, n, (float)alpha,
                                                  int_path, ys != nullptr);
  check_launch("hb_unary");
  HB_API_END
}

int hb_binary(uintptr_t ctx, int op, int dt_a, uintptr_t a, const int64_t* as, int dt_b, uintptr_t b,
              const int64_t* bs, int dt_y, uintptr_t y, const int64_t* shape, int rank) {
  HB_API_BEGIN
  Strided s = make_strided(shape, rank, as, bs, nullptr);
  int64_t n = numel(shape, rank);
  if (n == 0) return 0;
  bool cmp = op >= HB_BIN_EQ;
  int int_path = is_int_dt(dt_a) && is_int_dt(dt_b) && (cmp || is_int_dt(dt_y)) && op != HB_BIN_POW;
  binary_kernel<<<grid_for(n, 256), 256, 0, stream_of(ctx)>>>(op, dt_a, (const void*)a, dt_b, (const void*)b, dt_y,
                                                               (void*)y, s, n, int_path);
  check_launch("hb_binary");
  HB_API_END
}

int hb_where(uintptr_t ctx, uintptr_t cond, const int64_t* cs, int dt_a, uintptr_t a, const int64_t* as, int dt_b,
             uintptr_t b, const int64_t* bs, int dt_y, uintptr_t y, const int64_t* shape, int rank) {
  HB_API_BEGIN
  Strided s = make_strided(shape, rank, cs, as, bs);
  int64_t n = numel(shape, rank);
  if (n == 0) return 0;
  int int_path = is_int_dt(dt_a) && is_int_dt(dt_b) && is_int_dt(dt_y);
  where_kernel<<<grid_for(n, 256), 256, 0, stream_of(ctx)>>>((const uint8_t*)cond, dt_a, (const void*)a, dt_b,
                                                              (const void*)b, dt_y, (void*)y, s, n, int_path);
  check_launch("hb_where");
  HB_API_END
}

int hb_geglu(uintptr_t ctx, int dt_x, uintptr_t x, int64_t ldx, int dt_y, uintptr_t y, int64_t rows, int64_t F) {
  HB_API_BEGIN
  HB_REQUIRE(ldx >= 2 * F, "hb_geglu: ldx < 2F");
  int64_t n = rows * F;
  if (n == 0) return 0;
  geglu_kernel<<<grid_for(n, 256), 256, 0, stream_of(ctx)>>>(dt_x, (const void*)x, ldx, dt_y, (void*)y, rows, F);
  check_launch("hb_geglu");
  HB_API_END
}

int hb_gather(uintptr_t ctx, int dt, uintptr_t table, int64_t V, int64_t D, uintptr_t ids, int64_t n,
              int64_t batch_rows, int dt_out, uintptr_t out) {
  HB_API_BEGIN
  HB_REQUIRE(V > 0 || n == 0, "hb_gather: empty table");
  int64_t total = n * D;
  if (total == 0) return 0;
  const int es = dt_size(dt);
  if (dt == dt_out && (D * es) % 16 == 0 && table % 16 == 0 && out % 16 == 0) {
    gather16_kernel<<<grid_for(n * (D * es / 16), 256), 256, 0, stream_of(ctx)>>>(
        (const uint8_t*)table, V, D * es, (const int32_t*)ids, n, batch_rows, (uint8_t*)out);
    check_launch("hb_gather");
    return 0;
  }
  gather_kernel<<<grid_for(total, 256), 256, 0, stream_of(ctx)>>>(dt, (const void*)table, V, D,
                                                                   (const int32_t*)ids, n, batch_rows, dt_out,
                                                                   (void*)out);
  check_launch("hb_gather");
  HB_API_END
}

// Float sum / mean / max / min of contiguous rows of 64 or more values: one
// block of 256 threads per row, a wave tree and then the four waves in a
// fixed order.  Max and min keep reduce_kernel's rule: a NaN wins.
__device__ __forceinline__ float red_comb(int op, float a, float b) {
  if (op == HB_RED_SUM || op == HB_RED_MEAN) return a + b;
  if (op == HB_RED_MAX) return (b > a || b != b) ? b : a;
  return (b < a || b != b) ? b : a;
}

__global__ __launch_bounds__(256) void reduce_row_kernel(int op, int dt_x, const void* __restrict__ x, int64_t n,
                                                         int dt_y, void* __restrict__ y) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * n;
  const bool additive = op == HB_RED_SUM || op == HB_RED_MEAN;
  float acc = additive ? 0.f : load_f(x, base, dt_x);  // max / min: seeded with an element of the row
  for (int64_t j = threadIdx.x; j < n; j += 256) acc = red_comb(op, acc, load_f(x, base + j, dt_x));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc = red_comb(op, acc, __shfl_xor(acc, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x != 0) return;
  float v = red_comb(op, red_comb(op, red_comb(op, red[0], red[1]), red[2]), red[3]);
  if (op == HB_RED_MEAN) v /= (float)n;
  store_f(y, blockIdx.x, dt_y, v);
}

int hb_reduce(uintptr_t ctx, int op, int dt_x, uintptr_t x, int64_t outer, int64_t n, int64_t inner, int dt_y,
              uintptr_t y) {
  HB_API_BEGIN
  HB_REQUIRE(op >= HB_RED_SUM && op <= HB_RED_ARGMIN, "hb_reduce: bad op");
  HB_REQUIRE(n > 0 || op == HB_RED_SUM || op == HB_RED_MEAN, "hb_reduce: empty axis");
  int64_t total = outer * inner;
  if (total == 0) return 0;
  const bool fl = !is_int_dt(dt_x) || !is_int_dt(dt_y);  // reduce_kernel's float path
  if (fl && op <= HB_RED_MEAN && inner == 1 && n >= 64 && outer <= 0x7fffffff) {
    reduce_row_kernel<<<(unsigned)outer, 256, 0, stream_of(ctx)>>>(op, dt_x, (const void*)x, n, dt_y, (void*)y);
    check_launch("hb_reduce");
    return 0;
  }
  reduce_kernel<<<grid_for(total, 256), 256, 0, stream_of(ctx)>>>(op, dt_x, (const void*)x, outer, n, inner, dt_y,
                                                                   (void*)y);
  check_launch("hb_reduce");
  HB_API_END
}

// Softmax and sort of contiguous rows of 16..1024 values (the decision
// head's rows of marker scores): one block of 256 threads per row.  Softmax:
// block max and sum reductions in a fixed order.  Sort: the row goes through
// y in y's dtype first (the value scan_kernel sorts), then a bitonic sort in
// LDS on (value, original index) with NaN after every number and ties kept in
// their original order -- the result of scan_kernel's stable insertion
// sort, -0 / +0 order included.
constexpr int kRowMax = 1024;

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is free (a previous reduction has been read)
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : ((red[0] + red[1]) + red[2]) + red[3];
}

__global__ __launch_bounds__(256) void row_block_kernel(int op, int dt_x, const void* __restrict__ x, int64_t n,
                                                        int dt_y, void* __restrict__ y) {
  __shared__ float kf[kRowMax];
  __shared__ int32_t ki[kRowMax];
  __shared__ int32_t ix[kRowMax];
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * n;
  const int tid = threadIdx.x;
  if (op == HB_SCAN_SOFTMAX) {
    float m = -INFINITY;
    for (int64_t j = tid; j < n; j += 256) m = fmaxf(m, load_f(x, base + j, dt_x));
    m = block_reduce(m, true, red);
    float sum = 0.f;
    for (int64_t j = tid; j < n; j += 256) sum += expf(load_f(x, base + j, dt_x) - m);
    const float inv = 1.0f / block_reduce(sum, false, red);
    for (int64_t j = tid; j < n; j += 256) store_f(y, base + j, dt_y, expf(load_f(x, base + j, dt_x) - m) * inv);
    return;
  }
  const bool in_int = is_int_dt(dt_x), out_int = is_int_dt(dt_y);
  int P = 1;
  while (P < n) P <<= 1;
  for (int j = tid; j < P; j += 256) {
    if (j < n) {
      // through y's dtype, element by element in the same thread (no
      // cross-thread dependence on the global write)
      if (in_int) store_i(y, base + j, dt_y, load_i(x, base + j, dt_x));
      else store_f(y, base + j, dt_y, load_f(x, base + j, dt_x));
      if (out_int) ki[j] = load_i(y, base + j, dt_y);
      else kf[j] = load_f(y, base + j, dt_y);
    }
    ix[j] = j;  // j >= n: padding, after everything
  }
  __syncthreads();
  auto greater = [&](int a, int b) -> bool {  // slot a sorts after slot b
    const int ia = ix[a], ib = ix[b];
    const bool pa = ia >= n, pb = ib >= n;
    if (pa != pb) return pa;
    if (!pa) {
      if (out_int) {
        if (ki[a] != ki[b]) return ki[a] > ki[b];
      } else {
        const float fa = kf[a], fb = kf[b];
        const bool na = fa != fa, nb = fb != fb;
        if (na != nb) return na;
        if (!na && fa != fb) return fa > fb;
      }
    }
    return ia > ib;
  };
  for (int k = 2; k <= P; k <<= 1) {
    for (int jj = k >> 1; jj > 0; jj >>= 1) {
      for (int i = tid; i < P; i += 256) {
        const int l = i ^ jj;
        if (l > i && greater(i, l) == ((i & k) == 0)) {
          const int32_t t = ix[i];
          ix[i] = ix[l];
          ix[l] = t;
          if (out_int) {
            const int32_t u = ki[i];
            ki[i] = ki[l];
            ki[l] = u;
          } else {
            const float u = kf[i];
            kf[i] = kf[l];
            kf[l] = u;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int64_t j = tid; j < n; j += 256) {
    if (out_int) store_i(y, base + j, dt_y, ki[j]);
    else store_f(y, base + j, dt_y, kf[j]);
  }
}

int hb_scan(uintptr_t ctx, int op, int dt_x, uintptr_t x, int64_t outer, int64_t n, int64_t inner, int dt_y,
            uintptr_t y) {
  HB_API_BEGIN
  HB_REQUIRE(op >= HB_SCAN_SOFTMAX && op <= HB_SCAN_SORT, "hb_scan: bad op");
  int64_t total = outer * inner;
  if (total == 0 || n == 0) return 0;
  if (op != HB_SCAN_CUMSUM && inner == 1 && n >= 16 && n <= kRowMax && outer <= 0x7fffffff) {
    row_block_kernel<<<(unsigned)outer, 256, 0, stream_of(ctx)>>>(op, dt_x, (const void*)x, n, dt_y, (void*)y);
    check_launch("hb_scan");
    return 0;
  }
  scan_kernel<<<grid_for(total, 256), 256, 0, stream_of(ctx)>>>(op, dt_x, (const void*)x, outer, n, inner, dt_y,
                                                                 (void*)y);
  check_launch("hb_scan");
  HB_API_END
}

static void check_panel_args(const char* op, uintptr_t a, uintptr_t b, int64_t ld, int64_t M, int64_t K) {
  if (M < 0 || K <= 0 || K % 16 != 0 || ld < K || ld % 8 != 0 || a % 16 != 0 || b % 16 != 0)
    throw std::runtime_error(std::string(op) + ": needs K % 16 == 0, ld >= K, ld % 8 == 0 and 16-byte aligned buffers");
}

int hb_panel_pack(uintptr_t ctx, uintptr_t src, int64_t ld, uintptr_t dst, int64_t M, int64_t K) {
  HB_API_BEGIN
  check_panel_args("hb_panel_pack", src, dst, ld, M, K);
  const int64_t chunks = (M + 31) / 32 * 32 * (K / 8);
  if (chunks == 0) return 0;
  panel_pack_kernel<<<grid_for(chunks, 256), 256, 0, stream_of(ctx)>>>((const uint16_t*)src, ld, (uint4v*)dst, M, K,
                                                                        chunks);
  check_launch("hb_panel_pack");
  HB_API_END
}

int hb_panel_unpack(uintptr_t ctx, uintptr_t src, uintptr_t dst, int64_t ld, int64_t M, int64_t K) {
  HB_API_BEGIN
  check_panel_args("hb_panel_unpack", src, dst, ld, M, K);
  const int64_t chunks = (M + 31) / 32 * 32 * (K / 8);
  if (chunks == 0) return 0;
  panel_unpack_kernel<<<grid_for(chunks, 256), 256, 0, stream_of(ctx)>>>((const uint4v*)src, (uint16_t*)dst, ld, M,
                                                                          K, chunks);
  check_launch("hb_panel_unpack");
  HB_API_END
}

int hb_meanpool(uintptr_t ctx, int dt_x, uintptr_t x, uintptr_t mask, int64_t B, int64_t L, int64_t D,
                uintptr_t out) {
  HB_API_BEGIN
  int64_t total = B * D;
  if (total == 0) return 0;
  hipStream_t st = stream_of(ctx);
  if ((dt_x == HB_F16 || dt_x == HB_BF16) && D % 8 == 0 && x % 16 == 0 && L > 0 && B <= 65535) {
    // row slices: enough blocks to fill the device, at least 16 rows each
    const int64_t chunks = (D + 511) / 512;
    int64_t S = (4 * 256 + B * chunks - 1) / (B * chunks);
    S = S < 1 ? 1 : (S > 64 ? 64 : S);
    if (S > (L + 15) / 16) S = (L + 15) / 16;
    if (S < 1) S = 1;
    float* part = (float*)pool_alloc(ctx, (size_t)(S * B * D + S * B) * sizeof(float));
    float* cnt = part + S * B * D;
    dim3 grid((unsigned)chunks, (unsigned)S, (unsigned)B);
    if (dt_x == HB_BF16)
      meanpool16_partial<true><<<grid, 256, 0, st>>>((const uint16_t*)x, (const uint8_t*)mask, B, L, D, (int)S, part,
                                                     cnt);
    else
      meanpool16_partial<false><<<grid, 256, 0, st>>>((const uint16_t*)x, (const uint8_t*)mask, B, L, D, (int)S,
                                                      part, cnt);
    meanpool16_final<<<grid_for(total, 256), 256, 0, st>>>(part, cnt, B, D, (int)S, (float*)out);
    check_launch("hb_meanpool");
    pool_free(ctx, part);
    return 0;
  }
  meanpool_kernel<<<grid_for(total, 256), 256, 0, st>>>(dt_x, (const void*)x, (const uint8_t*)mask, B, L, D,
                                                        (float*)out);
  check_launch("hb_meanpool");
  HB_API_END
}

}  // extern "C"
