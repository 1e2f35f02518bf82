// Linear layers: y = x . w^T with f32 accumulation and fused epilogues, for
// 16-bit weights and for laya's quantized weight format (q8 / q4 with
// per-group scales and zeros).
//
// Three MFMA kernels, all on gfx950's v_mfma_f32_32x32x16_{f16,bf16} with the
// same operand order (W rows as the A operand, X rows as the B operand) and
// the same sequence of k16 steps, so a row's output bits do not depend on M:
// - gemm_mfma_arow (M >= 4096): persistent, 256 x 192 tiles, one wave per
//   SIMD; X rows in registers (loaded two stages ahead), W tiles
//   double-buffered in LDS; the output (and the residual, fetched into the
//   same LDS C tile) is staged in LDS and written during the first stages of
//   the block's next tile.  X and Y may be row-major or in panel order
//   (32-row x 16-column blocks of 1 KB laid out as MFMA operands);
// - gemm_slab (small M, K % 64 == 0): weight-stationary, the whole W slab of
//   a block in LDS, every X fragment in registers, one wait for memory;
// - gemm_mfma (the rest below M = 4096): 128 x 128 tiles, A and B
//   double-buffered in LDS, epilogue staged in LDS, 16-byte stores.
// W tiles are 64-wide K stages of 16-byte chunks XOR-swizzled by row so the
// fragment reads of consecutive rows spread over the LDS banks.  The
// epilogue adds the bias, rounds once to the storage type, applies GeGLU on
// (value, gate) column pairs held by the same lane, and adds the residual
// (y = round(round(x.w^T + b) + r), the linear-then-add order).  Quantized
// weights are dequantized to fl16(q*s + z) -- one correctly rounded f16 fma,
// the value host dequantization would upload -- by one routine (dequant8):
// in the 128 x 128 kernel's W loader, into the slab in LDS, and from
// M = 1024 on (unless the slab kernel takes the call) once per call into a
// pooled 16-bit copy that the 16-bit kernels then read (dequant_rows_kernel).
// Blocks walk the tile grid in an XCD-aware order: the hardware deals block b
// to XCD b % 8, so each XCD is given a contiguous run of row panels (their A
// rows and the whole W stay in that XCD's L2).
//
// gemm_simt is the f32 path (and the fallback for shapes the MFMA kernel's
// 16-byte loads cannot take: K or row strides not a multiple of 8).
#include <stdexcept>
#include <type_traits>

#include "gemm_kernels.h"

namespace hb {

const float* rope_table(uintptr_t ctx, int64_t L, int64_t D, double base);

// ------------------------------------------------------------------ SIMT kernel (f32 path, fallback)

struct QWs {  // quantized weight for the SIMT kernel (bits = 0: plain)
  const uint8_t* q;
  const void* scales;
  const void* zeros;
  int sdt;  // dtype of scales / zeros
  int G, group, bits, aff;
};

__device__ __forceinline__ float simt_w(int dt, const void* W, const QWs& qw, int64_t n, int k, int K) {
  if (qw.bits == 0) return load_f(W, n * K + k, dt);
  int code;
  if (qw.bits == 8) {
    uint8_t u = qw.q[n * K + k];
    code = qw.aff ? (int)u : (int)(int8_t)u;
  } else {
    uint8_t u = qw.q[n * (K / 2) + k / 2];
    int v = (k & 1) ? (u >> 4) : (u & 15);
    code = qw.aff ? v : ((v ^ 8) - 8);
  }
  int64_t gi = n * qw.G + k / qw.group;
  float s = load_f(qw.scales, gi, qw.sdt);
  // compose.ts:379-398: w = f32(f32(q*s) + z), rounded once to the compute dtype
  float w = (float)code * s;
  if (qw.aff) w = w + load_f(qw.zeros, gi, qw.sdt);
  return round_to(w, dt);
}

// 64x64 output tile, 256 threads x (4x4) outputs, K staged 16 at a time.
__global__ __launch_bounds__(256) void gemm_simt(int dt, const void* __restrict__ X, int64_t ldx,
                                                 const void* __restrict__ W, QWs qw, const void* __restrict__ bias,
                                                 const void* __restrict__ R, int64_t ldr, void* __restrict__ Y,
                                                 int64_t ldy, int M, int N, int K, int geglu) {
  __shared__ float As[16][64 + 1];
  __shared__ float Bs[2][16][64 + 1];
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[2][4][4] = {};
  const int nb = geglu ? 2 : 1;
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int q = tid; q < 16 * 64; q += 256) {
      int r = q / 16, kk = q % 16;
      int gm = m0 + r, gk = k0 + kk;
      As[kk][r] = (gm < M && gk < K) ? load_f(X, (int64_t)gm * ldx + gk, dt) : 0.f;
      for (int h = 0; h < nb; h++) {
        int gn = n0 + r;
        Bs[h][kk][r] = (gn < N && gk < K) ? simt_w(dt, W, qw, (int64_t)gn + (int64_t)h * N, gk, K) : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = As[kk][ty * 4 + i];
      for (int h = 0; h < nb; h++) {
#pragma unroll
        for (int j = 0; j < 4; j++) b[j] = Bs[h][kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) acc[h][i][j] = fmaf(a[i], b[j], acc[h][i][j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int gn = n0 + tx * 4 + j;
      if (gn >= N) continue;
      float v = acc[0][i][j] + (bias ? load_f(bias, gn, dt) : 0.f);
      v = round_to(v, dt);
      if (geglu) {
        float g = round_to(acc[1][i][j] + (bias ? load_f(bias, N + gn, dt) : 0.f), dt);
        v = gelu_erf(v) * g;
      }
      if (R) v = round_to(v, dt) + load_f(R, (int64_t)gm * ldr + gn, dt);
      store_f(Y, (int64_t)gm * ldy + gn, dt, v);
    }
  }
}

// Small outputs with a long K (M * N <= 16384, K >= 256: a classifier on
// pooled vectors, the decision head's layers): one wave per output element,
// lanes striding K with coalesced loads of the X row and the W row(s), then a
// wave reduction and gemm_simt's epilogue.  The tiled kernel would take one
// global round trip per 16 columns of K on a handful of blocks.
__global__ __launch_bounds__(256) void gemm_dot(int dt, const void* __restrict__ X, int64_t ldx,
                                                const void* __restrict__ W, QWs qw, const void* __restrict__ bias,
                                                const void* __restrict__ R, int64_t ldr, void* __restrict__ Y,
                                                int64_t ldy, int M, int N, int K, int geglu) {
  const int lane = threadIdx.x & 63;
  const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // output m * N + n, one per wave
  if (o >= (int64_t)M * N) return;                                   // whole waves
  const int m = (int)(o / N), n = (int)(o - (int64_t)m * N);
  float a0 = 0.f, a1 = 0.f;
  for (int k = lane; k < K; k += 64) {
    const float x = load_f(X, (int64_t)m * ldx + k, dt);
    a0 = fmaf(x, simt_w(dt, W, qw, n, k, K), a0);
    if (geglu) a1 = fmaf(x, simt_w(dt, W, qw, (int64_t)n + N, k, K), a1);
  }
  a0 = wave_sum(a0);
  a1 = wave_sum(a1);
  if (lane != 0) return;
  float v = a0 + (bias ? load_f(bias, n, dt) : 0.f);
  v = round_to(v, dt);
  if (geglu) {
    const float g = round_to(a1 + (bias ? load_f(bias, N + n, dt) : 0.f), dt);
    v = gelu_erf(v) * g;
  }
  if (R) v = round_to(v, dt) + load_f(R, (int64_t)m * ldr + n, dt);
  store_f(Y, (int64_t)m * ldy + n, dt, v);
}

static bool dot_shape(int64_t M, int64_t N, int64_t K) { return M * N <= 16384 && K >= 256; }

// Panel-order operands (HB_X_PANEL / HB_Y_PANEL) need K % 64 == 0 and one of
// the two kernels that take them: the large-M one (M >= 4096) or, for 16-bit
// weights, the small-M slab kernel (`slab`: the call takes it); a panel-order
// Y also a width of whole 16-column blocks and no residual.
static void check_panel(unsigned flags, bool mfma, bool slab, int64_t M, int64_t N_out, int64_t K, bool resid,
                        const char* op) {
  if (!(flags & (HB_X_PANEL | HB_Y_PANEL))) return;
  if (!mfma || !(arow_path(M) || slab) || K % 64 != 0)
    throw std::runtime_error(std::string(op) +
                             ": panel-order operands need f16/bf16, K % 64 == 0, 16-byte aligned operands and "
                             "M >= 4096, or (16-bit weights) the small-M slab kernel");
  if ((flags & HB_Y_PANEL) && (N_out % 16 != 0 || resid))
    throw std::runtime_error(std::string(op) + ": a panel-order y needs out % 16 == 0 and no residual");
}

static void check_linear_args(int dt, int64_t ldx, int64_t ldy, int64_t M, int64_t N, int64_t K, unsigned flags,
                              uintptr_t bias, uintptr_t resid, int64_t ldr) {
  HB_REQUIRE(dt == HB_F32 || dt == HB_F16 || dt == HB_BF16, "dtype must be f32, f16 or bf16");
  HB_REQUIRE(M >= 0 && N >= 0 && K >= 0, "negative size");
  HB_REQUIRE(M < (1ll << 31) && N < (1ll << 30) && K < (1ll << 30), "size too large");
  HB_REQUIRE(ldx >= K && ldy >= N, "leading dimension smaller than the row");
  HB_REQUIRE(!(flags & HB_EPI_BIAS) || bias, "bias flag without bias");
  HB_REQUIRE(!(flags & HB_EPI_RESID) || (resid && ldr >= N), "resid flag without resid");
}

}  // namespace hb

using namespace hb;

extern "C" int hb_linear(uintptr_t ctx, int dt, uintptr_t x, int64_t ldx, uintptr_t w, uintptr_t bias,
                         uintptr_t resid, int64_t ldr, uintptr_t y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                         unsigned flags) {
  HB_API_BEGIN
  try {
    check_linear_args(dt, ldx, ldy, M, N, K, flags, bias, resid, ldr);
  } catch (const std::exception& e) {
    throw std::runtime_error(std::string("hb_linear: ") + e.what());
  }
  bool geglu = flags & HB_EPI_GEGLU;
  const void* b = (flags & HB_EPI_BIAS) ? (const void*)bias : nullptr;
  const void* r = (flags & HB_EPI_RESID) ? (const void*)resid : nullptr;
  if (M == 0 || N == 0) return 0;
  hipStream_t st = stream_of(ctx);
  bool mfma = (dt == HB_F16 || dt == HB_BF16) && K > 0 && K % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 &&
              (!r || ldr % 8 == 0) && x % 16 == 0 && w % 16 == 0 && y % 16 == 0 && (!r || resid % 16 == 0);
  check_panel(flags, mfma, !arow_path(M) && slab_path(M, N, K, geglu, cu_count(ctx)), M, N, K, r != nullptr,
              "hb_linear");
  const unsigned pan = flags & (HB_X_PANEL | HB_Y_PANEL);
  if (mfma) {
    QW qw{nullptr, nullptr, nullptr, 0, 1};
    mfma_dtype<0, false, false>(dt, geglu, st, cu_count(ctx), pan, (const uint16_t*)x, ldx, (const uint16_t*)w, qw,
                                (const uint16_t*)b, (const uint16_t*)r, ldr, (uint16_t*)y, ldy, (int)M, (int)N, (int)K);
  } else {
    QWs qw{nullptr, nullptr, nullptr, 0, 0, 1, 0, 0};
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (dot_shape(M, N, K)) {
      gemm_dot<<<(unsigned)((M * N + 3) / 4), 256, 0, st>>>(dt, (const void*)x, ldx, (const void*)w, qw, b, r, ldr,
                                                           (void*)y, ldy, (int)M, (int)N, (int)K, geglu ? 1 : 0);
    } else {
      gemm_simt<<<grid, 256, 0, st>>>(dt, (const void*)x, ldx, (const void*)w, qw, b, r, ldr, (void*)y, ldy, (int)M,
                                      (int)N, (int)K, geglu ? 1 : 0);
    }
  }
  check_launch("hb_linear");
  HB_API_END
}

extern "C" int hb_linear_qkv(uintptr_t ctx, int dt, uintptr_t x, int64_t ldx, uintptr_t w, uintptr_t bias,
                             uintptr_t y, int64_t M, int64_t K, int64_t L, int64_t H, double rope_base,
                             unsigned flags) {
  HB_API_BEGIN
  HB_REQUIRE(dt == HB_F16 || dt == HB_BF16, "hb_linear_qkv: dtype must be f16 or bf16");
  HB_REQUIRE(arow_path(M) && M < (1ll << 31) && K > 0 && K % 64 == 0 && K < (1ll << 30),
             "hb_linear_qkv: needs M >= 4096 and K % 64 == 0");
  HB_REQUIRE(L > 0 && M % L == 0 && H > 0 && H < (1 << 20), "hb_linear_qkv: M must be a multiple of L, H > 0");
  HB_REQUIRE((flags & ~(unsigned)HB_X_PANEL) == 0 && bias == 0,
             "hb_linear_qkv: takes no bias and no flag but HB_X_PANEL");
  HB_REQUIRE(x % 16 == 0 && w % 16 == 0 && y % 16 == 0 && ((flags & HB_X_PANEL) || (ldx >= K && ldx % 8 == 0)),
             "hb_linear_qkv: operands must be 16-byte aligned (ldx % 8 == 0)");
  const float2* tab = rope_base > 0 ? (const float2*)rope_table(ctx, L, 64, rope_base) : nullptr;
  const QK qk{tab, (int)L, (int)H};
  const unsigned pan = flags & HB_X_PANEL;
  const int N = (int)(3 * H * 64);
  if (dt == HB_F16)
    launch_qkv<false>(stream_of(ctx), cu_count(ctx), pan, (const uint16_t*)x, ldx, (const uint16_t*)w, (uint16_t*)y,
                      (int)M, N, (int)K, qk);
  else
    launch_qkv<true>(stream_of(ctx), cu_count(ctx), pan, (const uint16_t*)x, ldx, (const uint16_t*)w, (uint16_t*)y,
                     (int)M, N, (int)K, qk);
  check_launch("hb_linear_qkv");
  HB_API_END
}

// Dequantizes rows [0, rows) of a quantized weight ([rows, K] codes, f16
// scales / zeros [rows, G]) into 16-bit weights, 8 per thread and step, with
// the GEMMs' own dequant8: the 16-bit GEMM on the result computes what the
// dequantizing kernels compute, bit for bit.
template <int QB, bool AFF, bool BF16>
__global__ __launch_bounds__(256) void dequant_rows_kernel(QW qw, uint16_t* __restrict__ out, int64_t rows, int K) {
  const int cpr = K >> 3;
  const int64_t n = rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cpr;
    const int c = (int)(i - r * cpr);
    uint32_t w0, w1 = 0;
    if constexpr (QB == 8) {
      const uint2v w = *(const uint2v*)(qw.q + r * K + 8 * c);
      w0 = w.x;
      w1 = w.y;
    } else {
      w0 = *(const uint32_t*)(qw.q + r * (K / 2) + 4 * c);
    }
    const int64_t gi = r * qw.G + (8 * c) / qw.group;
    const uint32_t sb = ((const uint16_t*)qw.scales)[gi], zb = AFF ? ((const uint16_t*)qw.zeros)[gi] : 0u;
    *(uint4v*)(out + r * K + 8 * c) = dequant8<QB, AFF, false, BF16>(w0, w1, sb, zb, 0.f, 0.f);
  }
}

template <int QB, bool AFF>
static void launch_dequant_rows(hipStream_t st, int cus, int dt, const QW& q, uint16_t* out, int64_t rows, int K) {
  const int64_t n = rows * (K / 8);
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, (int64_t)cus * 16);
  if (dt == HB_BF16) dequant_rows_kernel<QB, AFF, true><<<grid, 256, 0, st>>>(q, out, rows, K);
  else dequant_rows_kernel<QB, AFF, false><<<grid, 256, 0, st>>>(q, out, rows, K);
}

extern "C" int hb_qlinear(uintptr_t ctx, int dt, uintptr_t x, int64_t ldx, uintptr_t qw, uintptr_t scales,
                          uintptr_t zeros, uintptr_t bias, uintptr_t resid, int64_t ldr, uintptr_t y, int64_t ldy,
                          int64_t M, int64_t N, int64_t K, int bits, int group, int mode, unsigned flags) {
  HB_API_BEGIN
  try {
    check_linear_args(dt, ldx, ldy, M, N, K, flags, bias, resid, ldr);
  } catch (const std::exception& e) {
    throw std::runtime_error(std::string("hb_qlinear: ") + e.what());
  }
  HB_REQUIRE(bits == 8 || bits == 4, "hb_qlinear: bits must be 8 or 4");
  HB_REQUIRE(mode == 0 || mode == 1, "hb_qlinear: mode must be 0 (symmetric) or 1 (affine)");
  HB_REQUIRE(group > 0, "hb_qlinear: bad group size");
  HB_REQUIRE((K * bits) % 32 == 0, "hb_qlinear: in * bits must be a multiple of 32");
  HB_REQUIRE(qw && scales && (mode == 0 || zeros), "hb_qlinear: missing weight tensors");
  bool geglu = flags & HB_EPI_GEGLU;
  const void* b = (flags & HB_EPI_BIAS) ? (const void*)bias : nullptr;
  const void* r = (flags & HB_EPI_RESID) ? (const void*)resid : nullptr;
  if (M == 0 || N == 0) return 0;
  hipStream_t st = stream_of(ctx);
  int G = (int)((K + group - 1) / group);
  // scales / zeros are f16 [N, G]: the laya checkpoint format
  bool mfma = (dt == HB_F16 || dt == HB_BF16) && K > 0 && K % 8 == 0 && group % 8 == 0 && ldx % 8 == 0 &&
              ldy % 8 == 0 && (!r || ldr % 8 == 0) && x % 16 == 0 && y % 16 == 0 && (!r || resid % 16 == 0) &&
              qw % 8 == 0 && scales % 2 == 0 && zeros % 2 == 0;
  check_panel(flags, mfma, false, M, N, K, r != nullptr, "hb_qlinear");
  const unsigned pan = flags & (HB_X_PANEL | HB_Y_PANEL);
  if (mfma) {
    QW q{(const uint8_t*)qw, (const void*)scales, (const void*)zeros, G, group};
    const uint16_t* X = (const uint16_t*)x;
    const uint16_t* Bp = (const uint16_t*)b;
    const uint16_t* Rp = (const uint16_t*)r;
    uint16_t* Yp = (uint16_t*)y;
    int m = (int)M, n = (int)N, k = (int)K;
    const int cus0 = cu_count(ctx);
    const bool slab = slab_path(M, N, K, geglu, cus0) && qslab_ok(K, geglu ? 2 : 1, bits, mode == 1, q);
    if (arow_path(M) || (M >= 1024 && !slab && !thin_tiles(M, N, geglu, cus0))) {
      // At M >= 4096, and from M = 1024 where neither the slab kernel nor
      // 128 x 64 tiles take the call: the weight is dequantized once into a
      // pooled 16-bit copy and the 16-bit GEMM runs on it.  A loader that
      // dequantizes repeats the work for every row tile (at M = 8192:
      // 22-34% over 16-bit weights, against one bandwidth-bound pass over
      // the weight here).  With 128 x 64 tiles (many blocks, each a short
      // chain of K stages) the loader's dequantization is the faster of the
      // two (M = 2048: Wo 16.3 -> 14.6, Wqkv 27.9 -> 24.6 us).
      const int64_t rows = geglu ? 2 * N : N;
      struct PoolBlock {  // back to the pool when the call ends, by return or throw
        uintptr_t ctx;
        void* p;
        ~PoolBlock() { pool_free(ctx, p); }  // stream-ordered: reused only by work enqueued later
      } held{ctx, pool_alloc(ctx, (size_t)(rows * K * 2))};
      uint16_t* wd = (uint16_t*)held.p;
      const int cus = cu_count(ctx);
      if (bits == 8 && mode == 0) launch_dequant_rows<8, false>(st, cus, dt, q, wd, rows, k);
      else if (bits == 8) launch_dequant_rows<8, true>(st, cus, dt, q, wd, rows, k);
      else if (mode == 0) launch_dequant_rows<4, false>(st, cus, dt, q, wd, rows, k);
      else launch_dequant_rows<4, true>(st, cus, dt, q, wd, rows, k);
      check_launch("hb_qlinear (dequantize)");
      QW none{nullptr, nullptr, nullptr, 0, 1};
      mfma_dtype<0, false, false>(dt, geglu, st, cus, pan, X, ldx, wd, none, Bp, Rp, ldr, Yp, ldy, m, n, k);
    } else if (bits == 8 && mode == 0) mfma_dtype<8, false, false>(dt, geglu, st, cu_count(ctx), pan, X, ldx, nullptr, q, Bp, Rp, ldr, Yp, ldy, m, n, k);
    else if (bits == 8) mfma_dtype<8, true, false>(dt, geglu, st, cu_count(ctx), pan, X, ldx, nullptr, q, Bp, Rp, ldr, Yp, ldy, m, n, k);
    else if (mode == 0) mfma_dtype<4, false, false>(dt, geglu, st, cu_count(ctx), pan, X, ldx, nullptr, q, Bp, Rp, ldr, Yp, ldy, m, n, k);
    else mfma_dtype<4, true, false>(dt, geglu, st, cu_count(ctx), pan, X, ldx, nullptr, q, Bp, Rp, ldr, Yp, ldy, m, n, k);
  } else {
    QWs q{(const uint8_t*)qw, (const void*)scales, (const void*)zeros, HB_F16, G, group, bits, mode};
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (dot_shape(M, N, K)) {
      gemm_dot<<<(unsigned)((M * N + 3) / 4), 256, 0, st>>>(dt, (const void*)x, ldx, nullptr, q, b, r, ldr, (void*)y,
                                                           ldy, (int)M, (int)N, (int)K, geglu ? 1 : 0);
    } else {
      gemm_simt<<<grid, 256, 0, st>>>(dt, (const void*)x, ldx, nullptr, q, b, r, ldr, (void*)y, ldy, (int)M, (int)N,
                                      (int)K, geglu ? 1 : 0);
    }
  }
  check_launch("hb_qlinear");
  HB_API_END
}

// One dequantized table value: the code times its group's f16 scale (plus the
// f16 zero when affine).  f16 output: f16 arithmetic (an exact product rounded
// once, or one fused multiply-add); f32 output: one rounding of the exact value.
__device__ __forceinline__ float qg_value(int code, uint16_t s_bits, uint16_t z_bits, int aff, bool out_f16) {
  const float s = f16_bits_to_f32(s_bits);
  if (out_f16) {
    f16 sh = (f16)s, qh = (f16)(float)code;
    f16 w = aff ? __builtin_fmaf16(qh, sh, (f16)f16_bits_to_f32(z_bits)) : (f16)(qh * sh);
    return (float)w;
  }
  return aff ? fmaf((float)code, s, f16_bits_to_f32(z_bits)) : (float)code * s;  // q*s is exact in f32
}

__device__ __forceinline__ int qg_code(uint32_t u, int bits, int aff) {
  if (bits == 8) return aff ? (int)u : (int)(int8_t)(uint8_t)u;
  return aff ? (int)u : (((int)u ^ 8) - 8);
}

__global__ void qgather_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ scales,
                               const uint16_t* __restrict__ zeros, int64_t V, int64_t K, int bits, int G, int group,
                               int aff, const int32_t* __restrict__ ids, int64_t n, int dt_out,
                               void* __restrict__ out) {
  int64_t total = n * K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i / K, k = i - r * K;
    int64_t id = ids[r];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    uint32_t u;
    if (bits == 8) {
      u = q[id * K + k];
    } else {
      const uint8_t b = q[id * (K / 2) + k / 2];
      u = (k & 1) ? (b >> 4) : (b & 15);
    }
    int64_t gi = id * G + k / group;
    const float w = qg_value(qg_code(u, bits, aff), scales[gi], aff ? zeros[gi] : (uint16_t)0, aff,
                             dt_out == HB_F16);
    store_f(out, i, dt_out, w);
  }
}

// K % 8 == 0 and group % 8 == 0: one thread per 8 consecutive values of a
// row, which share one group.  One 8-byte (q8) or 4-byte (q4) code load, one
// scale (and zero) load, and 16-byte stores (one for f16, two for f32).  The
// values are qg_value's, as in qgather_kernel.
template <int BITS, bool OUT16>
__global__ __launch_bounds__(256) void qgather8_kernel(const uint8_t* __restrict__ q,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint16_t* __restrict__ zeros, int V, int K, int G,
                                                       int group, int aff, const int32_t* __restrict__ ids,
                                                       int chunks, void* __restrict__ out) {
  const int kc = K >> 3;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += gridDim.x * blockDim.x) {
    const int r = c / kc, k0 = (c - r * kc) << 3;
    int id = ids[r];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    uint32_t w0, w1 = 0;
    if (BITS == 8) {
      const uint2v v = *(const uint2v*)(q + (int64_t)id * K + k0);
      w0 = v.x;
      w1 = v.y;
    } else {
      w0 = *(const uint32_t*)(q + (int64_t)id * (K >> 1) + (k0 >> 1));
    }
    const int64_t gi = (int64_t)id * G + k0 / group;
    const uint16_t sb = scales[gi], zb = aff ? zeros[gi] : (uint16_t)0;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t u = BITS == 8 ? (((e < 4 ? w0 : w1) >> (8 * (e & 3))) & 255u) : ((w0 >> (4 * e)) & 15u);
      v[e] = qg_value(qg_code(u, BITS, aff), sb, zb, aff, OUT16);
    }
    const int64_t o = (int64_t)r * K + k0;
    if (OUT16) {
      uint4v pk;
      pk.x = (uint32_t)f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16);
      pk.y = (uint32_t)f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16);
      pk.z = (uint32_t)f32_to_f16_bits(v[4]) | ((uint32_t)f32_to_f16_bits(v[5]) << 16);
      pk.w = (uint32_t)f32_to_f16_bits(v[6]) | ((uint32_t)f32_to_f16_bits(v[7]) << 16);
      *(uint4v*)((uint16_t*)out + o) = pk;
    } else {
      float4v* d = (float4v*)((float*)out + o);
      d[0] = float4v{v[0], v[1], v[2], v[3]};
      d[1] = float4v{v[4], v[5], v[6], v[7]};
    }
  }
}

extern "C" int hb_qgather(uintptr_t ctx, uintptr_t qw, uintptr_t scales, uintptr_t zeros, int64_t V, int64_t K,
                          int bits, int group, int mode, uintptr_t ids, int64_t n, int dt_out, uintptr_t out) {
  HB_API_BEGIN
  HB_REQUIRE(bits == 8 || bits == 4, "hb_qgather: bits must be 8 or 4");
  HB_REQUIRE(group > 0 && V > 0, "hb_qgather: bad shape");
  HB_REQUIRE(mode == 0 || zeros, "hb_qgather: affine needs zeros");
  int64_t total = n * K;
  if (total == 0) return 0;
  int G = (int)((K + group - 1) / group);
  hipStream_t st = stream_of(ctx);
  const bool out16 = dt_out == HB_F16;
  if ((out16 || dt_out == HB_F32) && K % 8 == 0 && group % 8 == 0 && out % 16 == 0 && qw % (bits == 8 ? 8 : 4) == 0 &&
      ids % 4 == 0 && V < (1ll << 31) && K < (1ll << 30) && total / 8 < (1ll << 30)) {
    // chunks < 2^30: the grid-stride index stays below 2^31
    const int chunks = (int)(total / 8);
    const unsigned grid = grid_for(chunks, 256);
    const uint8_t* Q = (const uint8_t*)qw;
    const uint16_t *S = (const uint16_t*)scales, *Z = (const uint16_t*)zeros;
    const int32_t* I = (const int32_t*)ids;
    if (bits == 8 && out16)
      qgather8_kernel<8, true><<<grid, 256, 0, st>>>(Q, S, Z, (int)V, (int)K, G, group, mode, I, chunks, (void*)out);
    else if (bits == 8)
      qgather8_kernel<8, false><<<grid, 256, 0, st>>>(Q, S, Z, (int)V, (int)K, G, group, mode, I, chunks, (void*)out);
    else if (out16)
      qgather8_kernel<4, true><<<grid, 256, 0, st>>>(Q, S, Z, (int)V, (int)K, G, group, mode, I, chunks, (void*)out);
    else
      qgather8_kernel<4, false><<<grid, 256, 0, st>>>(Q, S, Z, (int)V, (int)K, G, group, mode, I, chunks, (void*)out);
    check_launch("hb_qgather");
    return 0;
  }
  qgather_kernel<<<grid_for(total, 256), 256, 0, st>>>((const uint8_t*)qw, (const uint16_t*)scales,
                                                                   (const uint16_t*)zeros, V, K, bits, G, group, mode,
                                                                   (const int32_t*)ids, n, dt_out, (void*)out);
  check_launch("hb_qgather");
  HB_API_END
}
