// MFMA GEMM kernels and their launchers (templates), shared by the
// translation units that instantiate them by weight format: gemm_f16.hip
// (16-bit weights), gemm_q8.hip and gemm_q4.hip (laya's quantized format);
// gemm.hip holds the entry points, the SIMT kernels and the dispatch.
#pragma once
#include <math.h>

#include <atomic>
#include <stdexcept>
#include <type_traits>

#include "common.h"

namespace hb {


// ------------------------------------------------------------------ helpers


template <bool BF16>
__device__ __forceinline__ float16v mfma32(const uint4v& a, const uint4v& b, float16v c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
  }
}

template <bool BF16>
__device__ __forceinline__ float to_f(uint32_t h) {
  return BF16 ? bf16_to_f32((uint16_t)h) : f16_bits_to_f32((uint16_t)h);
}
template <bool BF16>
__device__ __forceinline__ uint16_t from_f(float v) {
  return BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
}

// LDS element offset of 16-byte chunk c of row r in a [rows][64] u16 tile.
__device__ __forceinline__ int swz(int r, int c) { return r * 64 + ((c ^ (r & 7)) << 3); }

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane l
// fills LDS bytes [lds + 16 l, lds + 16 l + 16), `lds` being the wave's
// (wave-uniform) LDS byte address.  Issued from inline asm, so the compiler
// neither orders later LDS accesses behind it nor counts it in its own load
// waits (an extra load in flight only makes those waits stronger); the
// caller waits for it (vmcnt) before anything reads the destination.
__device__ __forceinline__ void lds_copy16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// Quantized code e (0..7) of a chunk: q8 codes are bytes of (w0, w1), q4
// codes nibbles of w0 (even column in the low nibble).
template <int QB, bool AFF>
__device__ __forceinline__ int qcode(uint32_t w0, uint32_t w1, int e) {
  if constexpr (QB == 8) {
    uint32_t w = e < 4 ? w0 : w1;
    int sh = 8 * (e & 3);
    return AFF ? (int)((w >> sh) & 0xff) : (int)(int8_t)((w >> sh) & 0xff);
  } else {
    int v = (int)((w0 >> (4 * e)) & 0xf);
    return AFF ? v : ((v ^ 8) - 8);
  }
}

// 8 dequantized weights as 16-bit values.  f16 with f16 scales: one f16 fma
// (q is exact in f16), so the weight is fl16(q*s + z) rounded once.  Other
// combinations compute in f32 and round once to the storage type.
template <int QB, bool AFF, bool SF32, bool BF16>
__device__ __forceinline__ uint4v dequant8(uint32_t w0, uint32_t w1, uint32_t sbits, uint32_t zbits, float sf,
                                           float zf) {
  uint32_t out[4];
  if constexpr (!SF32 && !BF16) {
    // Two codes per 32-bit word, each as the f16 1024 + c (c in 0..255 or
    // 0..15 is the low mantissa bits under the exponent of 1024, exact), then
    // one packed subtraction gives the code as f16 exactly and one packed
    // multiply (symmetric) or fma (affine) rounds q*s (+ z) once.
    const half2v s2 = __builtin_bit_cast(half2v, (sbits & 0xffffu) * 0x10001u);
    const half2v z2 = __builtin_bit_cast(half2v, (zbits & 0xffffu) * 0x10001u);
    uint32_t pr[4];  // value pairs (2e, 2e + 1) in the low bits of each half
    if constexpr (QB == 8) {
      // byte b of w0:w1 -> half (b & 1) of pair b / 2
      pr[0] = __builtin_amdgcn_perm(0u, w0, 0x0c010c00u);
      pr[1] = __builtin_amdgcn_perm(0u, w0, 0x0c030c02u);
      pr[2] = __builtin_amdgcn_perm(0u, w1, 0x0c010c00u);
      pr[3] = __builtin_amdgcn_perm(0u, w1, 0x0c030c02u);
    } else {
      // nibble e of w0 (e even: low nibble of byte e / 2)
      const uint32_t lo = w0 & 0x0f0f0f0fu, hi = (w0 >> 4) & 0x0f0f0f0fu;
#pragma unroll
      for (int p = 0; p < 4; p++) pr[p] = __builtin_amdgcn_perm(hi, lo, 0x0c040c00u + 0x00010001u * p);
    }
    // signed codes are stored offset by 2^(QB-1): q + 2^(QB-1) = c ^ 2^(QB-1)
    constexpr uint32_t flip = AFF ? 0u : (QB == 8 ? 0x00800080u : 0x00080008u);
    constexpr _Float16 base = AFF ? (_Float16)1024 : (_Float16)(1024 + (1 << (QB - 1)));
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const half2v q2 = __builtin_bit_cast(half2v, (pr[p] ^ flip) | 0x64006400u) - half2v{base, base};
      const half2v r2 = AFF ? __builtin_elementwise_fma(q2, s2, z2) : q2 * s2;
      out[p] = __builtin_bit_cast(uint32_t, r2);
    }
  } else {
    const float s = SF32 ? sf : f16_bits_to_f32((uint16_t)sbits);
    const float z = SF32 ? zf : f16_bits_to_f32((uint16_t)zbits);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float q0 = (float)qcode<QB, AFF>(w0, w1, e), q1 = (float)qcode<QB, AFF>(w0, w1, e + 1);
      float r0 = AFF ? fmaf(q0, s, z) : q0 * s;
      float r1 = AFF ? fmaf(q1, s, z) : q1 * s;
      out[e >> 1] = (uint32_t)from_f<BF16>(r0) | ((uint32_t)from_f<BF16>(r1) << 16);
    }
  }
  return uint4v{out[0], out[1], out[2], out[3]};
}

struct QW {  // quantized weight operand
  const uint8_t* q;
  const void* scales;
  const void* zeros;
  int G;      // groups per row
  int group;  // values per group
};

// The fused-projection epilogue (QKV): y = x . W^T with W the
// stacked [3 * H * 64, K] q / k / v projection, written head-major as
// [3][B][H][L][64] (B = M / L) with RoPE applied to the q and k parts.
struct QK {
  const float2* tab;  // RoPE cos / sin [L][32], or null: no rotation
  int L;              // sequence length (M = B * L)
  int H;              // heads (N = 3 * H * 64)
};

// Copies a [BM][BNO] 16-bit tile staged in LDS to Y with 16-byte coalesced
// stores; with a residual, y = round(tile + resid) (linear, then add).
template <bool BF16, int BM, int BNO, int NT>
__device__ __forceinline__ void write_tile(const uint16_t* Cs, int m0, int n0, int M, int N,
                                           const uint16_t* __restrict__ R, int64_t ldr, uint16_t* __restrict__ Y,
                                           int64_t ldy) {
  constexpr int CPR = BNO / 8;  // chunks per row
  for (int q = threadIdx.x; q < BM * CPR; q += NT) {
    const int r = q / CPR, c = q % CPR;
    const int gm = m0 + r, gn = n0 + c * 8;
    if (gm >= M || gn >= N) continue;
    uint4v v = *(const uint4v*)(Cs + r * BNO + c * 8);
    if (gn + 8 <= N) {
      if (R != nullptr) {
        uint4v rv = *(const uint4v*)(R + (int64_t)gm * ldr + gn);
        uint32_t vv[4] = {v.x, v.y, v.z, v.w};
        uint32_t rr[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          uint16_t lo = from_f<BF16>(to_f<BF16>(vv[e] & 0xffff) + to_f<BF16>(rr[e] & 0xffff));
          uint16_t hi = from_f<BF16>(to_f<BF16>(vv[e] >> 16) + to_f<BF16>(rr[e] >> 16));
          vv[e] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        v = uint4v{vv[0], vv[1], vv[2], vv[3]};
      }
      *(uint4v*)(Y + (int64_t)gm * ldy + gn) = v;
    } else {
      uint16_t vs[8];
      __builtin_memcpy(vs, &v, 16);
      for (int e = 0; e < 8 && gn + e < N; e++) {
        uint16_t o = vs[e];
        if (R != nullptr) o = from_f<BF16>(to_f<BF16>(o) + to_f<BF16>(R[(int64_t)gm * ldr + gn + e]));
        Y[(int64_t)gm * ldy + gn + e] = o;
      }
    }
  }
}

// ------------------------------------------------------------------ MFMA kernel

template <int BM, int BN, int WM, int WN, bool BF16, bool GEGLU, int QB, bool AFF, bool SF32>
__global__ __launch_bounds__(WM* WN * 64) void gemm_mfma(const uint16_t* __restrict__ X, int64_t ldx,
                                                         const uint16_t* __restrict__ W, QW qw,
                                                         const uint16_t* __restrict__ bias,
                                                         const uint16_t* __restrict__ R, int64_t ldr,
                                                         uint16_t* __restrict__ Y, int64_t ldy, int M, int N, int K,
                                                         int tiles_n) {
  constexpr int NT = WM * WN * 64;
  constexpr int BK = 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 blocks per wave
  constexpr int A_LD = BM * 8 / NT, B_LD = BN * 8 / NT;
  constexpr int BNO = GEGLU ? BN / 2 : BN;  // output columns per tile
  static_assert(A_LD * NT == BM * 8 && B_LD * NT == BN * 8, "tile/threads mismatch");
  static_assert(!GEGLU || (TN % 2 == 0), "GEGLU needs an even number of column blocks per wave");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* As = smem;                // [2][BM*64]
  uint16_t* Bs = smem + 2 * BM * BK;  // [2][BN*64]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int m0 = (tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BNO;  // first output column (pair index for GEGLU)

  // B tile row r -> W row (GEGLU: first half value rows, second half gate
  // rows).  wlane: byte offsets of the lane's W pieces from the tile's first
  // row of their half; load i holds rows 32i + tid/8, gate rows from
  // i = B_LD / 2 on.
  static_assert(!GEGLU || (B_LD % 2 == 0 && (B_LD / 2) * (NT / 8) == BN / 2), "GEGLU halves of the W loads");
  uint32_t wlane[B_LD];
#pragma unroll
  for (int i = 0; i < B_LD; i++) {
    const int q = tid + i * NT, r = q >> 3, c = q & 7;
    const int rr = GEGLU && r >= BN / 2 ? r - BN / 2 : r;
    wlane[i] = (uint32_t)(((int64_t)rr * K + c * 8) * 2);
  }
  auto w_row = [&](int r) -> int {
    if constexpr (GEGLU) return r < BN / 2 ? n0 + r : N + n0 + (r - BN / 2);
    else return n0 + r;
  };
  auto w_valid = [&](int r) -> bool {
    if constexpr (GEGLU) return n0 + (r < BN / 2 ? r : r - BN / 2) < N;
    else return n0 + r < N;
  };

  // One K stage in registers on its way to LDS.  16-bit weights: one set, a
  // stage loaded one stage before it is computed.  Quantized weights: two sets
  // rotate, a stage loaded two stages ahead, so the loads and the
  // dequantization behind them have two stages to complete (M = 512, q4:
  // 29 -> 23 us for Wqkv; the 16-bit kernel measured 1 us slower that way)
  struct RegSet {
    uint4v ra[A_LD], rb[B_LD];
    uint32_t rs[QB ? B_LD : 1], rz[QB ? B_LD : 1];
    float rsf[QB && SF32 ? B_LD : 1], rzf[QB && SF32 ? B_LD : 1];
  };
  auto load_regs = [&](RegSet& R, int k0) __attribute__((always_inline)) {
    uint4v(&ra)[A_LD] = R.ra;
    uint4v(&rb)[B_LD] = R.rb;
    auto& rs = R.rs;
    auto& rz = R.rz;
    auto& rsf = R.rsf;
    auto& rzf = R.rzf;
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      int q = tid + i * NT, r = q >> 3, c = q & 7;
      int k = k0 + c * 8;
      if (m0 + r < M && k < K) ra[i] = *(const uint4v*)(X + (int64_t)(m0 + r) * ldx + k);
      else ra[i] = uint4v{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int q = tid + i * NT, r = q >> 3, c = q & 7;
      int k = k0 + c * 8;
      bool ok = w_valid(r) && k < K;
      if constexpr (QB == 0) {
        rb[i] = ok ? *(const uint4v*)(W + (int64_t)w_row(r) * K + k) : uint4v{0, 0, 0, 0};
      } else {
        rb[i] = uint4v{0, 0, 0, 0};
        rs[i] = rz[i] = 0;
        if constexpr (SF32) rsf[i] = rzf[i] = 0.f;
        if (ok) {
          int64_t row = w_row(r);
          if constexpr (QB == 8) {
            uint2v w = *(const uint2v*)(qw.q + row * K + k);
            rb[i].x = w.x;
            rb[i].y = w.y;
          } else {
            rb[i].x = *(const uint32_t*)(qw.q + row * (K / 2) + k / 2);
          }
          int64_t gi = row * qw.G + k / qw.group;
          if constexpr (SF32) {
            rsf[i] = ((const float*)qw.scales)[gi];
            if constexpr (AFF) rzf[i] = ((const float*)qw.zeros)[gi];
          } else {
            rs[i] = ((const uint16_t*)qw.scales)[gi];
            if constexpr (AFF) rz[i] = ((const uint16_t*)qw.zeros)[gi];
          }
        }
      }
    }
  };
  auto store_lds = [&](int buf, const RegSet& R) __attribute__((always_inline)) {
    const uint4v(&ra)[A_LD] = R.ra;
    const uint4v(&rb)[B_LD] = R.rb;
    const auto& rs = R.rs;
    const auto& rz = R.rz;
    const auto& rsf = R.rsf;
    const auto& rzf = R.rzf;
    uint16_t* a = As + buf * BM * BK;
    uint16_t* b = Bs + buf * BN * BK;
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      int q = tid + i * NT, r = q >> 3, c = q & 7;
      *(uint4v*)(a + swz(r, c)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int q = tid + i * NT, r = q >> 3, c = q & 7;
      if constexpr (QB == 0) {
        *(uint4v*)(b + swz(r, c)) = rb[i];
      } else {
        float sf = 0.f, zf = 0.f;
        if constexpr (SF32) {
          sf = rsf[i];
          zf = rzf[i];
        }
        *(uint4v*)(b + swz(r, c)) = dequant8<QB, AFF, SF32, BF16>(rb[i].x, rb[i].y, rs[i], rz[i], sf, zf);
      }
    }
  };

  // column block tn of this wave -> tile column (B tile row)
  auto bcol = [&](int tn) -> int {
    if constexpr (GEGLU) {
      constexpr int H = TN / 2;
      return tn < H ? wn * (WTN / 2) + tn * 32 : BN / 2 + wn * (WTN / 2) + (tn - H) * 32;
    } else {
      return wn * WTN + tn * 32;
    }
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
  const int l32 = lane & 31, lg = lane >> 5;

  const int KT = (K + BK - 1) / BK;
  constexpr int AHEAD = QB ? 2 : 1;  // register sets, stages loaded ahead
  RegSet R0, R1;
  load_regs(R0, 0);
  if (AHEAD == 2 && KT > 1) load_regs(R1, BK);
  store_lds(0, R0);
  __syncthreads();
  // stage kt: loads stage kt + AHEAD into `rfree` (AHEAD = 2: its previous
  // stage is in LDS already; AHEAD = 1: rfree is rnext), computes stage kt
  // from LDS, stages kt + 1 (held in `rnext`) into the other LDS buffer
  auto stage = [&](int kt, RegSet& rnext, RegSet& rfree) __attribute__((always_inline)) {
    const int buf = kt & 1;
    if (kt + AHEAD < KT) load_regs(rfree, (kt + AHEAD) * BK);
    const uint16_t* a = As + buf * BM * BK;
    const uint16_t* b = Bs + buf * BN * BK;
    // k16 substeps in increasing k; W rows as the A operand and X rows as
    // the B operand, the order the large-M kernel uses, so both kernels
    // produce the same bits for a row whatever M is
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int c = 2 * s + lg;
      uint4v af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = *(const uint4v*)(a + swz(wm * WTM + i * 32 + l32, c));
#pragma unroll
      for (int j = 0; j < TN; j++) bf[j] = *(const uint4v*)(b + swz(bcol(j) + l32, c));
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = mfma32<BF16>(bf[j], af[i], acc[i][j]);
    }
    if (kt + 1 < KT) store_lds(buf ^ 1, rnext);
    __syncthreads();
  };
  if constexpr (AHEAD == 2) {
    for (int kt = 0; kt < KT; kt += 2) {
      stage(kt, R1, R0);
      if (kt + 1 < KT) stage(kt + 1, R0, R1);
    }
  } else {
    for (int kt = 0; kt < KT; kt++) stage(kt, R0, R0);
  }

  // ---- epilogue: bias, one rounding, GeGLU, stage in LDS as [BM][BNO];
  // lane l holds row l % 32 and columns 8*(r/4) + 4*(l/32) + {0..3}
  uint16_t* Cs = smem;
  constexpr int OUT_TN = GEGLU ? TN / 2 : TN;
  constexpr int WTNO = GEGLU ? WTN / 2 : WTN;
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int orow = wm * WTM + i * 32 + l32;
#pragma unroll
    for (int j = 0; j < OUT_TN; j++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int ocol = wn * WTNO + j * 32 + 8 * g + 4 * lg;  // tile output column of element 0
        uint16_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int gcol = n0 + ocol + e;
          float bv = 0.f, bg = 0.f;
          if (bias != nullptr && gcol < N) {
            bv = to_f<BF16>(bias[gcol]);
            if constexpr (GEGLU) bg = to_f<BF16>(bias[N + gcol]);
          }
          float v = to_f<BF16>(from_f<BF16>(acc[i][j][4 * g + e] + bv));
          if constexpr (GEGLU) {
            const float gt = to_f<BF16>(from_f<BF16>(acc[i][j + TN / 2][4 * g + e] + bg));
            v = pin_f32(gelu_fast(v) * gt);  // the f32 product, then one rounding to the storage type
          }
          o[e] = from_f<BF16>(v);
        }
        *(uint2v*)(Cs + orow * BNO + ocol) =
            uint2v{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      }
    }
  }
  __syncthreads();

  write_tile<BF16, BM, BNO, NT>(Cs, m0, n0, M, N, R, ldr, Y, ldy);
}

// ------------------------------------------------------------------ small-M MFMA kernel

// Small-M GEMM for 16-bit weights (M < 4096, K % 64 == 0): weight-stationary,
// one memory round trip.  A block of two or four waves owns a slab of
// 32*TN W rows (the output columns n0 .. n0 + 32*TNO, and with GeGLU their
// gate rows too) and one 32-row block of X per wave.  Everything a wave needs is
// requested at once before anything is waited for: its X fragments for P k16
// steps (P = K/16 when that fits in registers), its residual and bias values,
// and its share of the whole slab, which goes to LDS with direct-to-LDS loads
// (global_load_lds: 16 bytes per lane, whole 128-byte lines of 8 rows per
// instruction), so the kernel waits for memory once.  What bounds it is the
// X fragment loads (32 rows x 32 bytes per 1 KB instruction), which a CU's L1
// serves at about 15 bytes per clock; the launcher uses the kernel while its
// blocks fit one per CU (Wqkv at M = 128: 72 blocks, 11 us against 15 us for
// the 128 x 128 kernel, which ran 18 blocks).
// The k16 steps then run in ascending order with the same MFMA, operand
// order (W rows as the A operand, X rows as the B operand) and epilogue as
// the other kernels, so a row's bits do not depend on M.
// Slab layout: 1 KB blocks of 8 rows x 64 k, block (r/8)*KB + k/64 (KB = K/64),
// 16-byte chunk c of row r at slot (r%8)*8 + (c ^ (r%8)), so the 8 lanes of a
// fragment read that share a row group hit 8 distinct bank groups.  Blocks
// are numbered row-chunk-fastest and dealt to XCDs in contiguous runs: the
// blocks that read one slab share an XCD's L2.
//
// Quantized weights (QB = 8 or 4, f16 scales and zeros, groups a multiple of
// 8): the slab's codes (its rows are contiguous runs of the code matrix) and
// its scales and zeros go to LDS by direct-to-LDS loads beside the f16 slab,
// and after the one wait every thread dequantizes its share of the slab's
// 8-weight chunks into the f16 slab (dequant8, the other kernels' rounding),
// so the MFMA steps and their bits are those of the 16-bit path.
template <int TN, int P, bool BF16, bool GEGLU, int QB = 0, bool AFF = false>
__global__ __launch_bounds__(256) void gemm_slab(const uint16_t* __restrict__ X, int64_t ldx,
                                                 const uint16_t* __restrict__ W, QW qw,
                                                 const uint16_t* __restrict__ bias,
                                                 const uint16_t* __restrict__ R, int64_t ldr, uint16_t* __restrict__ Y,
                                                 int64_t ldy, int M, int N, int K, int chunks, int xpan, int ypan) {
  constexpr int TNO = GEGLU ? TN / 2 : TN;  // output column blocks
  constexpr int SR = 32 * TN;               // slab rows
  static_assert(!GEGLU || TN % 2 == 0, "GEGLU needs value and gate blocks");
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, lg = lane >> 5;
  const int nw = blockDim.x >> 6;  // waves per block (2 or 4): 32 rows of X each
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int nt = t / chunks, mc = t - nt * chunks;
  const int n0 = nt * 32 * TNO;
  const int KB = K >> 6, S = K >> 4;  // 64-wide k blocks, k16 steps
  const int row = (mc * nw + wave) * 32 + l32;  // this lane's output row
  // X row-major, or in panel order (xpan: 32-row x 16-column blocks of 1 KB
  // in MFMA operand order, rows padded to a multiple of 32), where one
  // fragment load reads one whole block; rows past the operand are clamped
  const int mlim = xpan ? (M + 31) & ~31 : M, rc = row < mlim ? row : mlim - 1;
  const int64_t xoff = xpan ? (int64_t)(rc >> 5) * 32 * K + (rc & 31) * 8 + 256 * lg : (int64_t)rc * ldx + 8 * lg;
  const int xstep = xpan ? 512 : 16;  // elements per k16 step

  uint4v xf[P];
#pragma unroll
  for (int p = 0; p < P; p++) xf[p] = *(const uint4v*)(X + xoff + xstep * p);
  // epilogue inputs: the residual and the bias of the lane's 4-column groups
  // (8-byte loads where aligned: R rows are, ldr % 8 == 0; the bias may be a
  // view at any offset, and its gate half starts at N)
  const bool bvec = bias != nullptr && ((uintptr_t)bias & 7) == 0 && (!GEGLU || (N & 3) == 0);
  uint2v rres[TNO][4], rb[TNO][4], rbg[TNO][4];
#pragma unroll
  for (int j = 0; j < TNO; j++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int col = n0 + 32 * j + 8 * g + 4 * lg;
      const bool whole = row < M && col + 4 <= N;
      rres[j][g] = R != nullptr && whole ? *(const uint2v*)(R + (int64_t)row * ldr + col) : uint2v{0, 0};
      rb[j][g] = bvec && col + 4 <= N ? *(const uint2v*)(bias + col) : uint2v{0, 0};
      rbg[j][g] = GEGLU && bvec && col + 4 <= N ? *(const uint2v*)(bias + N + col) : uint2v{0, 0};
    }
  // slab row r -> W row (GeGLU: gate rows from SR / 2 on); rows past N are
  // clamped, their outputs never stored
  auto slab_wrow = [&](int r) -> int {
    const bool gate = GEGLU && r >= SR / 2;
    const int cc = n0 + (gate ? r - SR / 2 : r);
    return (cc < N ? cc : N - 1) + (gate ? N : 0);
  };
  const int nq = (SR / 8) * KB;
  // quantized: codes [SR][K * QB / 8 bytes], then scales and zeros [SR][G],
  // each f16 in the low half of a 32-bit slot (a 2-byte direct-to-LDS load
  // writes lane l's value at 4 l), after the f16 slab
  constexpr int CRB = QB ? 8 / QB : 1;  // weights per code byte (QB = 4: 2)
  const int rowb = QB ? K / CRB : 0;     // code bytes per row
  uint8_t* codes = (uint8_t*)(smem + SR * K);
  uint32_t* szs = (uint32_t*)(codes + SR * rowb);
  if constexpr (QB == 0) {
    // the slab: DMA instruction q (of wave q % nw) fills block q, i.e. slab
    // rows 8 * (q / KB) + lane / 8, k block q % KB; lane l fetches chunk
    // (l%8) ^ (row%8)
    for (int q = wave; q < nq; q += nw) {
      const int rb8 = q / KB, kb = q - rb8 * KB;
      const int r = rb8 * 8 + (lane >> 3), c = (lane & 7) ^ (r & 7);
      __builtin_amdgcn_global_load_lds((const void*)(W + (int64_t)slab_wrow(r) * K + kb * 64 + c * 8),
                                       (__attribute__((address_space(3))) void*)(smem + q * 512), 16, 0, 0);
    }
  } else {
    // codes: instruction q fills bytes [1024 q, 1024 q + 1024) of the code
    // block, 16 of one row per lane (rowb % 16 == 0)
    const int ncq = SR * rowb / 1024;
    for (int q = wave; q < ncq; q += nw) {
      const int b = q * 1024 + lane * 16, r = b / rowb;
      __builtin_amdgcn_global_load_lds((const void*)(qw.q + (int64_t)slab_wrow(r) * rowb + (b - r * rowb)),
                                       (__attribute__((address_space(3))) void*)(codes + q * 1024), 16, 0, 0);
    }
    // scales (then zeros): 2 bytes per lane into 4-byte slots, instruction q
    // entries [64 q, 64 q + 64) of the slab's [SR][G]
    const int G = qw.G, nsq = (SR * G + 63) / 64;
    for (int q = wave; q < (AFF ? 2 : 1) * nsq; q += nw) {
      const bool zq = q >= nsq;
      const int e = (zq ? q - nsq : q) * 64 + lane, r = e / G;
      if (e < SR * G)
        __builtin_amdgcn_global_load_lds(
            (const void*)((const uint16_t*)(zq ? qw.zeros : qw.scales) + (int64_t)slab_wrow(r) * G + (e - r * G)),
            (__attribute__((address_space(3))) void*)(szs + (zq ? SR * G : 0) + (q - (zq ? nsq : 0)) * 64), 2, 0,
            0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): everything above has landed
  __syncthreads();
  if constexpr (QB != 0) {
    // dequantize: chunk i (8 weights) is slab row i / (K/8), chunk i % (K/8)
    // of the row, into the f16 slab's layout
    const int cpr = K >> 3, G = qw.G, nth = nw * 64;
    for (int i = tid; i < SR * cpr; i += nth) {
      const int r = i / cpr, c = i - r * cpr;
      uint32_t w0, w1 = 0;
      if constexpr (QB == 8) {
        const uint2v w = *(const uint2v*)(codes + r * rowb + 8 * c);
        w0 = w.x;
        w1 = w.y;
      } else {
        w0 = *(const uint32_t*)(codes + r * rowb + 4 * c);
      }
      const int gi = r * G + (8 * c) / qw.group;
      const uint32_t sb = szs[gi] & 0xffffu, zb = AFF ? szs[SR * G + gi] & 0xffffu : 0u;
      *(uint4v*)(smem + ((r >> 3) * KB + (c >> 3)) * 512 + (r & 7) * 64 + (((c & 7) ^ (r & 7)) << 3)) =
          dequant8<QB, AFF, false, BF16>(w0, w1, sb, zb, 0.f, 0.f);
    }
    __syncthreads();
  }
  if ((mc * nw + wave) * 32 >= M) return;  // a wave past the last row (after the barriers: its share is done)

  // W fragment of column block j, k16 step s (slab row 32 j + l32)
  auto wfrag = [&](int j, int s) __attribute__((always_inline)) -> uint4v {
    const int r = 32 * j + l32, c = (2 * s + lg) & 7;
    return *(const uint4v*)(smem + ((r >> 3) * KB + (s >> 2)) * 512 + (r & 7) * 64 + ((c ^ (r & 7)) << 3));
  };
  float16v acc[TN];
#pragma unroll
  for (int j = 0; j < TN; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[j][e] = 0.f;
  for (int s0 = 0; s0 < S; s0 += P) {  // S % P == 0
#pragma unroll
    for (int p = 0; p < P; p++) {
      uint4v b[TN];
#pragma unroll
      for (int j = 0; j < TN; j++) b[j] = wfrag(j, s0 + p);
#pragma unroll
      for (int j = 0; j < TN; j++) acc[j] = mfma32<BF16>(b[j], xf[p], acc[j]);
      if (s0 + P < S) xf[p] = *(const uint4v*)(X + xoff + xstep * (s0 + P + p));  // K longer than the registers
    }
  }

  // bias, one rounding, GeGLU on the lane's (value, gate) pair, the residual,
  // as the other kernels; lane l holds row l % 32 and columns 8*g + 4*(l/32) +
  // {0..3} of each column block
  if (row >= M) return;
#pragma unroll
  for (int j = 0; j < TNO; j++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int col = n0 + 32 * j + 8 * g + 4 * lg;
      if (col >= N) continue;
      const bool whole = col + 4 <= N;
      const uint32_t bw[2] = {rb[j][g].x, rb[j][g].y}, bgw[2] = {rbg[j][g].x, rbg[j][g].y};
      const uint32_t rw[2] = {rres[j][g].x, rres[j][g].y};
      uint16_t o[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float bv = 0.f, bg = 0.f;
        if (bias != nullptr) {
          if (whole && bvec) {
            bv = to_f<BF16>((bw[e >> 1] >> (16 * (e & 1))) & 0xffff);
            if constexpr (GEGLU) bg = to_f<BF16>((bgw[e >> 1] >> (16 * (e & 1))) & 0xffff);
          } else if (col + e < N) {
            bv = to_f<BF16>(bias[col + e]);
            if constexpr (GEGLU) bg = to_f<BF16>(bias[N + col + e]);
          }
        }
        float v = to_f<BF16>(from_f<BF16>(acc[j][4 * g + e] + bv));
        if constexpr (GEGLU) {
          const float gt = to_f<BF16>(from_f<BF16>(acc[j + TN / 2][4 * g + e] + bg));
          v = pin_f32(gelu_fast(v) * gt);  // the f32 product, then one rounding to the storage type
        }
        o[e] = from_f<BF16>(v);
        if (R != nullptr) {
          const uint16_t r16 = whole ? (uint16_t)((rw[e >> 1] >> (16 * (e & 1))) & 0xffff)
                                     : (col + e < N ? R[(int64_t)row * ldr + col + e] : (uint16_t)0);
          o[e] = from_f<BF16>(to_f<BF16>(o[e]) + to_f<BF16>(r16));
        }
      }
      // row-major, or panel order (ypan: N % 16 == 0, so the 4 columns are
      // whole and 8 bytes of one 16-byte chunk of a 1 KB block)
      uint16_t* yp = ypan ? Y + ((int64_t)(row >> 5) * (N >> 4) + (col >> 4)) * 512 +
                                (((col >> 3) & 1) * 32 + (row & 31)) * 8 + (col & 7)
                          : Y + (int64_t)row * ldy + col;
      if (whole) {
        *(uint2v*)yp = uint2v{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      } else {
        for (int e = 0; col + e < N; e++) yp[e] = o[e];
      }
    }
  }
}

// ------------------------------------------------------------------ large-M MFMA kernel


// Persistent GEMM over 256 x BN output tiles.  Four waves are stacked along
// M: each wave owns 64 rows and every column of the tile as 2 x (BN/32)
// blocks of v_mfma_f32_32x32x16 (on gfx950 the 32x32 MFMA runs at twice the
// rate of the 16x16x32 one, and reaches it from a single wave per SIMD).
// A wave's A rows are private, so they go from global memory straight into
// MFMA operand registers; only the weight tile is shared, through
// double-buffered LDS.
//
// One block per CU walks a list of tiles as one continuous stream of
// 64-wide K stages: loads run two stages ahead (three A and two W register
// sets rotating by name, issued between the MFMAs) and cross tile
// boundaries, so the next tile's first stages arrive while the current tile
// finishes.  Blocks on one XCD (block b runs on XCD b % 8) take consecutive
// tiles, which share A rows in that XCD's L2.
//
// The MFMA computes the transposed product (W rows as the A operand, X rows
// as the B operand): lane l then holds output row l % 32 and the four
// consecutive columns 8*(r/4) + 4*(l/32) + {0..3} of each accumulator, so the
// epilogue writes 8-byte pieces of Y straight from registers.
//
// QKV (16-bit weights, no GeGLU, no bias, no residual): the epilogue of the fused
// q / k / v projection (struct QK): each 64-column head of the tile is a pair
// of column blocks whose lanes hold the rotation partners d and d + 32 at the
// same register, so RoPE is applied in registers, and the tile leaves
// head-major.
template <int BN, bool BF16, bool GEGLU, bool KTAIL, bool QKV = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_mfma_arow(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ R, int64_t ldr, uint16_t* __restrict__ Y, int64_t ldy, int M, int N, int K,
    int tiles_n, int tiles, int xpan, int ypan, QK qk) {
  static_assert(!QKV || (!GEGLU && BN % 64 == 0), "QKV: no GeGLU, whole heads per tile");
  constexpr int NT = 256, BM = 256, BK = 64;
  constexpr int TM = 2, TN = BN / 32;  // 32x32 blocks per wave
  constexpr int KS = BK / 16;          // k16 substeps per stage
  constexpr int B_LD = BN * 8 / NT;
  constexpr int BNO = GEGLU ? BN / 2 : BN;
  static_assert(B_LD * NT == BN * 8 && BN % 32 == 0, "BN must be a multiple of 32");
  static_assert(!GEGLU || (TN % 2 == 0), "GEGLU needs an even number of column blocks");
  static_assert((BM * (BNO / 8)) % NT == 0, "write-out assumes whole rounds of chunks");

  constexpr int CPR = BNO / 8;           // 16-byte chunks per output row
  constexpr int RG = (CPR + 7) / 8;      // C tile: groups of 8 chunks per row
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* Bs = smem;               // [2][BN*64] W tiles
  uint16_t* Cs = smem + 2 * BN * BK;  // [RG][BM][8] 16-byte chunks: residual in, output out

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lg = lane >> 5;

  // This block's tiles (gridDim.x % 8 == 0).  XCD x owns the row panels
  // [mb0, mb1) with every column tile, and its blocks take the panel's tiles
  // column-tile-major: local tile l = slot + i * nx is row panel mb0 + l % mx,
  // column tile l / mx.  The tiles one XCD computes at a time then share a
  // few column tiles of W and cycle over the XCD's own rows of X, which stay
  // in its L2 from one column tile to the next.
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, nx = gridDim.x >> 3;
  const int tiles_m = tiles / tiles_n;
  const int mb0 = xcd * tiles_m / 8, mx = (xcd + 1) * tiles_m / 8 - mb0;
  const int nloc = mx * tiles_n;
  const int ntile = nloc > slot ? (nloc - slot + nx - 1) / nx : 0;
  if (ntile == 0) return;
  const int KT = (K + BK - 1) / BK;
  const int S = ntile * KT;  // stages in this block's stream
  auto tile_m0 = [&](int i) { return (mb0 + (slot + i * nx) % mx) * BM; };
  auto tile_n0 = [&](int i) { return ((slot + i * nx) / mx) * BNO; };

  // X is row-major (x[row * ldx + k]) or in panel order (xpan; 32-row x
  // 16-column blocks of 1 KB in MFMA operand order, rows padded to a multiple
  // of 32).  For k % 8 == 0 both are x[xs_hi * (row / 32) + xs_lo * (row % 32)
  // + xk * k]; in panel order one fragment load then reads one whole block.
  const int64_t xs_hi = xpan ? (int64_t)32 * K : (int64_t)32 * ldx;
  const int64_t xs_lo = xpan ? 8 : ldx;
  const int xk = xpan ? 32 : 1;
  const int mlim = xpan ? ((M + 31) & ~31) : M;
  // Loads are branch-free: addresses are clamped into the operand.  Rows past
  // M (A) or N (W) only feed outputs that are never stored, so they need no
  // zeroing; a K tail (K % 64 != 0, KTAIL, row-major X only) is zeroed.
  //
  // Without a K tail the loads are buffer loads: the resource's base is the
  // first row of the tile (wave-uniform, 64-bit), the lanes' offsets from it
  // are kernel constants and the K position is the scalar offset, so a stage
  // spends no vector instructions on addresses.  Rows past the operand lie
  // outside the resource's range and read 0.
  constexpr bool BUFX = !KTAIL, BUFW = !KTAIL;
  constexpr int BUF_FLAGS = 0x00020000;  // resource word 3: 32-bit raw data
  uint32_t xlane[TM];                    // byte offsets of the lane's rows in a tile
#pragma unroll
  for (int rb = 0; rb < TM; rb++) {
    const int lr = wave * 64 + rb * 32 + l32;
    xlane[rb] = (uint32_t)(((lr >> 5) * xs_hi + (lr & 31) * xs_lo + xk * lg * 8) * 2);
  }
  const int64_t x_elems = xpan ? (int64_t)mlim * K : (int64_t)(M - 1) * ldx + K;
  auto load_a = [&](int m0, int k0, uint4v (&a)[TM][KS]) {
    if constexpr (BUFX) {
      const int64_t base = xpan ? (int64_t)(m0 >> 5) * xs_hi : (int64_t)m0 * ldx;
      const int64_t left = (x_elems - base) * 2;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(X + base), (short)0, (int)(left < 0x7ffffff0 ? left : 0x7ffffff0), BUF_FLAGS);
#pragma unroll
      for (int rb = 0; rb < TM; rb++)
#pragma unroll
        for (int s = 0; s < KS; s++)
          a[rb][s] = __builtin_amdgcn_raw_buffer_load_b128(rs, xlane[rb], (k0 + s * 16) * xk * 2, 0);
      return;
    }
    const int arow = m0 + wave * 64 + l32;
#pragma unroll
    for (int rb = 0; rb < TM; rb++)
#pragma unroll
      for (int s = 0; s < KS; s++) {
        const int row = arow + rb * 32, k = k0 + s * 16 + lg * 8;
        const int rc = row < mlim ? row : mlim - 1;
        const uint4v v = *(const uint4v*)(X + (int64_t)(rc >> 5) * xs_hi + (int64_t)(rc & 31) * xs_lo +
                                          (int64_t)xk * (KTAIL && k >= K ? 0 : k));
        a[rb][s] = (KTAIL && k >= K) ? uint4v{0, 0, 0, 0} : v;
      }
  };

  struct BRegs {
    uint4v v[B_LD];
  };
  // B tile row r -> W row (GEGLU: first half value rows, second half gate
  // rows).  wlane: byte offsets of the lane's 16-byte W pieces from the
  // tile's first row of their half; load i holds rows 32i + tid/8, gate rows
  // from i = B_LD / 2 on.
  static_assert(!GEGLU || (B_LD % 2 == 0 && (B_LD / 2) * (NT / 8) == BN / 2), "GEGLU halves of the W loads");
  const int64_t wrow_b = (int64_t)K * 2;  // bytes per W row
  uint32_t wlane[B_LD];
#pragma unroll
  for (int i = 0; i < B_LD; i++) {
    const int q = tid + i * NT, r = q >> 3, c = q & 7;
    const int rr = GEGLU && r >= BN / 2 ? r - BN / 2 : r;
    wlane[i] = (uint32_t)(rr * wrow_b + c * 16);
  }
  auto load_b = [&](int n0, int k0, BRegs& br) {
    if constexpr (BUFW) {
      // value rows from W row n0, gate rows (GEGLU) from W row N + n0; each
      // resource ends with row N - 1 of its half
      const uint8_t* wb = (const uint8_t*)W;
      const int64_t left = (int64_t)(N - n0) * wrow_b;
      const int nrec = (int)(left < 0x7ffffff0 ? left : 0x7ffffff0);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc((void*)(wb + (int64_t)n0 * wrow_b), (short)0, nrec, BUF_FLAGS);
      const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(wb + (int64_t)((GEGLU ? N : 0) + n0) * wrow_b), (short)0, nrec, BUF_FLAGS);
#pragma unroll
      for (int i = 0; i < B_LD; i++) {
        const __amdgpu_buffer_rsrc_t rs = GEGLU && i >= B_LD / 2 ? rg : rv;
        br.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, wlane[i], k0 * 2, 0);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      const int q = tid + i * NT, r = q >> 3, c = q & 7;
      const int k = k0 + c * 8;
      const int nn = GEGLU ? n0 + (r < BN / 2 ? r : r - BN / 2) : n0 + r;
      const bool rv = nn < N;
      const int wr = GEGLU && r >= BN / 2 ? N + nn : nn;
      const uint4v v = *(const uint4v*)(W + (int64_t)(rv ? wr : 0) * K + (KTAIL && k >= K ? 0 : k));
      br.v[i] = (KTAIL && k >= K) ? uint4v{0, 0, 0, 0} : v;
    }
  };
  auto store_b = [&](int buf, const BRegs& br) {
    uint16_t* b = Bs + buf * BN * BK;
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int q = tid + i * NT, r = q >> 3, c = q & 7;
      *(uint4v*)(b + swz(r, c)) = br.v[i];
    }
  };

  // column block j of the tile -> W tile row (GEGLU: value blocks, then gate blocks)
  auto bcol = [&](int j) -> int {
    if constexpr (GEGLU) return j < TN / 2 ? j * 32 : BN / 2 + (j - TN / 2) * 32;
    else return j * 32;
  };

  // The C tile in LDS: 16-byte chunk c of tile row r sits in slot
  // (c/8)*BM*8 + r*8 + ((c%8) ^ (r%8)).  The epilogue's 8-byte accesses of 32
  // consecutive rows then spread over the banks, and 8 consecutive chunks of
  // a row are 8 distinct slots of one 128-byte span.  With a residual the
  // tile is first filled with R straight from global memory
  // (global_load_lds_dwordx4, issued at the tile's first K stage); the
  // epilogue adds the rounded linear output in place, and the whole tile
  // leaves with coalesced 16-byte stores (whole rows per instruction: partial
  // lines written from registers cost HBM write-backs twice over).
  auto r_slot = [&](int r, int c) { return (c >> 3) * (BM * 8) + r * 8 + ((c & 7) ^ (r & 7)); };
  // DMA instruction i of wave w fills slots (4i + w)*64 + lane, i.e. row
  // 32*(i%8) + 8w + lane/8, chunk 8*(i/8) + ((lane%8) ^ (lane/8)).  Every lane
  // writes its own slot, so slots outside the operand load a clamped,
  // in-bounds address (ldr % 8 == 0: a chunk starting below N lies inside the
  // row) and are never stored.
  // The copies are issued from inline asm (lds_copy16): the compiler then
  // does not take the fragment reads and W stores of the following stages for
  // possible readers of the C tile, each of which it would otherwise precede
  // with a wait for every load in flight.  The epilogue waits for them.
  //
  // They go out in six pieces (DMA_P instructions each), piece p at the end
  // of stage dma0 + p, after that stage's wait for its W tile.  The compiler
  // does not count them, so the first load wait issued after a piece also
  // waits for the piece: one stage later it has landed, whereas copies issued
  // at the start of a stage would hold that stage's own wait for the whole
  // residual tile.
  constexpr int DMA_N = RG * 8, DMA_P = (DMA_N + 5) / 6;
  auto dma_piece = [&](int m0, int n0, auto P_) __attribute__((always_inline)) {
    constexpr int P = decltype(P_)::value;
    int ln = lane, wv = wave;
    asm volatile("" : "+v"(ln), "+v"(wv));  // per-tile address math, not hoisted (see the epilogue)
    const int r_cx = (ln & 7) ^ (ln >> 3);
    const int rbase = m0 + wv * 8 + (ln >> 3), cbase = n0 + r_cx * 8;
    const uint32_t cs0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)Cs +
                         (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 1024u;
#pragma unroll
    for (int i = P * DMA_P; i < (P + 1) * DMA_P && i < DMA_N; i++) {
      const int row = rbase + (i & 7) * 32, col = cbase + (i >> 3) * 64;
      const bool cok = (i >> 3) * 8 + r_cx < CPR && col < N;
      lds_copy16(R + (int64_t)(row < M ? row : M - 1) * ldr + (cok ? col : 0), cs0 + (uint32_t)i * 4096u);
    }
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  // ---- epilogue: bias, one rounding to the storage type, GeGLU (value
  // block j and gate block j + TN/2 hold the same output columns), then the
  // residual add, y = round(round(x.w^T + b) + r), into the C tile
  constexpr int OUT_TN = GEGLU ? TN / 2 : TN;
  // The lane indices are re-read through an empty asm inside the epilogue,
  // the write-out and the residual DMA: the compiler then computes their
  // per-lane addresses there, once per tile, instead of hoisting all of them
  // out of the tile loop and spilling them to scratch (an HBM write per
  // spilled register).
  auto epilogue = [&](int n0, auto has_bias, auto has_r) {
    constexpr bool HB = decltype(has_bias)::value, HR = decltype(has_r)::value;
    int l32 = lane & 31, lg = lane >> 5, wv = wave;
    asm volatile("" : "+v"(l32), "+v"(lg), "+v"(wv));
#pragma unroll
    for (int j = 0; j < OUT_TN; j++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int col = j * 32 + 8 * g + 4 * lg;  // tile output column of element 0
        float bv[4] = {0.f, 0.f, 0.f, 0.f}, bg[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (HB) {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (n0 + col + e < N) {
              bv[e] = to_f<BF16>(bias[n0 + col + e]);
              if constexpr (GEGLU) bg[e] = to_f<BF16>(bias[N + n0 + col + e]);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
          uint16_t o[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float a = HB ? acc[i][j][4 * g + e] + bv[e] : acc[i][j][4 * g + e];
            if constexpr (GEGLU) {
              const float ag = HB ? acc[i][j + TN / 2][4 * g + e] + bg[e] : acc[i][j + TN / 2][4 * g + e];
              o[e] = from_f<BF16>(pin_f32(gelu_fast(to_f<BF16>(from_f<BF16>(a))) * to_f<BF16>(from_f<BF16>(ag))));
            } else {
              o[e] = from_f<BF16>(a);
            }
          }
          uint2v* cp = (uint2v*)(Cs + r_slot(wv * 64 + i * 32 + l32, col >> 3) * 8 + (col & 7));
          if constexpr (HR) {
            const uint2v rv = *cp;
            const uint16_t rr[4] = {(uint16_t)(rv.x & 0xffff), (uint16_t)(rv.x >> 16), (uint16_t)(rv.y & 0xffff),
                                    (uint16_t)(rv.y >> 16)};
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = from_f<BF16>(to_f<BF16>(o[e]) + to_f<BF16>(rr[e]));
          }
          *cp = uint2v{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
        }
      }
    }
  };
  // the C tile -> Y: thread t takes chunks t, t + 256, ...; consecutive
  // threads cover consecutive 16-byte pieces of a row (row-major Y) or of a
  // 1 KB block (panel-order Y, ypan: chunk q is row 32 * rb + q % 32, column
  // chunk 2 * nb + (q / 32) % 2 with (rb, nb) = divmod(q / 64, CPR / 2))
  static_assert(CPR % 2 == 0, "panel-order output needs whole 16-column blocks");
  const int yblk = (N + 15) >> 4;  // 16-column blocks per panel-order row block
  auto panel_chunk = [&](int q, int& r, int& c) -> int64_t {
    const int r32 = q & 31, h = (q >> 5) & 1, rest = q >> 6, rb = rest / (CPR / 2), nb = rest - rb * (CPR / 2);
    r = rb * 32 + r32;
    c = nb * 2 + h;
    return ((int64_t)rb * yblk + nb) * 512 + (h * 32 + r32) * 8;  // relative to the tile's first block
  };
  // output chunk c of C tile row r
  auto out_chunk = [&](int r, int c) __attribute__((always_inline)) -> uint4v {
    return *(const uint4v*)(Cs + r_slot(r, c) * 8);
  };
  auto write_out = [&](int m0, int n0) {
    int t0 = tid;
    asm volatile("" : "+v"(t0));
    if (ypan) {
      uint16_t* yb = Y + ((int64_t)(m0 >> 5) * yblk + (n0 >> 4)) * 512;
      const int rbl = ((M + 31) >> 5) - (m0 >> 5);  // row blocks of the padded output left from m0
      for (int q = t0; q < BM * CPR; q += NT) {
        int r, c;
        const int64_t o = panel_chunk(q, r, c);
        if ((r >> 5) >= rbl || n0 + c * 8 >= N) continue;
        *(uint4v*)(yb + o) = out_chunk(r, c);
      }
      return;
    }
    if (m0 + BM <= M && n0 + BNO <= N) {  // interior tile: no bounds checks
      // TPR threads per row, chunks c = t % TPR + TPR * j: a pass covers
      // NT / TPR rows (a multiple of 8, so a thread's C-tile slots differ
      // only by the pass: immediate LDS offsets), and every address is a
      // per-thread row pointer plus constants.  Two passes' LDS reads are
      // issued before their stores.
      constexpr int TPR = CPR % 8 == 0 ? 8 : 4, CPT = CPR / TPR, RPP = NT / TPR, NP = BM / RPP;
      static_assert(CPR % TPR == 0 && RPP % 8 == 0 && NP % 2 == 0, "interior write-out layout");
      const int tc = t0 % TPR, tr = t0 / TPR;
      uint16_t* yr = Y + (int64_t)(m0 + tr) * ldy + n0 + tc * 8;
      const int64_t ystep = (int64_t)RPP * ldy;
#pragma unroll
      for (int p = 0; p < NP; p += 2) {
        uint4v v[2][CPT];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
          for (int j = 0; j < CPT; j++) v[h][j] = out_chunk(tr + (p + h) * RPP, tc + TPR * j);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
          for (int j = 0; j < CPT; j++) *(uint4v*)(yr + h * ystep + TPR * 8 * j) = v[h][j];
        yr += 2 * ystep;
      }
      return;
    }
    for (int q = t0; q < BM * CPR; q += NT) {
      const int r = q / CPR, c = q - r * CPR;
      const int gm = m0 + r, gn = n0 + c * 8;
      if (gm >= M || gn >= N) continue;
      const uint4v v = out_chunk(r, c);
      uint16_t* yp = Y + (int64_t)gm * ldy + gn;
      if (gn + 8 <= N) {
        *(uint4v*)yp = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        for (int e = 0; gn + e < N; e++) yp[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      }
    }
  };

  // ---- spread write-out.  With several tiles per block, an interior tile
  // leaves the C tile during the next tile's first six stages instead of in
  // one burst: stage s stores chunks WO_PS * s .. WO_PS * s + WO_PS - 1 of
  // each thread's WO_N (those below WO_N), as buffer stores issued after the
  // stage's loads.
  // The wait counter counts loads and stores in issue order, so after a
  // burst the next tile's first load wait also waits for every store of the
  // tile, which all CUs issue at once; spread, a stage's stores are younger
  // than every load waited for until two stages later.  Those six stages are
  // a copy of the stage code of their own (the other stages carry no store
  // instructions); the resource's record count bounds every store to the
  // tile.
  //
  // Thread t's chunk q: row-major Y as in the interior burst below (WTPR
  // threads per row, chunk t % WTPR + WTPR * (q % WCPT) of row
  // t / WTPR + WRPP * (q / WCPT)); panel-order Y chunk t + NT q as in
  // panel_chunk, whose row block and block column are wave-uniform (lane
  // offset 16 * lane, scalar block offset).
  constexpr int WO_N = BM * CPR / NT, WO_PS = (WO_N + 5) / 6;
  constexpr int WTPR = CPR % 8 == 0 ? 8 : 4, WCPT = CPR / WTPR, WRPP = NT / WTPR;
  // The layout is a compile-time one, panel order for GeGLU (whose output
  // feeds the next linear) and row-major otherwise; an output in the other
  // layout leaves in a burst.
  constexpr bool YP = GEGLU;
  const bool spread = !QKV && ntile > 1 && KT >= 12 && (ypan != 0) == YP;
  // the pending output: its first element (row-major) or block (panel
  // order), and the bytes up to its last chunk (0: nothing pending)
  uint16_t* wo_base = Y;
  int wo_rec = 0;
  // Every address below is recomputed per stage from values re-read through
  // an empty asm: hoisted out of the stage loop, the addresses of the
  // chunks would each hold a register for the whole kernel.
  auto wo_part = [&](auto S_) __attribute__((always_inline)) {
    constexpr int S = decltype(S_)::value;
    int t0 = tid, wv = __builtin_amdgcn_readfirstlane(wave), ld2 = (int)ldy * 2, yb = yblk;
    asm volatile("" : "+v"(t0), "+s"(wv), "+s"(ld2), "+s"(yb));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)wo_base, (short)0, wo_rec, BUF_FLAGS);
    if constexpr (YP) {
      // chunk t + NT q: row block rb, block column nb of the tile (scalars)
      const int ln = t0 & 63, r32 = ln & 31, lx = (ln >> 5) ^ (r32 & 7);
#pragma unroll
      for (int u = 0; u < WO_PS; u++) {
        if (S * WO_PS + u >= WO_N) break;
        const int rest = wv + (NT / 64) * (S * WO_PS + u);
        const int rb = rest / (CPR / 2), nb = rest - rb * (CPR / 2);
        const int slot = (nb >> 2) * (BM * 8) + (rb * 32 + r32) * 8 + (((nb & 3) * 2) ^ lx);
        const uint4v v = *(const uint4v*)(Cs + slot * 8);
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, ln * 16, (rb * yb + nb) * 1024, 0);
      }
    } else {
      // tile row wtr + WRPP pass, chunk wtc + WTPR j
      const int wtc = t0 % WTPR, wtr = t0 / WTPR;
      const int voff = (wtr * ld2) + wtc * 16;
#pragma unroll
      for (int u = 0; u < WO_PS; u++) {
        if (S * WO_PS + u >= WO_N) break;
        const int q = S * WO_PS + u, pass = q / WCPT, j = q % WCPT;
        const int cr = wtc + WTPR * j;
        const int slot = (cr >> 3) * (BM * 8) + (wtr + WRPP * pass) * 8 + ((cr & 7) ^ (wtr & 7));
        const uint4v v = *(const uint4v*)(Cs + slot * 8);
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff, WRPP * pass * ld2 + WTPR * 16 * j, 0);
      }
    }
  };
  // sets the pending output to tile (m0, n0)
  auto wo_set = [&](int m0, int n0) {
    int64_t bytes;
    if constexpr (YP) {
      wo_base = Y + ((int64_t)(m0 >> 5) * yblk + (n0 >> 4)) * 512;
      bytes = ((int64_t)(BM / 32 - 1) * yblk + CPR / 2) * 1024;
    } else {
      wo_base = Y + (int64_t)m0 * ldy + n0;
      bytes = ((int64_t)(BM - 1) * ldy + BNO) * 2;
    }
    wo_rec = (int)(bytes < 0x7ffffff0 ? bytes : 0x7ffffff0);
  };

  // ---- QKV epilogue: one rounding to the storage type (the linear
  // output), then, for a head of q or k, the split-half rotation of that
  // rounded value in f32 and a second rounding (a separate Backend.rope),
  // into the C tile.  Head pair hp of the tile is column blocks 2hp (dims
  // 0..31) and 2hp + 1 (dims 32..63); a lane holds dims 8g + 4lg + e of both.
  auto epilogue_qkv = [&](int m0, int n0) {
    int l32 = lane & 31, lg = lane >> 5, wv = wave;
    asm volatile("" : "+v"(l32), "+v"(lg), "+v"(wv));
    // the QK fields are re-read here (through an empty asm), so what is
    // derived from them is computed per tile, not held across the K loop
    int L = qk.L, H = qk.H;
    const float2* tab = qk.tab;
    asm volatile("" : "+s"(L), "+s"(H), "+s"(tab));
    const int HD = H * 64;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int row = wv * 64 + i * 32 + l32;
      const int pos = (m0 + row < M ? m0 + row : M - 1) % L;
      // cos / sin of dims 8g + 4lg + 0..3 at this row's position
      float4v cs[4][2];
      if (tab != nullptr && n0 < 2 * HD) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4v* t = (const float4v*)(tab + (int64_t)pos * 32 + 8 * g + 4 * lg);
          cs[g][0] = t[0];
          cs[g][1] = t[1];
        }
      }
#pragma unroll
      for (int hp = 0; hp < TN / 2; hp++) {
        const int c0 = 64 * hp;                                   // tile column of the head's dim 0
        const bool rot = tab != nullptr && n0 + c0 < 2 * HD;     // a head of q or k
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int col = c0 + 8 * g + 4 * lg;  // tile column of dim 8g + 4lg
          uint16_t o0[4], o1[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            o0[e] = from_f<BF16>(acc[i][2 * hp][4 * g + e]);
            o1[e] = from_f<BF16>(acc[i][2 * hp + 1][4 * g + e]);
          }
          if (rot) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const float c = cs[g][e >> 1][2 * (e & 1)], sn = cs[g][e >> 1][2 * (e & 1) + 1];
              const float x0 = to_f<BF16>(o0[e]), x1 = to_f<BF16>(o1[e]);
              o0[e] = from_f<BF16>(pin_f32(fmaf(-x1, sn, x0 * c)));
              o1[e] = from_f<BF16>(pin_f32(fmaf(x0, sn, x1 * c)));
            }
          }
          *(uint2v*)(Cs + r_slot(row, col >> 3) * 8 + (col & 7)) =
              uint2v{(uint32_t)o0[0] | ((uint32_t)o0[1] << 16), (uint32_t)o0[2] | ((uint32_t)o0[3] << 16)};
          *(uint2v*)(Cs + r_slot(row, (col + 32) >> 3) * 8 + (col & 7)) =
              uint2v{(uint32_t)o1[0] | ((uint32_t)o1[1] << 16), (uint32_t)o1[2] | ((uint32_t)o1[3] << 16)};
        }
      }
    }
  };
  // ---- QKV write-out: 8 threads per tile row, thread t8 takes the 16-byte
  // chunk t8 of each head (dims 8 t8 .. 8 t8 + 7), so 8 threads write one
  // head row of 128 bytes and a wave 8 consecutive rows of one head
  auto write_out_qkv = [&](int m0, int n0) {
    int t0 = tid, L = qk.L, H = qk.H;
    asm volatile("" : "+v"(t0), "+s"(L), "+s"(H));
    const int t8 = t0 & 7, HD = H * 64, Bn = M / L;
#pragma unroll 1
    for (int r = t0 >> 3; r < BM; r += NT / 8) {
      const int gm = m0 + r;
      if (gm >= M) break;
      const int bb = gm / L, tt = gm - bb * L;
#pragma unroll
      for (int hp = 0; hp < BNO / 64; hp++) {
        const int gn = n0 + 64 * hp;  // the head's first column
        if (gn >= N) break;
        const int part = gn / HD, hh = (gn - part * HD) >> 6;
        uint16_t* dst = Y + ((((int64_t)part * Bn + bb) * H + hh) * L + tt) * 64 + 8 * t8;
        *(uint4v*)dst = out_chunk(r, 8 * hp + t8);
      }
    }
  };

  uint4v A0[TM][KS], A1[TM][KS], A2[TM][KS];
  BRegs B0, B1;
  // step g: MFMAs on `ac` and LDS buffer g&1; loads stage g+2 of the stream
  // into (al, bl); stages the W tile of g+1 (held in bs) into the other buffer.
  //
  // Origins of the block's current tile and of the tile after it, set per
  // tile, so that a stage finds the tile of the stage it loads with scalar
  // selects (for the last tile nxt = cur, nxt_kb = (KT - 1) * BK and
  // nxt_ks = 0: loads past the end of the stream repeat its last stage).
  int cur_m0 = 0, cur_n0 = 0, nxt_m0 = 0, nxt_n0 = 0, nxt_kb = 0, nxt_ks = 0;
  // The residual's pieces go out from stage dma0 on, once the C tile is free
  // (with a spread write-out pending it is read until stage 5), one per
  // stage up to stage dma0 + dpl, which sends the rest: the last piece then
  // has one more stage to land before the epilogue, if the tile has it.
  const int dma0 = spread ? 6 : 0;
  const int dpl = KT - 2 - dma0 < 0 ? 0 : (KT - 2 - dma0 < 5 ? KT - 2 - dma0 : 5);
  // S_: the stage's place in its group of six (a compile-time constant)
  // WO_: whether the stage stores its share of a pending write-out
  auto step = [&](auto S_, auto WO_, int g, int kin, uint4v (&ac)[TM][KS], uint4v (&al)[TM][KS], BRegs& bl,
                  BRegs& bs) __attribute__((always_inline)) {
    constexpr int SP = decltype(S_)::value;
    constexpr bool WO = decltype(WO_)::value && !QKV;
    // stage g + 2 of the stream: stage kin + 2 of this tile, or stage
    // kin + 2 - KT of the next (a block with several tiles has KT >= 6)
    const int k2 = __builtin_amdgcn_readfirstlane(kin + 2);
    const int wrap = __builtin_amdgcn_readfirstlane(k2 >= KT ? 1 : 0);
    const int m2 = __builtin_amdgcn_readfirstlane(wrap ? nxt_m0 : cur_m0);
    const int n2 = __builtin_amdgcn_readfirstlane(wrap ? nxt_n0 : cur_n0);
    const int k2b = __builtin_amdgcn_readfirstlane(wrap ? nxt_kb + (k2 - KT) * nxt_ks : k2 * BK);
    load_a(m2, k2b, al);
    load_b(n2, k2b, bl);
    const uint16_t* b = Bs + (g & 1) * BN * BK;
    uint4v bf[KS][TN];
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
      for (int j = 0; j < TN; j++) bf[s][j] = *(const uint4v*)(b + swz(bcol(j) + l32, 2 * s + lg));
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[i][j] = mfma32<BF16>(bf[s][j], ac[i][s], acc[i][j]);
    if constexpr (WO) wo_part(S_);
    // schedule: substep-0 fragment reads, then MFMA pairs, each preceded by
    // one global load (while any remain) and one fragment read of the next
    // substep; the write-out's C-tile reads ride with the last loads, its
    // stores follow every load; the W staging for the next stage goes last
    constexpr int NVMEM = TM * KS + B_LD, NPAIR = KS * TN, WOS = WO ? WO_PS : 0;
    // the stores two pairs after the last load, or as late as they fit
    constexpr int WST = NVMEM + 2 + WOS <= NPAIR ? NVMEM + 2 : NPAIR - WOS;
    static_assert(NVMEM <= NPAIR && WST > NVMEM - WOS && WST + WOS <= NPAIR, "write-out stores after their reads");
    __builtin_amdgcn_sched_group_barrier(0x100, TN, 0);
#pragma unroll
    for (int p = 0; p < NPAIR; p++) {
      if (p < NVMEM) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (p < (KS - 1) * TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (p >= NVMEM - WOS && p < NVMEM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (p >= WST && p < WST + WOS) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, TM, 0);
    }
    store_b((g + 1) & 1, bs);
    __builtin_amdgcn_sched_group_barrier(0x200, B_LD, 0);
    // the residual tile arrives in the C tile while the tile computes: piece
    // p at stage dma0 + min(p, dpl), the last ones together
    if (R != nullptr && kin - SP == dma0 && SP <= dpl) {
      dma_piece(cur_m0, cur_n0, S_);
      if (SP == dpl) {
        if constexpr (SP < 1) dma_piece(cur_m0, cur_n0, std::integral_constant<int, 1>{});
        if constexpr (SP < 2) dma_piece(cur_m0, cur_n0, std::integral_constant<int, 2>{});
        if constexpr (SP < 3) dma_piece(cur_m0, cur_n0, std::integral_constant<int, 3>{});
        if constexpr (SP < 4) dma_piece(cur_m0, cur_n0, std::integral_constant<int, 4>{});
        if constexpr (SP < 5) dma_piece(cur_m0, cur_n0, std::integral_constant<int, 5>{});
      }
    }
    __syncthreads();
  };

  {
    const int m0 = tile_m0(0), n0 = tile_n0(0);
    const int g1 = S > 1 ? 1 : 0, i1 = g1 / KT, k1 = (g1 - i1 * KT) * BK;
    load_a(m0, 0, A0);
    load_b(n0, 0, B0);
    store_b(0, B0);
    load_a(tile_m0(i1), k1, A1);
    load_b(tile_n0(i1), k1, B1);
    __syncthreads();
  }
  // The register rotation has period 6; a tile whose KT is not a multiple of
  // 6 ends with a tail that moves the next tile's registers back to phase 0.
  for (int it = 0; it < ntile; it++) {
    const int g0 = it * KT;
    cur_m0 = tile_m0(it);
    cur_n0 = tile_n0(it);
    const bool has_next = it + 1 < ntile;
    nxt_m0 = has_next ? tile_m0(it + 1) : cur_m0;
    nxt_n0 = has_next ? tile_n0(it + 1) : cur_n0;
    nxt_kb = has_next ? 0 : (KT - 1) * BK;
    nxt_ks = has_next ? BK : 0;
    // Six stages at a time (the register rotation's period), with no branch
    // between them: the compiler places its load waits by tracking which
    // registers have loads in flight, and where paths that ran different
    // numbers of stages join it must assume the union of their loads, which
    // makes a stage wait for the loads issued one stage earlier (for the
    // stage after next) and halves the latency the stream hides.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using I5 = std::integral_constant<int, 5>;
    using T = std::true_type;
    using F = std::false_type;
    int kt = 0;
    // a pending write-out leaves in the tile's first six stages (KT >= 12):
    // their own copy of the stage code, so that the other stages carry no
    // store instructions
    if (wo_rec != 0) {
      step(I0{}, T{}, g0, 0, A0, A2, B0, B1);
      step(I1{}, T{}, g0 + 1, 1, A1, A0, B1, B0);
      step(I2{}, T{}, g0 + 2, 2, A2, A1, B0, B1);
      step(I3{}, T{}, g0 + 3, 3, A0, A2, B1, B0);
      step(I4{}, T{}, g0 + 4, 4, A1, A0, B0, B1);
      step(I5{}, T{}, g0 + 5, 5, A2, A1, B1, B0);
      wo_rec = 0;
      kt = 6;
    }
    for (; kt + 6 <= KT; kt += 6) {
      step(I0{}, F{}, g0 + kt, kt, A0, A2, B0, B1);
      step(I1{}, F{}, g0 + kt + 1, kt + 1, A1, A0, B1, B0);
      step(I2{}, F{}, g0 + kt + 2, kt + 2, A2, A1, B0, B1);
      step(I3{}, F{}, g0 + kt + 3, kt + 3, A0, A2, B1, B0);
      step(I4{}, F{}, g0 + kt + 4, kt + 4, A1, A0, B0, B1);
      step(I5{}, F{}, g0 + kt + 5, kt + 5, A2, A1, B1, B0);
    }
    // The last q = KT % 6 stages.  Every load is drained after them, so the
    // join after this tail leaves the compiler's view of the loads in flight
    // exactly that of the loop above.  The next tile's first two stages are
    // then in registers named by phase q (its stage-0 X rows in set q % 3,
    // its stage-1 X rows in set (q + 1) % 3, its stage-1 W in set
    // (q + 1) % 2): they are moved to the names the tile loop starts from
    // (A0, A1, B1), so that every tile starts at phase 0 whatever KT is.
    if (kt < KT) {
      const int q = KT - kt;
      step(I0{}, F{}, g0 + kt, kt, A0, A2, B0, B1);
      if (q > 1) step(I1{}, F{}, g0 + kt + 1, kt + 1, A1, A0, B1, B0);
      if (q > 2) step(I2{}, F{}, g0 + kt + 2, kt + 2, A2, A1, B0, B1);
      if (q > 3) step(I3{}, F{}, g0 + kt + 3, kt + 3, A0, A2, B1, B0);
      if (q > 4) step(I4{}, F{}, g0 + kt + 4, kt + 4, A1, A0, B0, B1);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      if (has_next) {
        if (q % 3 == 1) {  // stage 0 in A1, stage 1 in A2 (A0 is free)
#pragma unroll
          for (int i = 0; i < TM; i++)
#pragma unroll
            for (int s = 0; s < KS; s++) {
              A0[i][s] = A1[i][s];
              A1[i][s] = A2[i][s];
            }
        } else if (q % 3 == 2) {  // stage 0 in A2, stage 1 in A0 (A1 is free)
#pragma unroll
          for (int i = 0; i < TM; i++)
#pragma unroll
            for (int s = 0; s < KS; s++) {
              A1[i][s] = A0[i][s];
              A0[i][s] = A2[i][s];
            }
        }
        if (q & 1) B1 = B0;  // stage-1 W in B0
      }
    }
    // The residual's last pieces went out at the end of stage dma0 + dpl, and
    // memory operations complete in issue order: they have landed once at
    // most the loads and stores of one later stage are outstanding (or none,
    // when they went out with the last stage).  The
    // barrier makes every wave's part of the C tile visible (and, without R,
    // keeps the previous tile's write-out reads ahead of this epilogue's
    // writes).
    constexpr int VM1 = TM * KS + B_LD;  // the loads of one stage (stages after the pieces store nothing)
    static_assert(VM1 <= 63, "vmcnt immediate");
    if (R != nullptr) {
      if (dma0 + dpl >= KT - 1) __builtin_amdgcn_s_waitcnt(0x0F70);
      else __builtin_amdgcn_s_waitcnt(0x0F70 | (VM1 & 15) | ((VM1 >> 4) << 14));
    }
    __syncthreads();
    {
      const int n0 = cur_n0;
      if constexpr (QKV) {
        epilogue_qkv(cur_m0, n0);
      } else if (bias == nullptr) {
        if (R == nullptr) epilogue(n0, F{}, F{});
        else epilogue(n0, F{}, T{});
      } else {
        if (R == nullptr) epilogue(n0, T{}, F{});
        else epilogue(n0, T{}, T{});
      }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    __syncthreads();
    if constexpr (QKV) {
      write_out_qkv(cur_m0, cur_n0);
    } else if (spread && has_next && cur_m0 + BM <= M && cur_n0 + BNO <= N) {
      wo_set(cur_m0, cur_n0);  // leaves during the next tile's first six stages
    } else {
      write_out(cur_m0, cur_n0);
      if (R != nullptr) __syncthreads();  // the next tile's residual DMA refills the C tile
    }
  }
}

// ------------------------------------------------------------------ launchers

template <int BM, int BN, int WM, int WN, bool BF16, bool GEGLU, int QB, bool AFF, bool SF32>
void launch_mfma(hipStream_t st, const uint16_t* x, int64_t ldx, const uint16_t* w, QW qw,
                        const uint16_t* bias, const uint16_t* r, int64_t ldr, uint16_t* y, int64_t ldy, int M, int N,
                        int K) {
  constexpr int BNO = GEGLU ? BN / 2 : BN;
  int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BNO - 1) / BNO;
  size_t stage = (size_t)2 * (BM + BN) * 64 * sizeof(uint16_t);
  size_t ctile = (size_t)BM * BNO * sizeof(uint16_t);
  size_t lds = stage > ctile ? stage : ctile;
  auto kern = gemm_mfma<BM, BN, WM, WN, BF16, GEGLU, QB, AFF, SF32>;
  static std::atomic<uint64_t> attr{0};
  once_per_device(attr, [&] {
    HB_CHECK_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  });
  kern<<<tiles_m * tiles_n, WM * WN * 64, lds, st>>>(x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K, tiles_n);
}

template <int BN, bool BF16, bool GEGLU, bool KTAIL, bool QKV = false>
void launch_arow(hipStream_t st, int cus, unsigned pan, const uint16_t* x, int64_t ldx, const uint16_t* w,
                 const uint16_t* bias, const uint16_t* r, int64_t ldr, uint16_t* y, int64_t ldy, int M, int N, int K,
                 QK qk = QK{nullptr, 1, 1}) {
  constexpr int BNO = GEGLU ? BN / 2 : BN;
  const int tiles_m = (M + 255) / 256, tiles_n = (N + BNO - 1) / BNO, tiles = tiles_m * tiles_n;
  // one persistent block per CU, a multiple of 8 (one per XCD), streaming
  // its tiles when they have a multiple of 6 or at least 12 K stages (the
  // shapes measured and tested).  Otherwise one tile per block: every XCD
  // gets as many blocks as the largest XCD share of tiles (ceil(tiles_m / 8)
  // row panels).
  const int KT = (K + 63) / 64;
  const bool stream = KT % 6 == 0 || KT >= 12;
  int grid = stream ? (tiles < cus ? tiles : cus) / 8 * 8 : 8 * (((tiles_m + 7) / 8) * tiles_n);
  HB_REQUIRE(grid >= 8, "hb_linear: large-M GEMM needs at least 8 tiles");
  constexpr int RG = (BNO / 8 + 7) / 8;
  // W tiles and the C tile
  const size_t lds = ((size_t)2 * BN * 64 + (size_t)RG * 256 * 64) * sizeof(uint16_t);
  auto kern = gemm_mfma_arow<BN, BF16, GEGLU, KTAIL, QKV>;
  static std::atomic<uint64_t> attr{0};
  once_per_device(attr, [&] {
    HB_CHECK_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  });
  kern<<<grid, 256, lds, st>>>(x, ldx, w, bias, r, ldr, y, ldy, M, N, K, tiles_n, tiles, (pan & HB_X_PANEL) ? 1 : 0,
                               (pan & HB_Y_PANEL) ? 1 : 0, qk);
}

// Waves per slab block (each takes 32 rows of X): two for slabs of at most
// 32 x 768 weights when those blocks fit one per CU, else four.  A launch
// spread over more CUs finishes sooner although X and the slabs are then read
// by more blocks (the k16 order per output is the same for any count), as
// long as a wave's share of the slab stays small: at two waves the 64-row
// GeGLU slab and the K = 1152 slab measured slower, and one wave per block
// (the whole slab to fetch) slower still.
inline int slab_waves(int64_t M, int64_t tiles_n, int64_t slab_elems, int cus) {
  return slab_elems <= 32 * 768 && tiles_n * ((M + 63) / 64) <= cus ? 2 : 4;
}

// Small-M launcher for 16-bit weights: slabs of 32 (GeGLU: 64) W rows, 64
// or 128 rows of X per block (slab_waves).  P (X steps held in registers)
// is the largest of 48, 36, 32, 24, 16 and 4 that divides K/16.
// LDS bytes of a slab block: the f16 slab of 32 tn rows, and for quantized
// weights the slab's codes and its scales (and zeros: aff), G per row in
// 4-byte slots
inline int64_t slab_lds(int64_t K, int tn, int qb, bool aff, int64_t G) {
  const int64_t sr = 32 * tn;
  return sr * K * 2 + (qb ? sr * K * qb / 8 + sr * G * 4 * (aff ? 2 : 1) : 0);
}

// Quantized weights on the slab kernel: f16 scales, groups a multiple of 8
// (a chunk of 8 weights in one group), K / 16 a multiple of 48 or 36 (the
// register depths instantiated for them), and the block's LDS within bounds.
inline bool qslab_ok(int64_t K, int tn, int qb, bool aff, const QW& qw) {
  return qw.group % 8 == 0 && ((K / 16) % 48 == 0 || (K / 16) % 36 == 0) &&
         slab_lds(K, tn, qb, aff, qw.G) <= 160 * 1024;
}

template <int TN, bool BF16, bool GEGLU, int QB = 0, bool AFF = false>
void launch_slab_t(hipStream_t st, int cus, QW qw, const uint16_t* x, int64_t ldx, const uint16_t* w,
                   const uint16_t* bias, const uint16_t* r, int64_t ldr, uint16_t* y, int64_t ldy, int M, int N,
                   int K, unsigned pan) {
  constexpr int TNO = GEGLU ? TN / 2 : TN;
  const int tiles_n = (N + 32 * TNO - 1) / (32 * TNO);
  const int nw = slab_waves(M, tiles_n, (int64_t)32 * TN * K, cus), chunks = (M + 32 * nw - 1) / (32 * nw);
  const int64_t lds = slab_lds(K, TN, QB, AFF, QB ? qw.G : 0);
  HB_REQUIRE(lds <= 160 * 1024, "hb_linear: weight slab too large for LDS");
  const int S = K / 16;
  auto go = [&](auto kern) {
    static std::atomic<uint64_t> attr{0};
    once_per_device(attr, [&] {
      HB_CHECK_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    });
    kern<<<tiles_n * chunks, 64 * nw, (size_t)lds, st>>>(x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K, chunks,
                                                          (pan & HB_X_PANEL) ? 1 : 0, (pan & HB_Y_PANEL) ? 1 : 0);
  };
  if constexpr (QB != 0) {
    HB_REQUIRE(S % 48 == 0 || S % 36 == 0, "hb_linear: quantized slab needs K a multiple of 768 or 576");
    if (S % 48 == 0) go(gemm_slab<TN, 48, BF16, GEGLU, QB, AFF>);
    else go(gemm_slab<TN, 36, BF16, GEGLU, QB, AFF>);
  } else {
    if (S % 48 == 0) go(gemm_slab<TN, 48, BF16, GEGLU>);
    else if (S % 36 == 0) go(gemm_slab<TN, 36, BF16, GEGLU>);
    else if (S % 32 == 0) go(gemm_slab<TN, 32, BF16, GEGLU>);
    else if (S % 24 == 0) go(gemm_slab<TN, 24, BF16, GEGLU>);
    else if (S % 16 == 0) go(gemm_slab<TN, 16, BF16, GEGLU>);
    else go(gemm_slab<TN, 4, BF16, GEGLU>);
  }
}

// The slab kernel pays off while its blocks fit one per CU: its X fragment
// loads (32 rows x 32 bytes each) are bound by the CU's L1 (about 15 bytes
// per clock for that pattern), so two blocks on one CU take twice as long and
// the 128 x 128 kernel, which stages X through LDS, is faster from there on.
inline bool slab_path(int64_t M, int64_t N_out, int64_t K, bool geglu, int cus) {
  const int64_t tiles_n = (N_out + 31) / 32, chunks = (M + 127) / 128;
  return K % 64 == 0 && K * 32 * (geglu ? 2 : 1) * 2 <= 160 * 1024 && tiles_n * chunks <= cus;
}

// The large-M kernel runs for M >= 4096.  It and the small-M slab kernel
// (16-bit weights) take panel-order operands; the entry points check that
// the call takes one of them before dispatching.
inline bool arow_path(int64_t M) { return M >= 4096; }

// Below M = 4096, without the slab kernel: 128 x 64 tiles (instead of
// 128 x 128) where 128 x 128 tiles would leave the GPU short of blocks.
// N_out: output columns (GeGLU: value / gate pairs).
inline bool thin_tiles(int64_t M, int64_t N_out, bool geglu, int cus) {
  const int64_t t128 = ((M + 127) / 128) * ((N_out + (geglu ? 63 : 127)) / (geglu ? 64 : 128));
  return t128 <= cus + cus / 8;
}

template <bool BF16, bool GEGLU, int QB, bool AFF, bool SF32>
void mfma_dispatch(hipStream_t st, int cus, unsigned pan, const uint16_t* x, int64_t ldx, const uint16_t* w,
                          QW qw, const uint16_t* bias, const uint16_t* r, int64_t ldr, uint16_t* y, int64_t ldy, int M,
                          int N, int K) {
  // large M: persistent 256 x 192 tiles with register-resident A rows (16-bit
  // weights: hb_qlinear dequantizes a quantized weight once and calls the
  // 16-bit path at large M); small M: weight-stationary slabs, else 128 x 128
  // tiles.  K % 64 != 0 takes the large-M variant with a K tail.
  if constexpr (QB == 0) {
    if (arow_path(M)) {
      // 128-column tiles where N is a multiple of 128 and not of 192 (N =
      // 1024: 8 whole tiles instead of 5 1/3 of 192 columns)
      if constexpr (!GEGLU) {
        if (N % 192 != 0 && N % 128 == 0) {
          if (K % 64 == 0)
            launch_arow<128, BF16, false, false>(st, cus, pan, x, ldx, w, bias, r, ldr, y, ldy, M, N, K);
          else
            launch_arow<128, BF16, false, true>(st, cus, pan, x, ldx, w, bias, r, ldr, y, ldy, M, N, K);
          return;
        }
      }
      if (K % 64 == 0)
        launch_arow<192, BF16, GEGLU, false>(st, cus, pan, x, ldx, w, bias, r, ldr, y, ldy, M, N, K);
      else
        launch_arow<192, BF16, GEGLU, true>(st, cus, pan, x, ldx, w, bias, r, ldr, y, ldy, M, N, K);
      return;
    }
  } else {
    HB_REQUIRE(!arow_path(M), "hb_qlinear: large-M quantized weights are dequantized before the GEMM");
  }
  {
    if constexpr (QB == 0 || !SF32) {
      if (slab_path(M, N, K, GEGLU, cus) && (QB == 0 || qslab_ok(K, GEGLU ? 2 : 1, QB, AFF, qw))) {
        launch_slab_t<GEGLU ? 2 : 1, BF16, GEGLU, QB, AFF>(st, cus, qw, x, ldx, w, bias, r, ldr, y, ldy, M, N, K,
                                                          pan);
        return;
      }
    }
    HB_REQUIRE(pan == 0, "hb_linear: panel-order operands on a kernel that does not take them");
    // Tiles of 128 x 64 (waves of 32 x 64) where 128 x 128 tiles would
    // leave the GPU short of blocks: the K stages of a block run one after
    // another (each one's loads, LDS staging and barrier), so a launch with
    // few blocks is bound by that chain; halving the tile halves the work
    // of each stage.  Measured (16-bit, M = 2048): attn Wo 18.2 -> 14.3 us,
    // mlp Wo 22.9 -> 18.1 us; at M = 3072 the 2304-column shapes are faster
    // with 128 x 128 tiles (27.0 against 32.8 us).  Every output keeps its
    // MFMA sequence and epilogue, so the bits do not change.  Quantized
    // weights take the same rule (their loader dequantizes each stage of
    // the thinner W tile; hb_qlinear calls with a quantized weight wherever
    // these tiles are taken below M = 4096).
    if (thin_tiles(M, N, GEGLU, cus)) {
      launch_mfma<128, 64, 4, 1, BF16, GEGLU, QB, AFF, SF32>(st, x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K);
      return;
    }
    launch_mfma<128, 128, 2, 2, BF16, GEGLU, QB, AFF, SF32>(st, x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K);
  }
}

template <int QB, bool AFF, bool SF32>
void mfma_dtype(int dt, bool geglu, hipStream_t st, int cus, unsigned pan, const uint16_t* x, int64_t ldx,
                       const uint16_t* w, QW qw, const uint16_t* bias, const uint16_t* r, int64_t ldr, uint16_t* y,
                       int64_t ldy, int M, int N, int K) {
  if (dt == HB_F16) {
    if (geglu) mfma_dispatch<false, true, QB, AFF, SF32>(st, cus, pan, x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K);
    else mfma_dispatch<false, false, QB, AFF, SF32>(st, cus, pan, x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K);
  } else {
    if (geglu) mfma_dispatch<true, true, QB, AFF, SF32>(st, cus, pan, x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K);
    else mfma_dispatch<true, false, QB, AFF, SF32>(st, cus, pan, x, ldx, w, qw, bias, r, ldr, y, ldy, M, N, K);
  }
}

// The fused q / k / v projection (16-bit weights, M >= 4096, K % 64 == 0):
// the large-M kernel with the QKV epilogue.
template <bool BF16>
void launch_qkv(hipStream_t st, int cus, unsigned pan, const uint16_t* x, int64_t ldx, const uint16_t* w,
                uint16_t* y, int M, int N, int K, QK qk) {
  launch_arow<192, BF16, false, false, true>(st, cus, pan, x, ldx, w, nullptr, nullptr, 0, y, 0, M, N, K, qk);
}

// Instantiated by gemm_f16.hip (QB = 0), gemm_q8.hip and gemm_q4.hip.
extern template void launch_qkv<false>(hipStream_t, int, unsigned, const uint16_t*, int64_t, const uint16_t*,
                                       uint16_t*, int, int, int, QK);
extern template void launch_qkv<true>(hipStream_t, int, unsigned, const uint16_t*, int64_t, const uint16_t*,
                                      uint16_t*, int, int, int, QK);
extern template void mfma_dtype<0, false, false>(int, bool, hipStream_t, int, unsigned, const uint16_t*, int64_t,
                                                 const uint16_t*, QW, const uint16_t*, const uint16_t*, int64_t,
                                                 uint16_t*, int64_t, int, int, int);
extern template void mfma_dtype<8, false, false>(int, bool, hipStream_t, int, unsigned, const uint16_t*, int64_t,
                                                 const uint16_t*, QW, const uint16_t*, const uint16_t*, int64_t,
                                                 uint16_t*, int64_t, int, int, int);
extern template void mfma_dtype<8, true, false>(int, bool, hipStream_t, int, unsigned, const uint16_t*, int64_t,
                                                const uint16_t*, QW, const uint16_t*, const uint16_t*, int64_t,
                                                uint16_t*, int64_t, int, int, int);
extern template void mfma_dtype<4, false, false>(int, bool, hipStream_t, int, unsigned, const uint16_t*, int64_t,
                                                 const uint16_t*, QW, const uint16_t*, const uint16_t*, int64_t,
                                                 uint16_t*, int64_t, int, int, int);
extern template void mfma_dtype<4, true, false>(int, bool, hipStream_t, int, unsigned, const uint16_t*, int64_t,
                                                const uint16_t*, QW, const uint16_t*, const uint16_t*, int64_t,
                                                uint16_t*, int64_t, int, int, int);

}  // namespace hb
