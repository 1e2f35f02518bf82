// Scaled dot-product attention (Backend.sdpa) with optional fused RoPE.
//
// sdpa_mfma: flash attention for head dim 64 in fp16 / bf16 on
// v_mfma_f32_16x16x32.  A block owns 128 queries of one (b, h); each of its
// eight waves owns 16 of them.  Per 64-key tile the wave computes
// S^T = K . Q^T, so a lane ends up holding the scores of ONE query for 8
// contiguous keys per 32-key half -- exactly the B-operand layout of
// O^T = V^T . P^T, so P never leaves registers.  The rows of K are fed to the
// MFMA in a permuted order that makes those 8 keys contiguous, which lets the
// lane read its 8 mask bytes with one load and its V^T fragment (V transposed
// in LDS) with one 16-byte read.  K and V^T tiles are double-buffered in LDS,
// loaded into registers two tiles ahead (waves 0-3 fetch K, waves 4-7 V).
// Softmax is online, in f32, in the log2 domain.  A pre-pass over the bool
// mask classes every (b, query tile, key tile, 16-query group) as skipped,
// all visible or masked: tiles no group needs are never staged, and a group
// skips the tiles it cannot see, so the sliding-window layers touch only the
// tiles inside the window (plus the full rows of padded queries, which see
// every valid key).  RoPE, when fused, rotates the Q and K tiles as they are
// staged and rounds them to the storage type, bit-identical to a separate
// Backend.rope.  The output is written row-major or, for the attention output
// projection, in the panel order of the GEMM's X operand.
//
// sdpa_simt: the f32 path and the fallback for other head dims / layouts.
//
// hb_sdpa_noalloc: hb_sdpa without RoPE for callers that cannot allocate; its
// mask summary goes to `scratch`, a file-scope device array.
#include <mutex>
#include <stdexcept>

#include "common.h"

// Scratch of hb_sdpa_noalloc: the mask summary (one byte per 16-query group
// of every 128-query x 64-key tile), for B * ceil(Lq/128) * ceil(Lk/64) <=
// 262144 tiles (B = 32 at Lq = Lk = 8192).  Every GPU the library runs on
// holds its own copy until the process ends.
constexpr size_t kSdpaScratchBytes = (size_t)2 << 20;
static __device__ __align__(256) uint8_t scratch[kSdpaScratchBytes];

namespace hb {

const float* rope_table(uintptr_t ctx, int64_t L, int64_t D, double base);

struct S4 {
  int64_t s[4];
};

static S4 s4(const int64_t* p) {
  S4 r;
  for (int i = 0; i < 4; i++) r.s[i] = p ? p[i] : 0;
  return r;
}

constexpr int kBQ = 128;  // queries per block
constexpr int kQB = 1;    // 16-query blocks per wave
constexpr int kNW = kBQ / (16 * kQB);  // waves per block
constexpr int kNT = kNW * 64;          // threads per block
constexpr int kBK = 64;   // keys per tile
constexpr int kMaxKeyTiles = 1024;  // Lk <= 65536 on the MFMA path

// ------------------------------------------------------------------ mask summary

// Class of every (batch, 16-query group, 64-key tile) block of a bool mask:
// 0 = no visible key (skipped), 1 = every key visible (no mask reads),
// 2 = mixed or running past Lk (per-element mask).  One byte per group, the
// 8 groups of a 128-query tile together: cls[((b * nqt + qt) * nkt + kt) * 8
// + group].  Computed once per mask tensor and reused by every layer that
// attends with it; the attention kernel skips a key tile for a wave whose
// group has class 0 and stages it only if some group needs it.
__global__ __launch_bounds__(256) void mask_class_kernel(const uint8_t* __restrict__ mask, S4 ms, int Lq, int Lk,
                                                         int nqt, int nkt, uint8_t* __restrict__ cls, int vec) {
  __shared__ int anyg[kNW], allg[kNW];
  const int kt = blockIdx.x, qt = blockIdx.y, b = blockIdx.z;
  const int q0 = qt * kBQ, k0 = kt * kBK;
  const int nq = min(kBQ, Lq - q0), nk = min(kBK, Lk - k0);
  const bool bcast = ms.s[2] == 0;  // a [B,1,1,L] mask has one row for every query
  if (threadIdx.x < kNW) {
    anyg[threadIdx.x] = 0;
    allg[threadIdx.x] = 1;
  }
  __syncthreads();
  if (vec && nk == kBK) {
    // 16-byte row chunks: rows x 4 chunks
    for (int i = threadIdx.x; i < nq * 4; i += blockDim.x) {
      const int q = i >> 2, c = i & 3;
      const uint4v w = *(const uint4v*)(mask + b * ms.s[0] + (int64_t)(bcast ? 0 : q0 + q) * ms.s[2] + k0 + c * 16);
      // any byte nonzero <=> word != 0; all visible when every byte == 1
      const uint32_t o = w.x | w.y | w.z | w.w, a = w.x & w.y & w.z & w.w;
      if (o != 0) atomicOr(&anyg[q >> 4], 1);
      if (a != 0x01010101u) atomicAnd(&allg[q >> 4], 0);
    }
  } else {
    for (int i = threadIdx.x; i < nq * nk; i += blockDim.x) {
      const int q = i / nk, k = i - q * nk;
      const uint8_t m = mask[b * ms.s[0] + (int64_t)(bcast ? 0 : q0 + q) * ms.s[2] + (int64_t)(k0 + k) * ms.s[3]];
      if (m != 0) atomicOr(&anyg[q >> 4], 1);
      else atomicAnd(&allg[q >> 4], 0);
    }
  }
  __syncthreads();
  if (threadIdx.x < kNW) {
    const int g = threadIdx.x;
    cls[(((int64_t)b * nqt + qt) * nkt + kt) * kNW + g] = !anyg[g] ? 0 : (allg[g] && nk == kBK ? 1 : 2);
  }
}

static size_t mask_info_bytes(int64_t B, int64_t Lq, int64_t Lk) {
  int64_t nqt = (Lq + kBQ - 1) / kBQ, nkt = (Lk + kBK - 1) / kBK;
  return (size_t)(B * nqt * nkt * kNW);
}

static void launch_mask_info(hipStream_t st, const uint8_t* mask, const S4& ms, int64_t B, int64_t Lq, int64_t Lk,
                             uint8_t* info) {
  int nqt = (int)((Lq + kBQ - 1) / kBQ), nkt = (int)((Lk + kBK - 1) / kBK);
  int vec = ms.s[3] == 1 && ((uintptr_t)mask % 16 == 0) && ms.s[0] % 16 == 0 && ms.s[2] % 16 == 0;
  mask_class_kernel<<<dim3(nkt, nqt, (unsigned)B), 256, 0, st>>>(mask, ms, (int)Lq, (int)Lk, nqt, nkt, info, vec);
}

// ------------------------------------------------------------------ MFMA kernel (D = 64)

template <bool BF16>
__device__ __forceinline__ float4v mfma16(const uint4v& a, const uint4v& b, float4v c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}
template <bool BF16>
__device__ __forceinline__ float tof(uint32_t h) {
  return BF16 ? bf16_to_f32((uint16_t)h) : f16_bits_to_f32((uint16_t)h);
}
template <bool BF16>
__device__ __forceinline__ uint32_t fromf(float v) {
  return BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
}

// Two f32 values packed as 16-bit (f16: v_cvt_pk_f16_f32; bf16: RNE).
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (BF16) {
    return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
  } else {
    typedef float float2v __attribute__((ext_vector_type(2)));
    half2v h = __builtin_convertvector((float2v){a, b}, half2v);
    return __builtin_bit_cast(uint32_t, h);
  }
}

// 4 mask bytes (any nonzero byte is true): bit 7 of each byte set iff the
// byte is nonzero (no carries between bytes)
__device__ __forceinline__ uint32_t mask_nz(uint32_t w) {
  return (((w & 0x7f7f7f7fu) + 0x7f7f7f7fu) | w) & 0x80808080u;
}

// Cross-lane exchanges for the 4 lanes that hold one query (lane, lane ^ 16,
// lane ^ 32, lane ^ 48): ds_swizzle in bit-mask mode (and 0x1f, xor 0x10)
// reads lane ^ 16 within each half-wave; v_permlane32_swap exchanges the
// two halves, returning (per lane) its own value and the one of lane ^ 32.
__device__ __forceinline__ float from_xor16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

__device__ __forceinline__ int qk_swz(int r, int c) { return r * 64 + ((c ^ (r & 7)) << 3); }
// K tiles: chunk c of row r at c ^ (4 * bit 1 of r + bits 3..4 of r).  A
// 16-lane pass of the S = K.Q^T fragment reads touches rows b + 8a (a, b in
// 0..3), which this spreads over all 64 banks, and the staging stores (rows
// r..r+3, chunks 0..3 or 4..7) hit disjoint banks too.
__device__ __forceinline__ int k_swz(int r, int c) { return r * 64 + ((c ^ ((((r >> 1) & 1) << 2) | ((r >> 3) & 3))) << 3); }
constexpr int kVtLd = 72;  // row stride (elements) of V^T in LDS
// V^T tiles: the 8-key chunk c of row d sits at c ^ (4 * bit 4 of d + 2 * bit 5
// of d), which makes the transposing staging stores (rows 8*vc + i, one
// 32-bit key pair per lane) hit 64 distinct banks; the fragment reads of one
// instruction share bits 4..5 of d, so they stay conflict-free.
__device__ __forceinline__ int vt_swz(int d, int c) {
  return d * kVtLd + ((c ^ ((((d >> 4) & 1) << 2) | (((d >> 5) & 1) << 1))) << 3);
}

// Raw chunks c and c + 4 (d in [8c, 8c+8) and the rotation partners d + 32)
// of one row of a [L, 64] operand; zero when the row is out of range.
__device__ __forceinline__ void load_pair(const uint16_t* __restrict__ src, bool valid, int c, uint4v& lo,
                                          uint4v& hi) {
  lo = uint4v{0, 0, 0, 0};
  hi = uint4v{0, 0, 0, 0};
  if (valid) {
    lo = *(const uint4v*)(src + c * 8);
    hi = *(const uint4v*)(src + 32 + c * 8);
  }
}

// cos / sin of the 8 rotation pairs (d, d + 32), d in [8c, 8c+8), at
// position `pos` of a RoPE table [L][32] (float2).
__device__ __forceinline__ void load_cs(const float2* __restrict__ tab, int pos, int c, float2 (&cs)[8]) {
  const float4v* t = (const float4v*)(tab + pos * 32 + c * 8);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float4v v = t[e];
    cs[2 * e] = float2{v[0], v[1]};
    cs[2 * e + 1] = float2{v[2], v[3]};
  }
}

// Rotates a loaded chunk pair by RoPE (when `rot`) with the pairs' cos / sin,
// rounding to the storage type like a separate Backend.rope, and writes it
// to the swizzled [rows][64] LDS tile.
template <bool BF16, bool KSWZ = false>
__device__ __forceinline__ void store_pair(uint4v lo, uint4v hi, bool rot, int c, const float2 (&cs)[8],
                                           uint16_t* lds, int row) {
  if (rot) {
    uint32_t* l = (uint32_t*)&lo;
    uint32_t* h = (uint32_t*)&hi;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float2 c0 = cs[2 * e], c1 = cs[2 * e + 1];
      float x0a = tof<BF16>(l[e] & 0xffff), x0b = tof<BF16>(l[e] >> 16);
      float x1a = tof<BF16>(h[e] & 0xffff), x1b = tof<BF16>(h[e] >> 16);
      l[e] = pack2<BF16>(pin_f32(fmaf(-x1a, c0.y, x0a * c0.x)), pin_f32(fmaf(-x1b, c1.y, x0b * c1.x)));
      h[e] = pack2<BF16>(pin_f32(fmaf(x0a, c0.y, x1a * c0.x)), pin_f32(fmaf(x0b, c1.y, x1b * c1.x)));
    }
  }
  *(uint4v*)(lds + (KSWZ ? k_swz(row, c) : qk_swz(row, c))) = lo;
  *(uint4v*)(lds + (KSWZ ? k_swz(row, c + 4) : qk_swz(row, c + 4))) = hi;
}

template <bool BF16>
__global__ __launch_bounds__(kNT) __attribute__((amdgpu_waves_per_eu(4))) void sdpa_mfma(const uint16_t* __restrict__ Q, S4 qs, const uint16_t* __restrict__ K,
                                                 S4 ks, const uint16_t* __restrict__ V, S4 vs,
                                                 const uint8_t* __restrict__ mask, S4 ms, int mask_vec,
                                                 const uint8_t* __restrict__ cls, uint16_t* __restrict__ O, S4 os,
                                                 int Lq, int Lk, float scale_log2, const float2* __restrict__ tabq,
                                                 const float2* __restrict__ tabk, int pK, int nqt, int nh) {
  // Q, and two buffers of K and V^T: tile t + 1 is staged while tile t computes
  __shared__ __attribute__((aligned(16))) uint16_t Qs[kBQ * 64];
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBK * 64];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][64 * kVtLd];
  __shared__ uint16_t cls_row[kMaxKeyTiles];  // 2 bits of class per 16-query group

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  // One block per (b, h, query tile) on a 1-D grid.  Blocks are dealt to the
  // 8 XCDs in turn (block i on XCD i % 8).  The query tiles of one (b, h)
  // read the same K / V rows and mask bytes, so they go to one XCD as
  // consecutive blocks of its share (they run together and share its L2),
  // and the (b, h) pairs are dealt to the XCDs in turn, which spreads
  // sequences of different lengths (and work) evenly over them.  Without a
  // multiple of 8 pairs the blocks take (b, h, query tile) in order.
  const int nbh = (int)(gridDim.x / nqt);
  int qt, bh;
  if ((nbh & 7) == 0) {
    const int x = blockIdx.x & 7, idx = blockIdx.x >> 3;
    qt = idx % nqt;
    bh = (idx / nqt) * 8 + x;
  } else {
    qt = blockIdx.x % nqt;
    bh = blockIdx.x / nqt;
  }
  const int h = bh % nh, b = bh / nh;
  const int nkt = (Lk + kBK - 1) / kBK;
  const int q0 = qt * kBQ;
  const uint16_t* Qb = Q + b * qs.s[0] + h * qs.s[1];
  const uint16_t* Kb = K + b * ks.s[0] + h * ks.s[1];
  const uint16_t* Vb = V + b * vs.s[0] + h * vs.s[1];
  // this block's Q rows (and their RoPE cos / sin) are requested first: they
  // do not depend on the tile classes, so their latency overlaps the class
  // row's
  constexpr int QR = kBQ * 4 / kNT;  // rounds of Q staging (4 threads per row)
  static_assert(QR * kNT == kBQ * 4, "Q staging: whole rounds");
  uint4v qlo[QR], qhi[QR];
  float2 qcs[QR][8];
#pragma unroll
  for (int u = 0; u < QR; u++) {
    const int t = tid + u * kNT, r = t >> 2, c = t & 3, q = q0 + r;
    load_pair(Qb + (int64_t)q * qs.s[2], q < Lq, c, qlo[u], qhi[u]);
    if (tabq != nullptr && q < Lq) load_cs(tabq, q, c, qcs[u]);
  }

  // tile classes of this (b, query tile) for each wave's 16-query group: 0
  // skip, 1 all visible, 2 per-element mask / key bound; staged in LDS once
  // (the host caps nkt at kMaxKeyTiles).  A tile is staged when some group
  // needs it.
  static_assert(kQB == 1 && kNW == 8, "one 16-query group per wave, 8 per tile");
  for (int t = tid; t < nkt; t += kNT) {
    uint32_t c;
    if (cls != nullptr) {
      const uint2v w = *(const uint2v*)(cls + (((int64_t)b * nqt + qt) * nkt + t) * kNW);
      c = 0;
#pragma unroll
      for (int gq = 0; gq < kNW; gq++) c |= (((gq < 4 ? w.x : w.y) >> (8 * (gq & 3))) & 3u) << (2 * gq);
    } else if (mask != nullptr) {
      c = 0xAAAAu;
    } else {
      c = (t + 1) * kBK <= Lk ? 0x5555u : 0xAAAAu;
    }
    cls_row[t] = (uint16_t)c;
  }
  auto tile_needed = [&](int kt) -> bool { return cls_row[kt] != 0; };
  auto wave_class = [&](int kt) -> int { return (cls_row[kt] >> (2 * wave)) & 3; };
  // (the same in every lane: read from the class row in LDS, made
  // wave-uniform so that the tile's address arithmetic is scalar)
  auto next_tile = [&](int kt) -> int {
    kt++;
    while (kt < nkt && !tile_needed(kt)) kt++;
    return __builtin_amdgcn_readfirstlane(kt);
  };
  __syncthreads();  // the class row is complete

  // A K tile is staged by the first 256 threads (row kr, chunk pair kc),
  // the V tile by the other 256 (key pair vj, chunk vc); loaded into
  // registers two tiles ahead and staged into LDS one tile ahead
  static_assert(kNT == 512, "K / V staging: 256 threads each");
  const bool kpart = tid < 256;  // whole waves
  const int kr = (tid & 255) >> 2, kc = tid & 3;
  const int vc = tid & 7, vj = 2 * ((tid & 255) >> 3);
  uint4v pr0, pr1;  // K threads: chunks kc and kc + 4 of row kr; V threads: keys vj and vj + 1
  float2 kcs[8];    // RoPE cos / sin of this thread's K row (fused RoPE)
  // The tile's first row is a scalar address (k0 is wave-uniform); a
  // thread's row within the tile adds a 24-bit product (row < 64, a row
  // stride below 2^24 elements: the host's condition for this kernel).
  auto prefetch = [&](int kt) {
    const int k0 = kt * kBK;
    if (kpart) {
      const uint16_t* kb = Kb + (int64_t)k0 * ks.s[2];
      load_pair(kb + __umul24(kr, (uint32_t)ks.s[2]), k0 + kr < Lk, kc, pr0, pr1);
      if (tabk != nullptr && k0 + kr < Lk) load_cs(tabk + (int64_t)k0 * 32, kr, kc, kcs);
    } else {
      const uint16_t* vb = Vb + (int64_t)k0 * vs.s[2] + vc * 8;
      const uint32_t vo = __umul24(vj, (uint32_t)vs.s[2]);
      pr0 = uint4v{0, 0, 0, 0};
      pr1 = uint4v{0, 0, 0, 0};
      if (k0 + vj < Lk) pr0 = *(const uint4v*)(vb + vo);
      if (k0 + vj + 1 < Lk) pr1 = *(const uint4v*)(vb + vo + (uint32_t)vs.s[2]);
    }
  };

  // this lane's mask bytes of a tile: 8 contiguous keys of its query (one per
  // 16-query block qb) in each 32-key half t
  auto load_mask = [&](int kt, uint2v (&mw)[kQB][2]) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int qb = 0; qb < kQB; qb++) {
      const int q = q0 + wave * 16 * kQB + qb * 16 + li;
      const uint8_t* mrow = mask + b * ms.s[0] + (int64_t)(q < Lq ? q : 0) * ms.s[2];
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int kbase = k0 + 32 * t + 8 * g;
        if (mask_vec && kbase + 8 <= Lk) {
          mw[qb][t] = *(const uint2v*)(mrow + kbase);
        } else {
          uint32_t w0 = 0, w1 = 0;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            uint32_t bit = (kbase + e < Lk) ? (mrow[(int64_t)(kbase + e) * ms.s[3]] != 0) : 0u;
            if (e < 4) w0 |= bit << (8 * e);
            else w1 |= bit << (8 * (e - 4));
          }
          mw[qb][t] = uint2v{w0, w1};
        }
      }
    }
  };

  // K tile `t` (rotated, as a separate Backend.rope would store it) and the
  // transposed V tile from the prefetch registers into LDS buffer `bf`
  auto store_kv = [&](int t, int bf) {
    if (kpart) {
      store_pair<BF16, true>(pr0, pr1, tabk != nullptr && t * kBK + kr < Lk, kc, kcs, Ks[bf], kr);
      return;
    }
    const uint32_t* pa = (const uint32_t*)&pr0;
    const uint32_t* pb = (const uint32_t*)&pr1;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      uint32_t lo = (pa[e] & 0xffff) | (pb[e] << 16);
      uint32_t hi = (pa[e] >> 16) | (pb[e] & 0xffff0000u);
      *(uint32_t*)(Vt[bf] + vt_swz(vc * 8 + 2 * e, vj >> 3) + (vj & 7)) = lo;
      *(uint32_t*)(Vt[bf] + vt_swz(vc * 8 + 2 * e + 1, vj >> 3) + (vj & 7)) = hi;
    }
  };

  // the first K / V tile (and its mask bytes) is requested before Q is
  // staged, so the two loads' latencies overlap
  int kt = next_tile(-1);
  uint2v mw[kQB][2], mwn[kQB][2];
  if (kt < nkt) {
    prefetch(kt);
    if (mask != nullptr && wave_class(kt) == 2) load_mask(kt, mw);
  }

  // ---- stage Q (rotated); this wave's B fragments of Q^T are read below
#pragma unroll
  for (int u = 0; u < QR; u++) {
    const int t = tid + u * kNT, r = t >> 2, c = t & 3, q = q0 + r;
    store_pair<BF16>(qlo[u], qhi[u], tabq != nullptr && q < Lq, c, qcs[u], Qs, r);
  }
  // the first tile into buffer 0; the second tile's loads start
  int nk = nkt;
  if (kt < nkt) {
    store_kv(kt, 0);
    nk = next_tile(kt);
    if (nk < nkt) prefetch(nk);
  }
  __syncthreads();
  uint4v qf[kQB][2];
#pragma unroll
  for (int qb = 0; qb < kQB; qb++)
#pragma unroll
    for (int s = 0; s < 2; s++)
      qf[qb][s] = *(const uint4v*)(Qs + qk_swz(wave * 16 * kQB + qb * 16 + li, s * 4 + g));


  float4v o[kQB][4];
  float m[kQB], l[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; qb++) {
#pragma unroll
    for (int d = 0; d < 4; d++) o[qb][d] = float4v{0.f, 0.f, 0.f, 0.f};
    m[qb] = -INFINITY;
    l[qb] = 0.f;
  }

  // online softmax of one 64-key tile for query block qb: scores st (raw,
  // -inf where hidden; lane key 32t + 8g + e is st[2t + e/4][e%4]) -> P
  // fragments, running max / sum, O rescale
  uint4v pf[kQB][2];
  auto softmax = [&](int qb, const float4v (&sq)[4], float mx) {
    mx = fmaxf(mx, from_xor16(mx));
    mx = max_xor32(mx);
    const float mnew = fmaxf(m[qb], mx);  // raw (unscaled) row max
    const float mc = mnew == -INFINITY ? 0.f : mnew * scale_log2;
    const float alpha = __builtin_amdgcn_exp2f(m[qb] * scale_log2 - mc);
    m[qb] = mnew;
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      uint32_t pk[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sq[2 * t + (e >> 2)][e & 3], scale_log2, -mc));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sq[2 * t + (e >> 2)][(e & 3) + 1], scale_log2, -mc));
        psum += p0 + p1;
        pk[e >> 1] = pack2<BF16>(p0, p1);
      }
      pf[qb][t] = uint4v{pk[0], pk[1], pk[2], pk[3]};
    }
    l[qb] = l[qb] * alpha + psum;
    // rescale O only when some row max of this wave moved
    if (!__all(alpha == 1.0f)) {
#pragma unroll
      for (int d = 0; d < 4; d++) o[qb][d] *= alpha;
    }
  };

  int buf = 0;
  while (kt < nkt) {
    const int k0 = kt * kBK;
    const int cl = wave_class(kt);  // this wave's class of the tile
    const uint16_t* Kc = Ks[buf];
    const uint16_t* Vc = Vt[buf];

    // ---- S^T = K . Q^T over 4 key blocks; block kb row i holds key
    // 32*(kb/2) + 8*(i/4) + (i%4) + 4*(kb%2) so a lane's 8 keys are contiguous
    // (a wave whose queries see no key of the tile skips its MFMAs and softmax)
    float4v st[kQB][4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      if (cl == 0) break;
      const int krow = 32 * (kb >> 1) + 8 * (li >> 2) + (li & 3) + 4 * (kb & 1);
      uint4v kf0 = *(const uint4v*)(Kc + k_swz(krow, g));
      uint4v kf1 = *(const uint4v*)(Kc + k_swz(krow, 4 + g));
#pragma unroll
      for (int qb = 0; qb < kQB; qb++) {
        float4v z = {0.f, 0.f, 0.f, 0.f};
        z = mfma16<BF16>(kf0, qf[qb][0], z);
        st[qb][kb] = mfma16<BF16>(kf1, qf[qb][1], z);
      }
    }

    // ---- the next tile into the other buffer (its loads were issued one
    // tile ago), the one after it into registers, the next mask bytes
    int nn = nkt;
    if (nk < nkt) {
      store_kv(nk, buf ^ 1);
      nn = next_tile(nk);
      if (nn < nkt) prefetch(nn);
      if (mask != nullptr && wave_class(nk) == 2) load_mask(nk, mwn);
    }

    // ---- mask (only for mixed tiles, in place), online softmax, P fragments
    if (cl != 0) {
#pragma unroll
      for (int qb = 0; qb < kQB; qb++) {
        if (cl == 2) {
#pragma unroll
          for (int t = 0; t < 2; t++) {
            const int kbase = k0 + 32 * t + 8 * g;  // this lane's 8 contiguous keys
            // bit 7 of byte e % 4 of word e / 4: key kbase + e is visible
            // (mask byte nonzero, key < Lk)
            uint32_t vx = 0x80808080u, vy = 0x80808080u;
            if (mask != nullptr) {
              vx = mask_nz(mw[qb][t].x);
              vy = mask_nz(mw[qb][t].y);
            }
            const int left = Lk - kbase;
            if (left < 8) {
              vx &= left >= 4 ? ~0u : (left <= 0 ? 0u : 0xffffffffu >> (8 * (4 - left)));
              vy &= left <= 4 ? 0u : 0xffffffffu >> (8 * (8 - left));
            }
            // a hidden score becomes -inf: the byte's bit 7 sign-extended to
            // a word mask, one bit-field insert per score
#pragma unroll
            for (int e = 0; e < 8; e++) {
              const uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)(e < 4 ? vx : vy), 8 * (e & 3) + 7, 1);
              const float sv = st[qb][2 * t + (e >> 2)][e & 3];
              st[qb][2 * t + (e >> 2)][e & 3] = __uint_as_float((__float_as_uint(sv) & m) | (~m & 0xff800000u));
            }
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
          for (int e = 0; e < 4; e++) mx = fmaxf(mx, st[qb][kb][e]);
        softmax(qb, st[qb], mx);
      }
    }

    // ---- O^T += V^T . P^T
#pragma unroll
    for (int d = 0; d < 4; d++) {
      if (cl == 0) break;
#pragma unroll
      for (int t = 0; t < 2; t++) {
        uint4v vf = *(const uint4v*)(Vc + vt_swz(d * 16 + li, 4 * t + g));
#pragma unroll
        for (int qb = 0; qb < kQB; qb++) o[qb][d] = mfma16<BF16>(vf, pf[qb][t], o[qb][d]);
      }
    }
#pragma unroll
    for (int qb = 0; qb < kQB; qb++)
#pragma unroll
      for (int t = 0; t < 2; t++) mw[qb][t] = mwn[qb][t];
    // this tile's buffer is free and the next one complete for every wave
    __syncthreads();
    buf ^= 1;
    kt = nk;
    nk = nn;
  }

  // ---- normalise and store (lane: one query, d = 16*dblk + 4g + 0..3)
#pragma unroll
  for (int qb = 0; qb < kQB; qb++) {
    float lt = l[qb];
    lt += from_xor16(lt);
    lt = sum_xor32(lt);
    const float inv = 1.0f / lt;
    const int q = q0 + wave * 16 * kQB + qb * 16 + li;
    if (q >= Lq) continue;
    // strided [B, H, Lq, D], or (pK > 0) panel order of the [B*Lq, pK]
    // matrix whose row b*Lq + q holds the heads side by side: columns
    // 64h + 16d + 4g.. are 16-column block 4h + d, half g/2, offset 4(g%2)
    uint16_t* op;
    int64_t dstep;
    if (pK > 0) {
      const int64_t m = (int64_t)b * Lq + q;
      op = O + ((m >> 5) * (pK >> 4) + 4 * h) * 512 + ((g >> 1) * 32 + (m & 31)) * 8 + 4 * (g & 1);
      dstep = 512;
    } else {
      op = O + b * os.s[0] + h * os.s[1] + (int64_t)q * os.s[2] + 4 * g;
      dstep = 16;
    }
#pragma unroll
    for (int d = 0; d < 4; d++) {
      uint2v w;
      w.x = fromf<BF16>(o[qb][d][0] * inv) | (fromf<BF16>(o[qb][d][1] * inv) << 16);
      w.y = fromf<BF16>(o[qb][d][2] * inv) | (fromf<BF16>(o[qb][d][3] * inv) << 16);
      *(uint2v*)(op + d * dstep) = w;
    }
  }
}

// ------------------------------------------------------------------ SIMT kernel (any dtype / D)

// One wave per query row: scores for every key into LDS, softmax in f32,
// then each lane accumulates its own output dims.
__device__ __forceinline__ float roped(int dt, const void* base, int64_t row, int64_t sd, int d, int D,
                                       const float2* tab, int pos) {
  float x = load_f(base, row + d * sd, dt);
  if (tab == nullptr) return x;
  int half = D / 2;
  int j = d < half ? d : d - half;
  float2 cs = tab[pos * half + j];
  float p = load_f(base, row + (d < half ? d + half : d - half) * sd, dt);
  // rotation rounded to the storage dtype, as a separate Backend.rope stores it
  float r = d < half ? fmaf(-p, cs.y, x * cs.x) : fmaf(p, cs.y, x * cs.x);
  return round_to(r, dt);
}

__global__ __launch_bounds__(64) void sdpa_simt(int dt, const void* __restrict__ Q, S4 qs,
                                                const void* __restrict__ K, S4 ks, const void* __restrict__ V, S4 vs,
                                                const uint8_t* __restrict__ mask, S4 ms, void* __restrict__ O, S4 os,
                                                int H, int Lq, int Lk, int D, float scale,
                                                const float2* __restrict__ tabq, const float2* __restrict__ tabk) {
  extern __shared__ float sc[];  // [Lk] scores, then [D] roped query
  float* qv = sc + Lk;
  const int lane = threadIdx.x;
  const int q = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t qrow = b * qs.s[0] + h * qs.s[1] + (int64_t)q * qs.s[2];
  for (int d = lane; d < D; d += 64) qv[d] = roped(dt, Q, qrow, qs.s[3], d, D, tabq, q);
  __syncthreads();
  float mx = -INFINITY;
  for (int j = lane; j < Lk; j += 64) {
    bool vis = mask == nullptr || mask[b * ms.s[0] + h * ms.s[1] + (int64_t)q * ms.s[2] + (int64_t)j * ms.s[3]];
    float s = -INFINITY;
    if (vis) {
      const int64_t krow = b * ks.s[0] + h * ks.s[1] + (int64_t)j * ks.s[2];
      float acc = 0.f;
      for (int d = 0; d < D; d++) acc = fmaf(qv[d], roped(dt, K, krow, ks.s[3], d, D, tabk, j), acc);
      s = acc * scale;
    }
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = lane; j < Lk; j += 64) {
    float p = sc[j] == -INFINITY ? 0.f : expf(sc[j] - mx);
    sc[j] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  __syncthreads();
  const float inv = 1.0f / sum;
  for (int d = lane; d < D; d += 64) {
    float acc = 0.f;
    for (int j = 0; j < Lk; j++) {
      float p = sc[j];
      if (p != 0.f) acc = fmaf(p, load_f(V, b * vs.s[0] + h * vs.s[1] + (int64_t)j * vs.s[2] + d * vs.s[3], dt), acc);
    }
    store_f(O, b * os.s[0] + h * os.s[1] + (int64_t)q * os.s[2] + d * os.s[3], dt, acc * inv);
  }
}

}  // namespace hb

using namespace hb;

extern "C" int hb_sdpa_mask_info_bytes(int64_t B, int64_t Lq, int64_t Lk, size_t* bytes) {
  HB_API_BEGIN
  HB_REQUIRE(bytes && B >= 0 && Lq >= 0 && Lk >= 0, "hb_sdpa_mask_info_bytes: bad arguments");
  *bytes = mask_info_bytes(B, Lq, Lk);
  HB_API_END
}

extern "C" int hb_sdpa_mask_info(uintptr_t ctx, uintptr_t mask, const int64_t* ms, int64_t B, int64_t Lq, int64_t Lk,
                                 uintptr_t info) {
  HB_API_BEGIN
  HB_REQUIRE(mask && ms && info, "hb_sdpa_mask_info: null argument");
  HB_REQUIRE(B >= 0 && Lq >= 0 && Lk >= 0 && B < 65536 && Lq < (1 << 30) && Lk < (1 << 30),
             "hb_sdpa_mask_info: bad shape");
  if (B == 0 || Lq == 0 || Lk == 0) return 0;
  launch_mask_info(stream_of(ctx), (const uint8_t*)mask, s4(ms), B, Lq, Lk, (uint8_t*)info);
  check_launch("hb_sdpa_mask_info");
  HB_API_END
}

// The MFMA kernel's conditions on a call (else sdpa_simt): 16-bit data,
// D = 64, unit inner strides, 16-byte aligned rows and 8-element strides, a
// mask that does not vary over heads, at most kMaxKeyTiles key tiles, and K /
// V row strides in [0, 2^24) (the kernel adds them as unsigned 24-bit
// products).  Lk == 0 takes the generic kernel: every row is fully masked,
// which it gives as 0/0 = NaN, as both kernels do for a row whose keys are
// all masked, and it needs no mask summary.
static bool sdpa_takes_mfma(int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks, uintptr_t v,
                            const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t o, const int64_t* os,
                            int64_t Lk, int64_t D) {
  return Lk > 0 && (dt == HB_F16 || dt == HB_BF16) && D == 64 && qs[3] == 1 && ks[3] == 1 && vs[3] == 1 &&
         os[3] == 1 && q % 16 == 0 && k % 16 == 0 && v % 16 == 0 && o % 8 == 0 && qs[2] % 8 == 0 &&
         ks[2] % 8 == 0 && vs[2] % 8 == 0 && qs[0] % 8 == 0 && qs[1] % 8 == 0 && ks[0] % 8 == 0 &&
         ks[1] % 8 == 0 && vs[0] % 8 == 0 && vs[1] % 8 == 0 && os[0] % 4 == 0 && os[1] % 4 == 0 &&
         os[2] % 4 == 0 && (mask == 0 || ms[1] == 0) && (Lk + kBK - 1) / kBK <= kMaxKeyTiles && ks[2] >= 0 &&
         ks[2] < (1 << 24) && vs[2] >= 0 && vs[2] < (1 << 24);
}

// The argument checks every sdpa entry point makes before it launches
// anything.
static void sdpa_check(int dt, const int64_t* qs, const int64_t* ks, const int64_t* vs, uintptr_t mask,
                       const int64_t* ms, const int64_t* os, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D) {
  HB_REQUIRE(dt == HB_F32 || dt == HB_F16 || dt == HB_BF16, "hb_sdpa: dtype must be f32, f16 or bf16");
  HB_REQUIRE(qs && ks && vs && os, "hb_sdpa: null strides");
  HB_REQUIRE(!mask || ms, "hb_sdpa: mask without strides");
  HB_REQUIRE(B >= 0 && H >= 0 && Lq >= 0 && Lk >= 0 && D > 0, "hb_sdpa: bad shape");
  HB_REQUIRE(B < 65536 && H < 65536 && Lq < (1 << 30) && Lk < (1 << 30), "hb_sdpa: shape too large");
}

// pK > 0: o is the panel-order [B*Lq, pK] matrix (pK = H*D), MFMA path only.
// A masked call on the MFMA path without a summary (mask_info == 0) builds
// one into a pool block, unless `noalloc`, where that is an error.
static void sdpa_impl(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks,
                      uintptr_t v, const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t mask_info,
                      uintptr_t o, const int64_t* os, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D,
                      float scale, double rope_q, double rope_k, int pK, bool noalloc = false) {
  sdpa_check(dt, qs, ks, vs, mask, ms, os, B, H, Lq, Lk, D);
  if (B == 0 || H == 0 || Lq == 0) return;
  HB_REQUIRE((rope_q <= 0 && rope_k <= 0) || D % 2 == 0, "hb_sdpa: rope needs an even head dim");
  HB_REQUIRE(!noalloc || (rope_q <= 0 && rope_k <= 0), "hb_sdpa_noalloc: no RoPE tables");
  hipStream_t st = stream_of(ctx);
  const float2* tq = rope_q > 0 ? (const float2*)rope_table(ctx, Lq, D, rope_q) : nullptr;
  const float2* tk = rope_k > 0 ? (const float2*)rope_table(ctx, Lk, D, rope_k) : nullptr;
  S4 Qs = s4(qs), Ks = s4(ks), Vs = s4(vs), Ms = s4(ms), Os = s4(os);
  const bool fast = sdpa_takes_mfma(dt, q, qs, k, ks, v, vs, mask, ms, o, os, Lk, D);
  if (pK > 0)
    HB_REQUIRE(fast && o % 16 == 0 && pK == H * D,
               "hb_sdpa_panel: needs the MFMA path (f16/bf16, D = 64, aligned operands, mask not varying over heads)");
  if (fast) {
    int nqt = (int)((Lq + kBQ - 1) / kBQ);
    uint8_t* info = (uint8_t*)mask_info;
    uint8_t* tmp = nullptr;
    int mask_vec = 0;
    if (mask) {
      if (!info) {
        HB_REQUIRE(!noalloc, "hb_sdpa_noalloc: no mask summary");
        tmp = (uint8_t*)pool_alloc(ctx, mask_info_bytes(B, Lq, Lk));
        launch_mask_info(st, (const uint8_t*)mask, Ms, B, Lq, Lk, tmp);
        check_launch("hb_sdpa(mask info)");
        info = tmp;
      }
      mask_vec = ms[3] == 1 && mask % 8 == 0 && ms[0] % 8 == 0 && ms[2] % 8 == 0;
    } else {
      info = nullptr;
    }
    const float sl2 = scale * 1.4426950408889634f;
    const int64_t nblk = (int64_t)nqt * H * B;
    HB_REQUIRE(nblk < ((int64_t)1 << 31), "hb_sdpa: too many (batch, head, query tile) blocks");
    const unsigned grid = (unsigned)nblk;
    if (dt == HB_F16)
      sdpa_mfma<false><<<grid, kNT, 0, st>>>((const uint16_t*)q, Qs, (const uint16_t*)k, Ks, (const uint16_t*)v, Vs,
                                             (const uint8_t*)mask, Ms, mask_vec, info, (uint16_t*)o, Os, (int)Lq,
                                             (int)Lk, sl2, tq, tk, pK, nqt, (int)H);
    else
      sdpa_mfma<true><<<grid, kNT, 0, st>>>((const uint16_t*)q, Qs, (const uint16_t*)k, Ks, (const uint16_t*)v, Vs,
                                            (const uint8_t*)mask, Ms, mask_vec, info, (uint16_t*)o, Os, (int)Lq,
                                            (int)Lk, sl2, tq, tk, pK, nqt, (int)H);
    check_launch("hb_sdpa");
    if (tmp) pool_free(ctx, tmp);
  } else {
    size_t lds = sizeof(float) * (size_t)(Lk + D);
    HB_REQUIRE(lds <= 160 * 1024, "hb_sdpa: sequence too long for the generic kernel");
    if (lds > 64 * 1024)
      HB_CHECK_HIP(hipFuncSetAttribute((const void*)sdpa_simt, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    dim3 grid((unsigned)Lq, (unsigned)H, (unsigned)B);
    sdpa_simt<<<grid, 64, lds, st>>>(dt, (const void*)q, Qs, (const void*)k, Ks, (const void*)v, Vs,
                                     (const uint8_t*)mask, Ms, (void*)o, Os, (int)H, (int)Lq, (int)Lk, (int)D, scale,
                                     tq, tk);
    check_launch("hb_sdpa(generic)");
  }
}

// The device address of `scratch` on each device, found once per device at
// hb_init (with that device current).  Host code passes these addresses to
// kernels; the array's name is only a host-side stand-in.
static std::mutex g_scratch_mu;
static void* g_scratch[64];

namespace hb {
void sdpa_scratch_init(int device) {
  HB_REQUIRE(device >= 0 && device < 64, "sdpa scratch: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device]) return;
  void* p = nullptr;
  HB_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  HB_REQUIRE(p != nullptr, "sdpa scratch: no device address");
  g_scratch[device] = p;
}
}  // namespace hb

extern "C" int hb_sdpa_noalloc(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks,
                               uintptr_t v, const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t o,
                               const int64_t* os, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D,
                               float scale) {
  HB_API_BEGIN
  sdpa_check(dt, qs, ks, vs, mask, ms, os, B, H, Lq, Lk, D);
  uintptr_t info = 0;
  // Only a masked call on the MFMA path reads a summary; the others launch
  // the generic kernel alone and have no size limit here.
  if (mask && B > 0 && H > 0 && Lq > 0 && sdpa_takes_mfma(dt, q, qs, k, ks, v, vs, mask, ms, o, os, Lk, D)) {
    const size_t need = mask_info_bytes(B, Lq, Lk);
    HB_REQUIRE(need <= kSdpaScratchBytes,
               "hb_sdpa_noalloc: the mask summary needs " + std::to_string(need) + " bytes, more than the " +
                   std::to_string(kSdpaScratchBytes) + "-byte scratch (B * ceil(Lq/128) * ceil(Lk/64) * 8); "
                   "use hb_sdpa for this shape");
    void* p;
    {
      std::lock_guard<std::mutex> lock(g_scratch_mu);
      p = g_scratch[device_of(ctx) & 63];
    }
    HB_REQUIRE(p, "hb_sdpa_noalloc: scratch not set up for this device (hb_init does it)");
    // every byte the attention kernel reads is written here: nothing to clear
    launch_mask_info(stream_of(ctx), (const uint8_t*)mask, s4(ms), B, Lq, Lk, (uint8_t*)p);
    check_launch("hb_sdpa_noalloc(mask info)");
    info = (uintptr_t)p;
  }
  sdpa_impl(ctx, dt, q, qs, k, ks, v, vs, mask, ms, info, o, os, B, H, Lq, Lk, D, scale, 0.0, 0.0, 0, true);
  HB_API_END
}

extern "C" int hb_sdpa(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks,
                       uintptr_t v, const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t mask_info,
                       uintptr_t o, const int64_t* os, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D,
                       float scale, double rope_q, double rope_k) {
  HB_API_BEGIN
  sdpa_impl(ctx, dt, q, qs, k, ks, v, vs, mask, ms, mask_info, o, os, B, H, Lq, Lk, D, scale, rope_q, rope_k, 0);
  HB_API_END
}

extern "C" int hb_sdpa_panel(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks,
                             uintptr_t v, const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t mask_info,
                             uintptr_t o, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, float scale,
                             double rope_q, double rope_k) {
  HB_API_BEGIN
  const int64_t os[4] = {0, 0, 0, 1};  // unused: the output is addressed in panel order
  sdpa_impl(ctx, dt, q, qs, k, ks, v, vs, mask, ms, mask_info, o, os, B, H, Lq, Lk, D, scale, rope_q, rope_k,
            (int)(H * D));
  HB_API_END
}
