// Scaled dot-product attention (Backend.sdpa) with optional fused RoPE.
//
// sdpa_mfma: flash attention for head dim 64 in fp16 / bf16 on
// v_mfma_f32_16x16x32.  A block owns 128 queries of one (b, h); each of its
// four waves owns 32 of them.  Per 64-key tile the wave computes
// S^T = K . Q^T, so a lane ends up holding the scores of ONE query for 8
// keys -- exactly the B-operand layout of O^T = V^T . P^T, so P never leaves
// registers.  The rows of K are fed to the MFMA in a permuted order that
// makes those 8 keys contiguous, which lets the lane read its 8 mask bytes
// with one load and its V^T fragment (V transposed in LDS) with one 16-byte
// read.  Softmax is online, in f32, in the log2 domain.  Key tiles outside
// the range where the (b, query tile) mask has any visible key are skipped:
// a pre-pass over the bool mask finds that range, so the sliding-window
// layers touch only the tiles inside the window (plus the full rows of
// padded queries, which see every valid key).  RoPE, when fused, rotates the
// Q and K tiles as they are staged and rounds them to the storage type,
// bit-identical to a separate Backend.rope.
//
// sdpa_simt: the f32 path and the fallback for other head dims / layouts.
#include <stdexcept>

#include "common.h"

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
constexpr int kBK = 64;   // keys per tile

// ------------------------------------------------------------------ mask pre-pass

// ranges[b * nqt + qt] = [first, last + 1) key TILE with any visible key for
// any query of the tile (any head).
__global__ __launch_bounds__(256) void mask_range_kernel(const uint8_t* __restrict__ mask, S4 ms, int H, int Lq,
                                                         int Lk, int nqt, int2* __restrict__ ranges) {
  __shared__ int lo, hi;
  const int qt = blockIdx.x, b = blockIdx.y;
  if (threadIdx.x == 0) {
    lo = Lk;
    hi = -1;
  }
  __syncthreads();
  const int q0 = qt * kBQ;
  const int nq = min(kBQ, Lq - q0);
  const int hn = ms.s[1] == 0 ? 1 : H;
  const int qn = ms.s[2] == 0 ? 1 : nq;
  int mylo = Lk, myhi = -1;
  const int64_t total = (int64_t)hn * qn * Lk;
  for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
    int k = (int)(i % Lk);
    int64_t rest = i / Lk;
    int q = (int)(rest % qn), h = (int)(rest / qn);
    if (mask[b * ms.s[0] + h * ms.s[1] + (int64_t)(q0 + q) * ms.s[2] + k * ms.s[3]]) {
      mylo = min(mylo, k);
      myhi = max(myhi, k);
    }
  }
  atomicMin(&lo, mylo);
  atomicMax(&hi, myhi);
  __syncthreads();
  if (threadIdx.x == 0) {
    int2 r;
    if (hi < 0) {
      r.x = 0;
      r.y = 0;
    } else {
      r.x = lo / kBK;
      r.y = hi / kBK + 1;
    }
    ranges[b * nqt + qt] = r;
  }
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

__device__ __forceinline__ int qk_swz(int r, int c) { return r * 64 + ((c ^ (r & 7)) << 3); }
constexpr int kVtLd = 72;  // row stride (elements) of V^T in LDS

// Loads row `row` (chunks c and c + 4, i.e. d in [8c, 8c+8) and the matching
// rotation partners d + 32) of a [L, 64] operand, rotating by RoPE at
// position `pos` when `tab` is set; writes both chunks to LDS.
template <bool BF16>
__device__ __forceinline__ void stage_pair(const uint16_t* __restrict__ src, bool valid, int c,
                                           const float2* __restrict__ tab, int pos, uint16_t* lds, int row) {
  uint4v lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
  if (valid) {
    lo = *(const uint4v*)(src + c * 8);
    hi = *(const uint4v*)(src + 32 + c * 8);
    if (tab != nullptr) {
      const float2* t = tab + pos * 32 + c * 8;
      uint32_t* l = (uint32_t*)&lo;
      uint32_t* h = (uint32_t*)&hi;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float2 c0 = t[2 * e], c1 = t[2 * e + 1];
        float x0a = tof<BF16>(l[e] & 0xffff), x0b = tof<BF16>(l[e] >> 16);
        float x1a = tof<BF16>(h[e] & 0xffff), x1b = tof<BF16>(h[e] >> 16);
        uint32_t oa = fromf<BF16>(pin_f32(fmaf(-x1a, c0.y, x0a * c0.x)));
        uint32_t ob = fromf<BF16>(pin_f32(fmaf(-x1b, c1.y, x0b * c1.x)));
        uint32_t pa = fromf<BF16>(pin_f32(fmaf(x0a, c0.y, x1a * c0.x)));
        uint32_t pb = fromf<BF16>(pin_f32(fmaf(x0b, c1.y, x1b * c1.x)));
        l[e] = oa | (ob << 16);
        h[e] = pa | (pb << 16);
      }
    }
  }
  *(uint4v*)(lds + qk_swz(row, c)) = lo;
  *(uint4v*)(lds + qk_swz(row, c + 4)) = hi;
}

template <bool BF16>
__global__ __launch_bounds__(256) void sdpa_mfma(const uint16_t* __restrict__ Q, S4 qs, const uint16_t* __restrict__ K,
                                                 S4 ks, const uint16_t* __restrict__ V, S4 vs,
                                                 const uint8_t* __restrict__ mask, S4 ms, int mask_vec,
                                                 const int2* __restrict__ ranges, uint16_t* __restrict__ O, S4 os,
                                                 int Lq, int Lk, float scale_log2, const float2* __restrict__ tabq,
                                                 const float2* __restrict__ tabk) {
  __shared__ __attribute__((aligned(16))) uint16_t Qs[kBQ * 64];
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBK * 64];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[64 * kVtLd];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int q0 = qt * kBQ;
  const uint16_t* Qb = Q + b * qs.s[0] + h * qs.s[1];
  const uint16_t* Kb = K + b * ks.s[0] + h * ks.s[1];
  const uint16_t* Vb = V + b * vs.s[0] + h * vs.s[1];

  // ---- stage Q (rotated) and build this wave's B fragments of Q^T
  for (int t = tid; t < kBQ * 4; t += 256) {
    int r = t >> 2, c = t & 3;
    int q = q0 + r;
    stage_pair<BF16>(Qb + (int64_t)q * qs.s[2], q < Lq, c, tabq, q, Qs, r);
  }
  __syncthreads();
  uint4v qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; qb++)
#pragma unroll
    for (int s = 0; s < 2; s++) qf[qb][s] = *(const uint4v*)(Qs + qk_swz(wave * 32 + qb * 16 + li, s * 4 + g));

  int kt0 = 0, kt1 = (Lk + kBK - 1) / kBK;
  if (ranges != nullptr) {
    int2 r = ranges[b * gridDim.x + qt];
    kt0 = r.x;
    kt1 = r.y;
  }

  float4v o[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; qb++)
#pragma unroll
    for (int d = 0; d < 4; d++) o[qb][d] = float4v{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};

  for (int kt = kt0; kt < kt1; kt++) {
    const int k0 = kt * kBK;
    __syncthreads();  // previous tile's K / V^T reads are done
    {  // K tile (rotated): 64 rows x 4 chunk pairs = one task per thread
      int r = tid >> 2, c = tid & 3;
      int kk = k0 + r;
      stage_pair<BF16>(Kb + (int64_t)kk * ks.s[2], kk < Lk, c, tabk, kk, Ks, r);
    }
    {  // V tile, transposed into V^T [d][key]: thread = (key pair, chunk)
      int c = tid & 7, jp = tid >> 3;
      int j0 = 2 * jp, kk = k0 + j0;
      uint4v a = {0, 0, 0, 0}, bb = {0, 0, 0, 0};
      if (kk < Lk) a = *(const uint4v*)(Vb + (int64_t)kk * vs.s[2] + c * 8);
      if (kk + 1 < Lk) bb = *(const uint4v*)(Vb + (int64_t)(kk + 1) * vs.s[2] + c * 8);
      const uint32_t* pa = (const uint32_t*)&a;
      const uint32_t* pb = (const uint32_t*)&bb;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        uint32_t lo = (pa[e] & 0xffff) | (pb[e] << 16);
        uint32_t hi = (pa[e] >> 16) | (pb[e] & 0xffff0000u);
        *(uint32_t*)(Vt + (c * 8 + 2 * e) * kVtLd + j0) = lo;
        *(uint32_t*)(Vt + (c * 8 + 2 * e + 1) * kVtLd + j0) = hi;
      }
    }
    __syncthreads();

    // ---- S^T = K . Q^T over 4 key blocks; block kb row i holds key
    // 32*(kb/2) + 8*(i/4) + (i%4) + 4*(kb%2) so a lane's 8 keys are contiguous
    float4v st[2][4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      const int krow = 32 * (kb >> 1) + 8 * (li >> 2) + (li & 3) + 4 * (kb & 1);
      uint4v kf0 = *(const uint4v*)(Ks + qk_swz(krow, g));
      uint4v kf1 = *(const uint4v*)(Ks + qk_swz(krow, 4 + g));
#pragma unroll
      for (int qb = 0; qb < 2; qb++) {
        float4v z = {0.f, 0.f, 0.f, 0.f};
        z = mfma16<BF16>(kf0, qf[qb][0], z);
        st[qb][kb] = mfma16<BF16>(kf1, qf[qb][1], z);
      }
    }

    // ---- mask, online softmax, P fragments
    uint4v pf[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
      const int q = q0 + wave * 32 + qb * 16 + li;
      float sv[2][8];
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int kbase = k0 + 32 * t + 8 * g;  // this lane's 8 contiguous keys
        uint8_t mb[8];
        if (mask != nullptr) {
          const uint8_t* mp = mask + b * ms.s[0] + (int64_t)(q < Lq ? q : 0) * ms.s[2] + kbase * ms.s[3];
          if (mask_vec && kbase + 8 <= Lk) {
            uint2v w = *(const uint2v*)mp;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              mb[e] = (w.x >> (8 * e)) & 0xff;
              mb[4 + e] = (w.y >> (8 * e)) & 0xff;
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; e++) mb[e] = (kbase + e < Lk) ? mp[e * ms.s[3]] : 0;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) mb[e] = 1;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
          float s = (e < 4 ? st[qb][2 * t][e] : st[qb][2 * t + 1][e - 4]) * scale_log2;
          bool vis = mb[e] != 0 && (kbase + e) < Lk;
          sv[t][e] = vis ? s : -INFINITY;
          mx = fmaxf(mx, sv[t][e]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m[qb], mx);
      const float muse = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = exp2f(m[qb] - muse);
      m[qb] = mnew;
      float psum = 0.f;
#pragma unroll
      for (int t = 0; t < 2; t++) {
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float p0 = exp2f(sv[t][e] - muse), p1 = exp2f(sv[t][e + 1] - muse);
          psum += p0 + p1;
          pk[e >> 1] = fromf<BF16>(p0) | (fromf<BF16>(p1) << 16);
        }
        pf[qb][t] = uint4v{pk[0], pk[1], pk[2], pk[3]};
      }
      l[qb] = l[qb] * alpha + psum;
#pragma unroll
      for (int d = 0; d < 4; d++) o[qb][d] *= alpha;
    }

    // ---- O^T += V^T . P^T
#pragma unroll
    for (int d = 0; d < 4; d++) {
#pragma unroll
      for (int t = 0; t < 2; t++) {
        uint4v vf = *(const uint4v*)(Vt + (d * 16 + li) * kVtLd + 32 * t + 8 * g);
#pragma unroll
        for (int qb = 0; qb < 2; qb++) o[qb][d] = mfma16<BF16>(vf, pf[qb][t], o[qb][d]);
      }
    }
  }

  // ---- normalise and store (lane: one query, d = 16*dblk + 4g + 0..3)
#pragma unroll
  for (int qb = 0; qb < 2; qb++) {
    float lt = l[qb];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const float inv = 1.0f / lt;
    const int q = q0 + wave * 32 + qb * 16 + li;
    if (q >= Lq) continue;
    uint16_t* op = O + b * os.s[0] + h * os.s[1] + (int64_t)q * os.s[2];
#pragma unroll
    for (int d = 0; d < 4; d++) {
      uint2v w;
      w.x = fromf<BF16>(o[qb][d][0] * inv) | (fromf<BF16>(o[qb][d][1] * inv) << 16);
      w.y = fromf<BF16>(o[qb][d][2] * inv) | (fromf<BF16>(o[qb][d][3] * inv) << 16);
      *(uint2v*)(op + d * 16 + 4 * g) = w;
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

extern "C" int hb_sdpa(uintptr_t ctx, int dt, uintptr_t q, const int64_t* qs, uintptr_t k, const int64_t* ks,
                       uintptr_t v, const int64_t* vs, uintptr_t mask, const int64_t* ms, uintptr_t o,
                       const int64_t* os, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, float scale,
                       double rope_q, double rope_k) {
  HB_API_BEGIN
  HB_REQUIRE(dt == HB_F32 || dt == HB_F16 || dt == HB_BF16, "hb_sdpa: dtype must be f32, f16 or bf16");
  HB_REQUIRE(qs && ks && vs && os, "hb_sdpa: null strides");
  HB_REQUIRE(!mask || ms, "hb_sdpa: mask without strides");
  HB_REQUIRE(B >= 0 && H >= 0 && Lq >= 0 && Lk >= 0 && D > 0, "hb_sdpa: bad shape");
  HB_REQUIRE(B < 65536 && H < 65536 && Lq < (1 << 30) && Lk < (1 << 30), "hb_sdpa: shape too large");
  if (B == 0 || H == 0 || Lq == 0) return 0;
  HB_REQUIRE((rope_q <= 0 && rope_k <= 0) || D % 2 == 0, "hb_sdpa: rope needs an even head dim");
  hipStream_t st = stream_of(ctx);
  int64_t Lt = Lq > Lk ? Lq : Lk;
  const float2* tq = rope_q > 0 ? (const float2*)rope_table(ctx, Lq, D, rope_q) : nullptr;
  const float2* tk = rope_k > 0 ? (const float2*)rope_table(ctx, Lk, D, rope_k) : nullptr;
  (void)Lt;
  S4 Qs = s4(qs), Ks = s4(ks), Vs = s4(vs), Ms = s4(ms), Os = s4(os);
  bool fast = (dt == HB_F16 || dt == HB_BF16) && D == 64 && qs[3] == 1 && ks[3] == 1 && vs[3] == 1 && os[3] == 1 &&
              q % 16 == 0 && k % 16 == 0 && v % 16 == 0 && o % 8 == 0 && qs[2] % 8 == 0 && ks[2] % 8 == 0 &&
              vs[2] % 8 == 0 && qs[0] % 8 == 0 && qs[1] % 8 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 &&
              vs[0] % 8 == 0 && vs[1] % 8 == 0 && os[0] % 4 == 0 && os[1] % 4 == 0 && os[2] % 4 == 0 &&
              (mask == 0 || ms[1] == 0);
  if (fast) {
    int nqt = (int)((Lq + kBQ - 1) / kBQ);
    int2* ranges = nullptr;
    int mask_vec = 0;
    if (mask) {
      ranges = (int2*)pool_alloc(ctx, sizeof(int2) * (size_t)(B * nqt));
      mask_range_kernel<<<dim3(nqt, (unsigned)B), 256, 0, st>>>((const uint8_t*)mask, Ms, (int)H, (int)Lq, (int)Lk,
                                                                 nqt, ranges);
      check_launch("hb_sdpa(mask ranges)");
      mask_vec = ms[3] == 1 && mask % 8 == 0 && ms[0] % 8 == 0 && ms[2] % 8 == 0;
    }
    const float sl2 = scale * 1.4426950408889634f;
    dim3 grid(nqt, (unsigned)H, (unsigned)B);
    if (dt == HB_F16)
      sdpa_mfma<false><<<grid, 256, 0, st>>>((const uint16_t*)q, Qs, (const uint16_t*)k, Ks, (const uint16_t*)v, Vs,
                                             (const uint8_t*)mask, Ms, mask_vec, ranges, (uint16_t*)o, Os, (int)Lq,
                                             (int)Lk, sl2, tq, tk);
    else
      sdpa_mfma<true><<<grid, 256, 0, st>>>((const uint16_t*)q, Qs, (const uint16_t*)k, Ks, (const uint16_t*)v, Vs,
                                            (const uint8_t*)mask, Ms, mask_vec, ranges, (uint16_t*)o, Os, (int)Lq,
                                            (int)Lk, sl2, tq, tk);
    check_launch("hb_sdpa");
    if (ranges) pool_free(ctx, ranges);
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
  HB_API_END
}
