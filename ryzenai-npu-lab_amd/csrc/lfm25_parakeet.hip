// Parakeet (FastConformer) encoder on gfx950: the reference's all-NPU encoder
// (experiments/pk_model.py, pk_engine.py, kernels/pk/pk_core.cc, pk_fast.cc)
// as four kernels per block phase kind, one stream:
//
//   GEMM      C = bf16(epi(A . B + bias)) on the matrix cores, 128 x 128 block
//             tiles (replaces gemm_step / pk_wx / epilogue,
//             pk_fast.cc:167-231, pk_core.cc:169-183)
//   LN        scaled residual + LayerNorm (+ a second LayerNorm)
//             (layer_norm / residual / ln_frame, pk_core.cc:55-116)
//   ATT       relative-position attention of one (sequence, head)
//             (att_queries / att_bd / att_keys / att_finish,
//             pk_core.cc:126-203, pk_fast.cc:71-116)
//   CONV      GLU + 9-tap depthwise conv + bias + Swish (conv_frames,
//             pk_fast.cc:119-154)
//
// and the 22-phase block order of build_phases (pk_model.py:132-161) on the
// host. Rounding points are those of the reference's BF16 mirror
// (experiments/012_layer_test.py:45-114): FP32 inside a phase, BF16 where the
// NPU stores a field. Weight matrices are stored output-major ([out x in],
// every row contiguous in the reduction dimension) so both GEMM operands are
// read as 16-byte runs along K.
#include <algorithm>
#include <cstring>
#include <vector>

#include "lfm25_host.h"
#include "lfm25_device.h"

namespace lfm25 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kD = 1024;
constexpr int kPkHeads = 8;
constexpr int kDk = 128;
constexpr int kPkFfn = 4096;
constexpr int kConvTapsPk = 9;
constexpr float kLnEps = 1.0e-5f;

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// Sum / maximum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (gfx950 row swaps).
__device__ __forceinline__ float sum_lanes16(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}
__device__ __forceinline__ float max_lanes16(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}

// ------------------------------------------------------------------ GEMM

// C[m][n] = bf16(epi(sum_k A[m][k] Bt[n][k] + bias[n])) for a (64 kWM) x 128
// tile per block (blockIdx.x: n tile, blockIdx.y: m tile, blockIdx.z: batch
// of independent products with element strides, or the K split). 2 kWM waves
// in kWM x 2, each 64 x 64 as 4 x 4 MFMA tiles (v_mfma_f32_16x16x32_bf16 with
// the weight tile as the first operand, so a lane's four results are four
// consecutive n of one row m and leave as one 8-byte store). kWM = 2 (128 x
// 128, two blocks per CU) by default; kWM = 4 (256 x 128, one block of 8
// waves per CU) for wide products with many rows: the tile loads, which bound
// this kernel through the L2 -> CU path, fall from 1/64 to 3/256 bytes per
// FLOP. K steps of 64
// go through double-buffered LDS: the next step's 16-byte global loads are
// in flight in registers while the current step multiplies, and land in the
// other buffer after it (one barrier per step). Rows m >= M read row M - 1
// (their results are never stored), so every load is unconditional.
//
// Split K (kSplit): block z covers K range [z * kchunk, (z + 1) * kchunk) and
// writes its FP32 partial tile to part[z][M][N]; k_pk_splitk sums the splits
// in index order and applies the epilogue, so the result does not depend on
// which blocks ran when.
constexpr int kBM = 128, kBN = 128, kBK = 64;  // kBM: the tile height of split products
// LDS holds each 64-wide K step of a tile row as eight 16-byte chunks; chunk
// c of row r sits at position c ^ ((r / 2) % 8) of the row, so the 16-byte
// reads of 16 consecutive rows at one chunk (an MFMA operand) and the
// row-contiguous 16-byte stores both spread over all 64 banks (no bank
// conflict cycles on gfx950; a one-chunk row padding leaves a third of the
// LDS cycles in conflicts).
constexpr int kRowChunks = 8;
__device__ __forceinline__ int lds_chunk(int r, int c) { return r * kRowChunks + (c ^ ((r >> 1) & 7)); }
constexpr int kSplitUnits = 256;  // split K until tiles x splits reaches this many blocks
// ... or this many for products of at most 256 rows (one window): there the
// FP32 partials of more splits cost more than the parallelism gains (a
// 128-row tile writes as many partial bytes as it reads operand bytes)
constexpr int kSplitUnitsFew = 64;
constexpr int kMinChunk = 128;    // smallest K range of a split
// FP32 partials: tiles x splits < 2 x kSplitUnits blocks of 128 x 128
constexpr size_t kPartBytes = (size_t)2 * kSplitUnits * kBM * kBN * sizeof(float);
enum PkEpi { EPI_NONE = 0, EPI_BIAS = 1, EPI_SWISH = 2 };

struct PkGemm {
  const uint16_t* A;
  const uint16_t* Bt;
  const uint16_t* bias;
  uint16_t* C;
  float* part;
  long long sa, sb, sc;  // per-z element strides (batched products)
  int lda, ldb, ldc, M, N, kchunk;
};

template <int EPI>
__device__ __forceinline__ float epilogue(float v, float b) {
  if (EPI == EPI_BIAS) v = v + b;
  if (EPI == EPI_SWISH) v = v * sigmoid_f32(v);
  return v;
}

// C = bf16(epi(A . B + bias)) per block tile of (64 kWM) x 128: kWM = 4 (256
// rows, 8 waves) for the tall unsplit products, kWM = 2 (128 rows, 4 waves)
// otherwise; each wave owns a 64 x 64 accumulator tile. The operands are
// copied from global memory straight into LDS (global_load_lds, 16 bytes per
// lane): no register staging and no LDS stores in the loop, three LDS stages
// of one K step each (48 or 32 KB apiece), the copies of step s + 2 issued as
// step s starts. A wave-instruction fills 64 consecutive 16-byte slots, so
// each lane loads the chunk whose swizzled slot (lds_chunk) it fills. With
// kSplit the block covers K range z and leaves its FP32 partial tile for
// k_pk_splitk / k_pk_reduce_ln; rows past M read row M - 1 and are not
// stored.
typedef __attribute__((address_space(3))) void PkLdsVoid;
typedef __attribute__((address_space(1))) void PkGlobalVoid;
template <int kWM>
struct PkGemmDmaLds {
  uint4 a[3][64 * kWM * kRowChunks];
  uint4 b[3][kBN * kRowChunks];
};
// One K step of 64 from LDS stage `buf` into the wave's 64 x 64 accumulators.
template <int kWM>
__device__ __forceinline__ void gemm_step_dma(const PkGemmDmaLds<kWM>& sh, int buf, int wm, int wn, int l,
                                              f32x4_t (&acc)[4][4]) {
#pragma unroll
  for (int ks = 0; ks < kBK / 32; ++ks) {
    const int kc = 4 * ks + (l >> 4);  // chunk of k = 32 ks + 8 (l / 16) .. + 7
    bf16x8_t xa[4], wb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xa[i] = __builtin_bit_cast(bf16x8_t, sh.a[buf][lds_chunk(64 * wm + 16 * i + (l & 15), kc)]);
      wb[i] = __builtin_bit_cast(bf16x8_t, sh.b[buf][lds_chunk(64 * wn + 16 * i + (l & 15), kc)]);
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb[nt], xa[mt], acc[nt][mt], 0, 0, 0);
  }
}

template <int EPI, bool kSplit, int kWM>
__global__ void __launch_bounds__(128 * kWM, 1) k_pk_gemm_dma(const PkGemm g) {
  constexpr int kTileM = 64 * kWM;
  constexpr int kAI = 4, kBI = 8 / kWM;  // copy instructions per wave and step: A, B
  __shared__ PkGemmDmaLds<kWM> sh;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kTileM, z = blockIdx.z;
  const int w = wave_id(), l = lane_id();
  const int wm = w % kWM, wn = w / kWM;
  const int kbeg = kSplit ? z * g.kchunk : 0;
  const uint16_t* A = g.A + (kSplit ? 0 : g.sa * z) + kbeg;
  const uint16_t* Bt = g.Bt + (kSplit ? 0 : g.sb * z) + kbeg;
  // this lane's source rows and chunks: A slots (kAI w + i) * 64 + l, B slots (kBI w + i) * 64 + l
  const uint16_t* pa[kAI];
  const uint16_t* pb[kBI];
#pragma unroll
  for (int i = 0; i < kAI; ++i) {
    const int p = (kAI * w + i) * kWave + l, r = p / kRowChunks, q = (p % kRowChunks) ^ ((r >> 1) & 7);
    pa[i] = A + (size_t)min(m0 + r, g.M - 1) * g.lda + 8 * q;
  }
#pragma unroll
  for (int i = 0; i < kBI; ++i) {
    const int p = (kBI * w + i) * kWave + l, r = p / kRowChunks, q = (p % kRowChunks) ^ ((r >> 1) & 7);
    pb[i] = Bt + (size_t)(n0 + r) * g.ldb + 8 * q;
  }
  const auto copy = [&](int step, int buf) {
    const int k = step * kBK;
#pragma unroll
    for (int i = 0; i < kAI; ++i)
      __builtin_amdgcn_global_load_lds((PkGlobalVoid*)(pa[i] + k), (PkLdsVoid*)&sh.a[buf][(kAI * w + i) * kWave], 16, 0,
                                       0);
#pragma unroll
    for (int i = 0; i < kBI; ++i)
      __builtin_amdgcn_global_load_lds((PkGlobalVoid*)(pb[i] + k), (PkLdsVoid*)&sh.b[buf][(kBI * w + i) * kWave], 16, 0,
                                       0);
  };
  const int steps = g.kchunk / kBK;
  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  copy(0, 0);
  if (steps > 1) copy(1, 1);
  int buf = 0;
  for (int s = 0; s < steps; ++s) {
    // this wave's copies of step s have landed (those of step s + 1, kAI +
    // kBI loads, may still be in flight); the barrier makes every wave's so,
    // and puts every wave's reads of step s - 1's buffer behind it
    if (s + 1 < steps) __builtin_amdgcn_s_waitcnt(0x0F70 | (kAI + kBI));  // vmcnt(kAI + kBI)
    else __builtin_amdgcn_s_waitcnt(0x0F70);                              // vmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (s + 2 < steps) copy(s + 2, buf == 0 ? 2 : buf - 1);
    gemm_step_dma<kWM>(sh, buf, wm, wn, l, acc);
    buf = buf == 2 ? 0 : buf + 1;
  }
  if (kSplit) {
    float* P = g.part + (size_t)z * g.M * g.N;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int n = n0 + 64 * wn + 16 * nt + 4 * (l >> 4);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int m = m0 + 64 * wm + 16 * mt + (l & 15);
        if (m < g.M) *reinterpret_cast<f32x4_t*>(P + (size_t)m * g.N + n) = acc[nt][mt];
      }
    }
    return;
  }
  uint16_t* C = g.C + g.sc * z;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = n0 + 64 * wn + 16 * nt + 4 * (l >> 4);
    float bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (EPI == EPI_BIAS) {
#pragma unroll
      for (int e = 0; e < 4; ++e) bs[e] = bf16_to_f32(g.bias[n + e]);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int m = m0 + 64 * wm + 16 * mt + (l & 15);
      if (m >= g.M) continue;
      u32x2_t pk;
      pk.x = (uint32_t)f32_to_bf16(epilogue<EPI>(acc[nt][mt][0], bs[0])) |
             ((uint32_t)f32_to_bf16(epilogue<EPI>(acc[nt][mt][1], bs[1])) << 16);
      pk.y = (uint32_t)f32_to_bf16(epilogue<EPI>(acc[nt][mt][2], bs[2])) |
             ((uint32_t)f32_to_bf16(epilogue<EPI>(acc[nt][mt][3], bs[3])) << 16);
      *reinterpret_cast<u32x2_t*>(C + (size_t)m * g.ldc + n) = pk;
    }
  }
}

// y += partials z .. z + G - 1 of a thread's NQ x 4 values (partial i at
// p + i * stride), those below `splits` only, added in index order after all
// G loads are issued; a load past the last partial repeats the last one.
template <int G, int NQ>
__device__ __forceinline__ void add_partials(f32x4_t (&y)[NQ], const float* p, size_t stride, int z, int splits) {
  f32x4_t t[G][NQ];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int zu = z + u < splits ? z + u : splits - 1;
#pragma unroll
    for (int q = 0; q < NQ; ++q) t[u][q] = *reinterpret_cast<const f32x4_t*>(p + zu * stride + 4 * q);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait
#pragma unroll
  for (int u = 0; u < G; ++u)
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const f32x4_t r = f32x4_t{y[q][0] + t[u][q][0], y[q][1] + t[u][q][1], y[q][2] + t[u][q][2],
                                y[q][3] + t[u][q][3]};
      y[q] = z + u < splits ? r : y[q];
    }
}
// y = the sum of partials 0 .. splits - 1 in index order, from -0 (x + -0 is
// x for every x, the sign of zero included), G partials' loads in flight per
// round trip. The host picks G from the split count (partial_group): one
// straight-line group per round trip, with no branch for the compiler to
// hoist a shared first load out of.
template <int G, int NQ>
__device__ __forceinline__ void sum_partials(f32x4_t (&y)[NQ], const float* p, size_t stride, int splits) {
#pragma unroll
  for (int q = 0; q < NQ; ++q) y[q] = f32x4_t{-0.0f, -0.0f, -0.0f, -0.0f};
  for (int z = 0; z < splits; z += G) add_partials<G>(y, p, stride, z, splits);
}
// Partials per round trip for `splits` of them: the next power of two, at
// most 8 (a one-window product has 8 splits).
inline int partial_group(int splits) { return splits <= 1 ? 1 : splits <= 2 ? 2 : splits <= 4 ? 4 : 8; }

// Sum of the `splits` FP32 partial products in index order (G of them per
// round trip), epilogue, BF16: one thread per four consecutive outputs of
// row blockIdx.x (blockIdx.y: the row's 1024-wide column range).
template <int EPI, int G>
__global__ void __launch_bounds__(256) k_pk_splitk(const float* __restrict__ part, int splits, int M, int N,
                                                   const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
                                                   int ldc) {
  const int m = blockIdx.x, n = 4 * (blockIdx.y * 256 + threadIdx.x);
  if (n >= N) return;
  float bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // loaded first: in flight with the partials
  if (EPI == EPI_BIAS) {
#pragma unroll
    for (int e = 0; e < 4; ++e) bs[e] = bf16_to_f32(bias[n + e]);
  }
  f32x4_t v[1];
  sum_partials<G>(v, part + (size_t)m * N + n, (size_t)M * N, splits);
  u32x2_t pk;
  pk.x = (uint32_t)f32_to_bf16(epilogue<EPI>(v[0][0], bs[0])) |
         ((uint32_t)f32_to_bf16(epilogue<EPI>(v[0][1], bs[1])) << 16);
  pk.y = (uint32_t)f32_to_bf16(epilogue<EPI>(v[0][2], bs[2])) |
         ((uint32_t)f32_to_bf16(epilogue<EPI>(v[0][3], bs[3])) << 16);
  *reinterpret_cast<u32x2_t*>(C + (size_t)m * ldc + n) = pk;
}

// ------------------------------------------------------------------ LayerNorm

// A lane's 16 BF16 values as loaded (two 16-byte words): unpacked where used,
// so a load issued early is not waited for until then.
struct Row16 {
  uint4 a, b;
};
__device__ __forceinline__ Row16 load_raw16(const uint16_t* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  return Row16{q[0], q[1]};
}
__device__ __forceinline__ void unpack16(const Row16& r, float* v) {
  const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = lo_f32(w[i]);
    v[2 * i + 1] = hi_f32(w[i]);
  }
}
__device__ __forceinline__ void load_row16(const uint16_t* p, float* v) { unpack16(load_raw16(p), v); }
__device__ __forceinline__ void store_row16(uint16_t* p, const float* v) {
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
  uint4* q = reinterpret_cast<uint4*>(p);
  q[0] = uint4{w[0], w[1], w[2], w[3]};
  q[1] = uint4{w[4], w[5], w[6], w[7]};
}

// bf16((v - mean) / sqrt(var + eps) * g + b) of one 1024-row held 16 per lane
// (lane l: elements 16l .. 16l + 15); mean and variance in FP32 (wave sums).
// g / b: the lane's 16 gammas and betas.
__device__ __forceinline__ void ln_apply(const float* v, const Row16& g, const Row16& b, float* out) {
  float gv[16], bv[16];
  unpack16(g, gv);
  unpack16(b, bv);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += v[i];
  const float mu = wave_sum(s) * (1.0f / (float)kD);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float d = v[i] - mu;
    q += d * d;
  }
  const float var = wave_sum(q) * (1.0f / (float)kD);
  const float den = sqrtf(var + kLnEps);
#pragma unroll
  for (int i = 0; i < 16; ++i) out[i] = round_bf16((v[i] - mu) / den * gv[i] + bv[i]);
}

// A lane's 16 gammas and betas of LN1 and, when g2 is given, of LN2: loaded
// before the row they norm is formed, so their loads overlap the row's.
struct LnLane {
  Row16 g1, b1, g2, b2;
  bool two;
};
__device__ __forceinline__ void load_ln(LnLane& p, const uint16_t* g1, const uint16_t* b1, const uint16_t* g2,
                                        const uint16_t* b2) {
  p.g1 = load_raw16(g1 + 16 * lane_id());
  p.b1 = load_raw16(b1 + 16 * lane_id());
  p.two = g2 != nullptr;
  if (p.two) {
    p.g2 = load_raw16(g2 + 16 * lane_id());
    p.b2 = load_raw16(b2 + 16 * lane_id());
  }
}

// The norm modes of one row m given x' (v, 16 per lane). "carry"
// (normed_x == 0): x <- x' when store_x, a <- LN1(x'). "normed"
// (normed_x == 1): x <- LN1(x') and, when LN2 is given, a <- LN2(x)
// (ln_frame's DOUBLE/FINAL, pk_core.cc:99-116).
__device__ __forceinline__ void ln_modes(uint16_t* x, int m, const float* v, bool store_x, const LnLane& p,
                                         int normed_x, uint16_t* a) {
  const size_t off = (size_t)m * kD + 16 * lane_id();
  float o[16];
  ln_apply(v, p.g1, p.b1, o);
  if (!normed_x) {
    if (store_x) store_row16(x + off, v);
    store_row16(a + off, o);
    return;
  }
  store_row16(x + off, o);
  if (p.two) {
    float o2[16];
    ln_apply(o, p.g2, p.b2, o2);
    store_row16(a + off, o2);
  }
}

// One wave per row (four rows per block). x' = y ? bf16(x + s * y) : x, then
// ln_modes.
constexpr int kLnRows = 4;
__global__ void __launch_bounds__(kLnRows* kWave) k_pk_ln(uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
                                                          float s, const uint16_t* __restrict__ g1,
                                                          const uint16_t* __restrict__ b1,
                                                          const uint16_t* __restrict__ g2,
                                                          const uint16_t* __restrict__ b2, int normed_x,
                                                          uint16_t* __restrict__ a, int rows) {
  const int m = blockIdx.x * kLnRows + wave_id();
  if (m >= rows) return;
  const size_t off = (size_t)m * kD + 16 * lane_id();
  LnLane p;
  load_ln(p, g1, b1, g2, b2);
  float v[16];
  load_row16(x + off, v);
  if (y != nullptr) {
    float yv[16];
    load_row16(y + off, yv);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = round_bf16(v[i] + s * yv[i]);
  }
  ln_modes(x, m, v, y != nullptr, p, normed_x, a);
}

// The end of a d-wide product whose `splits` FP32 partials sit in
// part[z][rows][1024]: y = bf16(sum of the partials in index order), then
// x' = bf16(x + s * y) and ln_modes (the GEMM's store, residual and
// LayerNorm phases of pk_core.cc:90-116 in one pass over the row). R rows
// (waves) per block: one when the product has few rows, so that a row's
// splits x 4 KB of partials are spread over as many CUs as there are rows
// (a CU's load rate, not HBM, bounds this pass).
template <int R, int G>
__global__ void __launch_bounds__(R* kWave) k_pk_reduce_ln(const float* __restrict__ part, int splits,
                                                                 uint16_t* __restrict__ x, float s,
                                                                 const uint16_t* __restrict__ g1,
                                                                 const uint16_t* __restrict__ b1,
                                                                 const uint16_t* __restrict__ g2,
                                                                 const uint16_t* __restrict__ b2, int normed_x,
                                                                 uint16_t* __restrict__ a, int rows) {
  const int m = blockIdx.x * R + wave_id();
  if (m >= rows) return;
  const size_t off = (size_t)m * kD + 16 * lane_id();
  const size_t stride = (size_t)rows * kD;
  // the residual row and the norms' parameters first: in flight with the partials
  LnLane p;
  load_ln(p, g1, b1, g2, b2);
  const Row16 xr = load_raw16(x + off);
  f32x4_t y[4];
  sum_partials<G>(y, part + off, stride, splits);
  float v[16];
  unpack16(xr, v);
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = round_bf16(v[i] + s * round_bf16(y[i / 4][i % 4]));
  ln_modes(x, m, v, true, p, normed_x, a);
}

// ------------------------------------------------------------------ attention

// Relative-position attention of sequence b (blockIdx.y), head h
// (blockIdx.x) over T = 128 frames, `valid` of them real (keys j >= valid
// masked), as the mirror computes it (012_layer_test.py:67-86):
//   bd_ij' = bf16(q_i . P_h[:, j'])            (j' < 2T, position scores)
//   qu = bf16(q + delta_h); s_ij = qu_i . k_j + bd_i,T-1-i+j;
//   p = softmax_j(s) in FP32; o_i = bf16(sum_j p_ij v_j).
// q (scaled, bias_v folded in), k, v come from the q|k|v rows [T x 3072];
// P_h^T is the head's [2T x 128] position table (last row zero).
//
// The block first requests everything it reads (P, K and V into LDS, each
// wave's 16 query rows into registers) in one round of 16-byte loads. Each
// wave then forms its queries' position scores and key scores from LDS on
// the matrix cores (BF16 operands, exact products, FP32 sums); after a
// barrier the position scores go to LDS as BF16 over the P region, so the
// shifted index T-1-i+j can be read per element. The probabilities stay FP32
// through the value product by splitting each into a BF16 high part and a
// BF16 remainder (two MFMA chains); V^T is the first operand, so a lane's four
// results are four consecutive dimensions of one query (one 8-byte store).
constexpr int kAttT = 128;
constexpr int kAttWaves = 8;
constexpr int kQT = kAttT / 16 / kAttWaves;  // 16-query tiles per wave: 1
constexpr int kAttThreads = kAttWaves * kWave;
constexpr int kAttRow = kDk + 8;           // bf16 per LDS row of P, K, V^T (272 bytes: conflict-free 16-byte reads)
constexpr int kBdRow = 2 * kAttT + 8;      // bf16 per LDS row of the position scores
// V^T rows of 130 bf16 (65 words: consecutive rows start one bank apart), so
// the transposing 2-byte stores of 16 dimensions at one key spread over the
// banks; the rows are 4-byte aligned, so the operand reads are 4-byte.
constexpr int kVtRow = kAttT + 2;
struct PkAttLds {
  union {
    uint16_t p[2 * kAttT][kAttRow];        // P_h^T [j'][d] while the position scores are formed
    uint16_t bd[kAttT][kBdRow];            // then the BF16 position scores [i][j']
  } u;
  uint16_t k[kAttT][kAttRow];              // K [j][d]
  uint16_t vt[kDk][kVtRow];                // V^T [d][j]
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }
__device__ __forceinline__ bf16x8_t lds_frag(const uint16_t* row, int col) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(row + col));
}

// kAttSplit blocks per (sequence, head), blockIdx.z taking query tiles
// [kAttWaves / kAttSplit z, + kAttWaves / kAttSplit): each block stages the
// whole P, K and V^T but forms only its queries' products, so at one window
// the 8 heads run on 16 CUs instead of 8.
constexpr int kAttSplit = 2;
constexpr int kAttBlockThreads = kAttThreads / kAttSplit;
__global__ void __launch_bounds__(kAttBlockThreads, 1)
    k_pk_attention(const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ pos,
                   const uint16_t* __restrict__ delta, uint16_t* __restrict__ out, int valid) {
  __shared__ PkAttLds sh;
  const int h = blockIdx.x, b = blockIdx.y;
  // w: the wave's query tile (16 kQT w ..) over the (sequence, head)'s kAttWaves
  const int t = threadIdx.x, w = wave_id() + (kAttWaves / kAttSplit) * blockIdx.z, l = lane_id();
  const uint16_t* base = qkv + (size_t)b * kAttT * 3 * kD;
  const uint16_t* ph = pos + (size_t)h * 2 * kAttT * kDk;
  // one round of loads: P (16 chunks per thread), K and V (8 each), this wave's q fragments
  constexpr int kRowChunks16 = kDk / 8;  // 16-byte chunks per 128-wide row
  uint4 pr[2 * kAttT * kRowChunks16 / kAttBlockThreads], kr[kAttT * kRowChunks16 / kAttBlockThreads],
      vr[kAttT * kRowChunks16 / kAttBlockThreads];
#pragma unroll
  for (int i = 0; i < 2 * kAttT * kRowChunks16 / kAttBlockThreads; ++i) {
    const int c = t + kAttBlockThreads * i;
    pr[i] = *reinterpret_cast<const uint4*>(ph + (size_t)(c / kRowChunks16) * kDk + 8 * (c % kRowChunks16));
  }
#pragma unroll
  for (int i = 0; i < kAttT * kRowChunks16 / kAttBlockThreads; ++i) {
    const int c = t + kAttBlockThreads * i;
    const uint16_t* row = base + (size_t)(c / kRowChunks16) * 3 * kD + h * kDk + 8 * (c % kRowChunks16);
    kr[i] = *reinterpret_cast<const uint4*>(row + kD);
    vr[i] = *reinterpret_cast<const uint4*>(row + 2 * kD);
  }
  uint4 qraw[kQT][kDk / 32];  // query 16 kQT w + 16qt + l%16, dimensions 32ds + 8(l/16) .. + 7
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
    for (int ds = 0; ds < kDk / 32; ++ds)
      qraw[qt][ds] = *reinterpret_cast<const uint4*>(base + (size_t)(16 * kQT * w + 16 * qt + (l & 15)) * 3 * kD +
                                                      h * kDk + 32 * ds + 8 * (l >> 4));
#pragma unroll
  for (int i = 0; i < 2 * kAttT * kRowChunks16 / kAttBlockThreads; ++i) {
    const int c = t + kAttBlockThreads * i;
    *reinterpret_cast<uint4*>(&sh.u.p[c / kRowChunks16][8 * (c % kRowChunks16)]) = pr[i];
  }
#pragma unroll
  for (int i = 0; i < kAttT * kRowChunks16 / kAttBlockThreads; ++i) {
    const int c = t + kAttBlockThreads * i;
    const int j = c / kRowChunks16, d0 = 8 * (c % kRowChunks16);
    *reinterpret_cast<uint4*>(&sh.k[j][d0]) = kr[i];
    const uint32_t vw[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sh.vt[d0 + 2 * e][j] = (uint16_t)(vw[e] & 0xffffu);
      sh.vt[d0 + 2 * e + 1][j] = (uint16_t)(vw[e] >> 16);
    }
  }
  lds_barrier();
  // position scores: bacc[pt][qt] lane holds j' = 16pt + 4(l/16) + e of query 16 kQT w + 16qt + l%16
  f32x4_t bacc[2 * kAttT / 16][kQT];
#pragma unroll
  for (int p = 0; p < 2 * kAttT / 16; ++p)
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) bacc[p][qt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ds = 0; ds < kDk / 32; ++ds)
#pragma unroll
    for (int p = 0; p < 2 * kAttT / 16; ++p) {
      const bf16x8_t pf = lds_frag(sh.u.p[16 * p + (l & 15)], 32 * ds + 8 * (l >> 4));
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
        bacc[p][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf, as_bf16x8(qraw[qt][ds]), bacc[p][qt], 0, 0, 0);
    }
  // key scores: acc[kt][qt] holds keys 16kt + 4(l/16) + e of query 16 kQT w + 16qt + l%16
  f32x4_t acc[8][kQT];
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) acc[kt][qt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ds = 0; ds < kDk / 32; ++ds) {
    const int d0 = 32 * ds + 8 * (l >> 4);
    const uint4 dl = *reinterpret_cast<const uint4*>(delta + h * kDk + d0);
    const uint32_t dw[4] = {dl.x, dl.y, dl.z, dl.w};
    bf16x8_t qf[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const uint32_t qw[4] = {qraw[qt][ds].x, qraw[qt][ds].y, qraw[qt][ds].z, qraw[qt][ds].w};
      uint32_t u[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        u[e] = (uint32_t)f32_to_bf16(lo_f32(qw[e]) + lo_f32(dw[e])) |
               ((uint32_t)f32_to_bf16(hi_f32(qw[e]) + hi_f32(dw[e])) << 16);
      qf[qt] = as_bf16x8(uint4{u[0], u[1], u[2], u[3]});
    }
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      const bf16x8_t kf = lds_frag(sh.k[16 * kt + (l & 15)], d0);
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) acc[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[qt], acc[kt][qt], 0, 0, 0);
    }
  }
  lds_barrier();  // every wave is done with P: its region takes the position scores
#pragma unroll
  for (int p = 0; p < 2 * kAttT / 16; ++p)
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      u32x2_t pk;
      pk.x = (uint32_t)f32_to_bf16(bacc[p][qt][0]) | ((uint32_t)f32_to_bf16(bacc[p][qt][1]) << 16);
      pk.y = (uint32_t)f32_to_bf16(bacc[p][qt][2]) | ((uint32_t)f32_to_bf16(bacc[p][qt][3]) << 16);
      *reinterpret_cast<u32x2_t*>(&sh.u.bd[16 * kQT * w + 16 * qt + (l & 15)][16 * p + 4 * (l >> 4)]) = pk;
    }
  // a wave reads back only the rows it wrote (its LDS operations complete in order)
  // position term, mask, softmax (FP32), per query row
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int i = 16 * kQT * w + 16 * qt + (l & 15);
    const uint16_t* bdr = &sh.u.bd[i][kAttT - 1 - i];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 16 * kt + 4 * (l >> 4) + e;
        float s = acc[kt][qt][e] + bf16_to_f32(bdr[j]);
        if (j >= valid) s = -INFINITY;
        acc[kt][qt][e] = s;
        mx = fmaxf(mx, s);
      }
    mx = max_lanes16(mx);
    float z = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = expf(acc[kt][qt][e] - mx);
        acc[kt][qt][e] = p;
        z += p;
      }
    z = sum_lanes16(z);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[kt][qt][e] = acc[kt][qt][e] / z;
  }
  // o^T = V^T . p^T: for key chunk c, a lane's eight k values are the keys
  // {16(2c) + 4(l/16) + e, 16(2c+1) + 4(l/16) + e} (e < 4) in both operands.
  f32x4_t o[kQT][8];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[qt][dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < kAttT / 32; ++c) {
    bf16x8_t phi[kQT], plo[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        uint16_t hi2[2], lo2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int e = 2 * e2 + u;
          const float p = e < 4 ? acc[2 * c][qt][e] : acc[2 * c + 1][qt][e - 4];
          hi2[u] = f32_to_bf16(p);
          lo2[u] = f32_to_bf16(p - bf16_to_f32(hi2[u]));
        }
        hw[e2] = (uint32_t)hi2[0] | ((uint32_t)hi2[1] << 16);
        lw[e2] = (uint32_t)lo2[0] | ((uint32_t)lo2[1] << 16);
      }
      phi[qt] = as_bf16x8(uint4{hw[0], hw[1], hw[2], hw[3]});
      plo[qt] = as_bf16x8(uint4{lw[0], lw[1], lw[2], lw[3]});
    }
    const int j0 = 32 * c + 4 * (l >> 4);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 16 * dt + (l & 15);
      const uint32_t* vr = reinterpret_cast<const uint32_t*>(&sh.vt[d][0]);
      const bf16x8_t vf = as_bf16x8(uint4{vr[j0 / 2], vr[j0 / 2 + 1], vr[j0 / 2 + 8], vr[j0 / 2 + 9]});
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, phi[qt], o[qt][dt], 0, 0, 0);
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, plo[qt], o[qt][dt], 0, 0, 0);
      }
    }
  }
  // o[qt][dt]: lane l holds dimensions 16dt + 4(l/16) + e of query 16 kQT w + 16qt + l%16
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    uint16_t* orow = out + (size_t)(b * kAttT + 16 * kQT * w + 16 * qt + (l & 15)) * kD + h * kDk + 4 * (l >> 4);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      u32x2_t pk;
      pk.x = (uint32_t)f32_to_bf16(o[qt][dt][0]) | ((uint32_t)f32_to_bf16(o[qt][dt][1]) << 16);
      pk.y = (uint32_t)f32_to_bf16(o[qt][dt][2]) | ((uint32_t)f32_to_bf16(o[qt][dt][3]) << 16);
      *reinterpret_cast<u32x2_t*>(orow + 16 * dt) = pk;
    }
  }
}

// ------------------------------------------------------------------ conv module

// GLU + depthwise conv of 16 channels (blockIdx.x) of sequence b
// (blockIdx.y), as the mirror (012_layer_test.py:92-100):
//   g_t = bf16(c_t[ch] * sigmoid(c_t[1024 + ch])) for t < valid, else 0;
//   y_t = sum_{j<9} g_{t+j-4} * dw[ch][j] (in order, zero outside the
//   frames) + bias[ch]; out = bf16(y * sigmoid(y)).
// A thread handles 8 adjacent channels: 16-byte loads of the GLU halves and
// the taps, 16-byte output stores. (16 channels a block: at one window that
// is 64 blocks, and a thread's GLU loads take about one round trip; with 64
// channels a block the 16 blocks' threads chained four or five.)
constexpr int kConvCh = 16;
constexpr int kConvThreads = 256;
__global__ void __launch_bounds__(kConvThreads) k_pk_conv(const uint16_t* __restrict__ c, const uint16_t* __restrict__ dw,
                                                          const uint16_t* __restrict__ dw_b,
                                                          uint16_t* __restrict__ out, int valid) {
  __shared__ float g[kAttT + 8][kConvCh];
  const int ch0 = blockIdx.x * kConvCh, b = blockIdx.y, t = threadIdx.x;
  for (int e = t; e < (kAttT + 8) * (kConvCh / 8); e += kConvThreads) {
    const int tt = e / (kConvCh / 8) - 4, q = e % (kConvCh / 8);
    float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (tt >= 0 && tt < valid) {
      const uint16_t* row = c + (size_t)(b * kAttT + tt) * 2 * kD + ch0 + 8 * q;
      const uint4 av = *reinterpret_cast<const uint4*>(row);
      const uint4 gv = *reinterpret_cast<const uint4*>(row + kD);
      const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = round_bf16(lo_f32(aw[i]) * sigmoid_f32(lo_f32(gw[i])));
        v[2 * i + 1] = round_bf16(hi_f32(aw[i]) * sigmoid_f32(hi_f32(gw[i])));
      }
    }
    float4* dst = reinterpret_cast<float4*>(&g[tt + 4][8 * q]);
    dst[0] = float4{v[0], v[1], v[2], v[3]};
    dst[1] = float4{v[4], v[5], v[6], v[7]};
  }
  // this thread's channels ch0 + 8q .. + 7: taps [8][9] and bias
  const int q = t % (kConvCh / 8);
  const int ch = ch0 + 8 * q;
  float wt[8][kConvTapsPk], bias[8];
  {
    const uint4* src = reinterpret_cast<const uint4*>(dw + (size_t)ch * kConvTapsPk);  // 72 values, 9 x 16 bytes
#pragma unroll
    for (int u = 0; u < kConvTapsPk; ++u) {
      const uint4 v = src[u];
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i0 = 8 * u + 2 * e;
        wt[i0 / kConvTapsPk][i0 % kConvTapsPk] = lo_f32(vw[e]);
        wt[(i0 + 1) / kConvTapsPk][(i0 + 1) % kConvTapsPk] = hi_f32(vw[e]);
      }
    }
    const uint4 bv = *reinterpret_cast<const uint4*>(dw_b + ch);
    const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bias[2 * e] = lo_f32(bw[e]);
      bias[2 * e + 1] = hi_f32(bw[e]);
    }
  }
  __syncthreads();
  for (int tt = t / (kConvCh / 8); tt < kAttT; tt += kConvThreads / (kConvCh / 8)) {
    float y[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = g[tt][8 * q + k] * wt[k][0];
#pragma unroll
    for (int j = 1; j < kConvTapsPk; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) y[k] = y[k] + g[tt + j][8 * q + k] * wt[k][j];
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float y0 = y[2 * e] + bias[2 * e], y1 = y[2 * e + 1] + bias[2 * e + 1];
      o[e] = (uint32_t)f32_to_bf16(y0 * sigmoid_f32(y0)) | ((uint32_t)f32_to_bf16(y1 * sigmoid_f32(y1)) << 16);
    }
    *reinterpret_cast<uint4*>(out + (size_t)(b * kAttT + tt) * kD + ch) = uint4{o[0], o[1], o[2], o[3]};
  }
}

// ------------------------------------------------------------------ host

// Number of K splits for an m x n x k product: doubled while the grid has
// fewer than kSplitUnits (kSplitUnitsFew) blocks, each split keeping >=
// kMinChunk of K.
inline bool use_tall(int m, int n, int splits);
int pick_splits(int m, int n, int k) {
  if (use_tall(m, n, 1)) return 1;
  const int tiles = (n / kBN) * ((m + kBM - 1) / kBM);
  int splits = 1;
  const int units = m <= 256 ? kSplitUnitsFew : kSplitUnits;
  while (tiles * splits < units && k % (2 * splits * kBK) == 0 && k / (2 * splits) >= kMinChunk) splits *= 2;
  return splits;
}

// Tall (256-row) tiles for an unsplit product with at least kTallTiles of
// them: fewer bytes per FLOP, and still about one block per CU.
constexpr int kTallTiles = 192;
inline bool use_tall(int m, int n, int splits) {
  return splits == 1 && (n / kBN) * ((m + 255) / 256) >= kTallTiles;
}

template <int EPI, int kWM>
void launch_gemm(const PkGemm& g, dim3 grid, bool split, hipStream_t s) {
  if (split)
    k_pk_gemm_dma<EPI, true, kWM><<<grid, 128 * kWM, 0, s>>>(g);
  else
    k_pk_gemm_dma<EPI, false, kWM><<<grid, 128 * kWM, 0, s>>>(g);
}

template <int EPI>
void launch_splitk(dim3 grid, const float* part, int splits, int m, int n, const uint16_t* bias, uint16_t* c, int ldc,
                   hipStream_t s) {
  switch (partial_group(splits)) {
    case 1: k_pk_splitk<EPI, 1><<<grid, 256, 0, s>>>(part, splits, m, n, bias, c, ldc); break;
    case 2: k_pk_splitk<EPI, 2><<<grid, 256, 0, s>>>(part, splits, m, n, bias, c, ldc); break;
    case 4: k_pk_splitk<EPI, 4><<<grid, 256, 0, s>>>(part, splits, m, n, bias, c, ldc); break;
    default: k_pk_splitk<EPI, 8><<<grid, 256, 0, s>>>(part, splits, m, n, bias, c, ldc); break;
  }
}

// C = epi(A . Bt^T + bias) for `batch` products at element strides sa / sb /
// sc, or (splits > 1, batch 1) as `splits` K ranges through `part`
// (splits x m x n floats) and k_pk_splitk.
int gemm(const uint16_t* a, int lda, long long sa, const uint16_t* bt, int ldb, long long sb, const uint16_t* bias,
         uint16_t* c, int ldc, long long sc, int m, int n, int k, int batch, int epi, int splits, float* part,
         hipStream_t s) {
  const bool split = splits > 1;
  const bool tall = batch == 1 && use_tall(m, n, splits);
  const int tile_m = tall ? 256 : kBM;
  const dim3 grid(n / kBN, (m + tile_m - 1) / tile_m, split ? splits : batch);
  PkGemm g{a, bt, bias, c, part, sa, sb, sc, lda, ldb, ldc, m, n, k / splits};
  switch (epi * 2 + (tall ? 1 : 0)) {
    case 2 * EPI_NONE: launch_gemm<EPI_NONE, 2>(g, grid, split, s); break;
    case 2 * EPI_NONE + 1: launch_gemm<EPI_NONE, 4>(g, grid, split, s); break;
    case 2 * EPI_BIAS: launch_gemm<EPI_BIAS, 2>(g, grid, split, s); break;
    case 2 * EPI_BIAS + 1: launch_gemm<EPI_BIAS, 4>(g, grid, split, s); break;
    case 2 * EPI_SWISH: launch_gemm<EPI_SWISH, 2>(g, grid, split, s); break;
    default: launch_gemm<EPI_SWISH, 4>(g, grid, split, s); break;
  }
  if (split) {
    const dim3 blocks((unsigned)m, (unsigned)((n / 4 + 255) / 256));
    switch (epi) {
      case EPI_NONE: launch_splitk<EPI_NONE>(blocks, part, splits, m, n, bias, c, ldc, s); break;
      case EPI_BIAS: launch_splitk<EPI_BIAS>(blocks, part, splits, m, n, bias, c, ldc, s); break;
      default: launch_splitk<EPI_SWISH>(blocks, part, splits, m, n, bias, c, ldc, s); break;
    }
  }
  return check_launch("parakeet gemm");
}

// One encoder product: split as pick_splits chooses, through the partial buffer.
int enc_gemm(const uint16_t* a, int lda, const uint16_t* bt, const uint16_t* bias, uint16_t* c, int ldc, int m, int n,
             int k, int epi, float* part, hipStream_t s) {
  return gemm(a, lda, 0, bt, k, 0, bias, c, ldc, 0, m, n, k, 1, epi, pick_splits(m, n, k), part, s);
}

struct ReduceLnArgs {
  const float* part;
  int splits;
  uint16_t* x;
  float scale;
  const uint16_t *g1, *b1, *g2, *b2;
  int normed_x;
  uint16_t* a;
  int rows;
};
template <int R, int G>
void launch_reduce_ln(const ReduceLnArgs& r, hipStream_t s) {
  k_pk_reduce_ln<R, G><<<(r.rows + R - 1) / R, R * kWave, 0, s>>>(r.part, r.splits, r.x, r.scale, r.g1, r.b1, r.g2,
                                                                   r.b2, r.normed_x, r.a, r.rows);
}

// A d-wide encoder product (m x 1024) whose end is a residual + LayerNorm:
// its FP32 partial products (one per K split, at least one) go to `part`
// and k_pk_reduce_ln finishes the row.
int enc_gemm_ln(const uint16_t* a, int lda, const uint16_t* bt, int m, int k, float* part, uint16_t* x, float scale,
                const uint16_t* ln1, const uint16_t* ln2, int normed_x, uint16_t* out_a, hipStream_t s) {
  const int splits = pick_splits(m, kD, k);
  const dim3 grid(kD / kBN, (m + kBM - 1) / kBM, splits);
  PkGemm g{a, bt, nullptr, nullptr, part, 0, 0, 0, lda, k, kD, m, kD, k / splits};
  k_pk_gemm_dma<EPI_NONE, true, 2><<<grid, 256, 0, s>>>(g);
  const ReduceLnArgs r{part, splits, x, scale, ln1, ln1 + kD, ln2, ln2 ? ln2 + kD : nullptr, normed_x, out_a, m};
  // A wave per block for few rows (latency-bound: all of a row's partials in
  // flight at once); blocks of kLnRows waves, at most two partials per round
  // trip, for many (a 16-window pass has two splits, and loading both at
  // once measured 1.1% faster on the pass than one at a time)
  if (m <= kSplitUnits) {
    switch (partial_group(splits)) {
      case 1: launch_reduce_ln<1, 1>(r, s); break;
      case 2: launch_reduce_ln<1, 2>(r, s); break;
      case 4: launch_reduce_ln<1, 4>(r, s); break;
      default: launch_reduce_ln<1, 8>(r, s); break;
    }
  } else if (splits >= 2) {
    launch_reduce_ln<kLnRows, 2>(r, s);
  } else {
    launch_reduce_ln<kLnRows, 1>(r, s);
  }
  return check_launch("parakeet gemm + layer norm");
}

// FP32 partial buffer of the encoder: split products stay under
// 2 * kSplitUnits tiles; an unsplit d-wide product needs rows x 1024 floats.
inline size_t pk_part_bytes(int rows) { return std::max(kPartBytes, (size_t)rows * kD * sizeof(float)); }

// Workspace of the encoder for `rows` = batch * 128 frames (bytes).
inline size_t pk_ws_bytes(int rows) {
  return pk_part_bytes(rows) + (size_t)rows * 2 * (kD /*a*/ + kPkFfn /*big*/ + kD /*o*/);
}

}  // namespace
}  // namespace lfm25

using namespace lfm25;

extern "C" {

int lfm25_pk_gemm(const uint16_t* a, int32_t lda, const uint16_t* bt, int32_t ldb, const uint16_t* bias, uint16_t* c,
                  int32_t ldc, int32_t m, int32_t n, int32_t k, int32_t epi, int32_t splits, void* workspace,
                  lfm25_stream_t stream) {
  LFM25_REQUIRE(a && bt && c, "pk gemm: null pointer");
  LFM25_REQUIRE(m >= 1 && n >= kBN && n % kBN == 0 && k >= kBK && k % kBK == 0,
                "pk gemm: need m >= 1, n a multiple of %d, k a multiple of %d (got %d, %d, %d)", kBN, kBK, m, n, k);
  LFM25_REQUIRE(lda >= k && ldb >= k && ldc >= n && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0,
                "pk gemm: leading dimensions too small or misaligned");
  LFM25_REQUIRE(aligned16(a) && aligned16(bt) && (reinterpret_cast<uintptr_t>(c) & 7) == 0,
                "pk gemm: a, bt must be 16-byte and c 8-byte aligned");
  LFM25_REQUIRE(epi >= EPI_NONE && epi <= EPI_SWISH, "pk gemm: epilogue must be 0 (none), 1 (bias) or 2 (swish)");
  LFM25_REQUIRE(epi != EPI_BIAS || bias != nullptr, "pk gemm: bias epilogue needs a bias");
  LFM25_REQUIRE(splits >= 1 && k % (splits * kBK) == 0,
                "pk gemm: splits must divide k into multiples of %d (got %d splits of %d)", kBK, splits, k);
  LFM25_REQUIRE(splits == 1 || (workspace && aligned16(workspace)),
                "pk gemm: a split product needs a 16-byte aligned workspace of splits * m * n floats");
  return gemm(a, lda, 0, bt, ldb, 0, bias, c, ldc, 0, m, n, k, 1, epi, splits, static_cast<float*>(workspace),
              reinterpret_cast<hipStream_t>(stream));
}

int lfm25_pk_layer_norm(uint16_t* x, const uint16_t* y, float scale, const uint16_t* gamma1, const uint16_t* beta1,
                        const uint16_t* gamma2, const uint16_t* beta2, int32_t normed_x, uint16_t* a, int32_t rows,
                        lfm25_stream_t stream) {
  LFM25_REQUIRE(x && gamma1 && beta1 && rows >= 1, "pk layer norm: null pointer or no rows");
  LFM25_REQUIRE(normed_x || a != nullptr, "pk layer norm: the carry mode writes a");
  LFM25_REQUIRE(!gamma2 || (beta2 && a && normed_x), "pk layer norm: a second norm needs normed_x, beta2 and a");
  LFM25_REQUIRE(aligned16(x) && (!y || aligned16(y)) && (!a || aligned16(a)) && aligned16(gamma1) &&
                    aligned16(beta1) && (!gamma2 || (aligned16(gamma2) && aligned16(beta2))),
                "pk layer norm: rows and norm parameters must be 16-byte aligned");
  k_pk_ln<<<(rows + kLnRows - 1) / kLnRows, kLnRows * kWave, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      x, y, scale, gamma1, beta1, gamma2, beta2, normed_x, a, rows);
  return check_launch("parakeet layer norm");
}

int lfm25_pk_attention(const uint16_t* qkv, const uint16_t* pos, const uint16_t* delta, uint16_t* out, int32_t batch,
                       int32_t frames, int32_t valid, lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv && pos && delta && out, "pk attention: null pointer");
  LFM25_REQUIRE(frames == kAttT, "pk attention: frames must be %d (one padded block), got %d", kAttT, frames);
  LFM25_REQUIRE(batch >= 1 && valid >= 1 && valid <= frames, "pk attention: need batch >= 1 and 1 <= valid <= frames");
  LFM25_REQUIRE(aligned16(qkv) && aligned16(pos) && aligned16(delta) && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
                "pk attention: qkv, pos, delta must be 16-byte and out 8-byte aligned");
  k_pk_attention<<<dim3(kPkHeads, batch, kAttSplit), kAttBlockThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(qkv, pos, delta,
                                                                                                  out, valid);
  return check_launch("parakeet attention");
}

int lfm25_pk_conv(const uint16_t* c, const uint16_t* dw, const uint16_t* dw_b, uint16_t* out, int32_t batch,
                  int32_t frames, int32_t valid, lfm25_stream_t stream) {
  LFM25_REQUIRE(c && dw && dw_b && out, "pk conv: null pointer");
  LFM25_REQUIRE(frames == kAttT, "pk conv: frames must be %d, got %d", kAttT, frames);
  LFM25_REQUIRE(batch >= 1 && valid >= 1 && valid <= frames, "pk conv: need batch >= 1 and 1 <= valid <= frames");
  LFM25_REQUIRE(aligned16(c) && aligned16(dw) && aligned16(dw_b) && aligned16(out), "pk conv: 16-byte alignment");
  k_pk_conv<<<dim3(kD / kConvCh, batch), kConvThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(c, dw, dw_b, out,
                                                                                                   valid);
  return check_launch("parakeet conv");
}

size_t lfm25_pk_workspace_bytes(int32_t batch, int32_t frames) {
  if (batch < 1 || frames != kAttT) return 0;
  return pk_ws_bytes(batch * frames);
}

int lfm25_pk_encoder(const lfm25_pk_layer* layers, int32_t n_layers, uint16_t* x, int32_t batch, int32_t frames,
                     int32_t valid, void* workspace, lfm25_stream_t stream) {
  LFM25_REQUIRE(layers && x && workspace && n_layers >= 1, "pk encoder: null argument");
  LFM25_REQUIRE(frames == kAttT && batch >= 1 && valid >= 1 && valid <= frames,
                "pk encoder: frames must be %d and 1 <= valid <= frames", kAttT);
  LFM25_REQUIRE(aligned16(x) && aligned16(workspace), "pk encoder: x and workspace must be 16-byte aligned");
  for (int i = 0; i < n_layers; ++i) {
    const lfm25_pk_layer& L = layers[i];
    LFM25_REQUIRE(L.ln && L.ff1_w1 && L.ff1_w2 && L.qkv && L.qkv_bias && L.att_delta && L.pos && L.out && L.pw1 &&
                      L.dw && L.dw_b && L.pw2 && L.ff2_w1 && L.ff2_w2,
                  "pk encoder: layer %d has a null tensor", i);
    LFM25_REQUIRE(aligned16(L.ln) && aligned16(L.ff1_w1) && aligned16(L.ff1_w2) && aligned16(L.qkv) &&
                      aligned16(L.att_delta) && aligned16(L.pos) && aligned16(L.out) && aligned16(L.pw1) &&
                      aligned16(L.dw) && aligned16(L.dw_b) && aligned16(L.pw2) && aligned16(L.ff2_w1) &&
                      aligned16(L.ff2_w2),
                  "pk encoder: layer %d tensors must be 16-byte aligned", i);
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int rows = batch * frames;
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws);
  uint16_t* a = reinterpret_cast<uint16_t*>(ws + pk_part_bytes(rows));
  uint16_t* big = a + (size_t)rows * kD;
  uint16_t* o = big + (size_t)rows * kPkFfn;
  int rc = LFM25_OK;
  auto ln_of = [](const lfm25_pk_layer& L, int which) { return L.ln + (size_t)which * 2 * kD; };
#define PK_TRY(call)               \
  do {                             \
    rc = (call);                   \
    if (rc != LFM25_OK) return rc; \
  } while (0)
  // a = LN_ff1(x) of the first layer; later layers get it from the previous
  // layer's last norm (LN_out, then the next LN_ff1, on the same row pass)
  k_pk_ln<<<(rows + kLnRows - 1) / kLnRows, kLnRows * kWave, 0, s>>>(x, nullptr, 0.0f, ln_of(layers[0], 0),
                                                                      ln_of(layers[0], 0) + kD, nullptr, nullptr, 0, a,
                                                                      rows);
  for (int i = 0; i < n_layers; ++i) {
    const lfm25_pk_layer& L = layers[i];
    const uint16_t* next_ln = i + 1 < n_layers ? ln_of(layers[i + 1], 0) : nullptr;
    // Macaron FFN 1: x = bf16(x + FFN(a) / 2), a = LN_att(x)
    PK_TRY(enc_gemm(a, kD, L.ff1_w1, nullptr, big, kPkFfn, rows, kPkFfn, kD, EPI_SWISH, part, s));
    PK_TRY(enc_gemm_ln(big, kPkFfn, L.ff1_w2, rows, kPkFfn, part, x, 0.5f, ln_of(L, 1), nullptr, 0, a, s));
    // relative-position self-attention: x = bf16(x + out(att)), a = LN_conv(x)
    PK_TRY(enc_gemm(a, kD, L.qkv, L.qkv_bias, big, 3 * kD, rows, 3 * kD, kD, EPI_BIAS, part, s));
    k_pk_attention<<<dim3(kPkHeads, batch, kAttSplit), kAttBlockThreads, 0, s>>>(big, L.pos, L.att_delta, o, valid);
    PK_TRY(enc_gemm_ln(o, kD, L.out, rows, kD, part, x, 1.0f, ln_of(L, 2), nullptr, 0, a, s));
    // conv module: x = bf16(x + pw2(conv(pw1(a)))), a = LN_ff2(x)
    PK_TRY(enc_gemm(a, kD, L.pw1, nullptr, big, 2 * kD, rows, 2 * kD, kD, EPI_NONE, part, s));
    k_pk_conv<<<dim3(kD / kConvCh, batch), kConvThreads, 0, s>>>(big, L.dw, L.dw_b, o, valid);
    PK_TRY(enc_gemm_ln(o, kD, L.pw2, rows, kD, part, x, 1.0f, ln_of(L, 3), nullptr, 0, a, s));
    // Macaron FFN 2 and the block's output norm: x = LN_out(bf16(x + FFN(a) / 2)),
    // a = LN_ff1 of the next layer (x)
    PK_TRY(enc_gemm(a, kD, L.ff2_w1, nullptr, big, kPkFfn, rows, kPkFfn, kD, EPI_SWISH, part, s));
    PK_TRY(enc_gemm_ln(big, kPkFfn, L.ff2_w2, rows, kPkFfn, part, x, 0.5f, ln_of(L, 4), next_ln, 1, a, s));
  }
#undef PK_TRY
  return check_launch("parakeet encoder");
}

}  // extern "C"
