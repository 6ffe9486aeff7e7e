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

// C[m][n] = bf16(epi(sum_k A[m][k] Bt[n][k] + bias[n])) for a 128 x 128 tile
// per block (blockIdx.x: n, blockIdx.y: m, blockIdx.z: batch of independent
// products with element strides). 4 waves in 2 x 2, each 64 x 64 as 4 x 4
// MFMA tiles (v_mfma_f32_16x16x32_bf16 with the weight tile as the first
// operand, so a lane's four results are four consecutive n of one row m and
// leave as one 8-byte store). K steps of 64 go through double-buffered LDS:
// the next step's global loads are in flight while the current one
// multiplies. Rows m >= M read zeros and are not stored; N % 128 == 0,
// K % 64 == 0.
constexpr int kGemmThreads = 256;
constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row: 144 bytes, conflict-free 16-byte reads
enum PkEpi { EPI_NONE = 0, EPI_BIAS = 1, EPI_SWISH = 2 };

struct PkGemmLds {
  uint16_t a[2][kBM][kLdsRow];
  uint16_t b[2][kBN][kLdsRow];
};

__device__ __forceinline__ uint4 load16_or_zero(const uint16_t* p, bool ok) {
  return ok ? *reinterpret_cast<const uint4*>(p) : uint4{0, 0, 0, 0};
}

template <int EPI>
__global__ void __launch_bounds__(kGemmThreads)
    k_pk_gemm(const uint16_t* __restrict__ A, int lda, long long sa, const uint16_t* __restrict__ Bt, int ldb,
              long long sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int ldc, long long sc,
              int M, int K) {
  __shared__ PkGemmLds sh;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM;
  A += sa * blockIdx.z;
  Bt += sb * blockIdx.z;
  C += sc * blockIdx.z;
  const int t = threadIdx.x, w = wave_id(), l = lane_id();
  const int wm = w & 1, wn = w >> 1;
  // global -> register staging of one K step: 4 chunks of 16 bytes per operand
  uint4 ra[4], rb[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + kGemmThreads * i;
      const int row = c >> 3, col = (c & 7) * 8;
      ra[i] = load16_or_zero(A + (size_t)(m0 + row) * lda + k0 + col, m0 + row < M);
      rb[i] = *reinterpret_cast<const uint4*>(Bt + (size_t)(n0 + row) * ldb + k0 + col);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + kGemmThreads * i;
      const int row = c >> 3, col = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&sh.a[buf][row][col]) = ra[i];
      *reinterpret_cast<uint4*>(&sh.b[buf][row][col]) = rb[i];
    }
  };
  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int steps = K / kBK;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) fetch((s + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      const int kc = 32 * ks + 8 * (l >> 4);
      bf16x8_t xa[4], wb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xa[i] = *reinterpret_cast<const bf16x8_t*>(&sh.a[buf][64 * wm + 16 * i + (l & 15)][kc]);
        wb[i] = *reinterpret_cast<const bf16x8_t*>(&sh.b[buf][64 * wn + 16 * i + (l & 15)][kc]);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb[nt], xa[mt], acc[nt][mt], 0, 0, 0);
    }
    if (s + 1 < steps) stash(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = n0 + 64 * wn + 16 * nt + 4 * (l >> 4);
    float bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (EPI == EPI_BIAS) {
#pragma unroll
      for (int e = 0; e < 4; ++e) bs[e] = bf16_to_f32(bias[n + e]);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int m = m0 + 64 * wm + 16 * mt + (l & 15);
      if (m >= M) continue;
      uint16_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[nt][mt][e];
        if (EPI == EPI_BIAS) v = v + bs[e];
        if (EPI == EPI_SWISH) v = v * sigmoid_f32(v);
        o[e] = f32_to_bf16(v);
      }
      u32x2_t pk;
      pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
      pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
      *reinterpret_cast<u32x2_t*>(C + (size_t)m * ldc + n) = pk;
    }
  }
}

// ------------------------------------------------------------------ LayerNorm

// bf16((v - mean) / sqrt(var + eps) * g + b) of one 1024-row held 16 per lane
// (lane l: elements 16l .. 16l + 15); mean and variance in FP32 (wave sums).
__device__ __forceinline__ void ln_lane(const float* v, const uint16_t* g, const uint16_t* b, float* out) {
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
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 16; ++i)
    out[i] = round_bf16((v[i] - mu) / den * bf16_to_f32(g[16 * l + i]) + bf16_to_f32(b[16 * l + i]));
}

__device__ __forceinline__ void load_row16(const uint16_t* p, float* v) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  const uint4 a = q[0], b = q[1];
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = lo_f32(w[i]);
    v[2 * i + 1] = hi_f32(w[i]);
  }
}
__device__ __forceinline__ void store_row16(uint16_t* p, const float* v) {
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
  uint4* q = reinterpret_cast<uint4*>(p);
  q[0] = uint4{w[0], w[1], w[2], w[3]};
  q[1] = uint4{w[4], w[5], w[6], w[7]};
}

// One wave per row. x' = y ? bf16(x + s * y) : x. Mode "carry" (ln2 == null,
// normed_x == 0): x <- x', a <- LN1(x'). Mode "normed" (normed_x == 1):
// x <- LN1(x') and, when ln2 is given, a <- LN2(x) (ln_frame's DOUBLE/FINAL,
// pk_core.cc:99-116).
__global__ void __launch_bounds__(kWave) k_pk_ln(uint16_t* __restrict__ x, const uint16_t* __restrict__ y, float s,
                                                 const uint16_t* __restrict__ g1, const uint16_t* __restrict__ b1,
                                                 const uint16_t* __restrict__ g2, const uint16_t* __restrict__ b2,
                                                 int normed_x, uint16_t* __restrict__ a) {
  const int m = blockIdx.x, l = lane_id();
  uint16_t* xr = x + (size_t)m * kD + 16 * l;
  float v[16], o[16];
  load_row16(xr, v);
  if (y != nullptr) {
    float yv[16];
    load_row16(y + (size_t)m * kD + 16 * l, yv);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = round_bf16(v[i] + s * yv[i]);
  }
  ln_lane(v, g1, b1, o);
  if (!normed_x) {
    if (y != nullptr) store_row16(xr, v);
    store_row16(a + (size_t)m * kD + 16 * l, o);
    return;
  }
  store_row16(xr, o);
  if (g2 != nullptr) {
    float o2[16];
    ln_lane(o, g2, b2, o2);
    store_row16(a + (size_t)m * kD + 16 * l, o2);
  }
}

// ------------------------------------------------------------------ attention

// Relative-position attention of sequence b (blockIdx.y), head h
// (blockIdx.x) over T = 128 frames, `valid` of them real (keys j >= valid
// masked), as the mirror computes it (012_layer_test.py:74-86):
//   qu = bf16(q + delta_h); s_ij = qu_i . k_j + bd[h][i][T - 1 - i + j];
//   p = softmax_j(s) in FP32; o_i = bf16(sum_j p_ij v_j).
// q (scaled, bias_v folded in), k, v come from the q|k|v rows [T x 3072];
// bd[h] is the position-score GEMM output [rows x 2T]. Scores use the
// matrix cores on BF16 operands (exact products, FP32 sums); the
// probabilities stay FP32 through the value product by splitting each into
// a BF16 high part and a BF16 remainder (two MFMA chains).
constexpr int kAttT = 128;
constexpr int kAttThreads = 256;
struct PkAttLds {
  uint16_t vt[kDk][kAttT + 8];  // V transposed: vt[d][j]
};

__global__ void __launch_bounds__(kAttThreads)
    k_pk_attention(const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ bd, const uint16_t* __restrict__ delta,
                   uint16_t* __restrict__ out, int valid, int rows) {
  __shared__ PkAttLds sh;
  const int h = blockIdx.x, b = blockIdx.y;
  const int t = threadIdx.x, w = wave_id(), l = lane_id();
  const uint16_t* base = qkv + (size_t)b * kAttT * 3 * kD;
  // V^T into LDS
  for (int c = t; c < kAttT * kDk / 8; c += kAttThreads) {
    const int j = c / (kDk / 8), d0 = (c % (kDk / 8)) * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(base + (size_t)j * 3 * kD + 2 * kD + h * kDk + d0);
    const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sh.vt[d0 + 2 * e][j] = (uint16_t)(vw[e] & 0xffffu);
      sh.vt[d0 + 2 * e + 1][j] = (uint16_t)(vw[e] >> 16);
    }
  }
  // scores: acc[kt][qt] holds keys 16kt + 4(l/16) + e of query 32w + 16qt + l%16
  f32x4_t acc[8][2];
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) acc[kt][qt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ds = 0; ds < kDk / 32; ++ds) {
    const int d0 = 32 * ds + 8 * (l >> 4);
    bf16x8_t qf[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int i = 32 * w + 16 * qt + (l & 15);
      const uint4 q = *reinterpret_cast<const uint4*>(base + (size_t)i * 3 * kD + h * kDk + d0);
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
      uint16_t u[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        u[2 * e] = f32_to_bf16(lo_f32(qw[e]) + bf16_to_f32(delta[h * kDk + d0 + 2 * e]));
        u[2 * e + 1] = f32_to_bf16(hi_f32(qw[e]) + bf16_to_f32(delta[h * kDk + d0 + 2 * e + 1]));
      }
      uint4 pk{(uint32_t)u[0] | ((uint32_t)u[1] << 16), (uint32_t)u[2] | ((uint32_t)u[3] << 16),
               (uint32_t)u[4] | ((uint32_t)u[5] << 16), (uint32_t)u[6] | ((uint32_t)u[7] << 16)};
      qf[qt] = __builtin_bit_cast(bf16x8_t, pk);
    }
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      const int j = 16 * kt + (l & 15);
      const bf16x8_t kf =
          __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(base + (size_t)j * 3 * kD + kD + h * kDk + d0));
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) acc[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[qt], acc[kt][qt], 0, 0, 0);
    }
  }
  // position term, mask, softmax (FP32), per query row
  const uint16_t* bdh = bd + (size_t)h * rows * (2 * kAttT);
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int i = 32 * w + 16 * qt + (l & 15);
    const uint16_t* bdr = bdh + (size_t)(b * kAttT + i) * (2 * kAttT);
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 16 * kt + 4 * (l >> 4) + e;
        float s = acc[kt][qt][e] + bf16_to_f32(bdr[kAttT - 1 - i + j]);
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
  __syncthreads();  // V^T complete
  // o = p . v: the probabilities of keys {16(2c) + 4(l/16) + e, 16(2c+1) + 4(l/16) + e}
  // (e < 4) are the eight k values of a lane for key chunk c, in both operands.
  f32x4_t o[2][8];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[qt][dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < kAttT / 32; ++c) {
    bf16x8_t phi[2], plo[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      uint16_t hi[8], lo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = e < 4 ? acc[2 * c][qt][e] : acc[2 * c + 1][qt][e - 4];
        hi[e] = f32_to_bf16(p);
        lo[e] = f32_to_bf16(p - bf16_to_f32(hi[e]));
      }
      uint4 ph{(uint32_t)hi[0] | ((uint32_t)hi[1] << 16), (uint32_t)hi[2] | ((uint32_t)hi[3] << 16),
               (uint32_t)hi[4] | ((uint32_t)hi[5] << 16), (uint32_t)hi[6] | ((uint32_t)hi[7] << 16)};
      uint4 pl{(uint32_t)lo[0] | ((uint32_t)lo[1] << 16), (uint32_t)lo[2] | ((uint32_t)lo[3] << 16),
               (uint32_t)lo[4] | ((uint32_t)lo[5] << 16), (uint32_t)lo[6] | ((uint32_t)lo[7] << 16)};
      phi[qt] = __builtin_bit_cast(bf16x8_t, ph);
      plo[qt] = __builtin_bit_cast(bf16x8_t, pl);
    }
    const int j0 = 32 * c + 4 * (l >> 4);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 16 * dt + (l & 15);
      const uint2 va = *reinterpret_cast<const uint2*>(&sh.vt[d][j0]);
      const uint2 vb = *reinterpret_cast<const uint2*>(&sh.vt[d][j0 + 16]);
      const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, uint4{va.x, va.y, vb.x, vb.y});
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(phi[qt], vf, o[qt][dt], 0, 0, 0);
        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(plo[qt], vf, o[qt][dt], 0, 0, 0);
      }
    }
  }
  // o[qt][dt]: lane l holds queries 32w + 16qt + 4(l/16) + e, dimension 16dt + l%16
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 32 * w + 16 * qt + 4 * (l >> 4) + e;
        out[(size_t)(b * kAttT + i) * kD + h * kDk + 16 * dt + (l & 15)] = f32_to_bf16(o[qt][dt][e]);
      }
}

// ------------------------------------------------------------------ conv module

// GLU + depthwise conv of 64 channels (blockIdx.x) of sequence b
// (blockIdx.y), as the mirror (012_layer_test.py:92-100):
//   g_t = bf16(c_t[ch] * sigmoid(c_t[1024 + ch])) for t < valid, else 0;
//   y_t = sum_{j<9} g_{t+j-4} * dw[ch][j] (in order, zero outside the
//   frames) + bias[ch]; out = bf16(y * sigmoid(y)).
constexpr int kConvCh = 64;
__global__ void __launch_bounds__(256) k_pk_conv(const uint16_t* __restrict__ c, const uint16_t* __restrict__ dw,
                                                 const uint16_t* __restrict__ dw_b, uint16_t* __restrict__ out,
                                                 int valid) {
  __shared__ float g[kAttT + 8][kConvCh];
  const int ch0 = blockIdx.x * kConvCh, b = blockIdx.y;
  for (int e = threadIdx.x; e < (kAttT + 8) * kConvCh; e += blockDim.x) {
    const int tt = e / kConvCh - 4, k = e % kConvCh;
    float v = 0.0f;
    if (tt >= 0 && tt < kAttT && tt < valid) {
      const uint16_t* row = c + (size_t)(b * kAttT + tt) * 2 * kD;
      v = round_bf16(bf16_to_f32(row[ch0 + k]) * sigmoid_f32(bf16_to_f32(row[kD + ch0 + k])));
    }
    g[tt + 4][k] = v;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kAttT * kConvCh; e += blockDim.x) {
    const int tt = e / kConvCh, k = e % kConvCh, ch = ch0 + k;
    float y = g[tt][k] * bf16_to_f32(dw[ch * kConvTapsPk]);
#pragma unroll
    for (int j = 1; j < kConvTapsPk; ++j) y = y + g[tt + j][k] * bf16_to_f32(dw[ch * kConvTapsPk + j]);
    y = y + bf16_to_f32(dw_b[ch]);
    out[(size_t)(b * kAttT + tt) * kD + ch] = f32_to_bf16(y * sigmoid_f32(y));
  }
}

// ------------------------------------------------------------------ host

int gemm(const uint16_t* a, int lda, long long sa, const uint16_t* bt, int ldb, long long sb, const uint16_t* bias,
         uint16_t* c, int ldc, long long sc, int m, int n, int k, int batch, int epi, hipStream_t s) {
  const dim3 grid(n / kBN, (m + kBM - 1) / kBM, batch);
  switch (epi) {
    case EPI_NONE: k_pk_gemm<EPI_NONE><<<grid, kGemmThreads, 0, s>>>(a, lda, sa, bt, ldb, sb, bias, c, ldc, sc, m, k); break;
    case EPI_BIAS: k_pk_gemm<EPI_BIAS><<<grid, kGemmThreads, 0, s>>>(a, lda, sa, bt, ldb, sb, bias, c, ldc, sc, m, k); break;
    default: k_pk_gemm<EPI_SWISH><<<grid, kGemmThreads, 0, s>>>(a, lda, sa, bt, ldb, sb, bias, c, ldc, sc, m, k); break;
  }
  return check_launch("parakeet gemm");
}

// Workspace of the encoder for `rows` = batch * 128 frames (bytes).
inline size_t pk_ws_bytes(int rows) {
  return (size_t)rows * 2 * (kD /*a*/ + kPkFfn /*big*/ + kD /*y*/ + kD /*o*/ + kPkHeads * 2 * kAttT /*bd*/);
}

}  // namespace
}  // namespace lfm25

using namespace lfm25;

extern "C" {

int lfm25_pk_gemm(const uint16_t* a, int32_t lda, const uint16_t* bt, int32_t ldb, const uint16_t* bias, uint16_t* c,
                  int32_t ldc, int32_t m, int32_t n, int32_t k, int32_t epi, lfm25_stream_t stream) {
  LFM25_REQUIRE(a && bt && c, "pk gemm: null pointer");
  LFM25_REQUIRE(m >= 1 && n >= kBN && n % kBN == 0 && k >= kBK && k % kBK == 0,
                "pk gemm: need m >= 1, n a multiple of %d, k a multiple of %d (got %d, %d, %d)", kBN, kBK, m, n, k);
  LFM25_REQUIRE(lda >= k && ldb >= k && ldc >= n && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0,
                "pk gemm: leading dimensions too small or misaligned");
  LFM25_REQUIRE(aligned16(a) && aligned16(bt) && (reinterpret_cast<uintptr_t>(c) & 7) == 0,
                "pk gemm: a, bt must be 16-byte and c 8-byte aligned");
  LFM25_REQUIRE(epi >= EPI_NONE && epi <= EPI_SWISH, "pk gemm: epilogue must be 0 (none), 1 (bias) or 2 (swish)");
  LFM25_REQUIRE(epi != EPI_BIAS || bias != nullptr, "pk gemm: bias epilogue needs a bias");
  return gemm(a, lda, 0, bt, ldb, 0, bias, c, ldc, 0, m, n, k, 1, epi, reinterpret_cast<hipStream_t>(stream));
}

int lfm25_pk_layer_norm(uint16_t* x, const uint16_t* y, float scale, const uint16_t* gamma1, const uint16_t* beta1,
                        const uint16_t* gamma2, const uint16_t* beta2, int32_t normed_x, uint16_t* a, int32_t rows,
                        lfm25_stream_t stream) {
  LFM25_REQUIRE(x && gamma1 && beta1 && rows >= 1, "pk layer norm: null pointer or no rows");
  LFM25_REQUIRE(normed_x || a != nullptr, "pk layer norm: the carry mode writes a");
  LFM25_REQUIRE(!gamma2 || (beta2 && a && normed_x), "pk layer norm: a second norm needs normed_x, beta2 and a");
  LFM25_REQUIRE(aligned16(x) && (!y || aligned16(y)) && (!a || aligned16(a)), "pk layer norm: rows must be 16-byte aligned");
  k_pk_ln<<<rows, kWave, 0, reinterpret_cast<hipStream_t>(stream)>>>(x, y, scale, gamma1, beta1, gamma2, beta2,
                                                                   normed_x, a);
  return check_launch("parakeet layer norm");
}

int lfm25_pk_attention(const uint16_t* qkv, const uint16_t* bd, const uint16_t* delta, uint16_t* out, int32_t batch,
                       int32_t frames, int32_t valid, lfm25_stream_t stream) {
  LFM25_REQUIRE(qkv && bd && delta && out, "pk attention: null pointer");
  LFM25_REQUIRE(frames == kAttT, "pk attention: frames must be %d (one padded block), got %d", kAttT, frames);
  LFM25_REQUIRE(batch >= 1 && valid >= 1 && valid <= frames, "pk attention: need batch >= 1 and 1 <= valid <= frames");
  LFM25_REQUIRE(aligned16(qkv), "pk attention: qkv must be 16-byte aligned");
  k_pk_attention<<<dim3(kPkHeads, batch), kAttThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      qkv, bd, delta, out, valid, batch * frames);
  return check_launch("parakeet attention");
}

int lfm25_pk_conv(const uint16_t* c, const uint16_t* dw, const uint16_t* dw_b, uint16_t* out, int32_t batch,
                  int32_t frames, int32_t valid, lfm25_stream_t stream) {
  LFM25_REQUIRE(c && dw && dw_b && out, "pk conv: null pointer");
  LFM25_REQUIRE(frames == kAttT, "pk conv: frames must be %d, got %d", kAttT, frames);
  LFM25_REQUIRE(batch >= 1 && valid >= 1 && valid <= frames, "pk conv: need batch >= 1 and 1 <= valid <= frames");
  k_pk_conv<<<dim3(kD / kConvCh, batch), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(c, dw, dw_b, out, valid);
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
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int rows = batch * frames;
  char* ws = static_cast<char*>(workspace);
  uint16_t* a = reinterpret_cast<uint16_t*>(ws);
  uint16_t* big = a + (size_t)rows * kD;
  uint16_t* y = big + (size_t)rows * kPkFfn;
  uint16_t* o = y + (size_t)rows * kD;
  uint16_t* bd = o + (size_t)rows * kD;
  const long long T2 = 2 * kAttT;
  int rc = LFM25_OK;
  auto ln_of = [](const lfm25_pk_layer& L, int which) { return L.ln + (size_t)which * 2 * kD; };
#define PK_TRY(call)             \
  do {                           \
    rc = (call);                 \
    if (rc != LFM25_OK) return rc; \
  } while (0)
  for (int i = 0; i < n_layers; ++i) {
    const lfm25_pk_layer& L = layers[i];
    // a = LN_ff1(x)  (for i > 0 the second half of the previous layer's LN_DOUBLE)
    k_pk_ln<<<rows, kWave, 0, s>>>(x, nullptr, 0.0f, ln_of(L, 0), ln_of(L, 0) + kD, nullptr, nullptr, 0, a);
    PK_TRY(gemm(a, kD, 0, L.ff1_w1, kD, 0, nullptr, big, kPkFfn, 0, rows, kPkFfn, kD, 1, EPI_SWISH, s));
    PK_TRY(gemm(big, kPkFfn, 0, L.ff1_w2, kPkFfn, 0, nullptr, y, kD, 0, rows, kD, kPkFfn, 1, EPI_NONE, s));
    k_pk_ln<<<rows, kWave, 0, s>>>(x, y, 0.5f, ln_of(L, 1), ln_of(L, 1) + kD, nullptr, nullptr, 0, a);
    PK_TRY(gemm(a, kD, 0, L.qkv, kD, 0, L.qkv_bias, big, 3 * kD, 0, rows, 3 * kD, kD, 1, EPI_BIAS, s));
    PK_TRY(gemm(big, 3 * kD, kDk, L.pos, kDk, T2 * kDk, nullptr, bd, (int)T2, (long long)rows * T2, rows, (int)T2,
                kDk, kPkHeads, EPI_NONE, s));
    k_pk_attention<<<dim3(kPkHeads, batch), kAttThreads, 0, s>>>(big, bd, L.att_delta, o, valid, rows);
    PK_TRY(gemm(o, kD, 0, L.out, kD, 0, nullptr, y, kD, 0, rows, kD, kD, 1, EPI_NONE, s));
    k_pk_ln<<<rows, kWave, 0, s>>>(x, y, 1.0f, ln_of(L, 2), ln_of(L, 2) + kD, nullptr, nullptr, 0, a);
    PK_TRY(gemm(a, kD, 0, L.pw1, kD, 0, nullptr, big, 2 * kD, 0, rows, 2 * kD, kD, 1, EPI_NONE, s));
    k_pk_conv<<<dim3(kD / kConvCh, batch), 256, 0, s>>>(big, L.dw, L.dw_b, o, valid);
    PK_TRY(gemm(o, kD, 0, L.pw2, kD, 0, nullptr, y, kD, 0, rows, kD, kD, 1, EPI_NONE, s));
    k_pk_ln<<<rows, kWave, 0, s>>>(x, y, 1.0f, ln_of(L, 3), ln_of(L, 3) + kD, nullptr, nullptr, 0, a);
    PK_TRY(gemm(a, kD, 0, L.ff2_w1, kD, 0, nullptr, big, kPkFfn, 0, rows, kPkFfn, kD, 1, EPI_SWISH, s));
    PK_TRY(gemm(big, kPkFfn, 0, L.ff2_w2, kPkFfn, 0, nullptr, y, kD, 0, rows, kD, kPkFfn, 1, EPI_NONE, s));
    k_pk_ln<<<rows, kWave, 0, s>>>(x, y, 0.5f, ln_of(L, 4), ln_of(L, 4) + kD, nullptr, nullptr, 1, nullptr);
  }
#undef PK_TRY
  return check_launch("parakeet encoder");
}

}  // extern "C"
