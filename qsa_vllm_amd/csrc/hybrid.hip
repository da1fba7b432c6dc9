// Hybrid decoder layers around the QSA path, gfx950: the gated RMSNorm of
// every decoder layer, the SwiGLU activation and the Gated DeltaNet (GDN)
// token mixer of the linear-attention layers.
//
// The plugin's model (model.py:60-98, 180-225) takes these from vLLM
// (RMSNorm, SiluAndMul, QwenGatedDeltaNetAttention with its fla kernels);
// they are restated here from their definitions:
//
//  * gated_norm_kernel: residual add (rounded to bf16), RMSNorm
//    bf16(bf16(x * rsqrt(mean(x^2) + eps)) * gamma), then the low-rank gate
//    n * bf16(sigmoid(bf16(up(bf16(silu(bf16(down(n)))))))) of YuLanGatedNorm,
//    16 tokens per workgroup, the rank-16 projections on MFMA;
//  * silu_mul_kernel: bf16(silu(g) * u) in fp32 (SiluAndMul);
//  * gdn_prep_kernel: per token, the depthwise causal convolution of the
//    projected q|k|v channels over the sequence's last K-1 inputs (from the
//    conv state before the chunk) with SiLU, rounded to bf16; l2-normalised
//    q (times dk^-1/2) and k in fp32; the gates g = -exp(A_log) *
//    softplus(a + dt_bias) and beta = sigmoid(b);
//  * gdn_conv_state_kernel: the new conv state (each sequence's last K-1
//    inputs), after the prep kernel has read the old one;
//  * gdn_recurrence_kernel: the gated delta rule per (sequence, value head)
//    over the sequence's tokens in order, state S [dk, dv] fp32 held in
//    registers (lane (w, l) of the 4 waves owns column 32 w + (l & 31),
//    rows 64 (l >> 5) .. + 63): S <- e^g S, u = beta (v - S^T k),
//    S <- S + k u^T, o = S^T q;
//  * gdn_norm_kernel: y = bf16(rmsnorm(o) * w * silu(z)) per (token, value head).
//
// Layouts: the GDN projection rows are grouped per key head as
// [q (128), k (128), v (r*128), z (r*128)] and [b (r), a (r)] (r value heads
// per key head); the conv channels are ordered [q of all key heads, k of all
// key heads, v of all value heads]; conv state [slots, K-1, channels] bf16
// (oldest row first); recurrent state [slots, value heads, 128, 128] fp32.
#include "qsa_common.h"
#include "../../include/qsa_hip.h"

namespace qsa {
namespace {

constexpr int kHeadDim = 128;

__device__ __forceinline__ float rbf(float x) { return bf16_lo(pack_bf16x2(x, 0.0f)); }
// Sigmoid and SiLU through the hardware exp2 and reciprocal, each within a
// couple of fp32 ulps before the results are rounded to bf16 (exp2 of a large
// argument is +inf, whose reciprocal is 0). The IEEE expf and fp32 division
// took ~25 VALU ops per element: the gate phase of the gated norm was
// VALU-bound on them.
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }

__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// ---------------------------------------------------------------------------
// Gated RMSNorm.
//
// A workgroup (4 to 16 waves) takes 16 tokens. With the v_mfma_f32_16x16x32_bf16
// operand layout (lane (m, g) = (lane & 15, lane >> 4) holds A[m][8 g .. +7]
// and B[8 g .. +7][m] of each 32-deep slice; the accumulator gives lane (n, g)
// rows 4 g .. 4 g + 3 of column n), lane (m, g) of wave w holds token m's
// columns 32 s + 8 g .. +7 for its wave's S column groups s (wave w: groups
// S w .. S w + S - 1), so the normalised rows stay in registers as A operands:
//  * down = n Wd^T: one MFMA per column group, B lane (j, g) reading
//    Wd[j][32 s + 8 g ..]; the four waves' partial 16x16 tiles meet in LDS;
//  * up^T = Wu s^T: two MFMAs per column group whose output rows are the
//    lane's own columns (row 4 g + i of MFMA h is column 32 s + 8 g + 4 h + i),
//    so the accumulator lands in the lane that holds n for the same
//    (token, column) and the epilogue needs no exchange. The rank-16 K
//    dimension is padded to 32 with zero lanes (g >= 2).
// Weights are read once per 16 tokens.
// ---------------------------------------------------------------------------
constexpr int kRank = 16;
constexpr int kNormTokens = 16;

struct GatedNormArgs {
  const uint16_t* x;
  int64_t x_stride;
  const uint16_t* res_in;  // null: no residual add
  int64_t res_in_stride;
  uint16_t* res_out;
  int64_t res_out_stride;
  const uint16_t* weight;     // [H]
  const uint16_t* gate_down;  // [16, H]
  const uint16_t* gate_up;    // [H, 16]
  const uint16_t* bias;       // [H]
  uint16_t* out;
  int64_t out_stride;
  int rows, hidden;
  float eps;
};

template <int S, int W>  // W waves of S column groups of 32: hidden = 32 S W
__global__ __launch_bounds__(64 * W) void gated_norm_kernel(const GatedNormArgs a) {
  __shared__ float ssq[W][kNormTokens];
  __shared__ float down_part[W][kNormTokens][kRank];
  __shared__ float gate_s[kNormTokens][kRank];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, g = lane >> 4;
  const int64_t t = (int64_t)blockIdx.x * kNormTokens + m;
  const bool ok = t < a.rows;
  const int col0 = 32 * S * wave + 8 * g;  // column of group s: col0 + 32 s
  u32x4 n[S];
  float ss = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    // Loads in batches of 4 groups: bounds the registers held by loads in flight.
    if (s % 4 == 0 && s > 0) __builtin_amdgcn_sched_barrier(0);
    const int col = col0 + 32 * s;
    u32x4 xv = {0, 0, 0, 0};
    if (ok) xv = load_u32x4(a.x + t * a.x_stride + col);
    float f[8];
    unpack8(xv, f);
    if (a.res_in) {
      u32x4 rv = {0, 0, 0, 0};
      if (ok) rv = load_u32x4(a.res_in + t * a.res_in_stride + col);
      float r[8];
      unpack8(rv, r);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = rbf(f[e] + r[e]);
      xv = pack8(f);
      if (ok) *reinterpret_cast<u32x4*>(a.res_out + t * a.res_out_stride + col) = xv;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    n[s] = xv;
  }
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if (g == 0) ssq[wave][m] = ss;
  lds_barrier();
  float sq = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) sq += ssq[w][m];
  const float inv = rsqrtf(sq / (float)a.hidden + a.eps);
  f32x4 down = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (s % 4 == 0 && s > 0) __builtin_amdgcn_sched_barrier(0);
    const int col = col0 + 32 * s;
    float f[8], w[8];
    unpack8(n[s], f);
    unpack8(load_u32x4(a.weight + col), w);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = rbf(rbf(f[e] * inv) * w[e]);
    n[s] = pack8(f);
    const u32x4 wd = load_u32x4(a.gate_down + (int64_t)m * a.hidden + col);  // B: rank m
    down = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, n[s]),
                                                   __builtin_bit_cast(bf16x8, wd), down, 0, 0, 0);
  }
  // down[token 4 g + i][rank m] partial over this wave's columns
#pragma unroll
  for (int i = 0; i < 4; ++i) down_part[wave][4 * g + i][m] = down[i];
  lds_barrier();
  if (threadIdx.x < kNormTokens * kRank) {
    const int tok = threadIdx.x >> 4, j = threadIdx.x & 15;
    float d = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) d += down_part[w][tok][j];
    gate_s[tok][j] = rbf(silu_f(rbf(d)));
  }
  lds_barrier();
  // B operand of the up projection: s^T, lane (m, g) = tokens m, ranks 8 g .. +7 (g < 2)
  u32x4 sb = {0, 0, 0, 0};
  if (g < 2) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = gate_s[m][8 * g + e];
    sb = pack8(f);
  }
  const u32x4 zero4 = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (s % 4 == 0 && s > 0) __builtin_amdgcn_sched_barrier(0);
    const int col = col0 + 32 * s;
    f32x4 up[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // A row m (this lane's load role) is column 32 s + 8 (m / 4) + 4 h + m % 4 of the wave's group
      const int arow = 32 * S * wave + 32 * s + 8 * (m >> 2) + 4 * h + (m & 3);
      const u32x4 wu = g < 2 ? load_u32x4(a.gate_up + (int64_t)arow * kRank + 8 * g) : zero4;
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      up[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wu),
                                                      __builtin_bit_cast(bf16x8, sb), z, 0, 0, 0);
    }
    float b[8], f[8];
    unpack8(load_u32x4(a.bias + col), b);
    unpack8(n[s], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float u = up[e >> 2][e & 3];
      f[e] = rbf(f[e] * rbf(sigmoid_f(rbf(u + b[e]))));
    }
    if (ok) *reinterpret_cast<u32x4*>(a.out + t * a.out_stride + col) = pack8(f);
  }
}

// ---------------------------------------------------------------------------
// Gated RMSNorm for small batches (fewer than kTokenNormRows tokens): the
// 16-token tiles above would run on a handful of CUs. One workgroup per token
// instead, hidden / 8 threads of 8 consecutive columns each, so a decode
// batch spreads over as many CUs as it has tokens, in one launch. The rank-16
// projections are per-thread dot products over the thread's columns:
//  * down: 16 partial sums per thread, summed across the wave by a transpose
//    reduction (each shuffle step halves the values a lane keeps: 17 shuffles
//    for 16 sums), then across waves in LDS; every wave forms
//    s = bf16(silu(bf16(down))) for the 16 ranks itself and broadcasts them
//    from lanes 0..15 into scalar registers;
//  * up: each of the thread's columns dots its 16 gate_up weights (32 B) with s.
// Every load that does not depend on the token's statistics (the row, the
// residual, gamma, the gate_down slices) is issued first; the gate_up slices
// and the bias go out before the down reduction. The 2 x 16 x hidden gate
// weights are read by every workgroup and come from L2 after the first ones.
// ---------------------------------------------------------------------------
constexpr int kTokenNormRows = 1024;
constexpr int kTokenNormMaxWaves = 8;  // hidden up to 4096

// Sum over the wave of v[j] for each j < 16: returns the total of rank
// j = (lane >> 2) & 15 (every lane holds one; lanes 4 j .. 4 j + 3 agree).
__device__ __forceinline__ float wave_transpose_sum16(float (&v)[kRank]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int half = 8, bit = 32; half >= 1; half >>= 1, bit >>= 1) {
    const bool upper = (lane & bit) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float keep = upper ? v[half + i] : v[i];
      const float give = upper ? v[i] : v[half + i];
      v[i] = keep + __shfl_xor(give, bit, 64);
    }
  }
  float r = v[0];
  r += __shfl_xor(r, 2, 64);
  r += __shfl_xor(r, 1, 64);
  return r;
}

__global__ __launch_bounds__(64 * kTokenNormMaxWaves) void token_norm_kernel(const GatedNormArgs a) {
  __shared__ float wsq[kTokenNormMaxWaves];
  __shared__ float wdown[kTokenNormMaxWaves][kRank];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int waves = blockDim.x >> 6;
  const int64_t t = blockIdx.x;
  const int col = 8 * tid;
  const u32x4 xv = load_u32x4(a.x + t * a.x_stride + col);
  u32x4 rv = {0, 0, 0, 0};
  if (a.res_in) rv = load_u32x4(a.res_in + t * a.res_in_stride + col);
  const u32x4 wv = load_u32x4(a.weight + col);
  u32x4 wd[kRank];
#pragma unroll
  for (int j = 0; j < kRank; ++j) wd[j] = load_u32x4(a.gate_down + (int64_t)j * a.hidden + col);
  float f[8];
  unpack8(xv, f);
  if (a.res_in) {
    float r[8];
    unpack8(rv, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = rbf(f[e] + r[e]);
    *reinterpret_cast<u32x4*>(a.res_out + t * a.res_out_stride + col) = pack8(f);
  }
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  if (lane == 0) wsq[wave] = ss;
  lds_barrier();
  float sq = 0.0f;
  for (int w = 0; w < waves; ++w) sq += wsq[w];
  const float inv = rsqrtf(sq / (float)a.hidden + a.eps);
  {
    float g[8];
    unpack8(wv, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = rbf(rbf(f[e] * inv) * g[e]);
  }
  u32x4 wu[2 * 8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wu[2 * e] = load_u32x4(a.gate_up + (int64_t)(col + e) * kRank);
    wu[2 * e + 1] = load_u32x4(a.gate_up + (int64_t)(col + e) * kRank + 8);
  }
  const u32x4 bv = load_u32x4(a.bias + col);
  float d[kRank];
#pragma unroll
  for (int j = 0; j < kRank; ++j) {
    float w[8];
    unpack8(wd[j], w);
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += f[e] * w[e];
    d[j] = acc;
  }
  const float dj = wave_transpose_sum16(d);
  if ((lane & 3) == 0) wdown[wave][lane >> 2] = dj;
  lds_barrier();
  float sj = 0.0f;
  if (lane < kRank) {
    for (int w = 0; w < waves; ++w) sj += wdown[w][lane];
    sj = rbf(silu_f(rbf(sj)));
  }
  float sr[kRank];
#pragma unroll
  for (int j = 0; j < kRank; ++j)
    sr[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), j));
  float b[8];
  unpack8(bv, b);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float u0[8], u1[8];
    unpack8(wu[2 * e], u0);
    unpack8(wu[2 * e + 1], u1);
    float u = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) u += sr[j] * u0[j];
#pragma unroll
    for (int j = 0; j < 8; ++j) u += sr[8 + j] * u1[j];
    f[e] = rbf(f[e] * rbf(sigmoid_f(rbf(u + b[e]))));
  }
  *reinterpret_cast<u32x4*>(a.out + t * a.out_stride + col) = pack8(f);
}

// ---------------------------------------------------------------------------
// SwiGLU activation.
// ---------------------------------------------------------------------------
struct SiluMulArgs {
  const uint16_t* gu;
  int64_t gu_stride;
  uint16_t* out;
  int64_t out_stride;
  int rows, inter;
};

__global__ __launch_bounds__(256) void silu_mul_kernel(const SiluMulArgs a) {
  const int64_t t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= a.inter) return;
  float g[8], u[8];
  unpack8(load_u32x4(a.gu + t * a.gu_stride + c), g);
  unpack8(load_u32x4(a.gu + t * a.gu_stride + a.inter + c), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) g[e] = silu_f(g[e]) * u[e];
  *reinterpret_cast<u32x4*>(a.out + t * a.out_stride + c) = pack8(g);
}

// ---------------------------------------------------------------------------
// GDN.
// ---------------------------------------------------------------------------
struct GdnShape {
  int key_heads, value_heads, r, group;  // group = 256 + 2 r 128 (projection row per key head)
  int channels;                          // 256 key_heads + 128 value_heads
  int kernel;                            // conv width K (2..4)
};

// Projection column of conv channel c (16 consecutive channels stay in one head).
__device__ __forceinline__ int gdn_column(int c, const GdnShape& s) {
  const int qk = s.key_heads * kHeadDim;
  if (c < qk) return (c >> 7) * s.group + (c & 127);
  c -= qk;
  if (c < qk) return (c >> 7) * s.group + kHeadDim + (c & 127);
  c -= qk;
  const int h = c >> 7, m = h / s.r;
  return m * s.group + 2 * kHeadDim + (h - m * s.r) * kHeadDim + (c & 127);
}

struct GdnPrepArgs {
  const uint16_t* qkvz;
  int64_t qkvz_stride;
  const uint16_t* ba;
  int64_t ba_stride;
  const uint16_t* conv_w;      // [channels, K]
  const uint16_t* conv_state;  // [slots, K-1, channels]
  const int* seq_start;        // [seqs + 1]
  const int* token_seq;        // [tokens]
  const int64_t* slots;        // [seqs]
  const float* A_log;
  const float* dt_bias;
  GdnShape s;
  int tokens, num_seqs, num_slots;
  float* q_out;  // [tokens, key_heads, 128]
  float* k_out;
  uint16_t* v_out;  // [tokens, value_heads, 128]
  float* g_out;     // [tokens, value_heads]
  float* beta_out;
};

__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// One token per workgroup; thread i covers channels 16 i .. 16 i + 15.
template <int K>
__global__ __launch_bounds__(1024) void gdn_prep_kernel(const GdnPrepArgs a) {
  const int t = blockIdx.x;
  const GdnShape& s = a.s;
  // A token whose sequence entry is out of range, or whose range does not
  // contain it, is treated as the first token of a sequence without state.
  const int seq_raw = a.token_seq[t];
  const bool seq_ok = seq_raw >= 0 && seq_raw < a.num_seqs;
  const int seq = seq_ok ? seq_raw : 0;
  int start = seq_ok ? a.seq_start[seq] : t;
  int64_t slot = seq_ok ? a.slots[seq] : -1;
  if (start < 0 || start > t) {
    start = t;
    slot = -1;
  }
  const int off = t - start;
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  const int c0 = 16 * threadIdx.x;
  const bool active = c0 < s.channels;
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
  if (active) {
    const int col = gdn_column(c0, s);
    // weights: 16 channels x K taps, channel-major (16 K contiguous bf16)
    float w[16][K];
    const uint16_t* wp = a.conv_w + (int64_t)c0 * K;
#pragma unroll
    for (int e = 0; e < 16; ++e)
#pragma unroll
      for (int j = 0; j < K; ++j) w[e][j] = __builtin_bit_cast(float, (uint32_t)wp[e * K + j] << 16);
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int src = off - (K - 1) + j;
      const uint16_t* row;
      bool ok = true;
      if (src >= 0) {
        row = a.qkvz + (int64_t)(start + src) * a.qkvz_stride + col;
      } else {
        ok = slot_ok;
        row = a.conv_state + (slot_ok ? (slot * (K - 1) + (K - 1 + src)) * s.channels + c0 : 0);
      }
      float x[16] = {};
      if (ok) {
        unpack8(load_u32x4(row), *reinterpret_cast<float(*)[8]>(&x[0]));
        unpack8(load_u32x4(row + 8), *reinterpret_cast<float(*)[8]>(&x[8]));
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] += w[e][j] * x[e];
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = rbf(silu_f(acc[e]));
  }
  // l2 norm over each 128-channel q/k head: 8 consecutive threads.
  const int qk = s.key_heads * kHeadDim;
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) ss += acc[e] * acc[e];
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  if (active) {
    if (c0 < 2 * qk) {
      const bool is_q = c0 < qk;
      const int cc = is_q ? c0 : c0 - qk;
      const float inv = rsqrtf(ss + 1e-6f);
      const float scale = is_q ? rsqrtf((float)kHeadDim) : 1.0f;
      float* dst = (is_q ? a.q_out : a.k_out) + ((int64_t)t * s.key_heads) * kHeadDim + cc;
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        f32x4 v;
        v[0] = acc[e] * inv * scale;
        v[1] = acc[e + 1] * inv * scale;
        v[2] = acc[e + 2] * inv * scale;
        v[3] = acc[e + 3] * inv * scale;
        *reinterpret_cast<f32x4*>(dst + e) = v;
      }
    } else {
      uint16_t* dst = a.v_out + (int64_t)t * s.value_heads * kHeadDim + (c0 - 2 * qk);
      *reinterpret_cast<u32x4*>(dst) = pack8(*reinterpret_cast<float(*)[8]>(&acc[0]));
      *reinterpret_cast<u32x4*>(dst + 8) = pack8(*reinterpret_cast<float(*)[8]>(&acc[8]));
    }
  }
  if ((int)threadIdx.x < s.value_heads) {
    const int h = threadIdx.x, m = h / s.r, hl = h - m * s.r;
    const uint16_t* bar = a.ba + (int64_t)t * a.ba_stride + m * 2 * s.r;
    const float b = __builtin_bit_cast(float, (uint32_t)bar[hl] << 16);
    const float av = __builtin_bit_cast(float, (uint32_t)bar[s.r + hl] << 16);
    a.g_out[(int64_t)t * s.value_heads + h] = -expf(a.A_log[h]) * softplus_f(av + a.dt_bias[h]);
    a.beta_out[(int64_t)t * s.value_heads + h] = sigmoid_f(b);
  }
}

struct GdnConvStateArgs {
  const uint16_t* qkvz;
  int64_t qkvz_stride;
  uint16_t* conv_state;
  const int* seq_start;
  const int64_t* slots;
  GdnShape s;
  int num_seqs, num_slots, tokens;
};

// One sequence per blockIdx.y; thread covers 16 channels. Reads every old
// row of its channels before writing, so the in-place shift is safe.
template <int K>
__global__ __launch_bounds__(256) void gdn_conv_state_kernel(const GdnConvStateArgs a) {
  const int seq = blockIdx.y;
  const int c0 = 16 * (blockIdx.x * 256 + threadIdx.x);
  const GdnShape& s = a.s;
  if (c0 >= s.channels) return;
  const int64_t slot = a.slots[seq];
  if (slot < 0 || slot >= a.num_slots) return;
  const int start = a.seq_start[seq], len = a.seq_start[seq + 1] - start;
  if (len <= 0 || start < 0 || start + len > a.tokens) return;
  uint16_t* base = a.conv_state + slot * (K - 1) * s.channels + c0;
  const int col = gdn_column(c0, s);
  u32x4 rows[K - 1][2];
#pragma unroll
  for (int i = 0; i < K - 1; ++i) {
    const int src = len - (K - 1) + i;  // offset in the chunk, or an old row K-1+src
    const uint16_t* p = src >= 0 ? a.qkvz + (int64_t)(start + src) * a.qkvz_stride + col
                                 : base + (int64_t)(K - 1 + src) * s.channels;
    rows[i][0] = load_u32x4(p);
    rows[i][1] = load_u32x4(p + 8);
  }
#pragma unroll
  for (int i = 0; i < K - 1; ++i) {
    *reinterpret_cast<u32x4*>(base + (int64_t)i * s.channels) = rows[i][0];
    *reinterpret_cast<u32x4*>(base + (int64_t)i * s.channels + 8) = rows[i][1];
  }
}

constexpr int kRecTokens = 16;  // tokens staged in LDS per block
constexpr int kChunkMin = 16;   // sequences this long take gdn_chunk_kernel

struct GdnRecurArgs {
  const float* q;  // [tokens, key_heads, 128]
  const float* k;
  const uint16_t* v;  // [tokens, value_heads, 128]
  const float* g;     // [tokens, value_heads]
  const float* beta;
  float* state;  // [slots, value_heads, 128, 128]
  const int* seq_start;
  const int64_t* slots;
  int num_seqs, key_heads, value_heads, num_slots, tokens;
  uint16_t* o;  // [tokens, value_heads, 128]
  int chunk_min;  // sequences this long go to gdn_chunk_kernel, shorter ones to the per-token kernel
};

__global__ __launch_bounds__(256) void gdn_recurrence_kernel(const GdnRecurArgs a) {
  __shared__ float sq[kRecTokens][kHeadDim];
  __shared__ float sk[kRecTokens][kHeadDim];
  __shared__ float sv[kRecTokens][kHeadDim];
  __shared__ float sg[kRecTokens], sb[kRecTokens];
  const int h = blockIdx.x % a.value_heads;
  const int seq = a.num_seqs - 1 - (int)(blockIdx.x / a.value_heads);  // longest (prefill) first
  const int m = h / (a.value_heads / a.key_heads);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = 32 * wave + (lane & 31);
  const int half = lane >> 5;
  const int start = a.seq_start[seq], len = a.seq_start[seq + 1] - start;
  if (len <= 0 || len >= a.chunk_min || start < 0 || start + len > a.tokens) return;
  const int64_t slot = a.slots[seq];
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  float* sp = a.state + ((slot_ok ? slot : 0) * a.value_heads + h) * (int64_t)(kHeadDim * kHeadDim) +
              (int64_t)(64 * half) * kHeadDim + j;
  float S[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) S[i] = slot_ok ? sp[(int64_t)i * kHeadDim] : 0.0f;
  for (int b0 = 0; b0 < len; b0 += kRecTokens) {
    const int nb = min(kRecTokens, len - b0);
    // stage: thread -> (token tt = tid / 16, 8 dims at 8 (tid % 16))
    {
      const int tt = threadIdx.x >> 4, d0 = 8 * (threadIdx.x & 15);
      if (tt < nb) {
        const int64_t t = start + b0 + tt;
        const float* qp = a.q + (t * a.key_heads + m) * kHeadDim + d0;
        const float* kp = a.k + (t * a.key_heads + m) * kHeadDim + d0;
        *reinterpret_cast<f32x4*>(&sq[tt][d0]) = *reinterpret_cast<const f32x4*>(qp);
        *reinterpret_cast<f32x4*>(&sq[tt][d0 + 4]) = *reinterpret_cast<const f32x4*>(qp + 4);
        *reinterpret_cast<f32x4*>(&sk[tt][d0]) = *reinterpret_cast<const f32x4*>(kp);
        *reinterpret_cast<f32x4*>(&sk[tt][d0 + 4]) = *reinterpret_cast<const f32x4*>(kp + 4);
        float vv[8];
        unpack8(load_u32x4(a.v + (t * a.value_heads + h) * kHeadDim + d0), vv);
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[tt][d0 + e] = vv[e];
        if ((threadIdx.x & 15) == 0) {
          sg[tt] = a.g[t * a.value_heads + h];
          sb[tt] = a.beta[t * a.value_heads + h];
        }
      }
    }
    __syncthreads();
    for (int tt = 0; tt < nb; ++tt) {
      const float* kr = &sk[tt][64 * half];
      float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
#pragma unroll
      for (int i = 0; i < 64; i += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(kr + i);
        p0 += kv[0] * S[i];
        p1 += kv[1] * S[i + 1];
        p2 += kv[2] * S[i + 2];
        p3 += kv[3] * S[i + 3];
      }
      const float ks = sum_wave_halves((p0 + p1) + (p2 + p3));
      const float decay = expf(sg[tt]);
      const float u = sb[tt] * (sv[tt][j] - decay * ks);
#pragma unroll
      for (int i = 0; i < 64; i += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(kr + i);
        S[i] = S[i] * decay + kv[0] * u;
        S[i + 1] = S[i + 1] * decay + kv[1] * u;
        S[i + 2] = S[i + 2] * decay + kv[2] * u;
        S[i + 3] = S[i + 3] * decay + kv[3] * u;
      }
      const float* qr = &sq[tt][64 * half];
      p0 = p1 = p2 = p3 = 0.0f;
#pragma unroll
      for (int i = 0; i < 64; i += 4) {
        const f32x4 qv = *reinterpret_cast<const f32x4*>(qr + i);
        p0 += qv[0] * S[i];
        p1 += qv[1] * S[i + 1];
        p2 += qv[2] * S[i + 2];
        p3 += qv[3] * S[i + 3];
      }
      const float os = sum_wave_halves((p0 + p1) + (p2 + p3));
      if (half == 0) {
        const int64_t t = start + b0 + tt;
        const __bf16 ob = (__bf16)os;
        a.o[(t * a.value_heads + h) * kHeadDim + j] = __builtin_bit_cast(uint16_t, ob);
      }
    }
    __syncthreads();
  }
  if (slot_ok) {
#pragma unroll
    for (int i = 0; i < 64; ++i) sp[(int64_t)i * kHeadDim] = S[i];
  }
}

// ---------------------------------------------------------------------------
// Chunked gated delta rule (sequences of kChunkMin tokens or more).
//
// The recurrence over a chunk of C = 64 tokens in its WY form. With G the
// in-chunk cumulative log decay, gamma = e^G and S the state at the chunk
// start:
//   A[t][s] = beta_t e^{G_t - G_s} k_t.k_s (s < t),  (I + A) U = beta V - beta gamma (K S)
//   O = gamma (Q S) + (e^{G_t - G_s} q_t.k_s)_{s <= t} U
//   S <- gamma_C S + (e^{G_C - G_s} k_s)^T U
// One workgroup (4 waves) per (sequence, value head). The state stays in
// registers as 16x16 MFMA accumulator tiles (wave w: value columns 32 w ..
// 32 w + 31, all 128 key rows) and feeds the K S / Q S products directly as
// the B operand: a 32-deep slice pairs key-row tiles 2 ks and 2 ks + 1, slice
// index 8 g + j being row 16 (2 ks + (j >> 2)) + 4 g + (j & 3) - exactly the
// accumulator elements lane (n, g) holds - and the A operand reads K with the
// same row order. Products run in bf16 with fp32 accumulation (the precision
// of the reference's chunk kernels); the state, gates and the triangular
// solve are fp32: 16-row blocks, each taking the earlier blocks' contribution
// and the inverse of its diagonal block as fp32 MFMA work.
// ---------------------------------------------------------------------------
constexpr int kChunk = 64;

struct ChunkLds {
  uint16_t q[kChunk][136];        // bf16 q (normalised, scaled)
  uint16_t k[kChunk][136];        // bf16 k
  uint16_t v[kChunk][136];        // bf16 v
  uint16_t kgt[kHeadDim][72];     // bf16 (e^{G_C - G_s} k_s)^T
  uint16_t p[kChunk][72];         // bf16 (e^{G_t - G_s} q_t.k_s), s <= t
  uint16_t ut[kHeadDim][72];      // bf16 U^T
  float a[kChunk][68];            // fp32 A (strict lower)
  float r[kChunk][132];           // fp32 right-hand side of the solve
  float tinv[4][16][17];          // fp32 inverses of the diagonal 16x16 blocks of I + A
  float G[kChunk], gam[kChunk], beta[kChunk];
};

__device__ __forceinline__ uint16_t bf16_bits(float x) {
  const __bf16 b = (__bf16)x;
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ bf16x8 lds_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}

// Two 4-element halves (8-byte aligned) as one 8-element operand.
__device__ __forceinline__ bf16x8 lds_bf16x4x2(const uint16_t* lo, const uint16_t* hi) {
  const u32x2 a = *reinterpret_cast<const u32x2*>(lo);
  const u32x2 b = *reinterpret_cast<const u32x2*>(hi);
  const u32x4 v = {a[0], a[1], b[0], b[1]};
  return __builtin_bit_cast(bf16x8, v);
}

__global__ __launch_bounds__(256) void gdn_chunk_kernel(const GdnRecurArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char chunk_lds_raw[];
  ChunkLds& L = *reinterpret_cast<ChunkLds*>(chunk_lds_raw);
  const int h = blockIdx.x % a.value_heads;
  const int seq = a.num_seqs - 1 - (int)(blockIdx.x / a.value_heads);
  const int mk = h / (a.value_heads / a.key_heads);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int m = lane & 15, g = lane >> 4;
  const int start = a.seq_start[seq], len = a.seq_start[seq + 1] - start;
  if (len < a.chunk_min || start < 0 || start + len > a.tokens) return;
  const int64_t slot = a.slots[seq];
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  float* state = a.state + ((slot_ok ? slot : 0) * a.value_heads + h) * (int64_t)(kHeadDim * kHeadDim);

  // S tiles: S[rt][nl] = rows 16 rt + 4 g + i, column 32 w + 16 nl + m.
  f32x4 S[8][2];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int nl = 0; nl < 2; ++nl)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        S[rt][nl][i] = slot_ok ? state[(16 * rt + 4 * g + i) * kHeadDim + 32 * w + 16 * nl + m] : 0.0f;

  // Inputs of a chunk: this thread's slice of row tid / 4 (dims 32 (tid % 4)
  // .. + 31) and the gates of row `lane`. The next chunk's are loaded as soon
  // as the current ones are staged, so they arrive during this chunk's work.
  // Loads are unconditional (rows past the sequence read its last token and
  // are zeroed when staged), so every wait count is static.
  const int row = tid >> 2, d0 = 32 * (tid & 3);
  f32x4 pq[8], pk[8];
  u32x4 pv[4];
  float pg, pb;
  auto load_chunk = [&](int c) {
    const int64_t t = start + min(c + row, len - 1);
    const float* qp = a.q + (t * a.key_heads + mk) * kHeadDim + d0;
    const float* kp = a.k + (t * a.key_heads + mk) * kHeadDim + d0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pq[e] = *reinterpret_cast<const f32x4*>(qp + 4 * e);
      pk[e] = *reinterpret_cast<const f32x4*>(kp + 4 * e);
    }
    const uint16_t* vp = a.v + (t * a.value_heads + h) * kHeadDim + d0;
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = load_u32x4(vp + 8 * e);
    const int64_t tg = start + min(c + lane, len - 1);
    pg = a.g[tg * a.value_heads + h];
    pb = a.beta[tg * a.value_heads + h];
  };
  load_chunk(0);

  for (int c0 = 0; c0 < len; c0 += kChunk) {
    const int nc = min(kChunk, len - c0);
    // 1. Stage the chunk from the registers loaded one chunk earlier.
    const bool live = row < nc;
    float kf[32];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 qv = live ? pq[e] : zero, kv = live ? pk[e] : zero;
      *reinterpret_cast<u32x2*>(&L.q[row][d0 + 4 * e]) = u32x2{pack_bf16x2(qv[0], qv[1]), pack_bf16x2(qv[2], qv[3])};
      *reinterpret_cast<u32x2*>(&L.k[row][d0 + 4 * e]) = u32x2{pack_bf16x2(kv[0], kv[1]), pack_bf16x2(kv[2], kv[3])};
#pragma unroll
      for (int j = 0; j < 4; ++j) kf[4 * e + j] = rbf(kv[j]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const u32x4 zero = {0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&L.v[row][d0 + 8 * e]) = live ? pv[e] : zero;
    }
    float gv = lane < nc ? pg : 0.0f;
    const float bv = lane < nc ? pb : 0.0f;
    load_chunk(c0 + kChunk);  // past the end: the last token again, never used
    if (w == 0) {  // gates of row `lane`, inclusive prefix sum of g
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float o = __shfl_up(gv, d, 64);
        if (lane >= d) gv += o;
      }
      L.G[lane] = gv;
      L.gam[lane] = expf(gv);
      L.beta[lane] = bv;
    }
    __syncthreads();
    {
      const float scale = expf(L.G[kChunk - 1] - L.G[row]);
#pragma unroll
      for (int e = 0; e < 32; ++e) L.kgt[d0 + e][row] = bf16_bits(kf[e] * scale);
    }
    // 2. K S and Q S: tiles (ct, nl), rows 16 ct + 4 g + i, columns 32 w + 16 nl + m.
    bf16x8 sb[4][2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int nl = 0; nl < 2; ++nl) {
        const u32x4 v = {pack_bf16x2(S[2 * ks][nl][0], S[2 * ks][nl][1]),
                         pack_bf16x2(S[2 * ks][nl][2], S[2 * ks][nl][3]),
                         pack_bf16x2(S[2 * ks + 1][nl][0], S[2 * ks + 1][nl][1]),
                         pack_bf16x2(S[2 * ks + 1][nl][2], S[2 * ks + 1][nl][3])};
        sb[ks][nl] = __builtin_bit_cast(bf16x8, v);
      }
    f32x4 KS[4][2], QS[4][2];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int nl = 0; nl < 2; ++nl) {
        KS[ct][nl] = f32x4{0.f, 0.f, 0.f, 0.f};
        QS[ct][nl] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int r = 16 * ct + m;
        const bf16x8 ak = lds_bf16x4x2(&L.k[r][32 * ks + 4 * g], &L.k[r][32 * ks + 16 + 4 * g]);
        const bf16x8 aq = lds_bf16x4x2(&L.q[r][32 * ks + 4 * g], &L.q[r][32 * ks + 16 + 4 * g]);
#pragma unroll
        for (int nl = 0; nl < 2; ++nl) {
          KS[ct][nl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, sb[ks][nl], KS[ct][nl], 0, 0, 0);
          QS[ct][nl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq, sb[ks][nl], QS[ct][nl], 0, 0, 0);
        }
      }
    // 3. K K^T and Q K^T for row tile w: rows 16 w + 4 g + i, columns 16 ct + m.
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 bk = lds_bf16x8(&L.k[16 * ct + m][32 * ks + 8 * g]);
        kk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lds_bf16x8(&L.k[16 * w + m][32 * ks + 8 * g]), bk, kk, 0, 0, 0);
        qk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lds_bf16x8(&L.q[16 * w + m][32 * ks + 8 * g]), bk, qk, 0, 0, 0);
      }
      const int sc = 16 * ct + m;
      const float Gs = L.G[sc];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tr = 16 * w + 4 * g + i;
        const float d = L.G[tr] - Gs;
        const float e = sc <= tr ? expf(d) : 0.0f;
        L.a[tr][sc] = sc < tr ? L.beta[tr] * e * kk[i] : 0.0f;
        L.p[tr][sc] = bf16_bits(e * qk[i]);
      }
    }
    // 3b. Wave w wrote rows 16 w .. 16 w + 15 of A above, so it inverts the
    // unit lower-triangular diagonal block w of I + A without a barrier: lane
    // j < 16 solves for column j by forward substitution.
    if (lane < 16) {
      const int j = lane;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float* arow = &L.a[16 * w + i][16 * w];
        float p0 = i == j ? 1.0f : 0.0f, p1 = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < i; ++s2) {
          if (s2 & 1) p1 -= arow[s2] * x[s2];
          else p0 -= arow[s2] * x[s2];
        }
        x[i] = p0 + p1;
        L.tinv[w][i][j] = x[i];
      }
    }
    // 4. Right-hand side beta (V - gamma K S).
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int nl = 0; nl < 2; ++nl)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tr = 16 * ct + 4 * g + i, col = 32 * w + 16 * nl + m;
          const float vv = __builtin_bit_cast(float, (uint32_t)L.v[tr][col] << 16);
          L.r[tr][col] = L.beta[tr] * (vv - L.gam[tr] * KS[ct][nl][i]);
        }
    __syncthreads();
    // 5. Solve (I + A) U = R in 16-row blocks, each wave its own 32 value
    // columns alone, with no barrier: block b takes the earlier blocks'
    // contribution, R_b - A[b][0 : 16 b] U[0 : 16 b], and multiplies it by the
    // inverse of its diagonal block, both as fp32 MFMA work
    // (v_mfma_f32_16x16x4f32: lane (m, kk) holds A[m][kk] and B[kk][m] of each
    // 4-deep slice). The wave reads back through LDS only what it wrote
    // itself, in issue order. U overwrites R (fp32) and goes to U^T (bf16) for
    // the products below, which read this wave's columns only.
    {
      const int kk = lane >> 4;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        f32x4 acc[2];
#pragma unroll
        for (int nl = 0; nl < 2; ++nl)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[nl][i] = L.r[16 * blk + 4 * g + i][32 * w + 16 * nl + m];
#pragma unroll
        for (int ks = 0; ks < 4 * blk; ++ks) {
          const float av = -L.a[16 * blk + m][4 * ks + kk];
#pragma unroll
          for (int nl = 0; nl < 2; ++nl)
            acc[nl] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                av, L.r[4 * ks + kk][32 * w + 16 * nl + m], acc[nl], 0, 0, 0);
        }
        if (blk > 0) {
#pragma unroll
          for (int nl = 0; nl < 2; ++nl)
#pragma unroll
            for (int i = 0; i < 4; ++i) L.r[16 * blk + 4 * g + i][32 * w + 16 * nl + m] = acc[nl][i];
        }
        f32x4 u[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const float tv = L.tinv[blk][m][4 * ks + kk];
#pragma unroll
          for (int nl = 0; nl < 2; ++nl)
            u[nl] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                tv, L.r[16 * blk + 4 * ks + kk][32 * w + 16 * nl + m], u[nl], 0, 0, 0);
        }
#pragma unroll
        for (int nl = 0; nl < 2; ++nl)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tr = 16 * blk + 4 * g + i, col = 32 * w + 16 * nl + m;
            L.r[tr][col] = u[nl][i];
            L.ut[col][tr] = bf16_bits(u[nl][i]);
          }
      }
    }
    // 6. O = gamma (Q S) + P U.
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      f32x4 o[2];
#pragma unroll
      for (int nl = 0; nl < 2; ++nl) o[nl] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 ap = lds_bf16x8(&L.p[16 * ct + m][32 * ks + 8 * g]);
#pragma unroll
        for (int nl = 0; nl < 2; ++nl)
          o[nl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              ap, lds_bf16x8(&L.ut[32 * w + 16 * nl + m][32 * ks + 8 * g]), o[nl], 0, 0, 0);
      }
#pragma unroll
      for (int nl = 0; nl < 2; ++nl)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tr = 16 * ct + 4 * g + i;
          if (tr < nc) {
            const float val = L.gam[tr] * QS[ct][nl][i] + o[nl][i];
            a.o[((start + c0 + tr) * (int64_t)a.value_heads + h) * kHeadDim + 32 * w + 16 * nl + m] =
                bf16_bits(val);
          }
        }
    }
    // 7. S <- gamma_C S + Kg^T U.
    const float gc = L.gam[kChunk - 1];
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
      for (int nl = 0; nl < 2; ++nl) S[rt][nl] = S[rt][nl] * gc;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 ak = lds_bf16x8(&L.kgt[16 * rt + m][32 * ks + 8 * g]);
#pragma unroll
        for (int nl = 0; nl < 2; ++nl)
          S[rt][nl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              ak, lds_bf16x8(&L.ut[32 * w + 16 * nl + m][32 * ks + 8 * g]), S[rt][nl], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  if (slot_ok) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int nl = 0; nl < 2; ++nl)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          state[(16 * rt + 4 * g + i) * kHeadDim + 32 * w + 16 * nl + m] = S[rt][nl][i];
  }
}

struct GdnNormArgs {
  const uint16_t* o;  // [tokens, value_heads, 128]
  const uint16_t* qkvz;
  int64_t qkvz_stride;
  const uint16_t* weight;  // [128]
  float eps;
  uint16_t* y;  // [tokens, value_heads, 128]
  GdnShape s;
  int tokens;
};

// Sixteen lanes per (token, value head), lane l covering dims 8 l .. 8 l + 7
// (one 16-byte load of o, z and the weight each), four rows per wave.
__global__ __launch_bounds__(256) void gdn_norm_kernel(const GdnNormArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  const GdnShape& s = a.s;
  const bool ok = row < (int64_t)a.tokens * s.value_heads;
  const int64_t t = ok ? row / s.value_heads : 0;
  const int h = ok ? (int)(row - t * s.value_heads) : 0;
  const int m = h / s.r, hl = h - m * s.r;
  u32x4 ov = {0, 0, 0, 0}, zv = {0, 0, 0, 0};
  if (ok) {
    ov = load_u32x4(a.o + row * kHeadDim + 8 * l);
    zv = load_u32x4(a.qkvz + t * a.qkvz_stride + m * s.group + 2 * kHeadDim + s.r * kHeadDim +
                    hl * kHeadDim + 8 * l);
  }
  float o[8], z[8], w[8];
  unpack8(ov, o);
  unpack8(zv, z);
  unpack8(load_u32x4(a.weight + 8 * l), w);
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += o[e] * o[e];
#pragma unroll
  for (int d = 1; d < 16; d <<= 1) ss += __shfl_xor(ss, d, 64);
  const float inv = rsqrtf(ss * (1.0f / kHeadDim) + a.eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = o[e] * inv * w[e] * silu_f(z[e]);
  if (ok) *reinterpret_cast<u32x4*>(a.y + row * kHeadDim + 8 * l) = pack8(y);
}

bool gdn_shape(int key_heads, int value_heads, int head_dim, int kernel, GdnShape* s,
               const char* what) {
  if (head_dim != kHeadDim) {
    fail(QSA_ERR_UNSUPPORTED, std::string(what) + ": GDN head dims must be 128");
    return false;
  }
  if (key_heads <= 0 || value_heads <= 0 || value_heads % key_heads) {
    fail(QSA_ERR_INVALID, std::string(what) + ": value heads must be a positive multiple of key heads");
    return false;
  }
  if (kernel < 2 || kernel > 4) {
    fail(QSA_ERR_UNSUPPORTED, std::string(what) + ": conv width must be 2..4");
    return false;
  }
  s->key_heads = key_heads;
  s->value_heads = value_heads;
  s->r = value_heads / key_heads;
  s->group = 2 * kHeadDim + 2 * s->r * kHeadDim;
  s->channels = 2 * key_heads * kHeadDim + value_heads * kHeadDim;
  s->kernel = kernel;
  if (s->channels / 16 > 1024) {
    fail(QSA_ERR_UNSUPPORTED, std::string(what) + ": more than 16384 conv channels");
    return false;
  }
  return true;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace qsa

using namespace qsa;

extern "C" size_t qsa_gated_norm_workspace_bytes(int rows, int hidden) {
  (void)rows;
  (void)hidden;
  return 0;  // no launch shape needs one
}

extern "C" int qsa_gated_norm(const void* x, int64_t x_stride, const void* residual_in,
                              int64_t residual_in_stride, void* residual_out,
                              int64_t residual_out_stride, const void* weight,
                              const void* gate_down, const void* gate_up, const void* gate_up_bias,
                              void* out, int64_t out_stride, int rows, int hidden, int rank,
                              float eps, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0) return fail(QSA_ERR_INVALID, "qsa_gated_norm: negative rows");
  if (rows == 0) return QSA_OK;
  if (!x || !weight || !gate_down || !gate_up || !gate_up_bias || !out ||
      (residual_in && !residual_out))
    return fail(QSA_ERR_INVALID, "qsa_gated_norm: null tensor pointer");
  if (rank != kRank) return fail(QSA_ERR_UNSUPPORTED, "qsa_gated_norm: gate rank must be 16");
  // One supported set for both launch paths (one workgroup per token below
  // kTokenNormRows rows, 16-token tiles above), so a hidden size that decodes
  // also prefills.
  if (hidden != 512 && hidden != 1024 && hidden != 2048 && hidden != 4096)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_gated_norm: hidden size must be 512, 1024, 2048 or 4096");
  const void* ptrs[] = {x, weight, gate_down, gate_up, gate_up_bias, out, residual_in, residual_out};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return fail(QSA_ERR_INVALID, "qsa_gated_norm: tensors must be 16-byte aligned");
  if ((x_stride | out_stride | residual_in_stride | residual_out_stride) & 7)
    return fail(QSA_ERR_INVALID, "qsa_gated_norm: row strides must be multiples of 8 elements");
  GatedNormArgs a{static_cast<const uint16_t*>(x), x_stride,
                  static_cast<const uint16_t*>(residual_in), residual_in_stride,
                  static_cast<uint16_t*>(residual_out), residual_out_stride,
                  static_cast<const uint16_t*>(weight), static_cast<const uint16_t*>(gate_down),
                  static_cast<const uint16_t*>(gate_up), static_cast<const uint16_t*>(gate_up_bias),
                  static_cast<uint16_t*>(out), out_stride, rows, hidden, eps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)workspace;
  (void)workspace_bytes;
  if (rows < kTokenNormRows) {
    hipLaunchKernelGGL(token_norm_kernel, dim3(rows), dim3(hidden / 8), 0, s, a);
    return check_launch("qsa_gated_norm (one workgroup per token)");
  }
  const dim3 grid((rows + kNormTokens - 1) / kNormTokens);
  switch (hidden / 512) {
    case 1: hipLaunchKernelGGL((gated_norm_kernel<4, 4>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((gated_norm_kernel<8, 4>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((gated_norm_kernel<8, 8>), grid, dim3(512), 0, s, a); break;
    case 8: hipLaunchKernelGGL((gated_norm_kernel<8, 16>), grid, dim3(1024), 0, s, a); break;
    default: return fail(QSA_ERR_UNSUPPORTED, "qsa_gated_norm: hidden size must be 512, 1024, 2048 or 4096");
  }
  return check_launch("qsa_gated_norm");
}

extern "C" int qsa_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out,
                            int64_t out_stride, int rows, int intermediate, void* stream) {
  if (rows < 0 || intermediate < 0) return fail(QSA_ERR_INVALID, "qsa_silu_mul: negative size");
  if (rows == 0 || intermediate == 0) return QSA_OK;
  if (!gate_up || !out) return fail(QSA_ERR_INVALID, "qsa_silu_mul: null tensor pointer");
  if (intermediate % 8 || (gate_up_stride | out_stride) & 7 || !aligned16(gate_up) || !aligned16(out))
    return fail(QSA_ERR_INVALID,
                "qsa_silu_mul: 16-byte aligned rows with sizes and strides multiples of 8 elements");
  if (rows > 65535) return fail(QSA_ERR_UNSUPPORTED, "qsa_silu_mul: more than 65535 rows");
  SiluMulArgs a{static_cast<const uint16_t*>(gate_up), gate_up_stride, static_cast<uint16_t*>(out),
                out_stride, rows, intermediate};
  const dim3 grid((intermediate / 8 + 255) / 256, rows);
  hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_silu_mul");
}

extern "C" int qsa_gdn_prep(const void* qkvz, int64_t qkvz_stride, const void* ba,
                            int64_t ba_stride, const void* conv_weight, const void* conv_state,
                            int num_slots, const int* query_start_loc, const int* token_to_seq,
                            const int64_t* slots, int num_seqs, const float* A_log,
                            const float* dt_bias, int key_heads, int value_heads, int head_dim,
                            int conv_kernel, int tokens, float* q_out, float* k_out, void* v_out,
                            float* g_out, float* beta_out, void* stream) {
  GdnShape s;
  if (!gdn_shape(key_heads, value_heads, head_dim, conv_kernel, &s, "qsa_gdn_prep")) return QSA_ERR_UNSUPPORTED;
  if (tokens < 0 || num_seqs < 0) return fail(QSA_ERR_INVALID, "qsa_gdn_prep: negative size");
  if (tokens == 0) return QSA_OK;
  if (!qkvz || !ba || !conv_weight || !conv_state || !query_start_loc || !token_to_seq || !slots ||
      !A_log || !dt_bias || !q_out || !k_out || !v_out || !g_out || !beta_out)
    return fail(QSA_ERR_INVALID, "qsa_gdn_prep: null tensor pointer");
  if (!aligned16(qkvz) || !aligned16(conv_state) || !aligned16(q_out) || !aligned16(k_out) ||
      !aligned16(v_out) || (qkvz_stride & 7))
    return fail(QSA_ERR_INVALID, "qsa_gdn_prep: 16-byte aligned rows with strides multiples of 8");
  GdnPrepArgs a{static_cast<const uint16_t*>(qkvz), qkvz_stride, static_cast<const uint16_t*>(ba),
                ba_stride, static_cast<const uint16_t*>(conv_weight),
                static_cast<const uint16_t*>(conv_state), query_start_loc, token_to_seq, slots,
                A_log, dt_bias, s, tokens, num_seqs, num_slots, q_out, k_out,
                static_cast<uint16_t*>(v_out), g_out, beta_out};
  const int threads = ((s.channels / 16 + 63) / 64) * 64;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (conv_kernel) {
    case 2: hipLaunchKernelGGL(gdn_prep_kernel<2>, dim3(tokens), dim3(threads), 0, st, a); break;
    case 3: hipLaunchKernelGGL(gdn_prep_kernel<3>, dim3(tokens), dim3(threads), 0, st, a); break;
    default: hipLaunchKernelGGL(gdn_prep_kernel<4>, dim3(tokens), dim3(threads), 0, st, a); break;
  }
  return check_launch("qsa_gdn_prep");
}

extern "C" int qsa_gdn_conv_state(const void* qkvz, int64_t qkvz_stride, int tokens,
                                  void* conv_state, int num_slots, const int* query_start_loc,
                                  const int64_t* slots, int num_seqs, int key_heads,
                                  int value_heads, int head_dim, int conv_kernel, void* stream) {
  GdnShape s;
  if (!gdn_shape(key_heads, value_heads, head_dim, conv_kernel, &s, "qsa_gdn_conv_state"))
    return QSA_ERR_UNSUPPORTED;
  if (num_seqs < 0 || tokens < 0) return fail(QSA_ERR_INVALID, "qsa_gdn_conv_state: negative size");
  if (num_seqs == 0 || tokens == 0) return QSA_OK;
  if (num_seqs > 65535) return fail(QSA_ERR_UNSUPPORTED, "qsa_gdn_conv_state: more than 65535 sequences");
  if (!qkvz || !conv_state || !query_start_loc || !slots)
    return fail(QSA_ERR_INVALID, "qsa_gdn_conv_state: null tensor pointer");
  if (!aligned16(qkvz) || !aligned16(conv_state) || (qkvz_stride & 7))
    return fail(QSA_ERR_INVALID, "qsa_gdn_conv_state: 16-byte aligned rows with strides multiples of 8");
  GdnConvStateArgs a{static_cast<const uint16_t*>(qkvz), qkvz_stride,
                     static_cast<uint16_t*>(conv_state), query_start_loc, slots, s, num_seqs,
                     num_slots, tokens};
  const dim3 grid((s.channels / 16 + 255) / 256, num_seqs);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (conv_kernel) {
    case 2: hipLaunchKernelGGL(gdn_conv_state_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL(gdn_conv_state_kernel<3>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(gdn_conv_state_kernel<4>, grid, dim3(256), 0, st, a); break;
  }
  return check_launch("qsa_gdn_conv_state");
}

extern "C" int qsa_gdn_recurrence(const float* q, const float* k, const void* v, const float* g,
                                  const float* beta, int tokens, float* state, int num_slots,
                                  const int* query_start_loc, const int64_t* slots, int num_seqs,
                                  int key_heads, int value_heads, int head_dim,
                                  int max_seq_tokens, void* o, void* stream) {
  GdnShape s;
  if (!gdn_shape(key_heads, value_heads, head_dim, 4, &s, "qsa_gdn_recurrence")) return QSA_ERR_UNSUPPORTED;
  if (num_seqs < 0 || tokens < 0) return fail(QSA_ERR_INVALID, "qsa_gdn_recurrence: negative size");
  if (num_seqs == 0 || tokens == 0) return QSA_OK;
  if (!q || !k || !v || !g || !beta || !state || !query_start_loc || !slots || !o)
    return fail(QSA_ERR_INVALID, "qsa_gdn_recurrence: null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(state))
    return fail(QSA_ERR_INVALID, "qsa_gdn_recurrence: tensors must be 16-byte aligned");
  if ((int64_t)num_seqs * value_heads > 0x7fffffffLL)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_gdn_recurrence: too many (sequence, head) pairs");
  // With no sequence of kChunkMin tokens (a decode batch, as the caller
  // states), the chunked kernel is not launched and the per-token kernel
  // takes every sequence, whatever its length: a wrong bound costs time only.
  const bool chunks = max_seq_tokens < 0 || max_seq_tokens >= kChunkMin;
  GdnRecurArgs a{q, k, static_cast<const uint16_t*>(v), g, beta, state, query_start_loc, slots,
                 num_seqs, key_heads, value_heads, num_slots, tokens, static_cast<uint16_t*>(o),
                 chunks ? kChunkMin : 0x7fffffff};
  if (chunks) {
    // Long sequences (chunks) first on the stream: their workgroups are the long ones.
    hipLaunchKernelGGL(gdn_chunk_kernel, dim3(num_seqs * value_heads), dim3(256), sizeof(ChunkLds),
                       static_cast<hipStream_t>(stream), a);
    const int st = check_launch("qsa_gdn_recurrence (chunks)");
    if (st != QSA_OK) return st;
  }
  hipLaunchKernelGGL(gdn_recurrence_kernel, dim3(num_seqs * value_heads), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_gdn_recurrence");
}

extern "C" int qsa_gdn_gated_norm(const void* o, const void* qkvz, int64_t qkvz_stride,
                                  const void* weight, float eps, int tokens, int key_heads,
                                  int value_heads, int head_dim, void* y, void* stream) {
  GdnShape s;
  if (!gdn_shape(key_heads, value_heads, head_dim, 4, &s, "qsa_gdn_gated_norm")) return QSA_ERR_UNSUPPORTED;
  if (tokens < 0) return fail(QSA_ERR_INVALID, "qsa_gdn_gated_norm: negative size");
  if (tokens == 0) return QSA_OK;
  if (!o || !qkvz || !weight || !y) return fail(QSA_ERR_INVALID, "qsa_gdn_gated_norm: null tensor pointer");
  if (!aligned16(o) || !aligned16(qkvz) || !aligned16(weight) || !aligned16(y) || (qkvz_stride & 7))
    return fail(QSA_ERR_INVALID,
                "qsa_gdn_gated_norm: 16-byte aligned tensors, qkvz stride a multiple of 8 elements");
  GdnNormArgs a{static_cast<const uint16_t*>(o), static_cast<const uint16_t*>(qkvz), qkvz_stride,
                static_cast<const uint16_t*>(weight), eps, static_cast<uint16_t*>(y), s, tokens};
  const int64_t rows = (int64_t)tokens * value_heads;
  if ((rows + 15) / 16 > 0x7fffffffLL)
    return fail(QSA_ERR_UNSUPPORTED, "qsa_gdn_gated_norm: too many (token, head) rows");
  hipLaunchKernelGGL(gdn_norm_kernel, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("qsa_gdn_gated_norm");
}
