// Prompt prefill for gfx950: every token of the prompt in one pass per layer.
//
// Kernels:
// - the int4 GEMM on MFMA, with a store or a SwiGLU epilogue;
// - the 4-tap causal conv over a sequence;
// - the chunked gated delta rule;
// - GatedRMSNorm over rows;
// - q/k RMSNorm + partial RoPE over rows, which also writes the KV cache;
// - causal GQA attention with the reference's bf16 softmax rounding.
//
// Every rounding point is the reference's forward over a sequence (reference.py:496-550,
// 610-677, 692-735). Only fp32 summation order differs.
#include <math.h>

#include "common.h"
#include "deltaforge_hip.h"
#include "int4_block.h"

namespace df {
namespace pf {

DF_DEVICE df_f32x4 mfma(const uint4& a, const uint4& b, df_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, a), __builtin_bit_cast(df_bf16x8, b),
                                                 c, 0, 0, 0);
}

DF_DEVICE float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// ---------------------------------------------------------------------------------------
// int4 GEMM: out[m][n] = bf16( sum_k x[m][k] * bf16((nibble - 8) * scale) ), fp32 sums
// ---------------------------------------------------------------------------------------
//
// The weight is in the library's device tiling (df_int4_repack). A 1 KB block is 16 columns x
// one 128-group, and lane L of a 64-lane read owns its bytes [16 L, 16 L + 16): four words of
// column L % 16. Word i holds k = 32 (L / 16) + 8 i + e, e < 8, with element e at bit
// 4 (e / 2), plus 16 when e is odd. That is exactly the B operand of
// v_mfma_f32_16x16x32_bf16 number i, whose A operand is then x[row][32 (L / 16) + 8 i ..+8].
// A workgroup computes a 128 x 128 tile; wave w owns all 128 rows and column tiles 2w, 2w + 1
// (8 x 2 products). Per 128-group:
// - only the x rows go through LDS, double-buffered (one barrier per group): the next
//   group's rows are stored from registers while this group's products run;
// - each wave loads its two weight blocks straight into registers a group ahead, in the
//   MFMA B layout, and dequantises them there with int4_block.h's exact dequant (19 VALU per
//   8 weights), so every weight is dequantised once and never staged.
// The products, and each output's order of summation, are those of a staged-B design.

constexpr int kGmBM = 128;
constexpr int kGmTiles = 8;           // 16-column tiles per workgroup (128 columns)
constexpr int kGmXPitch = 128 + 8;    // bf16 per staged x row (16-byte pad)

template <int EPI>
__global__ __launch_bounds__(256, 2) void int4_gemm_kernel(DfInt4GemmArgs p) {
  __shared__ __align__(16) uint16_t xs[2][kGmBM * kGmXPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * kGmBM, t0 = blockIdx.x * kGmTiles + 2 * wave;
  const int G = p.K / 128, ntiles = p.N / 16;
  df_f32x4 acc[8][2];
#pragma unroll
  for (int rb = 0; rb < 8; ++rb)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[rb][j] = df_f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 xr[8], wr[2];
  uint16_t sr[2];
  auto load_x = [&](int g) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // 128 rows x 16 chunks of 16 bytes
      const int ch = tid + 256 * i, r = ch >> 4, cc = ch & 15;
      xr[i] = m0 + r < p.M ? *reinterpret_cast<const uint4*>(p.x + (size_t)(m0 + r) * p.ldx + g * 128 + cc * 8)
                           : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ch = tid + 256 * i, r = ch >> 4, cc = ch & 15;
      *reinterpret_cast<uint4*>(&xs[buf][r * kGmXPitch + cc * 8]) = xr[i];
    }
  };
  auto load_w = [&](int g) {  // this wave's two blocks of group g (zeros past N)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      wr[j] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
      sr[j] = 0;
      if (t0 + j < ntiles) {
        const size_t blk = (size_t)(t0 + j) * G + g;
        wr[j] = *reinterpret_cast<const uint4*>(p.w + blk * 1024 + lane * 16);
        sr[j] = p.s[blk * 16 + (lane & 15)];
      }
    }
  };
  load_x(0);
  load_w(0);
  store_x(0);
  if (G > 1) load_x(1);
  const DqK K = dq_consts();
  for (int g = 0; g < G; ++g) {
    // xs[g & 1] is complete, and every wave is done with xs[(g + 1) & 1] (group g - 1)
    __syncthreads();
    uint4 b[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const GroupScale gs = group_scale(sr[j]);  // the exact bf16((n - 8) * scale) of the per-op GEMV
      b[j][0] = dequant8(wr[j].x, gs, K);
      b[j][1] = dequant8(wr[j].y, gs, K);
      b[j][2] = dequant8(wr[j].z, gs, K);
      b[j][3] = dequant8(wr[j].w, gs, K);
    }
    if (g + 1 < G) {
      store_x((g + 1) & 1);
      load_w(g + 1);
    }
    if (g + 2 < G) load_x(g + 2);
    const uint16_t* xb = xs[g & 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint4 a[8];
#pragma unroll
      for (int rb = 0; rb < 8; ++rb)
        a[rb] = *reinterpret_cast<const uint4*>(&xb[(rb * 16 + (lane & 15)) * kGmXPitch + (lane >> 4) * 32 + i * 8]);
#pragma unroll
      for (int rb = 0; rb < 8; ++rb)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[rb][j] = mfma(a[rb], b[j][i], acc[rb][j]);
    }
  }

  // lane holds D[4 (lane / 16) + r][lane % 16] of each 16 x 16 product
  const int col_in = lane & 15;
#pragma unroll
  for (int rb = 0; rb < 8; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + rb * 16 + (lane >> 4) * 4 + r;
      if (row >= p.M) continue;
      if (EPI == DF_EPI_SWIGLU) {
        // tiles alternate gate, up: this wave's pair (2w, 2w + 1);
        // bf16(bf16(silu(bf16(g))) * bf16(u)) (reference.py:692-693)
        if (t0 >= ntiles) continue;
        const float gv = round_bf(acc[rb][0][r]), uv = round_bf(acc[rb][1][r]);
        p.out[(size_t)row * p.ldo + (t0 / 2) * 16 + col_in] = f2bf(round_bf(silu(gv)) * uv);
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if (t0 + j >= ntiles) continue;
          p.out[(size_t)row * p.ldo + (t0 + j) * 16 + col_in] = f2bf(acc[rb][j][r]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// causal conv over the sequence (reference.py:496-510)
// ---------------------------------------------------------------------------------------

// out[t][c] = bf16(silu(bf16(sum_j w[c][j] x(p - 3 + j)))) for position p = pos0 + t, taps in
// order with fp32 sums (the decode step's arithmetic); x(q) is row q - pos0 of the input for
// q >= pos0, else the history ring (slot q mod 4, zero for positions before the first).
__global__ __launch_bounds__(256) void conv_seq_kernel(const uint16_t* __restrict__ x, int ldx, int tokens,
                                                       int channels, const uint16_t* __restrict__ w,
                                                       const uint16_t* __restrict__ ring, int pos0,
                                                       uint16_t* __restrict__ out, int ldo) {
#pragma clang fp contract(off)
  const int c = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
  if (c >= channels) return;
  const uint2 wt = *reinterpret_cast<const uint2*>(w + (size_t)c * 4);
  const float wk[4] = {__uint_as_float(wt.x << 16), __uint_as_float(wt.x & 0xFFFF0000u),
                       __uint_as_float(wt.y << 16), __uint_as_float(wt.y & 0xFFFF0000u)};
  float h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tt = t - 3 + j;
    h[j] = tt >= 0 ? bf2f(x[(size_t)tt * ldx + c]) : bf2f(ring[(size_t)c * 4 + ((pos0 + tt) & 3)]);
  }
  float acc = h[0] * wk[0];
  acc = acc + h[1] * wk[1];
  acc = acc + h[2] * wk[2];
  acc = acc + h[3] * wk[3];
  out[(size_t)t * ldo + c] = f2bf(silu(round_bf(acc)));
}

// The last three inputs into the ring (slot position mod 4), after conv_seq_kernel read it.
__global__ __launch_bounds__(256) void conv_ring_update_kernel(const uint16_t* __restrict__ x, int ldx, int tokens,
                                                               int channels, uint16_t* __restrict__ ring, int pos0) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= channels) return;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int t = tokens - 3 + j;
    if (t >= 0) ring[(size_t)c * 4 + ((pos0 + t) & 3)] = x[(size_t)t * ldx + c];
  }
}

// ---------------------------------------------------------------------------------------
// chunked gated delta rule (reference.py:403-461 over a sequence)
// ---------------------------------------------------------------------------------------
//
// Within a chunk of C = 64 tokens, with cumulative log-decay gamma_t = g_1 + ... + g_t and
// the chunk's initial state S0 (Dk x Dv), the token-by-token rule
//   S <- exp(g_t) S;  delta_t = beta_t (v_t - S^T k_t);  S <- S + k_t delta_t^T;  o_t = S^T q_t
// is, exactly in real arithmetic:
//   A'[t][j] = beta_t exp(gamma_t - gamma_j) (k_t . k_j), j < t      (strictly lower)
//   [Wv | Wk] = (I + A')^-1 [diag(beta) V | diag(beta e^gamma) K]      (forward substitution)
//   delta    = Wv - Wk S0
//   QK[t][j] = exp(gamma_t - gamma_j) (q_t . k_j), j <= t
//   O        = O_loc + Qx S0,   O_loc = QK Wv,   Qx = diag(e^gamma) Q - QK Wk
//   S_C      = e^gamma_C S0 + Kd^T delta,   Kd = diag(exp(gamma_C - gamma)) K
// with q, k the L2-normalised rows (q also / sqrt(Dk)). Everything but the three products
// with S0 is independent of the state, so it runs for every (chunk, head) at once
// (delta_prep_kernel, 2048 workgroups at 4096 tokens). The scan kernel then walks the chunks
// in order with the state slice in LDS and does only O, delta and the state update.
// Padding tokens past the prompt get g = beta = 0 and q = k = v = 0, which changes nothing.

constexpr int kCk = 64;          // tokens per chunk
constexpr int kDk = 128;         // key (and value) head dim
constexpr int kPitch = kDk + 4;  // fp32 row pitch in LDS
constexpr int kMat = kCk * kDk;  // floats of one chunk matrix in the scratch
constexpr int kPrepMats = 5;     // O_loc, Qx, Wv, Wk, Kd

DF_DEVICE size_t prep_base(int chunk, int h, int hv) { return ((size_t)chunk * hv + h) * kPrepMats * kMat; }

struct PrepLds {
  float Q[kCk][kPitch];
  float K[kCk][kPitch];
  float V[kCk][kPitch];
  float At[kCk][kCk];   // A' transposed: At[j][t] = A'[t][j] (beta_t-scaled, decayed, strictly lower)
  float QK[kCk][kCk];   // decayed, lower with the diagonal
  float gam[kCk], beta[kCk], eg[kCk], dec[kCk];
};

__global__ __launch_bounds__(256) void delta_prep_kernel(DfDeltaPrefillArgs p, float* __restrict__ scratch) {
  __shared__ __align__(16) PrepLds L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = blockIdx.x, h = blockIdx.y;
  const int c0 = chunk * kCk;
  const int kh = h / (p.num_v_heads / p.num_k_heads);
  const int key_dim = p.num_k_heads * kDk;
  const int qoff = kh * kDk, koff = key_dim + kh * kDk, voff = 2 * key_dim + h * kDk;
  const float qscale = sqrtf(static_cast<float>(kDk));

  // ---- normalised q, k rows; v rows; gates --------------------------------------------
  // wave w: tokens 16 w ..; all 16 tokens' loads are issued before any is used
  uint32_t qkv[16][3];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int T = c0 + wave * 16 + i;
    qkv[i][0] = qkv[i][1] = qkv[i][2] = 0u;
    if (T < p.tokens) {
      const uint16_t* row = p.mixed + (size_t)T * p.ld_mixed;
      qkv[i][0] = *reinterpret_cast<const uint32_t*>(row + qoff + 2 * lane);
      qkv[i][1] = *reinterpret_cast<const uint32_t*>(row + koff + 2 * lane);
      qkv[i][2] = *reinterpret_cast<const uint32_t*>(row + voff + 2 * lane);
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = wave * 16 + i;
    float q0 = 0.f, q1 = 0.f, k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    {
      const uint32_t qw = qkv[i][0], kw = qkv[i][1], vw = qkv[i][2];
      q0 = __uint_as_float(qw << 16);
      q1 = __uint_as_float(qw & 0xFFFF0000u);
      k0 = __uint_as_float(kw << 16);
      k1 = __uint_as_float(kw & 0xFFFF0000u);
      v0 = __uint_as_float(vw << 16);
      v1 = __uint_as_float(vw & 0xFFFF0000u);
    }
    const float rq = 1.0f / sqrtf(wave_sum(q0 * q0 + q1 * q1) + 1e-6f);
    const float rk = 1.0f / sqrtf(wave_sum(k0 * k0 + k1 * k1) + 1e-6f);
    L.Q[t][2 * lane] = (q0 * rq) / qscale;
    L.Q[t][2 * lane + 1] = (q1 * rq) / qscale;
    L.K[t][2 * lane] = k0 * rk;
    L.K[t][2 * lane + 1] = k1 * rk;
    L.V[t][2 * lane] = v0;
    L.V[t][2 * lane + 1] = v1;
  }
  if (wave == 0) {
    const int T = c0 + lane;
    float g = 0.0f, beta = 0.0f;
    if (T < p.tokens) {
      const float av = bf2f(p.a[(size_t)T * p.ld_ab + h]), bv = bf2f(p.b[(size_t)T * p.ld_ab + h]);
      beta = round_bf(sigmoid(bv));                                          // bf16 sigmoid
      g = -expf(bf2f(p.A_log[h])) * softplus(av + bf2f(p.dt_bias[h]));      // fp32 (reference.py:528-532)
    }
    float gam = g;  // inclusive prefix sum over the chunk
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(gam, off, 64);
      if (lane >= off) gam += o;
    }
    const float last = readlane(gam, 63);
    L.gam[lane] = gam;
    L.beta[lane] = beta;
    L.eg[lane] = expf(gam);
    L.dec[lane] = expf(last - gam);
    if (lane == 0) scratch[(size_t)gridDim.x * p.num_v_heads * kPrepMats * kMat + (size_t)chunk * p.num_v_heads + h] =
        expf(last);
  }
  __syncthreads();

  // ---- A' and QK (4 x 4 register tiles of the lower triangle) ---------------------------
  // The 136 tiles (tb, jb <= tb) go to threads p = 4 lane + wave < 136, spread evenly over
  // the waves; the other threads write the zero tiles above the diagonal.
  {
    const int pidx = 4 * lane + wave;
    int tb, jb;
    if (pidx < 136) {
      tb = 0;
      while ((tb + 1) * (tb + 2) / 2 <= pidx) ++tb;
      jb = pidx - tb * (tb + 1) / 2;
    } else {  // upper tiles: 120 of them, for the 120 threads 136 .. 255
      const int q = pidx - 136;  // (jb, tb) with tb < jb
      jb = 1;
      while (jb * (jb + 1) / 2 <= q) ++jb;
      tb = q - jb * (jb - 1) / 2;
    }
    float aa[4][4], qq[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) aa[r][c] = qq[r][c] = 0.0f;
    if (jb <= tb) {
      for (int k = 0; k < kDk; k += 4) {
        float4 kt[4], kj[4], qt[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          kt[r] = *reinterpret_cast<const float4*>(&L.K[tb * 4 + r][k]);
          qt[r] = *reinterpret_cast<const float4*>(&L.Q[tb * 4 + r][k]);
          kj[r] = *reinterpret_cast<const float4*>(&L.K[jb * 4 + r][k]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            aa[r][c] += kt[r].x * kj[c].x + kt[r].y * kj[c].y + kt[r].z * kj[c].z + kt[r].w * kj[c].w;
            qq[r][c] += qt[r].x * kj[c].x + qt[r].y * kj[c].y + qt[r].z * kj[c].z + qt[r].w * kj[c].w;
          }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int t = tb * 4 + r, j = jb * 4 + c;
        const float d = j <= t ? expf(L.gam[t] - L.gam[j]) : 0.0f;
        L.At[j][t] = j < t ? L.beta[t] * (aa[r][c] * d) : 0.0f;
        L.QK[t][j] = j <= t ? qq[r][c] * d : 0.0f;
      }
  }
  float* base = scratch + prep_base(chunk, h, p.num_v_heads);
  // Kd = diag(exp(gamma_C - gamma)) K, before K becomes a right-hand side
  for (int e = tid; e < kMat; e += 256) base[4 * kMat + e] = L.dec[e / kDk] * L.K[e / kDk][e % kDk];
  __syncthreads();
  for (int e = tid; e < kMat; e += 256) {
    const int t = e / kDk, k = e % kDk;
    L.V[t][k] *= L.beta[t];
    L.K[t][k] *= L.beta[t] * L.eg[t];
  }
  __syncthreads();

  // ---- forward substitution: X_t = R_t - sum_{j<t} A'[t][j] X_j, in place --------------
  // Lane = one of the 256 columns of [V | K] (wave w: columns 64 w ..), its 64 tokens in
  // registers. Once token t is final, t's multiple is taken off every later token u, with
  // A'[u][t] read from row t of At as uniform LDS broadcasts. Each token receives its terms in
  // the order j = 0, 1, .. with the same fmaf as a token-by-token solve, but every step's
  // updates are independent of each other.
  {
    float (*M)[kPitch] = wave < 2 ? L.V : L.K;
    const int col = (wave & 1) * 64 + lane;
    float x[kCk];
#pragma unroll
    for (int t = 0; t < kCk; ++t) x[t] = M[t][col];
#pragma unroll
    for (int t = 0; t < kCk - 1; ++t) {
#pragma unroll
      for (int u4 = (t + 1) & ~3; u4 < kCk; u4 += 4) {
        const float4 a = *reinterpret_cast<const float4*>(&L.At[t][u4]);
        const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (u4 + e > t) x[u4 + e] = fmaf(-av[e], x[t], x[u4 + e]);
      }
    }
#pragma unroll
    for (int t = 0; t < kCk; ++t) M[t][col] = x[t];
  }
  __syncthreads();

  // ---- O_loc = QK Wv and Qx = diag(e^gamma) Q - QK Wk; Wv, Wk out ----------------------
  {
    // token t = 4 (li % 16) + wave for li = tid / 4: each wave gets every fourth token, so the
    // triangular work (t + 1 terms) is spread evenly
    const int li = tid >> 2, t = 4 * (li & 15) + wave, cs = (tid & 3) * 32;
    float o[32], qx[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      o[c] = 0.0f;
      qx[c] = 0.0f;
    }
    for (int j = 0; j <= t; ++j) {
      const float w = L.QK[t][j];
#pragma unroll
      for (int c = 0; c < 32; c += 4) {
        const float4 wv = *reinterpret_cast<const float4*>(&L.V[j][cs + c]);
        const float4 wk = *reinterpret_cast<const float4*>(&L.K[j][cs + c]);
        o[c] += w * wv.x; o[c + 1] += w * wv.y; o[c + 2] += w * wv.z; o[c + 3] += w * wv.w;
        qx[c] += w * wk.x; qx[c + 1] += w * wk.y; qx[c + 2] += w * wk.z; qx[c + 3] += w * wk.w;
      }
    }
    const float egt = L.eg[t];
    float* orow = base + (size_t)t * kDk + cs;
    float* qrow = base + kMat + (size_t)t * kDk + cs;
#pragma unroll
    for (int c = 0; c < 32; c += 4) {
      *reinterpret_cast<float4*>(orow + c) = make_float4(o[c], o[c + 1], o[c + 2], o[c + 3]);
      *reinterpret_cast<float4*>(qrow + c) =
          make_float4(egt * L.Q[t][cs + c] - qx[c], egt * L.Q[t][cs + c + 1] - qx[c + 1],
                      egt * L.Q[t][cs + c + 2] - qx[c + 2], egt * L.Q[t][cs + c + 3] - qx[c + 3]);
    }
  }
  for (int e = tid; e < kMat; e += 256) {
    base[2 * kMat + e] = L.V[e / kDk][e % kDk];
    base[3 * kMat + e] = L.K[e / kDk][e % kDk];
  }
}

// The scan: one workgroup per (value head, 16 value columns), the chunks in order. Per chunk:
// O = O_loc + Qx S0 (tokens out as bf16), delta = Wv - Wk S0, S = e^gamma_C S0 + Kd^T delta,
// all on the fp32 MFMA (v_mfma_f32_16x16x4_f32):
// - O and delta: wave w owns tokens 16 w ..+15 (16 x 16 results over k = 128). Its A operands
//   (rows of Qx and Wk) come straight from the pre-pass scratch; B is S, shared through LDS
//   transposed (St[c][k]);
// - the update: wave w owns state rows k = 32 w ..+31 (two 16 x 16 tiles over the 64 tokens),
//   kept in registers in the MFMA result layout. A is Kd^T, read from the scratch; B is
//   delta, shared through LDS transposed (Dt[c][t]).
// Each lane takes k (or t) in runs of 4 (k = 16 s + 4 (lane / 16) + j for the MFMA j of
// group s), so its operands are 16-byte loads. Every global operand of the next chunk is
// loaded a chunk ahead (two register sets).
constexpr int kScanVs = 16;

struct ScanLds {
  float St[kScanVs][kDk + 4];   // S0 transposed
  float Dt[kScanVs][kCk + 4];   // delta transposed
};

struct ScanPre {                // one chunk's operands for one lane
  float4 qa[8], wa[8];          // Qx, Wk: row 16 w + lane % 16, k = 16 s + 4 (lane / 16) ..+3
  float kd[2][4][4];            // Kd[t = 16 s + 4 (lane / 16) + j][k = 32 w + 16 tile + lane % 16]
  float ol[4], wv[4];           // O_loc, Wv at (16 w + 4 (lane / 16) + r, column lane % 16)
};

DF_DEVICE df_f32x4 mfma4(float a, float b, df_f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

__global__ __launch_bounds__(256) void delta_scan_kernel(DfDeltaPrefillArgs p, const float* __restrict__ scratch) {
  __shared__ __align__(16) ScanLds L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x, vs = blockIdx.y;
  const int col0 = vs * kScanVs;
  const int nchunks = (p.tokens + kCk - 1) / kCk;
  const int n16 = lane & 15, q4 = lane >> 4;
  float* gstate = p.state + (size_t)h * kDk * kDk;
  const float* ecs = scratch + (size_t)nchunks * p.num_v_heads * kPrepMats * kMat;

  // this wave's state rows in the MFMA result layout: S[32 w + 16 tile + 4 q4 + r][n16]
  df_f32x4 S[2];
#pragma unroll
  for (int tl = 0; tl < 2; ++tl)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[tl][r] = gstate[(size_t)(32 * wave + 16 * tl + 4 * q4 + r) * kDk + col0 + n16];
  auto put_state = [&]() {
#pragma unroll
    for (int tl = 0; tl < 2; ++tl)
      *reinterpret_cast<float4*>(&L.St[n16][32 * wave + 16 * tl + 4 * q4]) = make_float4(S[tl][0], S[tl][1], S[tl][2], S[tl][3]);
  };
  auto fetch = [&](ScanPre& P, int chunk) {
    const float* base = scratch + prep_base(chunk, h, p.num_v_heads);
    const int row = 16 * wave + n16;
#pragma unroll
    for (int sg = 0; sg < 8; ++sg) {
      P.qa[sg] = *reinterpret_cast<const float4*>(base + kMat + (size_t)row * kDk + 16 * sg + 4 * q4);
      P.wa[sg] = *reinterpret_cast<const float4*>(base + 3 * kMat + (size_t)row * kDk + 16 * sg + 4 * q4);
    }
#pragma unroll
    for (int tl = 0; tl < 2; ++tl)
#pragma unroll
      for (int sg = 0; sg < 4; ++sg)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          P.kd[tl][sg][j] = base[4 * kMat + (size_t)(16 * sg + 4 * q4 + j) * kDk + 32 * wave + 16 * tl + n16];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const size_t e = (size_t)(16 * wave + 4 * q4 + r) * kDk + col0 + n16;
      P.ol[r] = base[e];
      P.wv[r] = base[2 * kMat + e];
    }
  };
  auto step = [&](const ScanPre& P, ScanPre& N, int chunk) {
    __syncthreads();  // St holds this chunk's S0
    if (chunk + 1 < nchunks) fetch(N, chunk + 1);
    // O and delta for tokens 16 w + 4 q4 + r, column n16
    df_f32x4 o = {P.ol[0], P.ol[1], P.ol[2], P.ol[3]}, d = {P.wv[0], P.wv[1], P.wv[2], P.wv[3]};
    df_f32x4 qs = {0.f, 0.f, 0.f, 0.f}, ws = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sg = 0; sg < 8; ++sg) {
      const float4 b = *reinterpret_cast<const float4*>(&L.St[n16][16 * sg + 4 * q4]);
      qs = mfma4(P.qa[sg].x, b.x, qs);
      qs = mfma4(P.qa[sg].y, b.y, qs);
      qs = mfma4(P.qa[sg].z, b.z, qs);
      qs = mfma4(P.qa[sg].w, b.w, qs);
      ws = mfma4(P.wa[sg].x, b.x, ws);
      ws = mfma4(P.wa[sg].y, b.y, ws);
      ws = mfma4(P.wa[sg].z, b.z, ws);
      ws = mfma4(P.wa[sg].w, b.w, ws);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      o[r] += qs[r];
      d[r] -= ws[r];
      const int T = chunk * kCk + 16 * wave + 4 * q4 + r;
      if (T < p.tokens) p.out[(size_t)T * p.ld_out + h * kDk + col0 + n16] = f2bf(o[r]);
    }
    *reinterpret_cast<float4*>(&L.Dt[n16][16 * wave + 4 * q4]) = make_float4(d[0], d[1], d[2], d[3]);
    __syncthreads();  // Dt complete; every wave is done reading St
    // S <- e^gamma_C S0 + Kd^T delta
    const float ec = ecs[(size_t)chunk * p.num_v_heads + h];
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) {
      df_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sg = 0; sg < 4; ++sg) {
        const float4 b = *reinterpret_cast<const float4*>(&L.Dt[n16][16 * sg + 4 * q4]);
        acc = mfma4(P.kd[tl][sg][0], b.x, acc);
        acc = mfma4(P.kd[tl][sg][1], b.y, acc);
        acc = mfma4(P.kd[tl][sg][2], b.z, acc);
        acc = mfma4(P.kd[tl][sg][3], b.w, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) S[tl][r] = ec * S[tl][r] + acc[r];
    }
    put_state();
  };
  put_state();
  ScanPre A, B;
  fetch(A, 0);
  for (int chunk = 0; chunk < nchunks; chunk += 2) {
    step(A, B, chunk);
    if (chunk + 1 < nchunks) step(B, A, chunk + 1);
  }
#pragma unroll
  for (int tl = 0; tl < 2; ++tl)
#pragma unroll
    for (int r = 0; r < 4; ++r) gstate[(size_t)(32 * wave + 16 * tl + 4 * q4 + r) * kDk + col0 + n16] = S[tl][r];
}

// ---------------------------------------------------------------------------------------
// GatedRMSNorm over rows (reference.py:115-121): one wave per (token, value head)
// ---------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void gated_norm_rows_kernel(const uint16_t* __restrict__ x, int ldx,
                                                              const uint16_t* __restrict__ z, int ldz,
                                                              const uint16_t* __restrict__ w, float eps, int tokens,
                                                              int heads, uint16_t* __restrict__ out, int ldo) {
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= tokens * heads) return;
  const int t = unit / heads, hh = unit % heads;
  const int d = hh * 128 + 2 * lane;
  const uint32_t xv = *reinterpret_cast<const uint32_t*>(x + (size_t)t * ldx + d);
  const uint32_t zv = *reinterpret_cast<const uint32_t*>(z + (size_t)t * ldz + d);
  const uint32_t wv = *reinterpret_cast<const uint32_t*>(w + 2 * lane);
  const float x0 = __uint_as_float(xv << 16), x1 = __uint_as_float(xv & 0xFFFF0000u);
  const float r = 1.0f / sqrtf(wave_sum(x0 * x0 + x1 * x1) / 128.0f + eps);
  const float n0 = round_bf(x0 * r), n1 = round_bf(x1 * r);
  const float y0 = round_bf(__uint_as_float(wv << 16) * n0), y1 = round_bf(__uint_as_float(wv & 0xFFFF0000u) * n1);
  const float g0 = silu(__uint_as_float(zv << 16)), g1 = silu(__uint_as_float(zv & 0xFFFF0000u));
  *reinterpret_cast<uint32_t*>(out + (size_t)t * ldo + d) =
      static_cast<uint32_t>(f2bf(y0 * g0)) | (static_cast<uint32_t>(f2bf(y1 * g1)) << 16);
}

// ---------------------------------------------------------------------------------------
// q/k RMSNorm (1 + w) + partial RoPE over rows; K/V cache rows written
// ---------------------------------------------------------------------------------------

constexpr int kHd = 256;

// The decode kernel's norm_rope4 arithmetic (attention.hip), from global rows: lane holds
// dims 4 lane .. 4 lane + 3.
DF_DEVICE void norm_rope_row(float x[4], const uint16_t* nw, float eps, const float* inv_freq, int rot, float posf,
                             int lane) {
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(kHd) + eps);
  float n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) n[i] = round_bf((x[i] * r) * (1.0f + bf2f(nw[lane * 4 + i])));
  const int half = rot / 2;
  float partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(n[i], half / 4, 64);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dim = lane * 4 + i;
    if (dim < rot) {
      const float ang = posf * inv_freq[dim % half];
      const float c = round_bf(cosf(ang)), s = round_bf(sinf(ang));
      const float rotated = dim < half ? -partner[i] : partner[i];
      x[i] = round_bf(round_bf(n[i] * c) + round_bf(rotated * s));
    } else {
      x[i] = n[i];
    }
  }
}

DF_DEVICE void load4(const uint16_t* src, float x[4]) {
  const uint2 v = *reinterpret_cast<const uint2*>(src);
  x[0] = __uint_as_float(v.x << 16);
  x[1] = __uint_as_float(v.x & 0xFFFF0000u);
  x[2] = __uint_as_float(v.y << 16);
  x[3] = __uint_as_float(v.y & 0xFFFF0000u);
}
DF_DEVICE void store4(uint16_t* dst, const float x[4]) {
  *reinterpret_cast<uint2*>(dst) =
      make_uint2(static_cast<uint32_t>(f2bf(x[0])) | (static_cast<uint32_t>(f2bf(x[1])) << 16),
                 static_cast<uint32_t>(f2bf(x[2])) | (static_cast<uint32_t>(f2bf(x[3])) << 16));
}

// One wave per (token, slot): slots < Hq are query heads (normed, roped -> q_out), the next Hkv
// are KV heads (key normed and roped, value copied, both into the cache at pos0 + t).
__global__ __launch_bounds__(256) void qk_rows_kernel(DfQkPrefillArgs p) {
  const int lane = threadIdx.x & 63;
  const int slots = p.num_q_heads + p.num_kv_heads;
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= p.tokens * slots) return;
  const int t = unit / slots, sl = unit % slots;
  const float posf = static_cast<float>(p.pos0 + t);
  const uint16_t* row = p.proj + (size_t)t * p.ld_proj;
  float x[4];
  if (sl < p.num_q_heads) {
    load4(row + sl * 2 * kHd + lane * 4, x);  // head sl's [query | gate]: the query half
    norm_rope_row(x, p.q_norm, p.eps, p.inv_freq, p.rotary_dim, posf, lane);
    store4(p.q_out + ((size_t)t * p.num_q_heads + sl) * kHd + lane * 4, x);
  } else {
    const int g = sl - p.num_q_heads;
    load4(row + p.k_col + g * kHd + lane * 4, x);
    norm_rope_row(x, p.k_norm, p.eps, p.inv_freq, p.rotary_dim, posf, lane);
    const size_t dst = ((size_t)g * p.max_len + p.pos0 + t) * kHd + lane * 4;
    store4(p.k_cache + dst, x);
    *reinterpret_cast<uint2*>(p.v_cache + dst) = *reinterpret_cast<const uint2*>(row + p.v_col + g * kHd + lane * 4);
  }
}

// ---------------------------------------------------------------------------------------
// causal GQA attention over the prompt (reference.py:645-677)
// ---------------------------------------------------------------------------------------
//
// scores = bf16(bf16(q . k) * scale), masked above the diagonal; p = bf16(softmax_fp32);
// o = bf16(p @ V); out = bf16(o * bf16(gate_fn(gate))). The bf16 rounding of p needs the
// row's final max and sum, so the keys are visited twice: pass 1 finds (max, sum), pass 2
// forms p and accumulates p V. A workgroup owns 16 query positions of one KV head; wave w is
// query head 4 g + w. Products run on v_mfma_f32_16x16x32_bf16 (query rows x keys, then
// query rows x head dims); keys are staged 64 at a time, V transposed for its B operand.

constexpr int kAtKeys = 64;
constexpr int kKsPitch = kHd + 8;
constexpr int kVtPitch = kAtKeys + 8;
constexpr int kPtPitch = kAtKeys + 8;

__global__ __launch_bounds__(256, 2) void attn_prefill_kernel(DfAttnPrefillArgs p) {
  __shared__ __align__(16) uint16_t Ks[kAtKeys * kKsPitch];
  __shared__ __align__(16) uint16_t Vt[kHd * kVtPitch];
  __shared__ __align__(16) uint16_t Pt[4][16 * kPtPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.y, h = g * 4 + wave;
  const int t0 = blockIdx.x * 16;
  const int rq = lane & 15, kq = lane >> 4;
  // A operands of q . k: row rq, dims 32 ds + 8 kq .. + 8
  uint4 qa[8];
  {
    const int t = t0 + rq;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
      qa[ds] = t < p.tokens
                   ? *reinterpret_cast<const uint4*>(p.q + ((size_t)t * p.num_q_heads + h) * kHd + ds * 32 + kq * 8)
                   : make_uint4(0u, 0u, 0u, 0u);
  }
  const int last_t = min(t0 + 16, p.tokens) - 1;
  const int nkeys = p.pos0 + last_t + 1;  // keys any row of the block attends
  const int nkb = (nkeys + kAtKeys - 1) / kAtKeys;
  const uint16_t* kbase = p.k_cache + (size_t)g * p.max_len * kHd;
  const uint16_t* vbase = p.v_cache + (size_t)g * p.max_len * kHd;
  // this lane's rows of the 16 x 16 products: 4 kq + r, at positions pos0 + t0 + 4 kq + r
  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
  }

  // Key block kb's K (and V) rows: loaded into registers one block ahead, stored into LDS
  // once the previous block's products are done with it. V is stored transposed (Vt[d][key],
  // the B operand of p V): thread (dim pair dp = tid % 128, half kh = tid / 128) loads dims
  // 2 dp, 2 dp + 1 of keys 32 kh + 8 q + j (4-byte loads, coalesced across the lanes) and
  // writes each dim's 8 keys with one 16-byte store.
  uint4 kr[8];
  uint32_t vr[32];
  auto load_rows = [&](uint4 (&rr)[8], const uint16_t* src, int kb) {  // K rows
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // 64 keys x 32 chunks of 16 bytes
      const int ch = tid + 256 * i, key = ch >> 5, cc = ch & 31;
      const int kg = kb * kAtKeys + key;
      rr[i] = make_uint4(0u, 0u, 0u, 0u);
      if (kg < nkeys) rr[i] = *reinterpret_cast<const uint4*>(src + (size_t)kg * kHd + cc * 8);
    }
  };
  auto put_k = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ch = tid + 256 * i, key = ch >> 5, cc = ch & 31;
      *reinterpret_cast<uint4*>(&Ks[key * kKsPitch + cc * 8]) = kr[i];
    }
  };
  const int vdp = tid & 127, vkh = tid >> 7;
  auto load_v = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int kg = kb * kAtKeys + 32 * vkh + i;
      vr[i] = kg < nkeys ? *reinterpret_cast<const uint32_t*>(vbase + (size_t)kg * kHd + 2 * vdp) : 0u;
    }
  };
  auto put_v = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t* w = vr + 8 * q;
      const uint4 lo = make_uint4((w[0] & 0xFFFFu) | (w[1] << 16), (w[2] & 0xFFFFu) | (w[3] << 16),
                                  (w[4] & 0xFFFFu) | (w[5] << 16), (w[6] & 0xFFFFu) | (w[7] << 16));
      const uint4 hi = make_uint4((w[0] >> 16) | (w[1] & 0xFFFF0000u), (w[2] >> 16) | (w[3] & 0xFFFF0000u),
                                  (w[4] >> 16) | (w[5] & 0xFFFF0000u), (w[6] >> 16) | (w[7] & 0xFFFF0000u));
      const int key0 = 32 * vkh + 8 * q;
      *reinterpret_cast<uint4*>(&Vt[(2 * vdp) * kVtPitch + key0]) = lo;
      *reinterpret_cast<uint4*>(&Vt[(2 * vdp + 1) * kVtPitch + key0]) = hi;
    }
  };
  // scores of key block kb for this lane: s[sb][r] (key kb*64 + 16 sb + lane % 16)
  auto scores = [&](int kb, float (&s)[4][4]) {
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      df_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) {
        const uint4 b = *reinterpret_cast<const uint4*>(&Ks[(sb * 16 + rq) * kKsPitch + ds * 32 + kq * 8]);
        acc = mfma(qa[ds], b, acc);
      }
      const int key = kb * kAtKeys + sb * 16 + rq;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = p.pos0 + t0 + kq * 4 + r;
        s[sb][r] = key <= pos ? round_bf(round_bf(acc[r]) * p.scale) : -INFINITY;
      }
    }
  };

  // ---- pass 1: row max and sum --------------------------------------------------------
  load_rows(kr, kbase, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    put_k();
    __syncthreads();
    if (kb + 1 < nkb) load_rows(kr, kbase, kb + 1);
    float s[4][4];
    scores(kb, s);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float mx = fmaxf(fmaxf(s[0][r], s[1][r]), fmaxf(s[2][r], s[3][r]));
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float mn = fmaxf(m[r], mx);
      float sum = 0.0f;
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) sum += s[sb][r] == -INFINITY ? 0.0f : expf(s[sb][r] - mn);
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
      l[r] = (m[r] == -INFINITY ? 0.0f : l[r] * expf(m[r] - mn)) + sum;
      m[r] = mn;
    }
    __syncthreads();
  }

  // ---- pass 2: p = bf16(exp(s - max) / sum), o += p V ----------------------------------
  df_f32x4 o[16];
#pragma unroll
  for (int db = 0; db < 16; ++db) o[db] = df_f32x4{0.f, 0.f, 0.f, 0.f};
  uint16_t* pt = Pt[wave];
  load_rows(kr, kbase, 0);
  load_v(0);
  for (int kb = 0; kb < nkb; ++kb) {
    put_k();
    put_v();
    __syncthreads();
    if (kb + 1 < nkb) {
      load_rows(kr, kbase, kb + 1);
      load_v(kb + 1);
    }
    float s[4][4];
    scores(kb, s);
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = s[sb][r] == -INFINITY ? 0.0f : expf(s[sb][r] - m[r]) / l[r];
        pt[(kq * 4 + r) * kPtPitch + sb * 16 + rq] = f2bf(pr);
      }
    __syncthreads();  // p rows are read back by other lanes of the wave in the A layout
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint4 pa = *reinterpret_cast<const uint4*>(&pt[rq * kPtPitch + ks * 32 + kq * 8]);
#pragma unroll
      for (int db = 0; db < 16; ++db) {
        const uint4 b = *reinterpret_cast<const uint4*>(&Vt[(db * 16 + rq) * kVtPitch + ks * 32 + kq * 8]);
        o[db] = mfma(pa, b, o[db]);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: bf16(o) * bf16(gate_fn(gate)) ----------------------------------------
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + kq * 4 + r;
    if (t >= p.tokens) continue;
    const uint16_t* gr = p.gate + (size_t)t * p.ld_gate + h * p.gate_head_stride;
    uint16_t* orow = p.out + (size_t)t * p.ld_out + h * kHd;
#pragma unroll
    for (int db = 0; db < 16; ++db) {
      const int d = db * 16 + rq;
      const float gx = bf2f(gr[d]);
      const float gv = round_bf(p.gate_kind == 0 ? sigmoid(gx) : silu(gx));
      orow[d] = f2bf(round_bf(o[db][r]) * gv);
    }
  }
}

}  // namespace pf
}  // namespace df

using namespace df;
using namespace df::pf;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

extern "C" {

int df_int4_gemm(const DfInt4GemmArgs* a, hipStream_t stream) {
  if (!a || !a->x || !a->w || !a->s || !a->out || a->M < 1 || a->K < 256 || a->K % 256 || a->N < 16 || a->N % 16)
    return DF_BAD_ARGUMENT;
  if (a->epilogue != DF_EPI_STORE && a->epilogue != DF_EPI_SWIGLU) return DF_BAD_ARGUMENT;
  if (a->epilogue == DF_EPI_SWIGLU && a->N % 32) return DF_BAD_ARGUMENT;
  const int out_cols = a->epilogue == DF_EPI_SWIGLU ? a->N / 2 : a->N;
  if (a->ldx < a->K || a->ldx % 8 || a->ldo < out_cols || !aligned16(a->x) || !aligned16(a->w))
    return DF_BAD_ARGUMENT;
  const dim3 grid((a->N / 16 + kGmTiles - 1) / kGmTiles, (a->M + kGmBM - 1) / kGmBM);
  if (grid.y > 65535) return DF_BAD_ARGUMENT;
  if (a->epilogue == DF_EPI_SWIGLU)
    hipLaunchKernelGGL(int4_gemm_kernel<DF_EPI_SWIGLU>, grid, dim3(256), 0, stream, *a);
  else
    hipLaunchKernelGGL(int4_gemm_kernel<DF_EPI_STORE>, grid, dim3(256), 0, stream, *a);
  DF_RETURN_LAUNCH_STATUS();
}

int df_causal_conv_prefill(const uint16_t* x, int ldx, int tokens, int channels, const uint16_t* weight,
                           uint16_t* ring, int pos0, uint16_t* out, int ldo, hipStream_t stream) {
  if (!x || !weight || !ring || !out || tokens < 1 || channels < 1 || ldx < channels || ldo < channels || pos0 < 0 ||
      (reinterpret_cast<uintptr_t>(weight) & 7) || tokens > 65535)
    return DF_BAD_ARGUMENT;
  const int cb = (channels + 255) / 256;
  hipLaunchKernelGGL(conv_seq_kernel, dim3(cb, tokens), dim3(256), 0, stream, x, ldx, tokens, channels, weight, ring,
                     pos0, out, ldo);
  hipLaunchKernelGGL(conv_ring_update_kernel, dim3(cb), dim3(256), 0, stream, x, ldx, tokens, channels, ring, pos0);
  DF_RETURN_LAUNCH_STATUS();
}

size_t df_delta_rule_prefill_workspace_bytes(int tokens, int num_v_heads) {
  if (tokens < 1 || num_v_heads < 1) return 0;
  const size_t chunks = (size_t)(tokens + kCk - 1) / kCk;
  return (chunks * num_v_heads * (kPrepMats * (size_t)kMat + 1)) * sizeof(float);
}

int df_delta_rule_prefill(const DfDeltaPrefillArgs* a, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!a || !a->mixed || !a->a || !a->b || !a->A_log || !a->dt_bias || !a->state || !a->out || a->tokens < 1)
    return DF_BAD_ARGUMENT;
  if (a->num_k_heads < 1 || a->num_v_heads < 1 || a->num_v_heads % a->num_k_heads) return DF_BAD_ARGUMENT;
  const int channels = 2 * a->num_k_heads * kDk + a->num_v_heads * kDk;
  if (a->ld_mixed < channels || a->ld_mixed % 2 || a->ld_out < a->num_v_heads * kDk || a->ld_out % 4 ||
      a->ld_ab < a->num_v_heads || (reinterpret_cast<uintptr_t>(a->mixed) & 3) ||
      (reinterpret_cast<uintptr_t>(a->out) & 7) || (reinterpret_cast<uintptr_t>(a->state) & 15))
    return DF_BAD_ARGUMENT;
  if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 15) ||
      workspace_bytes < df_delta_rule_prefill_workspace_bytes(a->tokens, a->num_v_heads))
    return DF_WORKSPACE_TOO_SMALL;
  const int chunks = (a->tokens + kCk - 1) / kCk;
  float* scratch = reinterpret_cast<float*>(workspace);
  hipLaunchKernelGGL(delta_prep_kernel, dim3(chunks, a->num_v_heads), dim3(256), 0, stream, *a, scratch);
  hipLaunchKernelGGL(delta_scan_kernel, dim3(a->num_v_heads, kDk / kScanVs), dim3(256), 0, stream, *a,
                     static_cast<const float*>(scratch));
  DF_RETURN_LAUNCH_STATUS();
}

int df_gated_rms_norm_rows(const uint16_t* x, int ldx, const uint16_t* z, int ldz, const uint16_t* weight, float eps,
                           int tokens, int heads, uint16_t* out, int ldo, hipStream_t stream) {
  if (!x || !z || !weight || !out || tokens < 1 || heads < 1 || ldx < heads * 128 || ldz < heads * 128 ||
      ldo < heads * 128 || ldx % 2 || ldz % 2 || ldo % 2 || (reinterpret_cast<uintptr_t>(x) & 3) ||
      (reinterpret_cast<uintptr_t>(z) & 3) || (reinterpret_cast<uintptr_t>(out) & 3) ||
      (reinterpret_cast<uintptr_t>(weight) & 3))
    return DF_BAD_ARGUMENT;
  const long units = (long)tokens * heads;
  hipLaunchKernelGGL(gated_norm_rows_kernel, dim3((units + 3) / 4), dim3(256), 0, stream, x, ldx, z, ldz, weight, eps,
                     tokens, heads, out, ldo);
  DF_RETURN_LAUNCH_STATUS();
}

int df_qk_norm_rope_prefill(const DfQkPrefillArgs* a, hipStream_t stream) {
  if (!a || !a->proj || !a->q_norm || !a->k_norm || !a->inv_freq || !a->q_out || !a->k_cache || !a->v_cache ||
      a->tokens < 1 || a->num_q_heads < 1 || a->num_kv_heads < 1 || a->pos0 < 0 ||
      a->pos0 + a->tokens > a->max_len)
    return DF_BAD_ARGUMENT;
  const int half = a->rotary_dim / 2;
  if (a->rotary_dim > kHd || half < 4 || (half & (half - 1))) return DF_BAD_ARGUMENT;
  if (a->ld_proj % 4 || a->k_col % 4 || a->v_col % 4 || (reinterpret_cast<uintptr_t>(a->proj) & 7) ||
      a->ld_proj < a->num_q_heads * 2 * kHd || a->k_col + a->num_kv_heads * kHd > a->ld_proj ||
      a->v_col + a->num_kv_heads * kHd > a->ld_proj)
    return DF_BAD_ARGUMENT;
  const long units = (long)a->tokens * (a->num_q_heads + a->num_kv_heads);
  hipLaunchKernelGGL(qk_rows_kernel, dim3((units + 3) / 4), dim3(256), 0, stream, *a);
  DF_RETURN_LAUNCH_STATUS();
}

int df_attention_prefill(const DfAttnPrefillArgs* a, hipStream_t stream) {
  if (!a || !a->q || !a->k_cache || !a->v_cache || !a->gate || !a->out || a->tokens < 1 || a->pos0 < 0 ||
      a->pos0 + a->tokens > a->max_len || a->num_kv_heads < 1 || a->num_q_heads != 4 * a->num_kv_heads)
    return DF_BAD_ARGUMENT;
  if (!aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache) || a->ld_out < a->num_q_heads * kHd ||
      a->gate_kind < 0 || a->gate_kind > 1)
    return DF_BAD_ARGUMENT;
  const int qb = (a->tokens + 15) / 16;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(qb, a->num_kv_heads), dim3(256), 0, stream, *a);
  DF_RETURN_LAUNCH_STATUS();
}

}  // extern "C"
