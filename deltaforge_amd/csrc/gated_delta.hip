// One decode token of Gated DeltaNet's middle section, fused, for gfx950.
//
// Per workgroup (batch b, value head h, value slice vs of 32 columns):
//   1. issue the loads of its fp32 state slice S[b,h,:,vs*32:+32] (16 KB) first;
//   2. 4-tap causal conv + SiLU for the 128 q and 128 k channels of key head h / groups
//      and its 32 v channels (fp32 sum in tap order, rounded to bf16, SiLU, bf16:
//      kernels/inline_causal_conv.py:114-123), and write the new history;
//   3. q, k L2-norm in fp32, q / sqrt(Dk); beta = bf16(sigmoid(b)); g = -exp(A_log)
//      softplus(a + dt_bias) (reference.py:528-532, 403-404, 432-437);
//   4. S *= exp(g); r = k^T S; delta = (v - r) beta; S += k delta^T; o = q^T S
//      (reference.py:450-458), with the state update rounded as the reference rounds it
//      (separate products and sums, no fused multiply-add);
//   5. store S and o (bf16).
//
// Conv history: mode 0 reads [B][C][3] and writes a separate [B][C][3] buffer; mode 1 is a
// 4-slot ring indexed by the device position, so the slot written (position % 4) is never
// one of the three read and workgroups sharing a key head's q/k channels cannot race.
#include "common.h"
#include "deltaforge_hip.h"

namespace df {

constexpr int kDk = 128;
constexpr int kVSlice = 32;
constexpr int kDeltaThreads = 256;

// The rule on one workgroup's 128 x 32 fp32 state slice, S held 4 rows x 4 columns per
// thread (thread t: rows 4 (t >> 3) .. +3, columns 4 (t & 7) .. +3), with q/k (128) and the
// slice's v (32) in LDS: S *= eg; r = k^T S; delta = (v - r) beta; S += k delta^T; o = q^T S
// (reference.py:450-458, in the reference's rounding: separate products and sums, no fused
// multiply-add). The updated slice goes to `sout` (row stride `ld`), o to store(col, o) for
// the slice's 32 columns.
template <class Store>
DF_DEVICE void delta_rule_slice(float4 (&S)[4], float* sout, int ld, const float* q_s, const float* k_s,
                                const float* v_s, float eg, float beta, float (&red)[2][4][kVSlice], int tid,
                                Store&& store) {
#pragma clang fp contract(off)
  const int lane = tid & 63, wave = tid >> 6;
  const int c4 = tid & 7, rg = tid >> 3;
  // Decay and recall.
  float kr[4], qr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    kr[r] = k_s[rg * 4 + r];
    qr[r] = q_s[rg * 4 + r];
  }
  float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    S[r].x = S[r].x * eg;
    S[r].y = S[r].y * eg;
    S[r].z = S[r].z * eg;
    S[r].w = S[r].w * eg;
    part[0] += S[r].x * kr[r];
    part[1] += S[r].y * kr[r];
    part[2] += S[r].z * kr[r];
    part[3] += S[r].w * kr[r];
  }
  // Reduce over the 8 row groups of a wave (lanes c4 + 8j), then over the 4 waves.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = part[j];
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    part[j] = v;
  }
  if (lane < 8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[0][wave][c4 * 4 + j] = part[j];
  }
  __syncthreads();
  float delta[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = c4 * 4 + j;
    const float recalled = red[0][0][col] + red[0][1][col] + red[0][2][col] + red[0][3][col];
    delta[j] = (v_s[col] - recalled) * beta;
  }

  // Rank-1 update and readout.
  float outp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float kv0 = kr[r] * delta[0], kv1 = kr[r] * delta[1], kv2 = kr[r] * delta[2], kv3 = kr[r] * delta[3];
    S[r].x = S[r].x + kv0;
    S[r].y = S[r].y + kv1;
    S[r].z = S[r].z + kv2;
    S[r].w = S[r].w + kv3;
    outp[0] += S[r].x * qr[r];
    outp[1] += S[r].y * qr[r];
    outp[2] += S[r].z * qr[r];
    outp[3] += S[r].w * qr[r];
    *reinterpret_cast<float4*>(sout + (size_t)(rg * 4 + r) * ld) = S[r];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = outp[j];
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    outp[j] = v;
  }
  if (lane < 8) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[1][wave][c4 * 4 + j] = outp[j];
  }
  __syncthreads();
  if (tid < kVSlice) store(tid, red[1][0][tid] + red[1][1][tid] + red[1][2][tid] + red[1][3][tid]);
}


__global__ __launch_bounds__(kDeltaThreads) void gated_delta_step_kernel(DfGatedDeltaArgs p) {
#pragma clang fp contract(off)
  __shared__ float q_s[kDk], k_s[kDk], v_s[kVSlice];
  __shared__ float red[2][4][kVSlice];
  __shared__ float scal[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int vsplits = p.head_v_dim / kVSlice;
  const int vs = blockIdx.x % vsplits;
  const int h = (blockIdx.x / vsplits) % p.num_v_heads;
  const int b = blockIdx.x / (vsplits * p.num_v_heads);
  const int groups = p.num_v_heads / p.num_k_heads;
  const int kh = h / groups;
  const int key_dim = p.num_k_heads * kDk;
  const int C = 2 * key_dim + p.num_v_heads * p.head_v_dim;

  // 1. State slice loads: thread -> 4 rows x 4 columns (float4 per row).
  const int c4 = tid & 7, rg = tid >> 3;  // rg: rows 4*rg .. 4*rg+3
  float* sbase = p.state + (((size_t)b * p.num_v_heads + h) * kDk) * p.head_v_dim + vs * kVSlice + c4 * 4;
  float4 S[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) S[r] = *reinterpret_cast<const float4*>(sbase + (size_t)(rg * 4 + r) * p.head_v_dim);

  // 2. Conv for 256 q/k channels (one per thread) and 32 v channels (threads 0..31).
  int slot_w = 0, slot0 = 0, slot1 = 0, slot2 = 0;
  if (p.conv_mode == 1) {
    const int pos = *p.position;
    slot_w = pos & 3;
    slot0 = (pos + 1) & 3;
    slot1 = (pos + 2) & 3;
    slot2 = (pos + 3) & 3;
  }
  auto conv = [&](int c, bool write_hist) -> float {
    const float x = bf2f(p.qkv[(size_t)b * p.ld_qkv + c]);
    const uint16_t* w = p.conv_w + (size_t)c * 4;
    float h0, h1, h2;
    if (p.conv_mode == 1) {
      const uint16_t* ring = p.conv_ring + ((size_t)b * C + c) * 4;
      h0 = bf2f(ring[slot0]);
      h1 = bf2f(ring[slot1]);
      h2 = bf2f(ring[slot2]);
    } else {
      const uint16_t* hist = p.conv_in + ((size_t)b * C + c) * 3;
      h0 = bf2f(hist[0]);
      h1 = bf2f(hist[1]);
      h2 = bf2f(hist[2]);
    }
    float acc = h0 * bf2f(w[0]);
    acc = acc + h1 * bf2f(w[1]);
    acc = acc + h2 * bf2f(w[2]);
    acc = acc + x * bf2f(w[3]);
    if (write_hist) {
      if (p.conv_mode == 1) {
        p.conv_ring[((size_t)b * C + c) * 4 + slot_w] = p.qkv[(size_t)b * p.ld_qkv + c];
      } else {
        uint16_t* o = p.conv_out + ((size_t)b * C + c) * 3;
        o[0] = f2bf(h1);
        o[1] = f2bf(h2);
        o[2] = p.qkv[(size_t)b * p.ld_qkv + c];
      }
    }
    return round_bf(silu(round_bf(acc)));
  };
  const bool owns_qk = (h % groups == 0) && vs == 0;
  {
    const int which = tid >> 7, e = tid & 127;  // 0: q, 1: k
    const int c = which * key_dim + kh * kDk + e;
    const float v = conv(c, owns_qk);
    if (which == 0) q_s[e] = v; else k_s[e] = v;
  }
  if (tid < kVSlice) v_s[tid] = conv(2 * key_dim + h * p.head_v_dim + vs * kVSlice + tid, true);

  // 3. Gates (thread 0) and the two L2 norms (waves 0 and 2 hold q and k).
  if (tid == 0) {
    const float a = bf2f(p.a[(size_t)b * p.ld_ab + h]);
    const float bb = bf2f(p.b[(size_t)b * p.ld_ab + h]);
    const float beta = round_bf(sigmoid(bb));
    const float g = -expf(bf2f(p.A_log[h])) * softplus(a + bf2f(p.dt_bias[h]));
    scal[0] = expf(g);
    scal[1] = beta;
  }
  __syncthreads();
  if (wave == 0 || wave == 2) {
    float* vec = wave == 0 ? q_s : k_s;
    const float x0 = vec[lane * 2], x1 = vec[lane * 2 + 1];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = 1.0f / sqrtf(ss + 1e-6f);
    float y0 = x0 * r, y1 = x1 * r;
    if (wave == 0) {
      const float scale = sqrtf(static_cast<float>(kDk));
      y0 = y0 / scale;
      y1 = y1 / scale;
    }
    vec[lane * 2] = y0;
    vec[lane * 2 + 1] = y1;
  }
  __syncthreads();

  // 4-5. The rule itself, shared with delta_rule_step_kernel.
  delta_rule_slice(S, sbase, p.head_v_dim, q_s, k_s, v_s, scal[0], scal[1], red, tid,
                   [&](int col, float o) {
                     p.out[((size_t)b * p.num_v_heads + h) * p.head_v_dim + vs * kVSlice + col] = f2bf(o);
                   });
}

// One delta-rule step on already-normalised fp32 inputs (the reference's
// deltaforge::delta_rule_step, kernels/gated_delta_step.py:109-186): per workgroup
// (batch b, head h, value slice vs of 32 columns), S = state_in slice; S *= exp(g);
// r = k^T S; delta = (v - r) beta; S += k delta^T; o = q^T S; state_out slice = S, out = o
// (fp32). state_out may alias state_in: each workgroup reads its slice before writing it.
__global__ __launch_bounds__(kDeltaThreads) void delta_rule_step_kernel(DfDeltaRuleArgs p) {
#pragma clang fp contract(off)
  __shared__ float q_s[kDk], k_s[kDk], v_s[kVSlice];
  __shared__ float red[2][4][kVSlice];
  const int tid = threadIdx.x;
  const int vsplits = p.value_dim / kVSlice;
  const int vs = blockIdx.x % vsplits;
  const int bh = blockIdx.x / vsplits;  // b * heads + h
  const int c4 = tid & 7, rg = tid >> 3;
  const size_t head = (size_t)bh * kDk * p.value_dim;
  const float* sin = p.state_in + head + vs * kVSlice + c4 * 4;
  float4 S[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) S[r] = *reinterpret_cast<const float4*>(sin + (size_t)(rg * 4 + r) * p.value_dim);
  if (tid < kDk) {
    q_s[tid] = p.query[(size_t)bh * kDk + tid];
    k_s[tid] = p.key[(size_t)bh * kDk + tid];
  }
  if (tid < kVSlice) v_s[tid] = p.value[(size_t)bh * p.value_dim + vs * kVSlice + tid];
  const float eg = expf(p.g[bh]);
  const float beta = p.beta[bh];
  __syncthreads();
  float* sout = p.state_out + head + vs * kVSlice + c4 * 4;
  delta_rule_slice(S, sout, p.value_dim, q_s, k_s, v_s, eg, beta, red, tid,
                   [&](int col, float o) { p.out[(size_t)bh * p.value_dim + vs * kVSlice + col] = o; });
}

// The inputs of delta_rule_step_kernel from one token of Gated DeltaNet, as the reference
// prepares them around its standalone step (kernels/gated_delta_step.py:189-213, 245-256):
// per workgroup (batch b, value head h; key head h / groups), wave 0 L2-normalises q and
// scales it by Dk^-1/2, wave 1 L2-normalises k, both in fp32 from the bf16 conv output; v is
// widened to fp32; beta = fp32(bf16(sigmoid(b))); g = -exp(A_log) softplus(a + dt_bias).
__global__ __launch_bounds__(2 * 64) void delta_step_inputs_kernel(DfDeltaInputsArgs p) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x % p.num_v_heads, b = blockIdx.x / p.num_v_heads;
  const int kh = h / (p.num_v_heads / p.num_k_heads);
  const int key_dim = p.num_k_heads * kDk;
  const uint16_t* row = p.mixed + (size_t)b * p.ld_mixed;
  const size_t bh = (size_t)b * p.num_v_heads + h;

  const uint16_t* src = row + wave * key_dim + kh * kDk;  // wave 0: q, wave 1: k
  const float x0 = bf2f(src[2 * lane]), x1 = bf2f(src[2 * lane + 1]);
  const float r = 1.0f / sqrtf(wave_sum(x0 * x0 + x1 * x1) + p.eps);
  float y0 = x0 * r, y1 = x1 * r;
  float* dst = (wave == 0 ? p.query : p.key) + bh * kDk;
  if (wave == 0) {
    const float scale = sqrtf(static_cast<float>(kDk));
    y0 = y0 / scale;
    y1 = y1 / scale;
  }
  dst[2 * lane] = y0;
  dst[2 * lane + 1] = y1;

  const uint16_t* vsrc = row + 2 * key_dim + (size_t)h * p.head_v_dim;
  for (int e = tid; e < p.head_v_dim; e += 2 * 64) p.value[bh * p.head_v_dim + e] = bf2f(vsrc[e]);
  if (tid == 0) {
    const float a = bf2f(p.a[(size_t)b * p.ld_ab + h]);
    const float bb = bf2f(p.b[(size_t)b * p.ld_ab + h]);
    p.beta[bh] = round_bf(sigmoid(bb));
    p.g[bh] = -expf(bf2f(p.A_log[h])) * softplus(a + bf2f(p.dt_bias[h]));
  }
}

}  // namespace df

extern "C" int df_delta_step_inputs(const DfDeltaInputsArgs* args, hipStream_t stream) {
  using namespace df;
  if (!args) return DF_BAD_ARGUMENT;
  const DfDeltaInputsArgs& a = *args;
  if (a.batch < 1 || a.head_k_dim != kDk || a.head_v_dim < 1 || a.num_k_heads < 1 || a.num_v_heads < 1 ||
      a.num_v_heads % a.num_k_heads || !a.mixed || !a.a || !a.b || !a.A_log || !a.dt_bias || !a.query ||
      !a.key || !a.value || !a.g || !a.beta)
    return DF_BAD_ARGUMENT;
  if (a.ld_mixed < 2 * a.num_k_heads * kDk + a.num_v_heads * a.head_v_dim || a.ld_ab < a.num_v_heads)
    return DF_BAD_ARGUMENT;
  hipLaunchKernelGGL(delta_step_inputs_kernel, dim3(a.batch * a.num_v_heads), dim3(2 * 64), 0, stream, a);
  DF_RETURN_LAUNCH_STATUS();
}

extern "C" int df_gated_delta_step(const DfGatedDeltaArgs* args, hipStream_t stream) {
  using namespace df;
  if (!args) return DF_BAD_ARGUMENT;
  const DfGatedDeltaArgs& a = *args;
  if (a.batch < 1 || a.head_k_dim != kDk || a.head_v_dim != kDk || a.num_k_heads < 1 ||
      a.num_v_heads % a.num_k_heads || !a.qkv || !a.a || !a.b || !a.A_log || !a.dt_bias || !a.conv_w ||
      !a.state || !a.out)
    return DF_BAD_ARGUMENT;
  if (a.conv_mode == 0) {
    if (!a.conv_in || !a.conv_out || a.conv_in == a.conv_out) return DF_BAD_ARGUMENT;
  } else if (a.conv_mode == 1) {
    if (!a.conv_ring || !a.position) return DF_BAD_ARGUMENT;
  } else {
    return DF_BAD_ARGUMENT;
  }
  const int C = 2 * a.num_k_heads * kDk + a.num_v_heads * a.head_v_dim;
  if (a.ld_qkv < C || a.ld_ab < a.num_v_heads) return DF_BAD_ARGUMENT;
  const int grid = a.batch * a.num_v_heads * (a.head_v_dim / kVSlice);
  hipLaunchKernelGGL(gated_delta_step_kernel, dim3(grid), dim3(kDeltaThreads), 0, stream, a);
  DF_RETURN_LAUNCH_STATUS();
}

extern "C" int df_delta_rule_step(const DfDeltaRuleArgs* args, hipStream_t stream) {
  using namespace df;
  if (!args) return DF_BAD_ARGUMENT;
  const DfDeltaRuleArgs& a = *args;
  if (a.batch < 1 || a.heads < 1 || a.key_dim != kDk || a.value_dim < kVSlice || a.value_dim % kVSlice ||
      !a.state_in || !a.state_out || !a.query || !a.key || !a.value || !a.g || !a.beta || !a.out)
    return DF_BAD_ARGUMENT;
  const int grid = a.batch * a.heads * (a.value_dim / kVSlice);
  hipLaunchKernelGGL(delta_rule_step_kernel, dim3(grid), dim3(kDeltaThreads), 0, stream, a);
  DF_RETURN_LAUNCH_STATUS();
}
