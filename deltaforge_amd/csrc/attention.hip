// Single-token gated GQA attention with split-KV for gfx950.
//
// Grid (split, kv_head, batch); 256 threads = 4 waves = the 4 query heads sharing the KV
// head (reference gqa_decode.py:95: q head h reads KV head h / groups), so every K/V byte is
// read once per split.
//
//   prologue  wave w: q_norm (RMSNorm(1+w) over 256) then partial RoPE of query head
//             4*kv + w, in the reference's bf16 op order (reference.py:632-643,
//             137-149, 189-200 with cos/sin = bf16(cos(position * inv_freq))); wave 0 does
//             the same for the new key, wave 1 stages the new value. The split that owns
//             `position` writes them into the cache (reference.py:645-650) and uses the
//             staged copies for that key.
//   per tile  64 keys: QK on MFMA (16x16x32 bf16, query heads as rows, keys as columns,
//             fp32 scores x head_dim^-0.5); fp32 online softmax per head; PV on VALU
//             with each lane owning 4 output dims for all 4 heads.
//   merge     each split writes (acc[256], m, l) per head with write-through stores; a second
//             kernel (attn_merge_kernel: one workgroup per batch row, query head and 64 output
//             dims, its 4 waves splitting the splits) combines them with the log-sum-exp
//             identity (flash_decode_splitkv.py:135-174), rounds to bf16 and applies the bf16
//             output gate (reference.py:558-568, 674-676). A single split finishes in place.
//
// Scores and probabilities stay fp32 (the reference rounds both to bf16); this is the
// more accurate function and is checked against the reference within tolerance.
#include "common.h"
#include "deltaforge_hip.h"

#include <mutex>

namespace df {

constexpr int kHd = 256;
constexpr int kQPerKv = 4;
constexpr int kTile = 64;
constexpr int kMaxSplits = 256;

struct AttnWs {
  float* acc;  // [B][Hq][S][256]
  float* ml;   // [B][Hq][S][2]
};

// Workspace layout: the split partials only. Every call writes all of its partials before
// the merge kernel reads them, so a workspace needs no clearing and serves calls of any shape.
inline AttnWs attn_ws(void* base, int batch, int hq, int splits) {
  AttnWs w;
  w.acc = reinterpret_cast<float*>(base);
  w.ml = w.acc + (size_t)batch * hq * splits * kHd;
  return w;
}

// RMSNorm(1+w) over 256 dims held 4 per lane, then partial RoPE over the first `rot` dims.
// The lane's norm weights (4 bf16) and inverse frequencies (of its dims' rotary pairs) come
// loaded, so the caller can issue those loads ahead of others.
DF_DEVICE void norm_rope4(float x[4], uint2 wraw, const float (&inv)[4], float eps, int rot, float posf, int lane) {
  const uint16_t norm_w4[4] = {static_cast<uint16_t>(wraw.x), static_cast<uint16_t>(wraw.x >> 16),
                               static_cast<uint16_t>(wraw.y), static_cast<uint16_t>(wraw.y >> 16)};
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(kHd) + eps);
  float n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float scaled = x[i] * r;
    n[i] = round_bf(scaled * (1.0f + bf2f(norm_w4[i])));
  }
  const int half = rot / 2;
  // dim d's partner d +- half sits half/4 lanes away; the xor reaches lane +- half/4 because
  // the launcher admits only rotary dims with rot/8 a power of two
  float partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(n[i], half / 4, 64);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dim = lane * 4 + i;
    if (dim < rot) {
      const float ang = posf * inv[i];
      const float c = round_bf(cosf(ang)), s = round_bf(sinf(ang));
      const float rotated = dim < half ? -partner[i] : partner[i];
      x[i] = round_bf(round_bf(n[i] * c) + round_bf(rotated * s));
    } else {
      x[i] = n[i];
    }
  }
}

struct NormIn {
  uint2 w;       // the lane's 4 norm weights (bf16)
  float inv[4];  // inverse frequency of each of its dims' rotary pairs
};
DF_DEVICE NormIn norm_in(const uint16_t* norm_w, const float* inv_freq, int rot, int lane) {
  NormIn n;
  n.w = *reinterpret_cast<const uint2*>(norm_w + lane * 4);
  const int half = rot / 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) n.inv[i] = inv_freq[(lane * 4 + i) % half];
  return n;
}

// What the plain entry point (no prologue, no gate: df_split_kv_decode_attention) changes in
// the kernel: the query comes ready as [B][Hq][D], every one of key_len cached keys is
// attended (no new key), the caller's scale applies, and the merged output is stored as is.
struct PlainAttn {
  int key_len;
  float scale;
};

template <bool PLAIN>
__global__ __launch_bounds__(256) void attn_decode_kernel(DfAttnDecodeArgs p, AttnWs ws, PlainAttn pl) {
  __shared__ __align__(16) uint16_t q_s[kQPerKv][kHd];
  __shared__ __align__(16) uint16_t knew[kHd];
  __shared__ __align__(16) uint16_t vnew[kHd];
  __shared__ float sc[kQPerKv][kTile];
  __shared__ float alpha_s[kQPerKv];
  __shared__ float red[kQPerKv][kQPerKv][kHd];
  __shared__ float ml_s[kQPerKv][2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int S = p.splits;
  // PLAIN: no new key (pos -1 matches no cache row), key_len keys.
  const int pos = PLAIN ? -1 : *p.position;
  // A position past the cache would write out of bounds; the host cannot see the device
  // scalar, so every workgroup refuses here (the output is left unwritten).
  if (!PLAIN && (pos < 0 || pos >= p.max_len)) return;
  const int nkeys = PLAIN ? pl.key_len : pos + 1;
  const int per = (nkeys + S - 1) / S;
  const int j0 = min(split * per, nkeys);
  const int j1 = min(j0 + per, nkeys);
  const float posf = static_cast<float>(pos);
  const size_t kv_base = ((size_t)b * p.num_kv_heads + kvh) * p.max_len;
  const int col = lane & 15, slot = lane >> 4;

  // A tile's K and V rows, all loads issued before any is used (one memory round trip): keys
  // past the split load row j1 - 1 instead (in bounds, ignored), and the new position's row
  // is replaced by the staged key / value. K rows use two register sets in turn, so the next
  // tile's keys are in flight while this one is computed; a tile's V rows are loaded when the
  // previous tile is done with the V registers, and the first tile's K and V rows go out
  // during the prologue, which they do not depend on. The loads are unconditional (rows clamp
  // into [0, j1), j1 >= 1): on every path the same loads are outstanding, so the compiler's
  // waits for one register set never include a younger one.
  auto load_k = [&](int t0, uint4 (&kb)[8]) {
    const int krow = min(t0 + wave * 16 + col, j1 - 1);
    const uint16_t* kp = p.k_cache + (kv_base + krow) * kHd + slot * 8;
#pragma unroll
    for (int d = 0; d < 8; ++d) kb[d] = *reinterpret_cast<const uint4*>(kp + d * 32);
  };
  auto load_v = [&](int t0, uint2 (&vb)[16]) {
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int vrow = min(t0 + wave * 16 + jj, j1 - 1);
      vb[jj] = *reinterpret_cast<const uint2*>(p.v_cache + (kv_base + vrow) * kHd + lane * 4);
    }
  };
  // Prologue: queries, new key, new value. Its operands are loaded first and the first tile's
  // rows after them, so the prologue's waits do not include the tile (a wave's loads complete
  // in order).
  const int hq = kvh * kQPerKv + wave;
  uint16_t qe[4], ke[4] = {0, 0, 0, 0}, ve[4] = {0, 0, 0, 0};
  NormIn qn{}, kn{};
  {
    const uint16_t* src = PLAIN ? p.q + ((size_t)b * p.num_q_heads + hq) * kHd + lane * 4
                                : p.q + (size_t)b * p.ld_q + (size_t)hq * 2 * kHd + lane * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) qe[i] = src[i];
  }
  if (!PLAIN) {
    qn = norm_in(p.q_norm_w, p.inv_freq, p.rotary_dim, lane);
    if (wave == 0) {
      const uint16_t* ks = p.k + (size_t)b * p.ld_kv + (size_t)kvh * kHd + lane * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) ke[i] = ks[i];
      kn = norm_in(p.k_norm_w, p.inv_freq, p.rotary_dim, lane);
    } else if (wave == 1) {
      const uint16_t* vsrc = p.v + (size_t)b * p.ld_kv + (size_t)kvh * kHd + lane * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) ve[i] = vsrc[i];
    }
  }
  uint4 kA[8], kB[8];
  uint2 vt[16];
  load_k(j0, kA);
  load_v(j0, vt);
  if (PLAIN) {
#pragma unroll
    for (int i = 0; i < 4; ++i) q_s[wave][lane * 4 + i] = qe[i];
  } else {
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = bf2f(qe[i]);
    norm_rope4(x, qn.w, qn.inv, p.eps, p.rotary_dim, posf, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) q_s[wave][lane * 4 + i] = f2bf(x[i]);
    if (wave == 0) {
      float kx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) kx[i] = bf2f(ke[i]);
      norm_rope4(kx, kn.w, kn.inv, p.eps, p.rotary_dim, posf, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) knew[lane * 4 + i] = f2bf(kx[i]);
    } else if (wave == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) vnew[lane * 4 + i] = ve[i];
    }
  }
  __syncthreads();
  const bool owner = !PLAIN && pos >= j0 && pos < j1;
  if (owner) {
    uint16_t* kd = p.k_cache + (kv_base + pos) * kHd;
    uint16_t* vd = p.v_cache + (kv_base + pos) * kHd;
    kd[tid] = knew[tid];
    vd[tid] = vnew[tid];
  }

  const float scale = PLAIN ? pl.scale : 1.0f / sqrtf(static_cast<float>(kHd));
  float m_run = -INFINITY, l_run = 0.0f;  // for head `wave`
  float acc[kQPerKv][4];
#pragma unroll
  for (int h = 0; h < kQPerKv; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[h][i] = 0.0f;

  auto tile = [&](int t0, const uint4 (&kb)[8], const uint2 (&vb)[16]) {
    // QK: wave covers keys t0 + 16*wave + col.
    {
      const int key = t0 + wave * 16 + col;
      const bool live = key < j1;
      df_f32x4 d4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        uint4 bw = make_uint4(0u, 0u, 0u, 0u);
        if (live) bw = key == pos ? *reinterpret_cast<const uint4*>(knew + d * 32 + slot * 8) : kb[d];
        uint4 aw = make_uint4(0u, 0u, 0u, 0u);
        if (col < kQPerKv) aw = *reinterpret_cast<const uint4*>(&q_s[col][d * 32 + slot * 8]);
        d4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, aw),
                                                     __builtin_bit_cast(df_bf16x8, bw), d4, 0, 0, 0);
      }
      if (slot == 0) {
#pragma unroll
        for (int i = 0; i < kQPerKv; ++i) sc[i][wave * 16 + col] = live ? d4[i] * scale : -INFINITY;
      }
    }
    __syncthreads();
    // Online softmax for head `wave`.
    {
      const float s = sc[wave][lane];
      const float tmax = wave_max(s);
      const float m_new = fmaxf(m_run, tmax);
      float pr = 0.0f, alpha = 1.0f;
      if (m_new != -INFINITY) {
        pr = s == -INFINITY ? 0.0f : expf(s - m_new);
        alpha = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
      }
      l_run = l_run * alpha + wave_sum(pr);
      m_run = m_new;
      sc[wave][lane] = pr;
      if (lane == 0) alpha_s[wave] = alpha;
    }
    __syncthreads();
    // PV: wave handles keys t0 + 16*wave .. +15 for all heads; lane owns dims 4*lane..+3.
    {
#pragma unroll
      for (int h = 0; h < kQPerKv; ++h) {
        const float a = alpha_s[h];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[h][i] *= a;
      }
      const uint2 vn = *reinterpret_cast<const uint2*>(vnew + lane * 4);
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int key = t0 + wave * 16 + jj;
        if (key >= j1) break;
        const uint2 raw = key == pos ? vn : vb[jj];
        const float v0 = __uint_as_float(raw.x << 16), v1 = __uint_as_float(raw.x & 0xFFFF0000u);
        const float v2 = __uint_as_float(raw.y << 16), v3 = __uint_as_float(raw.y & 0xFFFF0000u);
#pragma unroll
        for (int h = 0; h < kQPerKv; ++h) {
          const float pr = sc[h][wave * 16 + jj];
          acc[h][0] += pr * v0;
          acc[h][1] += pr * v1;
          acc[h][2] += pr * v2;
          acc[h][3] += pr * v3;
        }
      }
    }
    __syncthreads();
  };
  for (int t0 = j0; t0 < j1; t0 += 2 * kTile) {
    load_k(t0 + kTile, kB);
    tile(t0, kA, vt);
    if (t0 + kTile >= j1) break;
    load_v(t0 + kTile, vt);
    load_k(t0 + 2 * kTile, kA);
    tile(t0 + kTile, kB, vt);
    if (t0 + 2 * kTile >= j1) break;
    load_v(t0 + 2 * kTile, vt);
  }

  // Combine the four waves' PV partials; publish this split's (acc, m, l) per head.
#pragma unroll
  for (int h = 0; h < kQPerKv; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][h][lane * 4 + i] = acc[h][i];
  if (lane == 0) {
    ml_s[wave][0] = m_run;
    ml_s[wave][1] = l_run;
  }
  __syncthreads();
  const int hq0 = kvh * kQPerKv;
#pragma unroll
  for (int h = 0; h < kQPerKv; ++h) {
    const float total = red[0][h][tid] + red[1][h][tid] + red[2][h][tid] + red[3][h][tid];
    const size_t row = ((size_t)b * p.num_q_heads + hq0 + h) * S + split;
    store_through(ws.acc + row * kHd + tid, total);
    if (tid == 0) {
      store_through(ws.ml + row * 2, ml_s[h][0]);
      store_through(ws.ml + row * 2 + 1, ml_s[h][1]);
    }
  }
  if (S > 1) return;  // attn_merge_kernel combines the splits
  __syncthreads();

  // One split: normalise, round, gate (the same steps as attn_merge_kernel, over S = 1).
  float* wgt = &red[0][0][0];     // reuse: [2 * kQPerKv][kMaxSplits] = 2048 of the 4096 floats
  float* den_s = &red[3][0][0];   // past them
  for (int e = tid; e < kQPerKv * S; e += 256) {
    const int h = e / S, s = e % S;
    const size_t row = ((size_t)b * p.num_q_heads + hq0 + h) * S + s;
    const float m = load_through(ws.ml + row * 2), l = load_through(ws.ml + row * 2 + 1);
    wgt[h * kMaxSplits + s] = l > 0.0f ? m : -INFINITY;
    wgt[(kQPerKv + h) * kMaxSplits + s] = l;
  }
  __syncthreads();
  {
    const int h = wave;
    float mstar = -INFINITY;
    for (int s = lane; s < S; s += 64) mstar = fmaxf(mstar, wgt[h * kMaxSplits + s]);
    mstar = wave_max(mstar);
    float den = 0.0f;
    for (int s = lane; s < S; s += 64) {
      const float m = wgt[h * kMaxSplits + s];
      const float w = m == -INFINITY ? 0.0f : expf(m - mstar);
      den += w * wgt[(kQPerKv + h) * kMaxSplits + s];
      wgt[h * kMaxSplits + s] = w;
    }
    den = wave_sum(den);
    if (lane == 0) den_s[h] = den;
  }
  __syncthreads();
#pragma unroll 1
  for (int h = 0; h < kQPerKv; ++h) {
    const float* accp = ws.acc + (((size_t)b * p.num_q_heads + hq0 + h) * S) * kHd + tid;
    const float* w = wgt + h * kMaxSplits;
    float num0 = 0.0f, num1 = 0.0f, num2 = 0.0f, num3 = 0.0f;
    int s = 0;
    for (; s + 4 <= S; s += 4) {
      const float a0 = load_through(accp + (size_t)(s + 0) * kHd);
      const float a1 = load_through(accp + (size_t)(s + 1) * kHd);
      const float a2 = load_through(accp + (size_t)(s + 2) * kHd);
      const float a3 = load_through(accp + (size_t)(s + 3) * kHd);
      num0 += w[s] * a0;
      num1 += w[s + 1] * a1;
      num2 += w[s + 2] * a2;
      num3 += w[s + 3] * a3;
    }
    for (; s < S; ++s) num0 += w[s] * load_through(accp + (size_t)s * kHd);
    const float o = round_bf(((num0 + num1) + (num2 + num3)) / den_s[h]);
    if (PLAIN) {
      p.out[((size_t)b * p.num_q_heads + hq0 + h) * kHd + tid] = f2bf(o);
      continue;
    }
    const float gx = bf2f(p.q[(size_t)b * p.ld_q + (size_t)(hq0 + h) * 2 * kHd + kHd + tid]);
    const float gate = round_bf(p.gate == 0 ? sigmoid(gx) : silu(gx));
    p.out[(size_t)b * p.num_q_heads * kHd + (size_t)(hq0 + h) * kHd + tid] = f2bf(o * gate);
  }
}

// The splits' merge, after attn_decode_kernel: workgroup (chunk, query head, batch row), 64
// output dims each; wave w sums splits w, w + 4, ... of each dim and the 4 wave sums are added
// in wave order. Every wave issues its first 16 partial loads and wave 0 the (m, l) pairs of
// up to 256 splits before any of them is used, so for S <= 64 the merge is one memory round
// trip: wave 0 then turns the pairs into split weights w_s = exp(m_s - m*) (0 for an empty
// split) and the denominator, and later batches (S > 64) follow. The partials were written
// through to memory by workgroups on any XCD; they are read at system scope (a plain load
// could hit a line this XCD's L2 kept from an earlier call).
constexpr int kMergeBatch = 16;
template <bool PLAIN>
__global__ __launch_bounds__(256) void attn_merge_kernel(DfAttnDecodeArgs p, AttnWs ws) {
  __shared__ float w_s[kMaxSplits];
  __shared__ float part[kQPerKv][64];
  __shared__ float den_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
  const int S = p.splits;
  if (!PLAIN) {
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_len) return;  // the split kernel refused too
  }
  const size_t row0 = ((size_t)b * p.num_q_heads + hq) * S;
  const int d = chunk * 64 + lane;
  const float* accp = ws.acc + row0 * kHd + d;
  float a[kMergeBatch];
#pragma unroll
  for (int i = 0; i < kMergeBatch; ++i) {
    const int sp = wave + kQPerKv * i;
    a[i] = sp < S ? load_through(accp + (size_t)sp * kHd) : 0.0f;
  }
  if (wave == 0) {
    constexpr int kPer = kMaxSplits / 64;
    float m[kPer], l[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int sp = lane + 64 * j;
      m[j] = sp < S ? load_through(ws.ml + (row0 + sp) * 2) : -INFINITY;
      l[j] = sp < S ? load_through(ws.ml + (row0 + sp) * 2 + 1) : 0.0f;
    }
    float mstar = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPer; ++j) mstar = fmaxf(mstar, l[j] > 0.0f ? m[j] : -INFINITY);
    mstar = wave_max(mstar);
    float den = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int sp = lane + 64 * j;
      const float w = (l[j] > 0.0f && m[j] != -INFINITY) ? expf(m[j] - mstar) : 0.0f;
      den += w * l[j];
      if (sp < S) w_s[sp] = w;
    }
    den = wave_sum(den);
    if (lane == 0) den_s = den;
  }
  __syncthreads();
  float num = 0.0f;
#pragma unroll
  for (int i = 0; i < kMergeBatch; ++i) {
    const int sp = wave + kQPerKv * i;
    if (sp < S) num += w_s[sp] * a[i];
  }
  for (int s0 = wave + kQPerKv * kMergeBatch; s0 < S; s0 += kQPerKv * kMergeBatch) {
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const int sp = s0 + kQPerKv * i;
      a[i] = sp < S ? load_through(accp + (size_t)sp * kHd) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const int sp = s0 + kQPerKv * i;
      if (sp < S) num += w_s[sp] * a[i];
    }
  }
  part[wave][lane] = num;
  __syncthreads();
  if (wave == 0) {
    const float o = round_bf((((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]) / den_s);
    if (PLAIN) {
      p.out[((size_t)b * p.num_q_heads + hq) * kHd + d] = f2bf(o);
    } else {
      const float gx = bf2f(p.q[(size_t)b * p.ld_q + (size_t)hq * 2 * kHd + kHd + d]);
      const float gate = round_bf(p.gate == 0 ? sigmoid(gx) : silu(gx));
      p.out[(size_t)b * p.num_q_heads * kHd + (size_t)hq * kHd + d] = f2bf(o * gate);
    }
  }
}

// ---- the allocation-free variant -------------------------------------------------------
//
// df_attention_decode_static runs the same kernels with their workspace in this file-scope
// device array instead of a caller's buffer: room for kStaticPartialRows (batch x query head
// x split) partials of 258 floats. Each GPU the library runs on holds its own copy until the
// process ends. In host code the name `scratch` is only a stand-in: its device address comes
// from hipGetSymbolAddress, once per device, and only that address is handed to kernels.
constexpr int kStaticPartialRows = 8192;
constexpr size_t kStaticScratchBytes = (size_t)kStaticPartialRows * (kHd + 2) * sizeof(float);
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
struct StaticScratch {
  std::mutex lock;
  void* ptr[kMaxDevices] = {};
};
inline StaticScratch& static_scratch() {
  static StaticScratch s;
  return s;
}

// The current device's scratch address, looked up on the first call on that device.
inline void* scratch_for_current_device(int* device) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  StaticScratch& s = static_scratch();
  std::lock_guard<std::mutex> guard(s.lock);
  if (!s.ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    s.ptr[dev] = p;
  }
  *device = dev;
  return s.ptr[dev];
}

}  // namespace df

using namespace df;

extern "C" {

size_t df_attention_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                           int splits) {
  (void)num_kv_heads;
  return (size_t)batch * num_q_heads * splits * (head_dim + 2) * sizeof(float);
}

int df_attention_decode_splits(int batch, int num_kv_heads, int max_keys) {
  // Aim for ~512 workgroups (two resident per CU: 216 VGPRs, 21 KB of LDS), at least one
  // 64-key tile per split, at most 256 splits. Measured against ~1024: B=1 at 32k keys 40.7
  // against 48.9 us, B=8 at 4k keys 38.6 against 44.5 us; the same at B=1, 4k keys.
  if (batch < 1 || num_kv_heads < 1 || max_keys < 1) return 1;
  int s = 512 / (batch * num_kv_heads);
  const int tiles = (max_keys + kTile - 1) / kTile;
  if (s > tiles) s = tiles;
  if (s > 256) s = 256;
  return s < 1 ? 1 : s;
}

int df_attention_decode(const DfAttnDecodeArgs* args, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  if (!args) return DF_BAD_ARGUMENT;
  const DfAttnDecodeArgs& a = *args;
  if (a.head_dim != kHd || a.num_kv_heads < 1 || a.num_q_heads != a.num_kv_heads * kQPerKv || a.batch < 1 ||
      a.splits < 1 || a.splits > kMaxSplits || a.rotary_dim % 8 || a.rotary_dim > kHd || a.rotary_dim < 8 ||
      ((a.rotary_dim / 8) & (a.rotary_dim / 8 - 1)) || a.max_len < 1 ||
      !a.q || !a.k || !a.v || !a.q_norm_w || !a.k_norm_w || !a.inv_freq || !a.k_cache || !a.v_cache ||
      !a.position || !a.out || (a.gate != 0 && a.gate != 1))
    return DF_BAD_ARGUMENT;
  if (a.ld_q % 4 || a.ld_kv % 4) return DF_BAD_ARGUMENT;
  if (!workspace ||
      workspace_bytes < df_attention_decode_workspace_bytes(a.batch, a.num_q_heads, a.num_kv_heads, kHd, a.splits))
    return DF_WORKSPACE_TOO_SMALL;
  const AttnWs ws = attn_ws(workspace, a.batch, a.num_q_heads, a.splits);
  hipLaunchKernelGGL(attn_decode_kernel<false>, dim3(a.splits, a.num_kv_heads, a.batch), dim3(256), 0, stream, a,
                     ws, PlainAttn{0, 0.0f});
  if (a.splits > 1 && hipGetLastError() == hipSuccess)
    hipLaunchKernelGGL(attn_merge_kernel<false>, dim3(kHd / 64, a.num_q_heads, a.batch), dim3(256), 0, stream, a, ws);
  DF_RETURN_LAUNCH_STATUS();
}

int df_split_kv_decode_attention(const uint16_t* query, const uint16_t* key, const uint16_t* value, int batch,
                                 int num_q_heads, int num_kv_heads, int key_len, int head_dim, float scale,
                                 int splits, uint16_t* out, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  if (!query || !key || !value || !out || batch < 1 || num_kv_heads < 1 || num_q_heads != num_kv_heads * kQPerKv ||
      head_dim != kHd || key_len < 1 || splits < 1 || splits > kMaxSplits || !(scale == scale))
    return DF_BAD_ARGUMENT;
  if (!workspace ||
      workspace_bytes < df_attention_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, kHd, splits))
    return DF_WORKSPACE_TOO_SMALL;
  DfAttnDecodeArgs a{};
  a.q = query;
  a.k_cache = const_cast<uint16_t*>(key);  // read only in the plain kernel
  a.v_cache = const_cast<uint16_t*>(value);
  a.out = out;
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = kHd;
  a.max_len = key_len;
  a.splits = splits;
  const AttnWs ws = attn_ws(workspace, batch, num_q_heads, splits);
  hipLaunchKernelGGL(attn_decode_kernel<true>, dim3(splits, num_kv_heads, batch), dim3(256), 0, stream, a, ws,
                     PlainAttn{key_len, scale});
  if (splits > 1 && hipGetLastError() == hipSuccess)
    hipLaunchKernelGGL(attn_merge_kernel<true>, dim3(kHd / 64, num_q_heads, batch), dim3(256), 0, stream, a, ws);
  DF_RETURN_LAUNCH_STATUS();
}

size_t df_attention_decode_static_capacity(void) { return kStaticScratchBytes; }

int df_attention_decode_static(const DfAttnDecodeArgs* args, hipStream_t stream) {
  if (!args) return DF_BAD_ARGUMENT;
  const DfAttnDecodeArgs& a = *args;
  if (a.batch < 1 || a.num_q_heads < 1 || a.splits < 1 ||
      (size_t)a.batch * a.num_q_heads * a.splits > (size_t)kStaticPartialRows)
    return DF_WORKSPACE_TOO_SMALL;
  int dev = -1;
  void* base = scratch_for_current_device(&dev);
  if (!base) return DF_LAUNCH_FAILED;
  return df_attention_decode(args, base, kStaticScratchBytes, stream);
}

}  // extern "C"
