// Group-128 int4 dequantise-GEMV for gfx950, with fused norm prologues and epilogues.
//
// Interchange format (reference kernels/tiled_gemv.py:242-288): packed uint8 [K/2][N],
// byte [j][n] = nibble(k=j) | nibble(k=j+K/2) << 4, each stored +8; scales [K/128][N].
// At install time the weight is repacked once into a device tiling:
//
//   block (t, g) = 1024 bytes for output columns 16t..16t+15 and k in group g
//                = [slot s 0..3][column c 0..15][16 bytes]
//   16 bytes     = 4 dwords d; dword d holds k = 128g + 32s + 8d + e, e = 0..7, with
//                  nibble e=2j at bits 4j..4j+3 and e=2j+1 at bits 16+4j..16+4j+3.
//   blocks are ordered [t][g], so one tile's whole K range is contiguous.
//
// Work split: a workgroup of 8 waves owns NT 16-column tiles; the 8/NT waves that share a
// tile split its K range, and their fp32 partials are summed in LDS in a fixed order. Each
// wave keeps 12 groups (8 for the logits epilogue) in flight, 1 KB of weights each. Each group
// is one fully coalesced 1 KB load (64 lanes x 16 B).
//
// Arithmetic is the reference's (kernels/visible_int4_head.py:187-199): every weight is
// dequantised to bf16((nibble - 8) * scale) -- (nibble - 8) * scale is exact in fp32 and
// the bf16 conversion is one round-to-nearest-even (v_cvt_pk_bf16_f32) -- and multiplied by
// the bf16 activations with fp32 accumulation on MFMA (v_mfma_f32_16x16x32_bf16; up to 16
// activation rows, the dequantised weights as the B operand). Only the summation order
// differs from the reference.
//
// When even that leaves too few waves, the K range is also split across workgroups
// (blockIdx.y); those write fp32 partials and a second kernel sums them in split order and
// runs the epilogue. Nothing uses atomics, so results are bit-identical run to run.
#include "common.h"
#include "deltaforge_hip.h"
#include "int4_block.h"

namespace df {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxRows = 16;
// Groups in flight per wave. 12 puts a whole K range of the decode's MLP shapes (9 to 10
// groups per wave at 1 row, 9 to 20 at 16) in flight at once or nearly: MLP block 23.5 ->
// 22.3 us at 1 row and 35.4 -> 33.8 us at 16 rows, against 8. The head's 20-group ranges ran
// 1.6 to 2.7 % slower with 12 than with 8 (and 16 or 20 were slower everywhere), so the logits
// epilogue keeps 8.
template <int EPI>
constexpr int depth_of() { return EPI == DF_EPI_LOGITS ? 8 : 12; }
constexpr int kNormChunks = 3;  // RMSNorm prologue: K <= kNormChunks * kThreads * 8 = 12288
constexpr int kRowChunks = 5;   // ... one wave per row when K <= kRowChunks * 64 * 8 = 2560
constexpr int kGemvLds = 100 * 1024;  // LDS bytes a workgroup may take

struct GemvSmem {
  int xs_ld;  // bf16 elements per LDS row of x
  int ybuf_off, red_off, total;
};

// LDS holds the activation rows plus, when rows < 16, one zero row that the MFMA lanes of
// absent rows read (so the inner loop has no divergent branch).
__host__ __device__ inline GemvSmem gemv_smem(int rows, int kx, int nt) {
  GemvSmem s;
  s.xs_ld = kx + 8;
  const int rows_alloc = rows < kMaxRows ? rows + 1 : rows;
  const int xs_bytes = ((rows_alloc * s.xs_ld * 2) + 15) & ~15;
  s.ybuf_off = xs_bytes;
  s.red_off = s.ybuf_off + (kWaves / nt) * rows * nt * kTileCols * 4;
  s.total = s.red_off + 64;
  return s;
}

// ---------------------------------------------------------------------------------------
// Prologues: this workgroup's K range of the bf16 activation rows, into LDS.
// ---------------------------------------------------------------------------------------

template <int PRO, bool WROWS>
DF_DEVICE void gemv_prologue(const DfInt4GemvArgs& p, uint16_t* xs, int xs_ld, float* red, int k0, int kc) {
  const int tid = threadIdx.x;
  if (p.rows < kMaxRows) {
    for (int kk = tid * 8; kk < kc; kk += kThreads * 8)
      *reinterpret_cast<uint4*>(xs + p.rows * xs_ld + kk) = make_uint4(0u, 0u, 0u, 0u);
  }
  if constexpr (PRO == DF_PRO_NONE) {
    for (int m = 0; m < p.rows; ++m) {
      const uint16_t* src = p.x + (size_t)m * p.ldx + k0;
      for (int kk = tid * 8; kk < kc; kk += kThreads * 8)
        *reinterpret_cast<uint4*>(xs + m * xs_ld + kk) = load16(src + kk);
    }
  } else if constexpr (PRO == DF_PRO_RMSNORM || PRO == DF_PRO_ADD_RMSNORM) {
    // RMSNorm with the (1 + w) scale over the whole row (reference.py:92-96); with ADD the
    // row is first bf16(x + residual) (reference.py:735 feeding the next norm). Each thread
    // owns up to kNormChunks 8-element chunks of the row, loaded once (16-byte loads) and
    // kept in registers between the sum of squares and the scaling.
    const bool write_h =
        (PRO == DF_PRO_ADD_RMSNORM) && p.h_out && blockIdx.x == 0 && blockIdx.y == 0;
    const int nchunks = p.K / 8;
    if (WROWS && nchunks <= 64 * kRowChunks) {
      // Many rows (the WROWS instance): one wave per row (rows w, w + 8, ...), the row and the
      // norm weight of this workgroup's K range loaded at once into the wave's registers, its
      // sum of squares reduced within the wave. Rows proceed in parallel with no block-wide
      // reduction (and no second memory round trip) per row; the sum's order differs from the
      // block form's only in fp32 rounding. Few rows keep the block form: this one holds more
      // registers, and the occupancy it costs outweighs what it saves for one row.
      const int lane = tid & 63, wave = tid >> 6;
      for (int m = wave; m < p.rows; m += kWaves) {
        const uint16_t* xr = p.x + (size_t)m * p.ldx;
        const uint16_t* rr = p.x2 + (size_t)m * p.ldx2;
        uint32_t v[kRowChunks][4];
        uint4 wreg[kRowChunks];
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
          const int c = lane + 64 * j, k = c * 8;
          wreg[j] = make_uint4(0u, 0u, 0u, 0u);
          v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0u;
          if (c < nchunks) {
            const uint4 raw = load16(xr + k);
            v[j][0] = raw.x, v[j][1] = raw.y, v[j][2] = raw.z, v[j][3] = raw.w;
            if constexpr (PRO == DF_PRO_ADD_RMSNORM) {
              const uint4 rraw = load16(rr + k);
              const uint32_t rw[4] = {rraw.x, rraw.y, rraw.z, rraw.w};
#pragma unroll
              for (int e2 = 0; e2 < 4; ++e2) {
                const uint16_t lo = f2bf(bf2f(static_cast<uint16_t>(v[j][e2])) + bf2f(static_cast<uint16_t>(rw[e2])));
                const uint16_t hi = f2bf(bf2f(static_cast<uint16_t>(v[j][e2] >> 16)) +
                                         bf2f(static_cast<uint16_t>(rw[e2] >> 16)));
                v[j][e2] = lo | (static_cast<uint32_t>(hi) << 16);
              }
            }
            if (k >= k0 && k < k0 + kc) wreg[j] = load16(p.norm_w + k);
          }
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
          const int c = lane + 64 * j;
          if (c < nchunks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float val = bf2f(static_cast<uint16_t>(v[j][e >> 1] >> (16 * (e & 1))));
              ss += val * val;
            }
            if (write_h)
              *reinterpret_cast<uint4*>(p.h_out + (size_t)m * p.K + c * 8) = make_uint4(v[j][0], v[j][1], v[j][2], v[j][3]);
          }
        }
        ss = wave_sum(ss);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(p.K) + p.eps);
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
          const int c = lane + 64 * j, k = c * 8;
          if (c < nchunks && k >= k0 && k < k0 + kc) {
            const uint32_t ww[4] = {wreg[j].x, wreg[j].y, wreg[j].z, wreg[j].w};
            uint32_t o[4];
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              uint16_t pr[2];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const float scaled = bf2f(static_cast<uint16_t>(v[j][e2] >> (16 * h))) * r;
                pr[h] = f2bf(scaled * (1.0f + bf2f(static_cast<uint16_t>(ww[e2] >> (16 * h)))));
              }
              o[e2] = pr[0] | (static_cast<uint32_t>(pr[1]) << 16);
            }
            *reinterpret_cast<uint4*>(xs + m * xs_ld + (k - k0)) = make_uint4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    } else
    for (int m = 0; m < p.rows; ++m) {
      const uint16_t* xr = p.x + (size_t)m * p.ldx;
      const uint16_t* rr = p.x2 + (size_t)m * p.ldx2;
      uint32_t v[kNormChunks][4];  // the row as packed bf16 (bf16(x + r) is exact in bf16)
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < kNormChunks; ++j) {
        const int c = tid + j * kThreads;
        if (c < nchunks) {
          const uint4 raw = load16(xr + c * 8);
          v[j][0] = raw.x, v[j][1] = raw.y, v[j][2] = raw.z, v[j][3] = raw.w;
          if constexpr (PRO == DF_PRO_ADD_RMSNORM) {
            const uint4 rraw = load16(rr + c * 8);
            const uint32_t rw[4] = {rraw.x, rraw.y, rraw.z, rraw.w};
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              const uint16_t lo = f2bf(bf2f(static_cast<uint16_t>(v[j][e2])) + bf2f(static_cast<uint16_t>(rw[e2])));
              const uint16_t hi = f2bf(bf2f(static_cast<uint16_t>(v[j][e2] >> 16)) +
                                       bf2f(static_cast<uint16_t>(rw[e2] >> 16)));
              v[j][e2] = lo | (static_cast<uint32_t>(hi) << 16);
            }
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float val = bf2f(static_cast<uint16_t>(v[j][e >> 1] >> (16 * (e & 1))));
            ss += val * val;
          }
          if (write_h)
            *reinterpret_cast<uint4*>(p.h_out + (size_t)m * p.K + c * 8) = make_uint4(v[j][0], v[j][1], v[j][2], v[j][3]);
        }
      }
      ss = block_sum<kWaves>(ss, red);
      const float r = 1.0f / sqrtf(ss / static_cast<float>(p.K) + p.eps);
#pragma unroll
      for (int j = 0; j < kNormChunks; ++j) {
        const int c = tid + j * kThreads;
        const int k = c * 8;
        if (c < nchunks && k >= k0 && k < k0 + kc) {
          const uint4 wraw = load16(p.norm_w + k);
          const uint32_t ww[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
          uint32_t o[4];
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            uint16_t pr[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float scaled = bf2f(static_cast<uint16_t>(v[j][e2] >> (16 * h))) * r;
              pr[h] = f2bf(scaled * (1.0f + bf2f(static_cast<uint16_t>(ww[e2] >> (16 * h)))));
            }
            o[e2] = pr[0] | (static_cast<uint32_t>(pr[1]) << 16);
          }
          *reinterpret_cast<uint4*>(xs + m * xs_ld + (k - k0)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  } else {  // DF_PRO_GATED_RMSNORM: one 128-group == one value head (reference.py:115-121)
    // 8 elements per thread; a head is 16 consecutive lanes, reduced with lane shuffles.
    for (int m = 0; m < p.rows; ++m) {
      for (int c = tid; c < kc / 8; c += kThreads) {
        const int k = k0 + c * 8;
        const uint4 xraw = load16(p.x + (size_t)m * p.ldx + k);
        const uint4 zraw = load16(p.x2 + (size_t)m * p.ldx2 + k);
        const uint4 wraw = load16(p.norm_w + (k % kGroup));
        const uint32_t xw[4] = {xraw.x, xraw.y, xraw.z, xraw.w};
        const uint32_t zw[4] = {zraw.x, zraw.y, zraw.z, zraw.w};
        const uint32_t ww[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
        float v[8];
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e] = bf2f(static_cast<uint16_t>(xw[e >> 1] >> (16 * (e & 1))));
          ss += v[e] * v[e];
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) ss += __shfl_xor(ss, off, 64);
        const float r = 1.0f / sqrtf(ss / 128.0f + p.eps);
        uint32_t o[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          uint16_t pr[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int e = e2 * 2 + h;
            const float t = round_bf(bf2f(static_cast<uint16_t>(ww[e2] >> (16 * h))) * round_bf(v[e] * r));
            pr[h] = f2bf(t * silu(bf2f(static_cast<uint16_t>(zw[e2] >> (16 * h)))));
          }
          o[e2] = pr[0] | (static_cast<uint32_t>(pr[1]) << 16);
        }
        *reinterpret_cast<uint4*>(xs + m * xs_ld + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------
// Epilogues over the `cols` columns x rows results of this workgroup (fp32, in LDS).
// ---------------------------------------------------------------------------------------

template <int EPI>
DF_DEVICE void gemv_epilogue(const DfInt4GemvArgs& p, const float* y, int col0, int cols) {
  for (int e = threadIdx.x; e < p.rows * cols; e += blockDim.x) {
    const int m = e / cols, c = e % cols;
    const float v = y[m * cols + c];
    if constexpr (EPI == DF_EPI_STORE || EPI == DF_EPI_LOGITS) {
      p.out[(size_t)m * p.ldo + col0 + c] = f2bf(v);
    } else if constexpr (EPI == DF_EPI_RESIDUAL) {
      // bf16(residual + bf16(y)) (reference.py:730, 735). In place is allowed.
      const size_t at = (size_t)m * p.ldo + col0 + c;
      p.out[at] = f2bf(bf2f(p.res[at]) + round_bf(v));
    } else {  // DF_EPI_SWIGLU: 16-column gate / up tiles alternate
      if ((c & 16) == 0) {
        const float g = round_bf(v);
        const float u = round_bf(y[m * cols + c + 16]);
        const int oc = (col0 + c) / 32 * 16 + (c & 15);
        p.out[(size_t)m * p.ldo + oc] = f2bf(round_bf(silu(g)) * u);
      }
    }
  }
}

template <int PRO, int EPI, int NT, bool WROWS>
__global__ __launch_bounds__(kThreads) void w4_gemv_kernel(DfInt4GemvArgs p) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int KS = kWaves / NT;
  constexpr int kDepth = depth_of<EPI>();
  constexpr int COLS = NT * kTileCols;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tsub = wave % NT, kpart = wave / NT;
  const int G = p.K / kGroup;
  const int gx0 = blockIdx.y * p.groups_per_split;
  const int ngx = min(p.groups_per_split, G - gx0);
  const int per = (ngx + KS - 1) / KS;
  const int g_lo = min(kpart * per, ngx), g_hi = min(g_lo + per, ngx);
  const GemvSmem L = gemv_smem(p.rows, ngx * kGroup, NT);
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* ybuf = reinterpret_cast<float*>(smem + L.ybuf_off);
  float* red = reinterpret_cast<float*>(smem + L.red_off);

  const int tile = blockIdx.x * NT + tsub;
  const unsigned char* wp = p.w + ((size_t)tile * G + gx0) * kBlockBytes + lane * 16;
  const uint16_t* sp = p.s + ((size_t)tile * G + gx0) * kTileCols + (lane & 15);

  // Weights do not depend on the activations: put the first groups in flight before the
  // prologue so HBM is busy while the norm is computed. Refills are clamped to the last
  // group of the range (a repeat read of a cached block) so the pipeline is branch-free.
  const bool has_work = g_lo < g_hi;
  const int g_last = g_hi - 1;
  uint4 wb[kDepth];
  uint16_t sb[kDepth];
  if (has_work) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const int g = min(g_lo + u, g_last);
      wb[u] = load16(wp + (size_t)g * kBlockBytes);
      sb[u] = sp[g * kTileCols];
    }
  }

  gemv_prologue<PRO, WROWS>(p, xs, L.xs_ld, red, gx0 * kGroup, ngx * kGroup);

  const int col = lane & 15;   // A row, B/C column, scale column
  const int slot = lane >> 4;  // K slot of A and B; C row block
  const uint16_t* xrow = xs + min(col, p.rows) * L.xs_ld + slot * 32;  // absent rows read zeros
  df_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const DqK K = dq_consts();

  auto group_mac = [&](const uint4 wv, const uint16_t sraw, const int g) {
    const GroupScale gs = group_scale(sraw);
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint4 bw = dequant8(words[d], gs, K);
      const uint4 aw = *reinterpret_cast<const uint4*>(xrow + g * kGroup + d * 8);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, aw),
                                                    __builtin_bit_cast(df_bf16x8, bw), acc, 0, 0, 0);
    }
  };

  int g0 = g_lo;
  for (; g0 + kDepth <= g_hi; g0 += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const uint4 wv = wb[u];
      const uint16_t sv = sb[u];
      const int gn = min(g0 + u + kDepth, g_last);
      wb[u] = load16(wp + (size_t)gn * kBlockBytes);
      sb[u] = sp[gn * kTileCols];
      group_mac(wv, sv, g0 + u);
    }
  }
  // Tail: the remaining groups are already in wb[0 .. g_hi - g0).
#pragma unroll
  for (int u = 0; u < kDepth; ++u) {
    if (g0 + u < g_hi) group_mac(wb[u], sb[u], g0 + u);
  }

  // K parts of a tile -> LDS, then a fixed-order sum.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = slot * 4 + i;
    if (m < p.rows) ybuf[(kpart * p.rows + m) * COLS + tsub * kTileCols + col] = acc[i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < p.rows * COLS; e += kThreads) {
    float v = ybuf[e];
#pragma unroll
    for (int k = 1; k < KS; ++k) v += ybuf[k * p.rows * COLS + e];
    ybuf[e] = v;
  }
  __syncthreads();
  const int col0 = blockIdx.x * COLS;
  if (gridDim.y == 1) {
    gemv_epilogue<EPI>(p, ybuf, col0, COLS);
  } else {
    for (int e = threadIdx.x; e < p.rows * COLS; e += kThreads) {
      const int m = e / COLS, c = e % COLS;
      p.part[((size_t)blockIdx.y * p.rows + m) * p.N + col0 + c] = ybuf[e];
    }
  }
}

// Sum of the cross-workgroup K splits (in split order) + the epilogue. 64 columns per block.
template <int EPI>
__global__ __launch_bounds__(256) void w4_reduce_kernel(DfInt4GemvArgs p) {
  __shared__ float y[kMaxRows * 64];
  const int col0 = blockIdx.x * 64;
  for (int e = threadIdx.x; e < p.rows * 64; e += 256) {
    const int m = e / 64, c = e % 64;
    const float* src = p.part + (size_t)m * p.N + col0 + c;
    const size_t stride = (size_t)p.rows * p.N;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    int s = 0;
    for (; s + 4 <= p.ksplit; s += 4) {
      const float a0 = src[(s + 0) * stride], a1 = src[(s + 1) * stride];
      const float a2 = src[(s + 2) * stride], a3 = src[(s + 3) * stride];
      v[0] = ((v[0] + a0) + a1) + a2;
      v[0] = v[0] + a3;
    }
    for (; s < p.ksplit; ++s) v[0] += src[s * stride];
    y[e] = v[0];
  }
  __syncthreads();
  gemv_epilogue<EPI>(p, y, col0, 64);
}

// ---------------------------------------------------------------------------------------
// Install-time repack and the bit-exact dequant (debug / parity entry point).
// ---------------------------------------------------------------------------------------

__global__ void w4_repack_kernel(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
                                 int K, int N, uint32_t* __restrict__ wt, uint16_t* __restrict__ st) {
  const int G = K / kGroup;
  const size_t total = (size_t)(N / kTileCols) * G * 256;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int d = idx & 3, lane = (idx >> 2) & 63;
  const size_t tg = idx >> 8;
  const int g = tg % G, t = tg / G;
  const int s = lane >> 4, c = lane & 15, n = t * kTileCols + c;
  const int half = K / 2;
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = g * kGroup + s * 32 + d * 8 + e;
    const uint32_t byte = k < half ? packed[(size_t)k * N + n] : packed[(size_t)(k - half) * N + n];
    const uint32_t nib = k < half ? (byte & 15u) : (byte >> 4);
    const int pos = (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
    word |= nib << pos;
  }
  wt[idx] = word;
  if (s == 0 && d == 0) st[tg * kTileCols + c] = scale[(size_t)g * N + n];
}

// W[k][n] = bf16((nibble - 8) * scale), read back from the tiled layout with the GEMV's own
// dequant routine: proves the repack and the dequant arithmetic together (reference
// tiled_gemv.py:281-288 then .to(bf16)).
__global__ void w4_dequant_kernel(const uint32_t* __restrict__ wt, const uint16_t* __restrict__ st, int K,
                                  int N, uint16_t* __restrict__ out) {
  const int G = K / kGroup;
  const size_t total = (size_t)(N / kTileCols) * G * 256;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int d = idx & 3, lane = (idx >> 2) & 63;
  const size_t tg = idx >> 8;
  const int g = tg % G, t = tg / G;
  const int s = lane >> 4, c = lane & 15, n = t * kTileCols + c;
  const uint4 q = dequant8(wt[idx], group_scale(st[tg * kTileCols + c]), dq_consts());
  const uint32_t pairs[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = g * kGroup + s * 32 + d * 8 + e;
    out[(size_t)k * N + n] = static_cast<uint16_t>(pairs[e >> 1] >> (16 * (e & 1)));
  }
}

template <int PRO, int EPI, int NT>
static hipError_t launch_gemv(const DfInt4GemvArgs& a, hipStream_t stream) {
  const int G = a.K / kGroup;
  const int gps = a.groups_per_split;
  const GemvSmem L = gemv_smem(a.rows, min(gps, G) * kGroup, NT);
  dim3 grid(a.N / (NT * kTileCols), a.ksplit);
  constexpr bool kNorm = PRO == DF_PRO_RMSNORM || PRO == DF_PRO_ADD_RMSNORM;
  if (kNorm && a.rows > 4 && a.K <= kRowChunks * 64 * 8)
    hipLaunchKernelGGL((w4_gemv_kernel<PRO, EPI, NT, kNorm>), grid, dim3(kThreads), L.total, stream, a);
  else
    hipLaunchKernelGGL((w4_gemv_kernel<PRO, EPI, NT, false>), grid, dim3(kThreads), L.total, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.ksplit == 1) return e;
  hipLaunchKernelGGL((w4_reduce_kernel<EPI>), dim3(a.N / 64), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int PRO, int EPI>
static hipError_t launch_nt(const DfInt4GemvArgs& a, hipStream_t stream) {
  switch (a.tiles_per_workgroup) {
    case 1: return launch_gemv<PRO, EPI, 1>(a, stream);
    case 2: return launch_gemv<PRO, EPI, 2>(a, stream);
    case 4: return launch_gemv<PRO, EPI, 4>(a, stream);
    case 8: return launch_gemv<PRO, EPI, 8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace df

using namespace df;

extern "C" {

size_t df_int4_gemv_workspace_bytes(int rows, int N, int ksplit) {
  return ksplit > 1 ? (size_t)ksplit * rows * N * sizeof(float) : 0;
}

int df_int4_gemv_plan(int rows, int K, int N, int epilogue, int target_waves, int* tiles_per_workgroup,
                      int* ksplit, int* groups_per_split, size_t* workspace_bytes) {
  if (rows < 1 || rows > kMaxRows || K % 256 || N % 64 || K <= 0 || !tiles_per_workgroup || !ksplit ||
      !groups_per_split || !workspace_bytes)
    return DF_BAD_ARGUMENT;
  if (target_waves <= 0) target_waves = 2048;
  const int G = K / kGroup;
  const int tiles = N / kTileCols;
  // Widest workgroup (most tiles, least K splitting) that divides the tiles and still
  // reaches the wave target; SwiGLU pairs a gate tile with an up tile, so at least 2.
  const int min_nt = epilogue == DF_EPI_SWIGLU ? 2 : 1;
  // A workgroup's LDS (the activation rows of its K range, partial sums) must fit kGemvLds of
  // gfx950's 160 KB: 16 rows of K = 2560 fit, so that shape needs no K split, partials or
  // reduce launch.
  auto split_for = [&](int nt_, int& gps_, int& ks_) {
    gps_ = G;
    while (gps_ > 1 && gemv_smem(rows, gps_ * kGroup, nt_).total > kGemvLds) --gps_;
    ks_ = (G + gps_ - 1) / gps_;
    gps_ = (G + ks_ - 1) / ks_;
  };
  int nt = 8;
  while (nt > min_nt && (tiles % nt || (tiles / nt) * kWaves < target_waves)) nt /= 2;
  if (rows > 4) {
    // Many rows: every workgroup stages all rows of its K range, so fewer, wider workgroups
    // stage them fewer times. Take the most workgroups up to one per CU (measured best at 8
    // and 16 rows: gate|up 2560 x 18432 in 144 workgroups of 8 tiles, 17.7 against 23.9 us at
    // 16 rows and 16.2 against 20.3 us at 8 rows with 288 of 4; down 9216 x 2560 in 160
    // workgroups, 13.8 against 20.7 us at 16 rows (4 tiles x 4 K splits, not 1 tile) and 14.0
    // against 16.1 us at 8 rows (2 tiles x 2 splits)).
    int best = 0, best_wgs = 0;
    for (int c = 8; c >= min_nt; c /= 2) {
      if (tiles % c) continue;
      int gps_, ks_;
      split_for(c, gps_, ks_);
      const int wgs = (tiles / c) * ks_;
      if (wgs <= 256 && wgs > best_wgs) best = c, best_wgs = wgs;
    }
    if (best) nt = best;
  }
  int gps, ks;
  split_for(nt, gps, ks);
  *tiles_per_workgroup = nt;
  *ksplit = ks;
  *groups_per_split = gps;
  *workspace_bytes = df_int4_gemv_workspace_bytes(rows, N, ks);
  return DF_OK;
}

int df_int4_gemv(const DfInt4GemvArgs* args, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!args) return DF_BAD_ARGUMENT;
  DfInt4GemvArgs a = *args;
  const int G = a.K / kGroup;
  if (a.rows < 1 || a.rows > kMaxRows || a.K <= 0 || a.K % 256 || a.N <= 0 || a.N % 64 || !a.w || !a.s || !a.x ||
      !a.out)
    return DF_BAD_ARGUMENT;
  const int nt = a.tiles_per_workgroup;
  if (nt != 1 && nt != 2 && nt != 4 && nt != 8) return DF_BAD_ARGUMENT;
  if ((a.N / kTileCols) % nt) return DF_BAD_ARGUMENT;
  if (a.ksplit < 1 || a.groups_per_split < 1 || (long)a.ksplit * a.groups_per_split < G ||
      (long)(a.ksplit - 1) * a.groups_per_split >= G)
    return DF_BAD_ARGUMENT;
  if (a.ldx < a.K || a.ldx % 8) return DF_BAD_ARGUMENT;
  if (a.epilogue == DF_EPI_SWIGLU && (nt < 2 || a.N % 32)) return DF_BAD_ARGUMENT;
  const int out_cols = a.epilogue == DF_EPI_SWIGLU ? a.N / 2 : a.N;
  if (a.ldo < out_cols) return DF_BAD_ARGUMENT;
  if (gemv_smem(a.rows, min(a.groups_per_split, G) * kGroup, nt).total > kGemvLds) return DF_BAD_ARGUMENT;
  if ((a.prologue == DF_PRO_ADD_RMSNORM || a.prologue == DF_PRO_GATED_RMSNORM) && !a.x2) return DF_BAD_ARGUMENT;
  if (a.prologue != DF_PRO_NONE && !a.norm_w) return DF_BAD_ARGUMENT;
  if (a.epilogue == DF_EPI_RESIDUAL && !a.res) return DF_BAD_ARGUMENT;
  if (reinterpret_cast<uintptr_t>(a.x) % 16 || reinterpret_cast<uintptr_t>(a.w) % 16) return DF_BAD_ARGUMENT;
  // The norm prologues read x2 and the norm weight with 16-byte loads.
  if (a.prologue != DF_PRO_NONE && reinterpret_cast<uintptr_t>(a.norm_w) % 16) return DF_BAD_ARGUMENT;
  if ((a.prologue == DF_PRO_ADD_RMSNORM || a.prologue == DF_PRO_GATED_RMSNORM) &&
      (reinterpret_cast<uintptr_t>(a.x2) % 16 || a.ldx2 % 8))
    return DF_BAD_ARGUMENT;
  if ((a.prologue == DF_PRO_RMSNORM || a.prologue == DF_PRO_ADD_RMSNORM) && a.K > kNormChunks * kThreads * 8)
    return DF_BAD_ARGUMENT;
  if (a.h_out && reinterpret_cast<uintptr_t>(a.h_out) % 16) return DF_BAD_ARGUMENT;
  if (a.ksplit > 1) {
    if (!workspace || workspace_bytes < df_int4_gemv_workspace_bytes(a.rows, a.N, a.ksplit))
      return DF_WORKSPACE_TOO_SMALL;
    a.part = reinterpret_cast<float*>(workspace);
  }
  hipError_t e = hipErrorInvalidValue;
#define DF_GEMV_CASE(PRO, EPI) \
  if (a.prologue == PRO && a.epilogue == EPI) e = launch_nt<PRO, EPI>(a, stream);
  DF_GEMV_CASE(DF_PRO_NONE, DF_EPI_STORE)
  DF_GEMV_CASE(DF_PRO_NONE, DF_EPI_RESIDUAL)
  DF_GEMV_CASE(DF_PRO_NONE, DF_EPI_SWIGLU)
  DF_GEMV_CASE(DF_PRO_RMSNORM, DF_EPI_STORE)
  DF_GEMV_CASE(DF_PRO_RMSNORM, DF_EPI_SWIGLU)
  DF_GEMV_CASE(DF_PRO_RMSNORM, DF_EPI_LOGITS)
  DF_GEMV_CASE(DF_PRO_ADD_RMSNORM, DF_EPI_STORE)
  DF_GEMV_CASE(DF_PRO_ADD_RMSNORM, DF_EPI_LOGITS)
  DF_GEMV_CASE(DF_PRO_GATED_RMSNORM, DF_EPI_STORE)
  DF_GEMV_CASE(DF_PRO_GATED_RMSNORM, DF_EPI_RESIDUAL)
#undef DF_GEMV_CASE
  if (e == hipErrorInvalidValue) return DF_BAD_ARGUMENT;
  return e == hipSuccess ? DF_OK : DF_LAUNCH_FAILED;
}

int df_int4_repack(const uint8_t* packed, const uint16_t* scale, int K, int N, uint8_t* w_tiled,
                   uint16_t* s_tiled, hipStream_t stream) {
  if (!packed || !scale || !w_tiled || !s_tiled || K % 256 || N % kTileCols || K <= 0 || N <= 0)
    return DF_BAD_ARGUMENT;
  const size_t total = (size_t)(N / kTileCols) * (K / kGroup) * 256;
  hipLaunchKernelGGL(w4_repack_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, packed, scale, K, N,
                     reinterpret_cast<uint32_t*>(w_tiled), s_tiled);
  DF_RETURN_LAUNCH_STATUS();
}

int df_int4_dequant(const uint8_t* w_tiled, const uint16_t* s_tiled, int K, int N, uint16_t* out,
                    hipStream_t stream) {
  if (!w_tiled || !s_tiled || !out || K % 256 || N % kTileCols || K <= 0 || N <= 0) return DF_BAD_ARGUMENT;
  const size_t total = (size_t)(N / kTileCols) * (K / kGroup) * 256;
  hipLaunchKernelGGL(w4_dequant_kernel, dim3((total + 255) / 256), dim3(256), 0, stream,
                     reinterpret_cast<const uint32_t*>(w_tiled), s_tiled, K, N, out);
  DF_RETURN_LAUNCH_STATUS();
}

}  // extern "C"
