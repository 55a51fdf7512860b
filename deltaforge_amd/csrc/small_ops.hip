// Elementwise / row ops of the slot surface and the decode-loop glue, for gfx950.
#include "common.h"
#include "deltaforge_hip.h"

namespace df {

// One workgroup per row: RMSNorm(1+w) (reference.py:92-96); with `residual` the row is
// bf16(x + residual) first and that sum is also stored (fused_rmsnorm_residual.py:56-89).
template <bool ADD>
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ residual,
                                                       const uint16_t* __restrict__ w, float eps, int n,
                                                       uint16_t* __restrict__ resid_out,
                                                       uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  const uint16_t* xr = x + row * n;
  float ss = 0.0f;
  for (int k = threadIdx.x; k < n; k += 256) {
    float v = bf2f(xr[k]);
    if constexpr (ADD) {
      v = round_bf(v + bf2f(residual[row * n + k]));
      resid_out[row * n + k] = f2bf(v);
    }
    ss += v * v;
  }
  ss = block_sum<4>(ss, red);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
  for (int k = threadIdx.x; k < n; k += 256) {
    float v = bf2f(xr[k]);
    if constexpr (ADD) v = round_bf(v + bf2f(residual[row * n + k]));
    const float scaled = v * r;
    out[row * n + k] = f2bf(scaled * (1.0f + bf2f(w[k])));
  }
}

__global__ void silu_mul_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up, size_t n,
                                uint16_t* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f2bf(round_bf(silu(bf2f(gate[i]))) * bf2f(up[i]));
}

// One wave per (b, h, s) row of head_dim; rotary part in the reference's bf16 op order.
__global__ void partial_rope_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ cos,
                                    const uint16_t* __restrict__ sin, int heads, int seq, int head_dim,
                                    int rot, uint16_t* __restrict__ out, int rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int b = row / (heads * seq), s = row % seq;
  const uint16_t* cr = cos + ((size_t)b * seq + s) * rot;
  const uint16_t* sr = sin + ((size_t)b * seq + s) * rot;
  const uint16_t* xr = x + (size_t)row * head_dim;
  const int half = rot / 2;
  for (int d = lane; d < head_dim; d += 64) {
    if (d < rot) {
      const float xv = bf2f(xr[d]);
      const float partner = d < half ? -bf2f(xr[d + half]) : bf2f(xr[d - half]);
      out[(size_t)row * head_dim + d] =
          f2bf(round_bf(xv * bf2f(cr[d])) + round_bf(partner * bf2f(sr[d])));
    } else {
      out[(size_t)row * head_dim + d] = xr[d];
    }
  }
}

// Conv step at seq_len 1, history [B][C][3] in place (inline_causal_conv.py:98-129).
__global__ void causal_conv_step_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ hist,
                                        const uint16_t* __restrict__ w, int channels, size_t total,
                                        uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c = i % channels;
  uint16_t* h = hist + i * 3;
  const uint16_t* wc = w + (size_t)c * 4;
  const float h0 = bf2f(h[0]), h1 = bf2f(h[1]), h2 = bf2f(h[2]), xv = bf2f(x[i]);
  float acc = h0 * bf2f(wc[0]);
  acc = acc + h1 * bf2f(wc[1]);
  acc = acc + h2 * bf2f(wc[2]);
  acc = acc + xv * bf2f(wc[3]);
  out[i] = f2bf(silu(round_bf(acc)));
  h[0] = h[1];
  h[1] = h[2];
  h[2] = x[i];
}

// Tied embedding row from the tiled int4 head: one thread per (group, slot, dword). The
// token is tokens[b], or prompt[b * prompt_len + *position] in prompt mode (prefill).
__global__ void embed_int4_kernel(const int64_t* __restrict__ tokens, const int64_t* __restrict__ prompt,
                                  int prompt_len, const int* __restrict__ position,
                                  const uint32_t* __restrict__ wt, const uint16_t* __restrict__ st, int hidden,
                                  int vocab, uint16_t* __restrict__ out) {
  const int b = blockIdx.y;
  const int G = hidden / 128;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // g*16 + s*4 + d
  if (idx >= G * 16) return;
  int64_t tok;
  if (prompt) {
    const int pos = *position;
    if (pos < 0 || pos >= prompt_len) return;
    tok = prompt[(size_t)b * prompt_len + pos];
  } else {
    tok = tokens[b];
  }
  if (tok < 0 || tok >= vocab) return;
  const int g = idx / 16, s = (idx / 4) & 3, d = idx & 3;
  const int t = static_cast<int>(tok / 16), c = static_cast<int>(tok % 16);
  const size_t block = (size_t)t * G + g;
  const uint32_t word = wt[block * 256 + (s * 16 + c) * 4 + d];
  const float sc = bf2f(st[block * 16 + c]);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int pos = (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
    const int q = static_cast<int>((word >> pos) & 15u) - 8;
    out[(size_t)b * hidden + g * 128 + s * 32 + d * 8 + e] = f2bf(static_cast<float>(q) * sc);
  }
}

// One 16-byte chunk of the row per thread.
__global__ void embed_bf16_kernel(const int64_t* __restrict__ tokens, const int64_t* __restrict__ prompt,
                                  int prompt_len, const int* __restrict__ position,
                                  const uint4* __restrict__ table, int hidden, int vocab, uint4* __restrict__ out) {
  const int b = blockIdx.y;
  const int chunk = blockIdx.x * blockDim.x + threadIdx.x;
  const int chunks = hidden / 8;
  if (chunk >= chunks) return;
  int64_t tok;
  if (prompt) {
    const int pos = *position;
    if (pos < 0 || pos >= prompt_len) return;
    tok = prompt[(size_t)b * prompt_len + pos];
  } else {
    tok = tokens[b];
  }
  if (tok < 0 || tok >= vocab) return;
  out[(size_t)b * chunks + chunk] = table[(size_t)tok * chunks + chunk];
}

// argmax with torch's tie rule (first index of the maximum). Each workgroup reduces a
// chunk of one row to (value, index); the last workgroup reduces the chunks in order.
constexpr int kArgmaxChunk = 1024;

DF_DEVICE void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__global__ __launch_bounds__(256) void argmax_kernel(const uint16_t* __restrict__ logits, int rows, int n,
                                                     int64_t* __restrict__ tokens, int64_t* __restrict__ log,
                                                     int log_stride, int* position, int advance, int* step,
                                                     float* pv, int* pi, int* counter) {
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ int last;
  const int chunks = (n + kArgmaxChunk - 1) / kArgmaxChunk;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const uint16_t* lr = logits + (size_t)row * n;
  float v = -INFINITY;
  int idx = 0x7FFFFFFF;
  const int end = min(n, (chunk + 1) * kArgmaxChunk);
  float vals[kArgmaxChunk / 256];
#pragma unroll
  for (int j = 0; j < kArgmaxChunk / 256; ++j) {
    const int k = chunk * kArgmaxChunk + j * 256 + threadIdx.x;
    vals[j] = k < end ? bf2f(lr[k]) : -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < kArgmaxChunk / 256; ++j) {
    const int k = chunk * kArgmaxChunk + j * 256 + threadIdx.x;
    if (k < end) argmax_merge(v, idx, vals[j], k);
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    argmax_merge(v, idx, ov, oi);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) argmax_merge(v, idx, sv[w], si[w]);
    store_through(pv + row * chunks + chunk, v);
    store_through(pi + row * chunks + chunk, idx);
    publish_wait();
    last = arrive(counter) == rows * chunks - 1;
  }
  __syncthreads();
  if (!last) return;
  // Final reduction per row: every thread takes chunk partials at once, then lanes and
  // waves merge (the tie rule keeps the lowest index, so the order does not matter).
  for (int r = 0; r < rows; ++r) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int c = threadIdx.x; c < chunks; c += 256)
      argmax_merge(bv, bi, load_through(pv + r * chunks + c), load_through(pi + r * chunks + c));
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      argmax_merge(bv, bi, ov, oi);
    }
    __syncthreads();
    if (lane == 0) {
      sv[wave] = bv;
      si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < 4; ++w) argmax_merge(bv, bi, sv[w], si[w]);
      tokens[r] = bi;
      if (log && step) log[(size_t)r * log_stride + *step] = bi;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if (position) *position += advance;
    if (step) *step += 1;
    *counter = 0;
  }
}

}  // namespace df

using namespace df;

extern "C" {

int df_rms_norm(const uint16_t* x, const uint16_t* w, float eps, int rows, int n, uint16_t* out, hipStream_t stream) {
  if (!x || !w || !out || rows < 1 || n < 1) return DF_BAD_ARGUMENT;
  hipLaunchKernelGGL(rms_norm_kernel<false>, dim3(rows), dim3(256), 0, stream, x, nullptr, w, eps, n, nullptr, out);
  DF_RETURN_LAUNCH_STATUS();
}

int df_add_rms_norm(const uint16_t* x, const uint16_t* residual, const uint16_t* w, float eps, int rows, int n,
                    uint16_t* resid_out, uint16_t* out, hipStream_t stream) {
  if (!x || !residual || !w || !resid_out || !out || rows < 1 || n < 1) return DF_BAD_ARGUMENT;
  hipLaunchKernelGGL(rms_norm_kernel<true>, dim3(rows), dim3(256), 0, stream, x, residual, w, eps, n, resid_out,
                     out);
  DF_RETURN_LAUNCH_STATUS();
}

int df_silu_mul(const uint16_t* gate, const uint16_t* up, size_t n, uint16_t* out, hipStream_t stream) {
  if (!gate || !up || !out) return DF_BAD_ARGUMENT;
  if (n == 0) return DF_OK;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, gate, up, n, out);
  DF_RETURN_LAUNCH_STATUS();
}

int df_partial_rope(const uint16_t* x, const uint16_t* cos, const uint16_t* sin, int batch, int heads, int seq,
                    int head_dim, int rotary_dim, uint16_t* out, hipStream_t stream) {
  if (!x || !cos || !sin || !out || batch < 1 || heads < 1 || seq < 1 || head_dim < 1 || rotary_dim % 2 ||
      rotary_dim > head_dim || rotary_dim < 0)
    return DF_BAD_ARGUMENT;
  const int rows = batch * heads * seq;
  hipLaunchKernelGGL(partial_rope_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, x, cos, sin, heads, seq,
                     head_dim, rotary_dim, out, rows);
  DF_RETURN_LAUNCH_STATUS();
}

int df_causal_conv_step(const uint16_t* x, uint16_t* conv_cache, const uint16_t* weight, int batch, int channels,
                        uint16_t* out, hipStream_t stream) {
  if (!x || !conv_cache || !weight || !out || batch < 1 || channels < 1) return DF_BAD_ARGUMENT;
  const size_t total = (size_t)batch * channels;
  hipLaunchKernelGGL(causal_conv_step_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, x, conv_cache,
                     weight, channels, total, out);
  DF_RETURN_LAUNCH_STATUS();
}

int df_embed_int4(const int64_t* tokens, const int64_t* prompt, int prompt_len, const int* position, int batch,
                  const uint8_t* w_tiled, const uint16_t* s_tiled, int hidden, int vocab, uint16_t* out,
                  hipStream_t stream) {
  if ((!tokens && !prompt) || (prompt && (!position || prompt_len < 1)) || !w_tiled || !s_tiled || !out ||
      batch < 1 || hidden % 256 || vocab % 16)
    return DF_BAD_ARGUMENT;
  const int work = hidden / 128 * 16;
  hipLaunchKernelGGL(embed_int4_kernel, dim3((work + 255) / 256, batch), dim3(256), 0, stream, tokens, prompt,
                     prompt_len, position, reinterpret_cast<const uint32_t*>(w_tiled), s_tiled, hidden, vocab, out);
  DF_RETURN_LAUNCH_STATUS();
}

int df_embed_bf16(const int64_t* tokens, const int64_t* prompt, int prompt_len, const int* position, int batch,
                  const uint16_t* table, int hidden, int vocab, uint16_t* out, hipStream_t stream) {
  if ((!tokens && !prompt) || (prompt && (!position || prompt_len < 1)) || !table || !out || batch < 1 ||
      hidden % 8 || vocab < 1)
    return DF_BAD_ARGUMENT;
  const int chunks = hidden / 8;
  hipLaunchKernelGGL(embed_bf16_kernel, dim3((chunks + 255) / 256, batch), dim3(256), 0, stream, tokens, prompt,
                     prompt_len, position, reinterpret_cast<const uint4*>(table), hidden, vocab,
                     reinterpret_cast<uint4*>(out));
  DF_RETURN_LAUNCH_STATUS();
}

size_t df_argmax_workspace_bytes(int rows, int n) {
  const size_t chunks = (size_t)(n + kArgmaxChunk - 1) / kArgmaxChunk;
  return 256 + rows * chunks * (sizeof(float) + sizeof(int));
}

int df_argmax(const uint16_t* logits, int rows, int n, int64_t* tokens, int64_t* token_log, int log_stride,
              int* position, int advance, int* step, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!logits || !tokens || rows < 1 || rows > 256 || n < 1) return DF_BAD_ARGUMENT;
  if (token_log && !step) return DF_BAD_ARGUMENT;
  if (!workspace || workspace_bytes < df_argmax_workspace_bytes(rows, n)) return DF_WORKSPACE_TOO_SMALL;
  const int chunks = (n + kArgmaxChunk - 1) / kArgmaxChunk;
  char* p = reinterpret_cast<char*>(workspace);
  int* counter = reinterpret_cast<int*>(p);
  float* pv = reinterpret_cast<float*>(p + 256);
  int* pi = reinterpret_cast<int*>(pv + (size_t)rows * chunks);
  hipLaunchKernelGGL(argmax_kernel, dim3(chunks, rows), dim3(256), 0, stream, logits, rows, n, tokens, token_log,
                     log_stride, position, advance, step, pv, pi, counter);
  DF_RETURN_LAUNCH_STATUS();
}

}  // extern "C"
