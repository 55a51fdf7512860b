// Persistent bs=1 decode for gfx950: every phase of every token in one cooperative launch.
//
// Partitioning (8-way tensor parallelism over the 8 XCDs, 32 workgroups each; workgroup
// i runs on XCD i % 8, checked against HW_REG_XCC_ID):
//   Gated DeltaNet layer  XCD x: key heads 2x, 2x+1, value heads 4x..4x+3. in_proj is
//                         column-parallel (1552 columns per XCD), the conv + delta step
//                         runs on the XCD's own heads, out_proj is row-parallel over the
//                         XCD's 512 value channels.
//   gated attention layer XCD x: query heads 2x, 2x+1 (KV head x/2, shared by the XCD
//                         pair, written by the even XCD). q|k|v column-parallel (1536
//                         columns), 32 KV splits = the 32 workgroups, o_proj row-parallel.
//   MLP                   gate|up column-parallel (inter/8 columns of each), down
//                         row-parallel over the same inter/8 channels.
//   head                  vocab/8 columns per XCD; argmax over 256 workgroup candidates.
// Row-parallel outputs are the only data crossing XCDs: each XCD writes its fp32 partial
// of the hidden vector with write-through stores, each workgroup sums one 1/32 slice of
// the 8 partials in XCD order, adds the residual and publishes the new hidden vector to
// its XCD. Every other hand-off stays inside one XCD's L2 (plain stores, agent-scope
// loads, a per-workgroup epoch flag), which costs ~0.4 us instead of ~3 us across XCDs.
//
// Workgroup = 8 compute waves + 1 control wave. On gfx9 vector loads retire in order, so a
// wave that has weight loads in flight cannot see a flag or an activation before those
// weights land. The compute waves therefore only issue weight / state / KV prefetches
// and then work out of LDS and registers; the control wave polls the hand-offs, stages
// activations and norm weights into LDS, and does the output stores and the signalling.
// Each phase's weights are requested before its input hand-off is awaited.
//
// Arithmetic is the per-op kernels' (int4_gemv.hip, gated_delta.hip, attention.hip,
// small_ops.hip), with the reference's rounding points; only fp32 summation orders differ.
#include "common.h"
#include "deltaforge_hip.h"
#include "int4_block.h"

namespace df {
namespace pd {

constexpr int kXcd = 8;
constexpr int kPerXcd = 32;
constexpr int kNwg = kXcd * kPerXcd;
constexpr int kCompute = 8;
constexpr int kCtl = kCompute;                      // wave index of the control wave
constexpr int kThreads = (kCompute + 1) * 64;       // 576
constexpr int kCThreads = kCompute * 64;            // 512 compute threads
constexpr int kMaxHidden = 2560;
constexpr int kMaxNb = 12;                          // weight blocks per compute wave per phase
constexpr int kMaxWgTiles = 8;
constexpr int kDepthH = 8;                          // head pipeline depth (blocks per wave)
constexpr int kColparMax = 2304;
// Gated DeltaNet geometry
constexpr int kKH = 16, kVH = 32, kDk = 128;
constexpr int kKeyDim = kKH * kDk;                  // 2048
constexpr int kConvCh = 2 * kKeyDim + kVH * kDk;    // 8192
constexpr int kLinCols = 1552;
constexpr int kLinQ = 0, kLinK = 256, kLinV = 512, kLinZ = 1024, kLinA = 1536, kLinB = 1540;
// attention geometry
constexpr int kQH = 16, kKVH = 4, kHd = 256, kRot = 64;
constexpr int kAttnCols = 1536;
constexpr int kAttnK = 1024, kAttnV = 1280;
constexpr int kApHead = kHd + 2;                    // acc[256], m, l
constexpr int kTileKeys = kCompute * 16;            // 128 keys per attention tile

constexpr uint64_t kTimeout = 50000000ull;          // 0.5 s of s_memrealtime (100 MHz)
constexpr int kRegBase = 4;                         // ctl[4..11]: per-XCD registration tickets

enum Err : int { kErrNone = 0, kErrTimeout = 1, kErrXcd = 2, kErrPosition = 3, kErrToken = 4 };

struct Ws {
  int* ctl;          // [16]: epoch, abort, error, -, 8 registration tickets, -
  int* flags;        // [8][32] last epoch each workgroup finished
  float* colpar;     // [8][2][kColparMax] column-parallel partial outputs, 2 slots
  uint16_t* hloc;    // [8][hidden] the hidden vector, one copy per XCD
  uint16_t* core;    // [8][512] DeltaNet core / merged attention output of the XCD
  float* apart;      // [8][32 splits][2 heads][kApHead]
  uint64_t* rowpar;  // [2][8][hidden] (fp32 value, u32 epoch) row-parallel partials
  uint64_t* cand;    // [256] argmax candidates (value, index, epoch bits)
};

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

__host__ __device__ inline size_t ws_layout(int hidden, Ws* w, char* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = align256(off + bytes);
    return base ? base + at : nullptr;
  };
  char* ctl = take(16 * sizeof(int));
  char* flags = take((size_t)kXcd * kPerXcd * sizeof(int));
  char* colpar = take((size_t)kXcd * 2 * kColparMax * sizeof(float));
  char* hloc = take((size_t)kXcd * hidden * sizeof(uint16_t));
  char* core = take((size_t)kXcd * 512 * sizeof(uint16_t));
  char* apart = take((size_t)kXcd * kPerXcd * 2 * kApHead * sizeof(float));
  char* rowpar = take((size_t)2 * kXcd * hidden * sizeof(uint64_t));
  char* cand = take((size_t)kNwg * sizeof(uint64_t));
  if (w) {
    w->ctl = reinterpret_cast<int*>(ctl);
    w->flags = reinterpret_cast<int*>(flags);
    w->colpar = reinterpret_cast<float*>(colpar);
    w->hloc = reinterpret_cast<uint16_t*>(hloc);
    w->core = reinterpret_cast<uint16_t*>(core);
    w->apart = reinterpret_cast<float*>(apart);
    w->rowpar = reinterpret_cast<uint64_t*>(rowpar);
    w->cand = reinterpret_cast<uint64_t*>(cand);
  }
  return off;
}

// ---------------------------------------------------------------------------------------
// memory helpers
// ---------------------------------------------------------------------------------------

DF_DEVICE uint64_t now() { return __builtin_amdgcn_s_memrealtime(); }
template <class T>
DF_DEVICE T ld_agent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
DF_DEVICE T ld_sys(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
template <class T>
DF_DEVICE void st_sys(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// bf16 pair loads of XCD-local data (bypassing the CU's L1)
DF_DEVICE uint32_t ld_agent_u32(const uint16_t* p) { return ld_agent(reinterpret_cast<const uint32_t*>(p)); }

DF_DEVICE uint64_t pack_epoch(float v, uint32_t epoch) {
  return (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v);
}
DF_DEVICE uint64_t pack_cand(float v, int index, uint32_t epoch) {
  return (static_cast<uint64_t>(__float_as_uint(v)) << 32) | (static_cast<uint32_t>(index) << 14) | (epoch & 0x3FFFu);
}

// ---------------------------------------------------------------------------------------
// per-workgroup context and LDS
// ---------------------------------------------------------------------------------------

struct Ctx {
  DfPersistModel M;
  Ws w;
  int xcd, r, tid, wave, lane;
  bool control;
  uint32_t epoch;   // last epoch this workgroup reached (all workgroups agree on the sequence)
  int ar;           // row-parallel all-reduce counter (selects the rowpar buffer)
  int pos;          // position of the token being decoded
  uint64_t* tr;     // phase trace of the traced step (workgroup (0, 0), control wave), or null
  int tn;
};

// Phase trace of the traced step: s_memrealtime << 8 | tag (tags: 1-15 phase starts, 20
// staged after the hand-off, 30 signalled).
enum Tag : int { kTProj = 1, kTDelta, kTOut, kTAttn, kTMerge, kTOProj, kTGateUp, kTDown, kTHead, kTEmbed,
                 kTReduce, kTStaged = 20, kTSignal = 30 };
DF_DEVICE void stamp(Ctx& c, int tag) {
  if (c.tr) {
    if (c.control && c.lane == 0 && c.xcd == 0 && c.r == 0 && c.tn < c.M.trace_capacity)
      c.tr[c.tn] = (now() << 8) | static_cast<uint64_t>(tag);
    c.tn += 1;
  }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void gbl_void;

struct Lds {
  uint16_t h[kMaxHidden];                        // the hidden vector (bf16)
  __align__(16) uint16_t x[2][kMaxHidden + 8];   // GEMV activation row; row 1 stays zero
  __align__(16) uint16_t nw[kMaxHidden];         // staged norm weight
  float part[kMaxWgTiles][kCompute][16];         // per-wave tile partials
  float gated_z[512];                            // SiLU inputs of the GatedRMSNorm
  float red[64];
  int ok;
  int token;
  struct {                                       // head
    __align__(16) uint16_t logit[kMaxWgTiles * 8 * 16];  // up to 64 tiles
    float bv[kCompute];
    int bi[kCompute];
  } hd;
  union {
    // weight blocks of the current GEMV phase (or the head's ring), written by LDS DMA;
    // wave w owns wblk[w]
    struct {
      __align__(16) uint4 wblk[kCompute][kMaxNb][64];
      uint32_t sblk[kCompute][kMaxNb][64];       // scale dwords: lane i holds columns 2(i/2 % 8) +0/+1
    } wq;
    struct {                                     // Gated DeltaNet step
      float qkv_in[272];                         // pre-conv inputs: q 128, k 128, v 16
      float q[kDk], k[kDk], v[16];
      float sred[kCompute][16];
      float ab8[8];                              // a of the XCD's 4 value heads, then b
      float scal[4];
    } dn;
    struct {                                     // attention split
      __align__(16) uint16_t q[2][kHd];
      __align__(16) uint16_t knew[kHd];
      __align__(16) uint16_t vnew[kHd];
      float qraw[2][kHd];
      float kraw[kHd];
      float vraw[kHd];
      __align__(16) uint16_t qn_w[kHd];
      __align__(16) uint16_t kn_w[kHd];
      float inv[kRot / 2];
      float sc[2][kTileKeys];
      float alpha[2];
      float ml[2][2];
      float red[kCompute][2][kHd];               // 16 KB
    } at;
    struct {                                     // split merge
      float m[kPerXcd], l[kPerXcd], wgt[kPerXcd];
      float acc[kPerXcd][16];
      float gate[16];
      float den;
    } mg;
    struct {                                     // all-reduce slice
      float y[kXcd][128];
    } rd;
  } u;
};

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int N>
DF_DEVICE void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Re-derive the thread's coordinates at the start of a phase behind an opaque asm, so the
// compiler cannot hoist each phase's lane- and workgroup-derived addresses out of the layer
// loop (keeping every phase's values live at once spills hundreds of registers). The wave
// index is read back as a scalar so role branches stay uniform.
DF_DEVICE void fence(Ctx& c, int tag = 0) {
  int tid = threadIdx.x, xcd = c.xcd, r = c.r;
  asm volatile("" : "+v"(tid), "+v"(xcd), "+v"(r));
  c.tid = tid;
  c.lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  c.control = c.wave == kCtl;
  c.xcd = __builtin_amdgcn_readfirstlane(xcd);
  c.r = __builtin_amdgcn_readfirstlane(r);
  if (tag) stamp(c, tag);
}

DF_DEVICE void raise_abort(const Ctx& c, int err) {
  st_sys(c.w.ctl + 2, err);
  st_sys(c.w.ctl + 1, 1);
}

// Control wave: wait until the 32 workgroups of this XCD have reached `epoch`.
DF_DEVICE bool wait_local(const Ctx& c, uint32_t epoch) {
  const int* f = c.w.flags + c.xcd * kPerXcd;
  const uint64_t t0 = now();
  for (;;) {
    const int v = c.lane < kPerXcd ? ld_agent(f + c.lane) : static_cast<int>(epoch);
    if (__all(v >= static_cast<int>(epoch))) return true;
    if (ld_sys(c.w.ctl + 1)) return false;
    if (now() - t0 > kTimeout) {
      raise_abort(c, kErrTimeout);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// All threads: make this workgroup's stores visible, then the control wave publishes `epoch`.
DF_DEVICE void signal_local(Ctx& c, uint32_t epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  stamp(c, kTSignal);
  if (c.control && c.lane == 0) {
    // a plain store lands in this XCD's L2, where the agent-scope polls of the other
    // workgroups of the XCD read it
    *reinterpret_cast<volatile int*>(c.w.flags + c.xcd * kPerXcd + c.r) = static_cast<int>(epoch);
  }
}

// ---------------------------------------------------------------------------------------
// block reductions over all 9 waves (LDS only)
// ---------------------------------------------------------------------------------------

DF_DEVICE float block_sum9(float v, Lds& L, const Ctx& c) {
  v = wave_sum(v);
  __syncthreads();
  if (c.lane == 0) L.red[c.wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i <= kCompute; ++i) t += L.red[i];
  return t;
}

// x row 0 = RMSNorm(h) * (1 + w) over `hidden` (w staged in L.nw); row 1 zero.
DF_DEVICE void norm_prologue(Lds& L, const Ctx& c, int hidden, float eps) {
  float ss = 0.0f;
  for (int k = c.tid; k < hidden; k += kThreads) {
    const float v = bf2f(L.h[k]);
    ss += v * v;
  }
  ss = block_sum9(ss, L, c);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
  for (int k = c.tid; k < hidden; k += kThreads) {
    const float scaled = bf2f(L.h[k]) * r;
    L.x[0][k] = f2bf(scaled * (1.0f + bf2f(L.nw[k])));
    L.x[1][k] = 0;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------
// GEMV phase over a block range of this XCD's slice
// ---------------------------------------------------------------------------------------

struct Gemv {
  const uint8_t* w;
  const uint16_t* s;
  int G;       // groups per tile in the stored matrix
  int tile0;   // first tile of the XCD slice
  int g0, ng;  // group slice
  int b_lo, b_hi;  // this workgroup's block range (relative to the slice, tile-major)
};

struct WaveBlocks {
  int lo, n;
};

// One block (1 KB of nibbles) and its 16 scales into ring slot (wave, slot) by LDS DMA
// (dword granularity: lane i loads the scale pair holding its column i % 16).
DF_DEVICE void dma_block(const uint8_t* w, const uint16_t* s, size_t blk, int wave, int slot, int lane, Lds& L) {
  __builtin_amdgcn_global_load_lds((gbl_void*)(w + blk * kBlockBytes + lane * 16),
                                   (lds_void*)&L.u.wq.wblk[wave][slot][0], 16, 0, 0);
  __builtin_amdgcn_global_load_lds((gbl_void*)(s + blk * kTileCols + (lane & 14)),
                                   (lds_void*)&L.u.wq.sblk[wave][slot][0], 4, 0, 0);
}
DF_DEVICE uint16_t block_scale(const Lds& L, int wave, int slot, int lane) {
  return static_cast<uint16_t>(L.u.wq.sblk[wave][slot][lane] >> (16 * (lane & 1)));
}

DF_DEVICE void wave_range(const Gemv& g, int wave, int& lo, int& n) {
  const int len = g.b_hi - g.b_lo;
  lo = g.b_lo + (len * wave) / kCompute;
  n = g.b_lo + (len * (wave + 1)) / kCompute - lo;
}

// Compute waves: request this wave's blocks (issued before the phase's hand-off wait).
// Weights and scales go straight to this wave's LDS region (global_load_lds: lane i's
// bytes land at offset size * i, so a block keeps its register layout).
DF_DEVICE void gemv_issue(const Gemv& g, const Ctx& c, WaveBlocks& B, Lds& L) {
  wave_range(g, c.wave, B.lo, B.n);
#pragma unroll 1
  for (int i = 0; i < B.n; ++i) {
    const int b = B.lo + i;
    const int t = g.tile0 + b / g.ng, gg = g.g0 + b % g.ng;
    dma_block(g.w, g.s, (size_t)t * g.G + gg, c.wave, i, c.lane, L);
  }
}

// Compute waves: MFMA over the requested blocks with x row 0 of L.x (the K slice of the
// phase, index k - 128 * g0); per-tile partials of row 0 go to L.part[tile - first][wave].
DF_DEVICE void gemv_compute(const Gemv& g, const Ctx& c, const WaveBlocks& B, Lds& L) {
  wait_vm<0>();  // this wave's weight blocks and scales have landed
  const int col = c.lane & 15, slot = c.lane >> 4;
  const uint16_t* xrow = &L.x[col == 0 ? 0 : 1][slot * 32];
  const int t_first = g.b_lo / g.ng;
  df_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int cur = B.n > 0 ? B.lo / g.ng : 0;
#pragma unroll 1
  for (int i = 0; i < B.n; ++i) {
    const int b = B.lo + i;
    const int t = b / g.ng, gl = b % g.ng;
    if (t != cur) {
      if (c.lane < 16) L.part[cur - t_first][c.wave][c.lane] = acc[0];
      acc = df_f32x4{0.f, 0.f, 0.f, 0.f};
      cur = t;
    }
    const uint4 wv = L.u.wq.wblk[c.wave][i][c.lane];
    const GroupScale gs = group_scale(block_scale(L, c.wave, i, c.lane));
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint4 bw = dequant8(words[d], gs);
      const uint4 aw = *reinterpret_cast<const uint4*>(xrow + gl * kGroup + d * 8);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, aw),
                                                    __builtin_bit_cast(df_bf16x8, bw), acc, 0, 0, 0);
    }
  }
  if (B.n > 0 && c.lane < 16) L.part[cur - t_first][c.wave][c.lane] = acc[0];
}

DF_DEVICE void zero_part(Lds& L, const Ctx& c) {
  for (int e = c.tid; e < kMaxWgTiles * kCompute * 16; e += kThreads) (&L.part[0][0][0])[e] = 0.0f;
}

// Sum of the waves' partials for relative tile t (fixed wave order).
DF_DEVICE float part_sum(const Lds& L, int t, int col) {
  float v = 0.0f;
#pragma unroll
  for (int wv = 0; wv < kCompute; ++wv) v += L.part[t][wv][col];
  return v;
}

// ---------------------------------------------------------------------------------------
// Phase drivers. Each follows the same barrier schedule on every wave:
//   compute waves: issue loads | control: wait + stage   -> sync
//   all: prologue (LDS)                                  -> sync
//   compute waves: compute                               -> sync
//   all: epilogue stores; signal
// ---------------------------------------------------------------------------------------

// ---- control-wave staging: every load of a hand-off is issued before any is used -------

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int df_i4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int df_i2;
constexpr int kCpPlain = 0, kCpAgent = 16, kCpSystem = 17;  // buffer cache policy: -, sc1, sc0|sc1

DF_DEVICE __amdgpu_buffer_rsrc_t rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, 0x00020000);
}
template <int CP>
DF_DEVICE uint4 ld16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CP));
}
template <int CP>
DF_DEVICE uint64_t ld8(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, CP));
}

// n bf16 (n % 8 == 0, n <= 512 K) from global memory into LDS.
template <int K, int CP>
DF_DEVICE void stage16(uint16_t* dst, const uint16_t* src, int n, int lane) {
  const auto r = rsrc(src);
  uint4 v[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = lane + 64 * k;
    if (ch * 8 < n) v[k] = ld16<CP>(r, ch * 16);
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = lane + 64 * k;
    if (ch * 8 < n) *reinterpret_cast<uint4*>(dst + ch * 8) = v[k];
  }
}
constexpr int kHidChunks = (kMaxHidden / 8 + 63) / 64;  // 16-byte chunks per lane of a hidden row

// A run of XCD-local columns [j0, j0 + n) of the column-parallel outputs (j0, n multiples of
// 4), delivered as bf16-rounded slot sums into dst.
struct Seg {
  int j0, n;
  float* dst;
};

// Up to NS segments, K 16-byte chunks per lane and slot.
template <int NS, int K>
DF_DEVICE void gather_colpar(const Ctx& c, const Seg (&seg)[NS]) {
  const auto r = rsrc(c.w.colpar + (size_t)c.xcd * 2 * kColparMax);
  int start[NS + 1];
  start[0] = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) start[s + 1] = start[s] + seg[s].n / 4;
  uint4 a[K], b[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = c.lane + 64 * k;
    if (ch < start[NS]) {
      int col = 0;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        if (ch >= start[s] && ch < start[s + 1]) col = seg[s].j0 + 4 * (ch - start[s]);
      a[k] = ld16<kCpAgent>(r, col * 4);
      b[k] = ld16<kCpAgent>(r, (kColparMax + col) * 4);
    }
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = c.lane + 64 * k;
    if (ch < start[NS]) {
      float* d = nullptr;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        if (ch >= start[s] && ch < start[s + 1]) d = seg[s].dst + 4 * (ch - start[s]);
      d[0] = round_bf(__uint_as_float(a[k].x) + __uint_as_float(b[k].x));
      d[1] = round_bf(__uint_as_float(a[k].y) + __uint_as_float(b[k].y));
      d[2] = round_bf(__uint_as_float(a[k].z) + __uint_as_float(b[k].z));
      d[3] = round_bf(__uint_as_float(a[k].w) + __uint_as_float(b[k].w));
    }
  }
}

// The down projection's input: act = bf16(bf16(silu(g)) * u) over the XCD's inter_x gate|up
// column pairs (16-column gate tile, then its up tile), straight from the column-parallel
// slots. Chunk ch (4 columns) of pair ch / 8 is a gate chunk for ch % 8 < 4; its up
// partner is chunk ch + 4, held 4 lanes up.
template <int K>
DF_DEVICE void stage_act(const Ctx& c, int inter_x, Lds& L) {
  const auto r = rsrc(c.w.colpar + (size_t)c.xcd * 2 * kColparMax);
  const int chunks = inter_x / 2;
  uint4 a[K], b[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = c.lane + 64 * k;
    if (ch < chunks) {
      a[k] = ld16<kCpAgent>(r, ch * 16);
      b[k] = ld16<kCpAgent>(r, kColparMax * 4 + ch * 16);
    }
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = c.lane + 64 * k;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ch < chunks) {
      v[0] = round_bf(__uint_as_float(a[k].x) + __uint_as_float(b[k].x));
      v[1] = round_bf(__uint_as_float(a[k].y) + __uint_as_float(b[k].y));
      v[2] = round_bf(__uint_as_float(a[k].z) + __uint_as_float(b[k].z));
      v[3] = round_bf(__uint_as_float(a[k].w) + __uint_as_float(b[k].w));
    }
    float u[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = __shfl(v[e], (c.lane + 4) & 63, 64);
    if (ch < chunks && (c.lane & 7) < 4) {
      const int j = (ch / 8) * 16 + (ch % 8) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) L.x[0][j + e] = f2bf(round_bf(silu(v[e])) * u[e]);
    }
  }
}

// Column-parallel epilogue: this workgroup's partial of each tile it touched into its slot
// (r & 1); tiles wholly inside its range also zero the other slot.
DF_DEVICE void colpar_epilogue(const Gemv& g, const Ctx& c, const Lds& L) {
  const int t_first = g.b_lo / g.ng, t_last = (g.b_hi - 1) / g.ng;
  const int nt = t_last - t_first + 1;
  float* cp = c.w.colpar + (size_t)c.xcd * 2 * kColparMax;
  const int mine = c.r & 1;
  for (int e = c.tid; e < nt * 16; e += kThreads) {
    const int tr = e / 16, col = e % 16;
    const int t = t_first + tr;
    const float v = part_sum(L, tr, col);
    const int j = t * 16 + col;
    cp[mine * kColparMax + j] = v;
    const bool whole = t * g.ng >= g.b_lo && (t + 1) * g.ng <= g.b_hi;
    if (whole) cp[(mine ^ 1) * kColparMax + j] = 0.0f;
  }
}

// Row-parallel epilogue: the XCD's partial of hidden columns [16 t_first, ...) with epoch.
DF_DEVICE void rowpar_epilogue(const Gemv& g, const Ctx& c, const Lds& L, int hidden) {
  const int t_first = g.b_lo / g.ng, nt = (g.b_hi - g.b_lo) / g.ng;
  uint64_t* rp = c.w.rowpar + ((size_t)(c.ar & 1) * kXcd + c.xcd) * hidden;
  for (int e = c.tid; e < nt * 16; e += kThreads) {
    const int tr = e / 16, col = e % 16;
    st_sys(rp + (t_first + tr) * 16 + col, pack_epoch(part_sum(L, tr, col), c.epoch));
  }
}

// The all-reduce after a row-parallel phase (control wave polls, all waves finish):
// slice [sl0, sl0 + ns) of y = sum over XCDs (in order); h = bf16(h + bf16(y)); publish
// the slice to this XCD's copy of h; wait for the XCD; read all of h back into LDS.
DF_DEVICE bool allreduce_residual(Ctx& c, Lds& L, int hidden) {
  fence(c, kTReduce);
  const int ns = hidden / kPerXcd;  // <= 128
  const int sl0 = c.r * ns;
  const uint64_t* rp = c.w.rowpar + (size_t)(c.ar & 1) * kXcd * hidden;
  if (c.control) {
    // slice [sl0, sl0 + ns) of the 8 XCD partials: item i = (x = i / ns, column i % ns)
    constexpr int K = (kXcd * (kMaxHidden / kPerXcd) + 63) / 64;
    const auto r = rsrc(rp);
    const int items = kXcd * ns;
    uint64_t v[K];
    bool ok = true;
    const uint64_t t0 = now();
    for (;;) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = c.lane + 64 * k;
        if (i < items) v[k] = ld8<kCpSystem>(r, ((i / ns) * hidden + sl0 + i % ns) * 8);
      }
      bool ready = true;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = c.lane + 64 * k;
        if (i < items) ready = ready && static_cast<uint32_t>(v[k] >> 32) == c.epoch;
      }
      if (__all(ready)) break;
      if (ld_sys(c.w.ctl + 1)) { ok = false; break; }
      if (now() - t0 > kTimeout) { raise_abort(c, kErrTimeout); ok = false; break; }
      __builtin_amdgcn_s_sleep(1);
    }
    if (ok) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = c.lane + 64 * k;
        if (i < items) L.u.rd.y[i / ns][i % ns] = __uint_as_float(static_cast<uint32_t>(v[k]));
      }
    }
    if (c.lane == 0) L.ok = ok;
  }
  __syncthreads();
  if (!L.ok) return false;
  // h slice update (one thread per column)
  uint16_t* hx = c.w.hloc + (size_t)c.xcd * hidden;
  if (c.tid < ns) {
    float y = 0.0f;
#pragma unroll
    for (int x = 0; x < kXcd; ++x) y += L.u.rd.y[x][c.tid];
    const int k = sl0 + c.tid;
    const uint16_t hn = f2bf(bf2f(L.h[k]) + round_bf(y));
    hx[k] = hn;
  }
  c.ar += 1;
  c.epoch += 1;
  signal_local(c, c.epoch);
  if (c.control) {
    const bool ok = wait_local(c, c.epoch);
    if (ok) stage16<kHidChunks, kCpAgent>(L.h, hx, hidden, c.lane);
    if (c.lane == 0) L.ok = ok;
  }
  __syncthreads();
  return L.ok;
}

// ---------------------------------------------------------------------------------------
// Gated DeltaNet step for (value head 4x + r/8, value columns 16 (r%8) ..+15)
// ---------------------------------------------------------------------------------------

struct DnPre {
  float4 S;          // state row k = tid/4, columns 4 (tid%4) ..+3 of the slice
  float w[4];        // conv taps of this thread's channel (tid < 272)
  float h[3];        // its three history values (oldest first)
};

DF_DEVICE int dn_channel(const Ctx& c, int i) {
  // i in 0..271: q (128), k (128), v slice (16) of this workgroup's unit -> global channel
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int kh = 2 * c.xcd + (hvl >> 1), hv = 4 * c.xcd + hvl;
  if (i < 128) return kh * kDk + i;
  if (i < 256) return kKeyDim + kh * kDk + (i - 128);
  return 2 * kKeyDim + hv * kDk + vs * 16 + (i - 256);
}

DF_DEVICE void dn_issue(const Ctx& c, const DfPersistLayer& Lr, DnPre& P) {
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int hv = 4 * c.xcd + hvl;
  const int k = c.tid >> 2, c4 = c.tid & 3;
  P.S = *reinterpret_cast<const float4*>(Lr.state + ((size_t)hv * kDk + k) * kDk + vs * 16 + c4 * 4);
  if (c.tid < 272) {
    const int ch = dn_channel(c, c.tid);
    const uint2 wt = *reinterpret_cast<const uint2*>(Lr.conv_w + (size_t)ch * 4);
    P.w[0] = __uint_as_float(wt.x << 16);
    P.w[1] = __uint_as_float(wt.x & 0xFFFF0000u);
    P.w[2] = __uint_as_float(wt.y << 16);
    P.w[3] = __uint_as_float(wt.y & 0xFFFF0000u);
    const uint16_t* ring = Lr.conv_ring + (size_t)ch * 4;
    // ring slots (pos+1)&3, (pos+2)&3, (pos+3)&3 hold positions pos-3, pos-2, pos-1;
    // read at agent scope: another workgroup of the XCD writes the q/k slots
    const uint64_t rv = ld_agent(reinterpret_cast<const uint64_t*>(ring));
    const uint16_t sl[4] = {static_cast<uint16_t>(rv), static_cast<uint16_t>(rv >> 16),
                            static_cast<uint16_t>(rv >> 32), static_cast<uint16_t>(rv >> 48)};
    P.h[0] = bf2f(sl[(c.pos + 1) & 3]);
    P.h[1] = bf2f(sl[(c.pos + 2) & 3]);
    P.h[2] = bf2f(sl[(c.pos + 3) & 3]);
  }
}

// After the control wave staged the pre-conv inputs and gates (L.u.dn.qkv_in, ab).
DF_DEVICE void dn_compute(const Ctx& c, const DfPersistLayer& Lr, DnPre& P, Lds& L) {
#pragma clang fp contract(off)
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int hv = 4 * c.xcd + hvl;
  auto& D = L.u.dn;
  // conv + SiLU (fp32 sum in tap order, bf16, SiLU, bf16)
  if (c.tid < 272) {
    const float x = D.qkv_in[c.tid];
    float acc = P.h[0] * P.w[0];
    acc = acc + P.h[1] * P.w[1];
    acc = acc + P.h[2] * P.w[2];
    acc = acc + x * P.w[3];
    const float y = round_bf(silu(round_bf(acc)));
    if (c.tid < 128) D.q[c.tid] = y;
    else if (c.tid < 256) D.k[c.tid - 128] = y;
    else D.v[c.tid - 256] = y;
    // history: this unit owns its v slice; the (even value head, slice 0) unit owns the
    // key head's q/k channels
    const bool owner = c.tid >= 256 || ((hvl & 1) == 0 && vs == 0);
    if (owner) {
      uint16_t* ring = Lr.conv_ring + (size_t)dn_channel(c, c.tid) * 4;
      ring[c.pos & 3] = f2bf(x);
    }
  }
  if (c.tid == 0) {
    const float a = D.ab8[hvl], b = D.ab8[4 + hvl];
    const float beta = round_bf(sigmoid(b));
    const float g = -expf(bf2f(Lr.A_log[hv])) * softplus(a + bf2f(Lr.dt_bias[hv]));
    D.scal[0] = expf(g);
    D.scal[1] = beta;
  }
  __syncthreads();
  // L2 norms: wave 0 q, wave 1 k (2 values per lane)
  if (c.wave < 2) {
    float* vec = c.wave == 0 ? D.q : D.k;
    const float x0 = vec[c.lane * 2], x1 = vec[c.lane * 2 + 1];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float rr = 1.0f / sqrtf(ss + 1e-6f);
    float y0 = x0 * rr, y1 = x1 * rr;
    if (c.wave == 0) {
      const float scale = sqrtf(static_cast<float>(kDk));
      y0 = y0 / scale;
      y1 = y1 / scale;
    }
    vec[c.lane * 2] = y0;
    vec[c.lane * 2 + 1] = y1;
  }
  __syncthreads();
  const float eg = D.scal[0], beta = D.scal[1];
  const int k = c.tid >> 2, c4 = c.tid & 3;
  float part[4] = {0.f, 0.f, 0.f, 0.f};
  float kr = 0.f, qr = 0.f;
  if (!c.control) {
    kr = D.k[k];
    qr = D.q[k];
    P.S.x = P.S.x * eg;
    P.S.y = P.S.y * eg;
    P.S.z = P.S.z * eg;
    P.S.w = P.S.w * eg;
    part[0] = P.S.x * kr;
    part[1] = P.S.y * kr;
    part[2] = P.S.z * kr;
    part[3] = P.S.w * kr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = part[j];
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      part[j] = v;
    }
    if (c.lane < 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) D.sred[c.wave][c4 * 4 + j] = part[j];
    }
  }
  __syncthreads();
  float delta[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = c4 * 4 + j;
    float recalled = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kCompute; ++wv) recalled += D.sred[wv][col];
    delta[j] = (D.v[col] - recalled) * beta;
  }
  __syncthreads();  // sred is reused below
  if (!c.control) {
    P.S.x = P.S.x + kr * delta[0];
    P.S.y = P.S.y + kr * delta[1];
    P.S.z = P.S.z + kr * delta[2];
    P.S.w = P.S.w + kr * delta[3];
    float o[4] = {P.S.x * qr, P.S.y * qr, P.S.z * qr, P.S.w * qr};
    *reinterpret_cast<float4*>(Lr.state + ((size_t)hv * kDk + k) * kDk + vs * 16 + c4 * 4) = P.S;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = o[j];
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      o[j] = v;
    }
    if (c.lane < 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) D.sred[c.wave][c4 * 4 + j] = o[j];
    }
  }
  __syncthreads();
  if (c.tid < 16) {
    float o = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kCompute; ++wv) o += D.sred[wv][c.tid];
    c.w.core[(size_t)c.xcd * 512 + hvl * kDk + vs * 16 + c.tid] = f2bf(o);
  }
}

// ---------------------------------------------------------------------------------------
// attention split r of [0, pos] for query heads 2x, 2x+1
// ---------------------------------------------------------------------------------------

// RMSNorm(1+w) over 256 dims held 4 per lane, then partial RoPE (attention.hip's order).
DF_DEVICE void norm_rope4_lds(float x[4], const uint16_t* nw, float eps, const float* inv, float posf, int lane) {
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(kHd) + eps);
  float n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) n[i] = round_bf((x[i] * r) * (1.0f + bf2f(nw[lane * 4 + i])));
  constexpr int half = kRot / 2;
  float partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(n[i], half / 4, 64);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dim = lane * 4 + i;
    if (dim < kRot) {
      const float ang = posf * inv[dim % half];
      const float cs = round_bf(cosf(ang)), sn = round_bf(sinf(ang));
      const float rotated = dim < half ? -partner[i] : partner[i];
      x[i] = round_bf(round_bf(n[i] * cs) + round_bf(rotated * sn));
    } else {
      x[i] = n[i];
    }
  }
}

struct AtPre {
  uint4 kb[8];   // K rows: this lane's key (t0 + 16 wave + col), dims d*32 + slot*8 ..+7
  uint2 vb[16];  // V rows: keys t0 + 16 wave + j, dims 4 lane ..+3
};

DF_DEVICE void at_keys(const Ctx& c, int& j0, int& j1) {
  const int nkeys = c.pos + 1;
  const int per = (nkeys + kPerXcd - 1) / kPerXcd;
  j0 = min(c.r * per, nkeys);
  j1 = min(j0 + per, nkeys);
}

// Compute waves: prefetch the split's first tile of keys/values (not the new position).
DF_DEVICE void at_issue_tile(const Ctx& c, const DfPersistLayer& Lr, int t0, int j1, AtPre& P) {
  const int col = c.lane & 15, slot = c.lane >> 4;
  const int kvh = c.xcd >> 1;
  const size_t base = (size_t)kvh * c.M.max_len;
  const int key = t0 + c.wave * 16 + col;
  if (key < j1 && key != c.pos) {
    const uint16_t* kp = Lr.k_cache + (base + key) * kHd + slot * 8;
#pragma unroll
    for (int d = 0; d < 8; ++d) P.kb[d] = load16(kp + d * 32);
  }
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    const int kk = t0 + c.wave * 16 + jj;
    if (kk < j1 && kk != c.pos) P.vb[jj] = *reinterpret_cast<const uint2*>(Lr.v_cache + (base + kk) * kHd + c.lane * 4);
  }
}

// One 128-key tile: QK (MFMA), online softmax (waves 0 / 1 for heads 0 / 1), PV.
DF_DEVICE void at_tile(const Ctx& c, int t0, int j1, const AtPre& P, float acc[2][4], float& m_run,
                       float& l_run, Lds& L) {
  auto& A = L.u.at;
  const int col = c.lane & 15, slot = c.lane >> 4;
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  if (!c.control) {
    const int key = t0 + c.wave * 16 + col;
    const bool live = key < j1;
    df_f32x4 d4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      uint4 bw = make_uint4(0u, 0u, 0u, 0u);
      if (live) bw = key == c.pos ? *reinterpret_cast<const uint4*>(A.knew + d * 32 + slot * 8) : P.kb[d];
      uint4 aw = make_uint4(0u, 0u, 0u, 0u);
      if (col < 2) aw = *reinterpret_cast<const uint4*>(&A.q[col][d * 32 + slot * 8]);
      d4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, aw), __builtin_bit_cast(df_bf16x8, bw),
                                                   d4, 0, 0, 0);
    }
    if (slot == 0) {
      A.sc[0][c.wave * 16 + col] = live ? d4[0] * scale : -INFINITY;
      A.sc[1][c.wave * 16 + col] = live ? d4[1] * scale : -INFINITY;
    }
  }
  __syncthreads();
  if (c.wave < 2) {
    const int h = c.wave;
    const float s0 = A.sc[h][c.lane], s1 = A.sc[h][c.lane + 64];
    const float tmax = wave_max(fmaxf(s0, s1));
    const float mo = A.ml[h][0];
    const float m_new = fmaxf(mo, tmax);
    float p0 = 0.f, p1 = 0.f, alpha = 1.0f;
    if (m_new != -INFINITY) {
      p0 = s0 == -INFINITY ? 0.0f : expf(s0 - m_new);
      p1 = s1 == -INFINITY ? 0.0f : expf(s1 - m_new);
      alpha = mo == -INFINITY ? 0.0f : expf(mo - m_new);
    }
    const float lsum = wave_sum(p0 + p1);
    A.sc[h][c.lane] = p0;
    A.sc[h][c.lane + 64] = p1;
    if (c.lane == 0) {
      A.ml[h][0] = m_new;
      A.ml[h][1] = A.ml[h][1] * alpha + lsum;
      A.alpha[h] = alpha;
    }
  }
  __syncthreads();
  if (!c.control) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float a = A.alpha[h];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[h][i] *= a;
    }
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int kk = t0 + c.wave * 16 + jj;
      if (kk < j1) {
        const uint2 raw = kk == c.pos ? *reinterpret_cast<const uint2*>(A.vnew + c.lane * 4) : P.vb[jj];
        const float v0 = __uint_as_float(raw.x << 16), v1 = __uint_as_float(raw.x & 0xFFFF0000u);
        const float v2 = __uint_as_float(raw.y << 16), v3 = __uint_as_float(raw.y & 0xFFFF0000u);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float pr = A.sc[h][c.wave * 16 + jj];
          acc[h][0] += pr * v0;
          acc[h][1] += pr * v1;
          acc[h][2] += pr * v2;
          acc[h][3] += pr * v3;
        }
      }
    }
  }
  __syncthreads();
  (void)m_run;
  (void)l_run;
}

// ---------------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void decode_kernel(DfPersistModel M, Ws w, int steps, int teacher_forced) {
  __shared__ Lds L;
  Ctx c;
  c.M = M;
  c.w = w;
  c.ar = 0;
  const int hidden = M.hidden;
  const int G = hidden / kGroup;

  // Role = (XCD this workgroup runs on, its ticket among that XCD's workgroups). The
  // dispatcher spreads a launch round-robin over the XCDs but not from XCD 0 every time,
  // so the XCD comes from HW_REG_XCC_ID and the rank from a per-XCD counter that the
  // launcher clears before each launch.
  if (threadIdx.x == 0) {
    L.ok = 1;
    const int xcc = __builtin_amdgcn_s_getreg(0x1814) & 0xF;  // HW_REG_XCC_ID
    int ticket = kPerXcd;
    if (xcc < kXcd) ticket = atomicAdd(w.ctl + kRegBase + xcc, 1);
    if (ticket >= kPerXcd) {
      st_sys(w.ctl + 2, static_cast<int>(kErrXcd));
      st_sys(w.ctl + 1, 1);
      L.ok = 0;
    }
    L.token = xcc * kPerXcd + ticket;
  }
  __syncthreads();
  if (!L.ok) return;
  c.xcd = L.token / kPerXcd;
  c.r = L.token % kPerXcd;
  c.tr = nullptr;
  c.tn = 0;
  fence(c);
  __syncthreads();
  const uint32_t epoch0 = static_cast<uint32_t>(w.ctl[0]);
  c.epoch = epoch0;
  const int pos0 = *M.position;
  const int step0 = M.step ? *M.step : 0;
  if (pos0 < 0 || pos0 + steps > M.max_len || (teacher_forced && pos0 + steps > M.prompt_len) ||
      (!teacher_forced && M.token_log && step0 + steps > M.log_capacity)) {
    if (c.tid == 0 && c.xcd == 0 && c.r == 0) raise_abort(c, kErrPosition);
    return;
  }
  int64_t token = M.tokens[0];

  // per-XCD geometry of the phases
  const int inter_x = M.inter / kXcd;                  // intermediate channels per XCD
  const int gu_tiles = 2 * inter_x / kTileCols;         // gate|up tiles per XCD
  const int row_tiles = hidden / kTileCols;             // output tiles of row-parallel GEMVs
  const int rp_lo = (c.r * row_tiles) / kPerXcd, rp_hi = ((c.r + 1) * row_tiles) / kPerXcd;
  const int vocab_tiles = M.vocab / kTileCols / kXcd;

  for (int step = 0; step < steps; ++step) {
    c.pos = pos0 + step;
    c.tr = (M.trace && step == M.trace_step) ? M.trace : nullptr;
    c.tn = 0;
    // ---- embedding of the step's token (every workgroup, into L.h) --------------------
    fence(c, kTEmbed);
    if (teacher_forced) token = M.prompt[c.pos];
    if (token < 0 || token >= M.vocab) {
      if (c.tid == 0 && c.xcd == 0 && c.r == 0) raise_abort(c, kErrToken);
      return;
    }
    {
      const int tt = static_cast<int>(token / 16), cc = static_cast<int>(token % 16);
      const uint32_t* wt = reinterpret_cast<const uint32_t*>(M.head_w);
      for (int idx = c.tid; idx < G * 16; idx += kThreads) {  // idx = g*16 + s*4 + d
        const int g = idx / 16, s = (idx / 4) & 3, d = idx & 3;
        const size_t block = (size_t)tt * G + g;
        const uint32_t word = wt[block * 256 + (s * 16 + cc) * 4 + d];
        const float sc = bf2f(M.head_s[block * 16 + cc]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int sh = (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
          const int q = static_cast<int>((word >> sh) & 15u) - 8;
          L.h[g * 128 + s * 32 + d * 8 + e] = f2bf(static_cast<float>(q) * sc);
        }
      }
    }
    __syncthreads();

    for (int li = 0; li < M.num_layers; ++li) {
      const DfPersistLayer Lr = M.layers[li];
      // ================= input projection (column-parallel) =========================
      {
        fence(c, kTProj);
        const int cols = Lr.kind == 0 ? kLinCols : kAttnCols;
        const int nt = cols / kTileCols;
        Gemv g{Lr.proj_w, Lr.proj_s, G, c.xcd * nt, 0, G, 0, 0};
        const int B = nt * G;
        g.b_lo = (c.r * B) / kPerXcd;
        g.b_hi = ((c.r + 1) * B) / kPerXcd;
        WaveBlocks wb;
        if (!c.control) gemv_issue(g, c, wb, L);
        else stage16<kHidChunks, kCpPlain>(L.nw, Lr.in_norm, hidden, c.lane);  // h is already in LDS
        zero_part(L, c);
        __syncthreads();
        norm_prologue(L, c, hidden, M.eps);
        if (!c.control) gemv_compute(g, c, wb, L);
        __syncthreads();
        colpar_epilogue(g, c, L);
        c.epoch += 1;
        signal_local(c, c.epoch);
      }
      if (Lr.kind == 0) {
        // ================= conv + gated delta step ===================================
        fence(c, kTDelta);
        DnPre P;
        if (!c.control) dn_issue(c, Lr, P);
        if (c.control) {
          bool ok = wait_local(c, c.epoch);
          if (ok) {
            const int hvl = c.r >> 3, vs = c.r & 7, khl = hvl >> 1;
            const Seg seg[4] = {{kLinQ + khl * 128, 128, L.u.dn.qkv_in},
                                {kLinK + khl * 128, 128, L.u.dn.qkv_in + 128},
                                {kLinV + hvl * 128 + vs * 16, 16, L.u.dn.qkv_in + 256},
                                {kLinA, 8, L.u.dn.ab8}};
            gather_colpar<4, 2>(c, seg);
          }
          if (c.lane == 0) L.ok = ok;
        }
        __syncthreads();
        if (!L.ok) return;
        stamp(c, kTStaged);
        dn_compute(c, Lr, P, L);
        c.epoch += 1;
        signal_local(c, c.epoch);
        // ================= gated norm + out_proj (row-parallel) ======================
        {
          fence(c, kTOut);
          Gemv g{Lr.out_w, Lr.out_s, 4096 / kGroup, 0, c.xcd * 4, 4, 0, 0};
          g.b_lo = rp_lo * 4;
          g.b_hi = rp_hi * 4;
          WaveBlocks wb;
          if (!c.control) gemv_issue(g, c, wb, L);
          if (c.control) {
            bool ok = wait_local(c, c.epoch);
            if (ok) {
              // core (512) and z (512) of the XCD's four value heads
              stage16<1, kCpAgent>(L.x[0], c.w.core + (size_t)c.xcd * 512, 512, c.lane);
              const Seg seg[1] = {{kLinZ, 512, L.gated_z}};
              gather_colpar<1, 2>(c, seg);
              stage16<1, kCpPlain>(L.nw, Lr.gnorm_w, kDk, c.lane);
            }
            if (c.lane == 0) L.ok = ok;
          }
          zero_part(L, c);
          __syncthreads();
          if (!L.ok) return;
          stamp(c, kTStaged);
          // GatedRMSNorm per 128-head: 8 elements per thread of the first 64 threads of
          // each of waves 0..3 is simpler as one element per thread over 512 threads.
          {
            const int i = c.tid;  // 0..575; 512 elements
            float v = 0.f;
            if (i < 512) v = bf2f(L.x[0][i]);
            float ss = v * v;
            // a head is 128 consecutive elements = 2 waves; reduce within each wave, then pair
            ss = wave_sum(ss);
            if (c.lane == 0) L.red[c.wave] = ss;
            __syncthreads();
            if (i < 512) {
              const int h = i >> 7;
              const float tot = L.red[2 * h] + L.red[2 * h + 1];
              const float rr = 1.0f / sqrtf(tot / 128.0f + M.eps);
              const float t = round_bf(bf2f(L.nw[i & 127]) * round_bf(v * rr));
              L.x[0][i] = f2bf(t * silu(L.gated_z[i]));
              L.x[1][i] = 0;
            }
            __syncthreads();
          }
          if (!c.control) gemv_compute(g, c, wb, L);
          __syncthreads();
          c.epoch += 1;
          rowpar_epilogue(g, c, L, hidden);
          if (!allreduce_residual(c, L, hidden)) return;
        }
      } else {
        // ================= attention split ===========================================
        fence(c, kTAttn);
        int j0, j1;
        at_keys(c, j0, j1);
        AtPre P;
        if (!c.control && j0 < j1) at_issue_tile(c, Lr, j0, j1, P);
        auto& A = L.u.at;
        if (c.control) {
          bool ok = wait_local(c, c.epoch);
          if (ok) {
            const Seg seg[3] = {{0, kHd, A.qraw[0]}, {512, kHd, A.qraw[1]}, {kAttnK, 2 * kHd, A.kraw}};
            gather_colpar<3, 4>(c, seg);  // kraw and vraw are adjacent in LDS
            stage16<1, kCpPlain>(A.qn_w, Lr.q_norm, kHd, c.lane);
            stage16<1, kCpPlain>(A.kn_w, Lr.k_norm, kHd, c.lane);
            if (c.lane < kRot / 2) A.inv[c.lane] = M.inv_freq[c.lane];
            if (c.lane < 2) {
              A.ml[c.lane][0] = -INFINITY;
              A.ml[c.lane][1] = 0.0f;
            }
          }
          if (c.lane == 0) L.ok = ok;
        }
        __syncthreads();
        if (!L.ok) return;
        stamp(c, kTStaged);
        const float posf = static_cast<float>(c.pos);
        if (c.wave < 3) {
          float x[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = c.wave < 2 ? A.qraw[c.wave][c.lane * 4 + i] : A.kraw[c.lane * 4 + i];
          norm_rope4_lds(x, c.wave < 2 ? A.qn_w : A.kn_w, M.eps, A.inv, posf, c.lane);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (c.wave < 2) A.q[c.wave][c.lane * 4 + i] = f2bf(x[i]);
            else A.knew[c.lane * 4 + i] = f2bf(x[i]);
          }
        } else if (c.wave == 3) {
#pragma unroll
          for (int i = 0; i < 4; ++i) A.vnew[c.lane * 4 + i] = f2bf(A.vraw[c.lane * 4 + i]);
        }
        __syncthreads();
        // the even XCD of the pair writes the new key/value (write-through: the odd XCD
        // reads this row in later steps)
        if ((c.xcd & 1) == 0 && c.pos >= j0 && c.pos < j1 && c.tid < kHd / 2) {
          const size_t row = ((size_t)(c.xcd >> 1) * M.max_len + c.pos) * kHd;
          const uint32_t kw = static_cast<uint32_t>(A.knew[2 * c.tid]) | (static_cast<uint32_t>(A.knew[2 * c.tid + 1]) << 16);
          const uint32_t vw = static_cast<uint32_t>(A.vnew[2 * c.tid]) | (static_cast<uint32_t>(A.vnew[2 * c.tid + 1]) << 16);
          st_sys(reinterpret_cast<uint32_t*>(Lr.k_cache + row) + c.tid, kw);
          st_sys(reinterpret_cast<uint32_t*>(Lr.v_cache + row) + c.tid, vw);
        }
        float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        float m_run = -INFINITY, l_run = 0.f;
        for (int t0 = j0; t0 < j1; t0 += kTileKeys) {
          if (t0 != j0 && !c.control) at_issue_tile(c, Lr, t0, j1, P);
          at_tile(c, t0, j1, P, acc, m_run, l_run, L);
        }
        // combine the waves' PV partials; publish (acc, m, l) of both heads
        if (!c.control) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) A.red[c.wave][h][c.lane * 4 + i] = acc[h][i];
        }
        __syncthreads();
        {
          float* ap = c.w.apart + ((size_t)c.xcd * kPerXcd + c.r) * 2 * kApHead;
          for (int e = c.tid; e < 2 * kHd; e += kThreads) {
            const int h = e / kHd, d = e % kHd;
            float s = 0.0f;
#pragma unroll
            for (int wv = 0; wv < kCompute; ++wv) s += A.red[wv][h][d];
            ap[h * kApHead + d] = s;
          }
          if (c.tid < 2) {
            ap[c.tid * kApHead + kHd] = A.ml[c.tid][0];
            ap[c.tid * kApHead + kHd + 1] = A.ml[c.tid][1];
          }
        }
        c.epoch += 1;
        signal_local(c, c.epoch);
        // ================= merge the 32 splits: head r/16, dims 16 (r%16) ..+15 =======
        {
          fence(c, kTMerge);
          auto& Mg = L.u.mg;
          const int hl = c.r >> 4, d0 = (c.r & 15) * 16;
          if (c.control) {
            bool ok = wait_local(c, c.epoch);
            if (ok) {
              // split s: (m, l) of head hl and its accumulator dims d0 .. d0+15 (4 chunks)
              const float* ap = c.w.apart + (size_t)c.xcd * kPerXcd * 2 * kApHead + hl * kApHead;
              const auto r = rsrc(ap);
              uint64_t ml = 0;
              uint4 av[2];
              if (c.lane < kPerXcd) ml = ld8<kCpAgent>(r, (c.lane * 2 * kApHead + kHd) * 4);
#pragma unroll
              for (int k = 0; k < 2; ++k) {
                const int ch = c.lane + 64 * k;  // 128 chunks: split ch / 4, dims 4 (ch % 4)
                av[k] = ld16<kCpAgent>(r, ((ch / 4) * 2 * kApHead + d0 + 4 * (ch % 4)) * 4);
              }
              if (c.lane < kPerXcd) {
                Mg.m[c.lane] = __uint_as_float(static_cast<uint32_t>(ml));
                Mg.l[c.lane] = __uint_as_float(static_cast<uint32_t>(ml >> 32));
              }
#pragma unroll
              for (int k = 0; k < 2; ++k) {
                const int ch = c.lane + 64 * k;
                *reinterpret_cast<uint4*>(&Mg.acc[ch / 4][4 * (ch % 4)]) = av[k];
              }
              const Seg seg[1] = {{hl * 512 + kHd + d0, 16, Mg.gate}};
              gather_colpar<1, 1>(c, seg);
            }
            if (c.lane == 0) L.ok = ok;
          }
          __syncthreads();
          if (!L.ok) return;
          stamp(c, kTStaged);
          if (c.wave == 0) {
            const float mm = c.lane < kPerXcd && Mg.l[c.lane] > 0.0f ? Mg.m[c.lane] : -INFINITY;
            const float mstar = wave_max(mm);
            const float wgt = mm == -INFINITY ? 0.0f : expf(mm - mstar);
            const float den = wave_sum(c.lane < kPerXcd ? wgt * Mg.l[c.lane] : 0.0f);
            if (c.lane < kPerXcd) Mg.wgt[c.lane] = wgt;
            if (c.lane == 0) Mg.den = den;
          }
          __syncthreads();
          if (c.tid < 16) {
            float num = 0.0f;
            for (int s = 0; s < kPerXcd; ++s) num += Mg.wgt[s] * Mg.acc[s][c.tid];
            const float o = round_bf(num / Mg.den);
            const float gx = Mg.gate[c.tid];
            const float gate = round_bf(M.gate_kind == 0 ? sigmoid(gx) : silu(gx));
            c.w.core[(size_t)c.xcd * 512 + hl * kHd + d0 + c.tid] = f2bf(o * gate);
          }
          c.epoch += 1;
          signal_local(c, c.epoch);
        }
        // ================= o_proj (row-parallel) =====================================
        {
          fence(c, kTOProj);
          Gemv g{Lr.out_w, Lr.out_s, 4096 / kGroup, 0, c.xcd * 4, 4, 0, 0};
          g.b_lo = rp_lo * 4;
          g.b_hi = rp_hi * 4;
          WaveBlocks wb;
          if (!c.control) gemv_issue(g, c, wb, L);
          if (c.control) {
            bool ok = wait_local(c, c.epoch);
            if (ok) stage16<1, kCpAgent>(L.x[0], c.w.core + (size_t)c.xcd * 512, 512, c.lane);
            if (c.lane == 0) L.ok = ok;
          }
          zero_part(L, c);
          for (int i = c.tid; i < 512; i += kThreads) L.x[1][i] = 0;
          __syncthreads();
          if (!L.ok) return;
          stamp(c, kTStaged);
          if (!c.control) gemv_compute(g, c, wb, L);
          __syncthreads();
          c.epoch += 1;
          rowpar_epilogue(g, c, L, hidden);
          if (!allreduce_residual(c, L, hidden)) return;
        }
      }
      // ================= gate|up + SwiGLU (column-parallel) ============================
      {
        fence(c, kTGateUp);
        Gemv g{Lr.gu_w, Lr.gu_s, G, c.xcd * gu_tiles, 0, G, 0, 0};
        const int B = gu_tiles * G;
        g.b_lo = (c.r * B) / kPerXcd;
        g.b_hi = ((c.r + 1) * B) / kPerXcd;
        WaveBlocks wb;
        if (!c.control) gemv_issue(g, c, wb, L);
        else stage16<kHidChunks, kCpPlain>(L.nw, Lr.post_norm, hidden, c.lane);
        zero_part(L, c);
        __syncthreads();
        norm_prologue(L, c, hidden, M.eps);
        if (!c.control) gemv_compute(g, c, wb, L);
        __syncthreads();
        colpar_epilogue(g, c, L);
        c.epoch += 1;
        signal_local(c, c.epoch);
      }
      // ================= down (row-parallel) ===========================================
      {
        fence(c, kTDown);
        const int ngx = inter_x / kGroup;
        Gemv g{Lr.down_w, Lr.down_s, M.inter / kGroup, 0, c.xcd * ngx, ngx, 0, 0};
        g.b_lo = rp_lo * ngx;
        g.b_hi = rp_hi * ngx;
        WaveBlocks wb;
        if (!c.control) gemv_issue(g, c, wb, L);
        if (c.control) {
          bool ok = wait_local(c, c.epoch);
          if (ok) stage_act<(kColparMax / 4 + 63) / 64>(c, inter_x, L);
          if (c.lane == 0) L.ok = ok;
        }
        zero_part(L, c);
        for (int i = c.tid; i < inter_x; i += kThreads) L.x[1][i] = 0;
        __syncthreads();
        if (!L.ok) return;
        stamp(c, kTStaged);
        if (!c.control) gemv_compute(g, c, wb, L);
        __syncthreads();
        c.epoch += 1;
        rowpar_epilogue(g, c, L, hidden);
        if (!allreduce_residual(c, L, hidden)) return;
      }
    }

    // ================= final norm + tied head + argmax =================================
    {
      fence(c, kTHead);
      const int t_lo = c.xcd * vocab_tiles + (c.r * vocab_tiles) / kPerXcd;
      const int t_hi = c.xcd * vocab_tiles + ((c.r + 1) * vocab_tiles) / kPerXcd;
      auto& H = L.hd;
      // Compute waves own whole tiles t_lo + wave + 8 j; their (tile, group) blocks form one
      // stream through an 8-block LDS ring (LDS DMA), the first 8 requested before the norm.
      const int ntw = c.control ? 0 : (t_hi - t_lo - c.wave + kCompute - 1) / kCompute;
      const int nblk = ntw > 0 ? ntw * G : 0;
      auto blk_idx = [&](int q) -> size_t {
        const int t = t_lo + c.wave + (q / G) * kCompute;
        return (size_t)t * G + q % G;
      };
      if (!c.control) {
#pragma unroll 1
        for (int u = 0; u < kDepthH && u < nblk; ++u) dma_block(M.head_w, M.head_s, blk_idx(u), c.wave, u, c.lane, L);
      } else {
        stage16<kHidChunks, kCpPlain>(L.nw, M.final_norm, hidden, c.lane);
      }
      __syncthreads();
      norm_prologue(L, c, hidden, M.eps);
      float bv = -INFINITY;
      int bi = 0x7FFFFFFF;
      if (!c.control) {
        const int col = c.lane & 15, slot = c.lane >> 4;
        const uint16_t* xrow = &L.x[col == 0 ? 0 : 1][slot * 32];
        df_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int q0 = 0; q0 < nblk; q0 += kDepthH) {
#pragma unroll
          for (int u = 0; u < kDepthH; ++u) {
            const int q = q0 + u;
            if (q < nblk) {
              // block q has landed once at most the 7 later blocks (weights + scales each)
              // are still in flight; near the end of the stream, wait for everything
              if (q + kDepthH - 1 < nblk) wait_vm<2 * (kDepthH - 1)>();
              else wait_vm<0>();
              const uint4 wv = L.u.wq.wblk[c.wave][u][c.lane];
              const uint16_t sv = block_scale(L, c.wave, u, c.lane);
              const int gl = q % G;
              const GroupScale gs = group_scale(sv);
              const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
              df_f32x4 a2 = acc;
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                const uint4 bw = dequant8(words[d], gs);
                const uint4 aw = *reinterpret_cast<const uint4*>(xrow + gl * kGroup + d * 8);
                a2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, aw),
                                                             __builtin_bit_cast(df_bf16x8, bw), a2, 0, 0, 0);
              }
              acc = a2;
              const int qn = q + kDepthH;
              if (qn < nblk) dma_block(M.head_w, M.head_s, blk_idx(qn), c.wave, u, c.lane, L);  // refill the slot
              if (gl == G - 1) {  // tile complete: logits of 16 columns in lanes 0..15
                const int t = t_lo + c.wave + (q / G) * kCompute;
                const uint16_t lb = f2bf(acc[0]);
                if (c.lane < 16) {
                  H.logit[(t - t_lo) * 16 + c.lane] = lb;
                  const float lv = bf2f(lb);
                  const int li = t * 16 + c.lane;
                  if (lv > bv || (lv == bv && li < bi)) {
                    bv = lv;
                    bi = li;
                  }
                }
                acc = df_f32x4{0.f, 0.f, 0.f, 0.f};
              }
            }
          }
        }
        for (int off = 8; off > 0; off >>= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (c.lane == 0) {
          H.bv[c.wave] = bv;
          H.bi[c.wave] = bi;
        }
      }
      __syncthreads();
      // logits out (this workgroup's columns) and its candidate
      if (M.logits) {
        for (int e = c.tid; e < (t_hi - t_lo) * 16; e += kThreads) M.logits[(size_t)t_lo * 16 + e] = H.logit[e];
      }
      c.epoch += 1;
      if (c.tid == 0) {
        float v = H.bv[0];
        int i = H.bi[0];
        for (int wv = 1; wv < kCompute; ++wv) {
          if (H.bv[wv] > v || (H.bv[wv] == v && H.bi[wv] < i)) {
            v = H.bv[wv];
            i = H.bi[wv];
          }
        }
        // one atomic word: value, 18-bit index, the epoch's low 14 bits (a slot is rewritten
        // once per token, so its previous epoch differs by the phases per token)
        st_sys(reinterpret_cast<uint64_t*>(w.cand) + blockIdx.x, pack_cand(v, i, c.epoch));
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      // every workgroup reduces the 256 candidates (control wave)
      if (c.control) {
        const auto r = rsrc(w.cand);
        uint64_t v[kNwg / 64];
        bool ok = true;
        const uint64_t t0 = now();
        for (;;) {
#pragma unroll
          for (int k = 0; k < kNwg / 64; ++k) v[k] = ld8<kCpSystem>(r, (c.lane + 64 * k) * 8);
          bool ready = true;
#pragma unroll
          for (int k = 0; k < kNwg / 64; ++k) ready = ready && (static_cast<uint32_t>(v[k]) & 0x3FFFu) == (c.epoch & 0x3FFFu);
          if (__all(ready)) break;
          if (ld_sys(w.ctl + 1)) { ok = false; break; }
          if (now() - t0 > kTimeout) { raise_abort(c, kErrTimeout); ok = false; break; }
          __builtin_amdgcn_s_sleep(1);
        }
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int k = 0; k < kNwg / 64; ++k) {
          const float cv = __uint_as_float(static_cast<uint32_t>(v[k] >> 32));
          const int ci = static_cast<int>((static_cast<uint32_t>(v[k]) >> 14) & 0x3FFFFu);
          if (cv > bv || (cv == bv && ci < bi)) {
            bv = cv;
            bi = ci;
          }
        }
        for (int off = 32; off > 0; off >>= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (c.lane == 0) {
          L.ok = ok;
          L.token = bi;
        }
      }
      __syncthreads();
      if (!L.ok) return;
      token = L.token;
      if (c.xcd == 0 && c.r == 0 && c.tid == 0 && !teacher_forced && M.token_log) M.token_log[step0 + step] = token;
    }
  }
  if (c.xcd == 0 && c.r == 0 && c.tid == 0) {
    M.tokens[0] = token;
    *M.position = pos0 + steps;
    if (M.step && !teacher_forced) *M.step = step0 + steps;
    w.ctl[0] = static_cast<int>(c.epoch);
  }
}

__global__ void register_reset_kernel(int* ctl) {
  if (threadIdx.x < kXcd) ctl[kRegBase + threadIdx.x] = 0;
}

}  // namespace pd
}  // namespace df

using namespace df;

extern "C" size_t df_decode_persistent_workspace_bytes(int hidden) {
  if (hidden <= 0 || hidden > pd::kMaxHidden) return 0;
  return pd::ws_layout(hidden, nullptr, nullptr);
}

extern "C" int df_decode_persistent(const DfPersistModel* model, int steps, int teacher_forced, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  using namespace df::pd;
  if (!model || !workspace || steps < 0) return DF_BAD_ARGUMENT;
  DfPersistModel m = *model;
  if (m.hidden <= 0 || m.hidden > kMaxHidden || m.hidden % 512 || m.inter <= 0 || m.inter % 1024 ||
      m.vocab <= 0 || m.vocab % 128 || m.vocab > (1 << 18) || m.num_layers < 1 || m.max_len < 1 || !m.layers || !m.head_w || !m.head_s ||
      !m.final_norm || !m.inv_freq || !m.position || !m.tokens)
    return DF_BAD_ARGUMENT;
  if (2 * (m.inter / kXcd) > kColparMax) return DF_BAD_ARGUMENT;
  if ((m.vocab / kTileCols / kXcd + kPerXcd - 1) / kPerXcd > kMaxWgTiles * kCompute) return DF_BAD_ARGUMENT;
  if (teacher_forced && !m.prompt) return DF_BAD_ARGUMENT;
  // per-wave register budgets: blocks per wave of every GEMV phase <= kMaxNb, and tiles
  // per workgroup range <= kMaxWgTiles
  const int G = m.hidden / kGroup;
  auto fits = [&](int blocks, int ng) {
    const int per_wg = (blocks + kPerXcd - 1) / kPerXcd;
    return (per_wg + kCompute - 1) / kCompute <= kMaxNb && per_wg / ng + 2 <= kMaxWgTiles;
  };
  const int gu_tiles = 2 * (m.inter / kXcd) / kTileCols;
  const int row_tiles = m.hidden / kTileCols;
  if (!fits((kLinCols / kTileCols) * G, G) || !fits((kAttnCols / kTileCols) * G, G) || !fits(gu_tiles * G, G) ||
      !fits(row_tiles * 4, 4) || !fits(row_tiles * (m.inter / kXcd / kGroup), m.inter / kXcd / kGroup))
    return DF_BAD_ARGUMENT;
  if (workspace_bytes < ws_layout(m.hidden, nullptr, nullptr)) return DF_WORKSPACE_TOO_SMALL;
  if (steps == 0) return DF_OK;
  Ws w;
  ws_layout(m.hidden, &w, reinterpret_cast<char*>(workspace));
  hipLaunchKernelGGL(register_reset_kernel, dim3(1), dim3(64), 0, stream, w.ctl);
  if (hipGetLastError() != hipSuccess) return DF_LAUNCH_FAILED;
  void* args[] = {&m, &w, &steps, &teacher_forced};
  const hipError_t e =
      hipLaunchCooperativeKernel(reinterpret_cast<const void*>(decode_kernel), dim3(kNwg), dim3(kThreads), args, 0, stream);
  return e == hipSuccess ? DF_OK : DF_LAUNCH_FAILED;
}
