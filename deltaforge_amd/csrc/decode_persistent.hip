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
// loads, a per-workgroup epoch flag).
//
// Weight stream. Workgroup = 8 compute waves + 1 control wave. Each compute wave owns a
// fixed sequence of 1 KB weight blocks per token (its share of every GEMV phase of every
// layer, then of the head) and keeps the next kRing of them in flight or landed in its
// own LDS ring (LDS DMA), refilling a slot as soon as it has consumed it. The stream runs
// across phase and layer boundaries, so HBM keeps streaming while workgroups wait on
// hand-offs; it pauses only before each attention layer's output projection, until that
// layer's KV-cache loads are consumed. On gfx9 vector memory operations of a wave retire
// in order (one vmcnt counter), so a compute wave never waits for anything behind its
// ring: hand-off polls, activation staging, the recurrent state and every hand-off store
// belong to the control wave, which also signals. Ring slots are read with inline-asm
// ds_read so the compiler does not insert a vmcnt(0) before them (it cannot tell which
// slot a DMA targets); the kernel waits explicitly for exactly the block it consumes.
//
// GEMV arithmetic (bf16 MFMA). Each lane dequantises the 32 weights it holds of a block with
// dequant8 (int4_block.h): bf16((n - 8) s), the reference's expression bit for bit, 19 VALU ops
// per 8 weights. The input row is staged in bf16 as it is, so any bf16 activation is taken as
// it comes, and v_mfma_f32_16x16x32_bf16 sums the exact products in fp32 (row 0 of the
// 16-row product; rows 1..15 are don't-cares).
//
// Other arithmetic is the per-op kernels' (gated_delta.hip, attention.hip, small_ops.hip),
// with the reference's rounding points; only fp32 summation orders differ.
#include "common.h"
#include "deltaforge_hip.h"
#include "int4_block.h"

#include <algorithm>
#include <cstdlib>

namespace df {
namespace pd {

constexpr int kXcd = 8;
constexpr int kPerXcd = 32;
constexpr int kNwg = kXcd * kPerXcd;
constexpr int kCompute = 8;
constexpr int kCtl = kCompute;                      // wave index of the control wave
constexpr int kThreads = (kCompute + 1) * 64;       // 576
constexpr int kMaxHidden = 2560;
#ifndef DF_RING
#define DF_RING 8
#endif
constexpr int kRing = DF_RING;                      // weight blocks in flight per compute wave
static_assert(kRing >= 4 && (kRing & (kRing - 1)) == 0, "ring slots wrap with a mask");
constexpr int kMaxWgTiles = 8;                      // output tiles of a workgroup's GEMV range
constexpr int kMaxGroups = 24;                      // 128-groups of a GEMV phase's input row
constexpr int kMaxHeadTiles = 64;                   // head tiles per workgroup
constexpr int kColparMax = 2304;
// Gated DeltaNet geometry
constexpr int kKH = 16, kDk = 128;
constexpr int kKeyDim = kKH * kDk;                  // 2048
constexpr int kLinCols = 1552;
constexpr int kLinQ = 0, kLinK = 256, kLinV = 512, kLinZ = 1024, kLinA = 1536;
constexpr int kDnCh = 2 * kDk + 16;                 // conv channels of one delta unit: q, k, v slice
// attention geometry
constexpr int kHd = 256, kRot = 64;
constexpr int kAttnCols = 1536;
constexpr int kAttnK = 1024;
constexpr int kApHead = kHd + 2;                    // acc[256], m, l
constexpr int kTileKeys = kCompute * 16;            // 128 keys per attention tile
constexpr int kSplits = 2 * kPerXcd;                // key splits of a KV head over its XCD pair
constexpr int kPairHeads = 4;                       // query heads of a KV head (2 per XCD of the pair);
                                                    // an XCD's own two are its slots 0, 1
// int4 dot product: B = the reference's dequantised weights bf16((n - 8) s) (dequant8), the
// input row staged in bf16 as it is (see the file comment).
// Two bf16 values (already bf16-rounded floats) as one packed dword, k order.
DF_DEVICE uint32_t pack_x2(float a, float b) { return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xFFFF0000u); }

constexpr uint64_t kTimeout = 50000000ull;          // 0.5 s of s_memrealtime (100 MHz)
constexpr int kRegBase = 4;                         // ctl[4..11]: per-XCD registration tickets

enum Err : int { kErrNone = 0, kErrTimeout = 1, kErrXcd = 2, kErrPosition = 3, kErrToken = 4, kErrSchedule = 5 };

struct Ws {
  int* ctl;          // [16]: epoch, abort, error, -, 8 registration tickets, -
  int* flags;        // [8][32] last epoch each workgroup finished
  uint64_t* colpar;  // [8][2][kColparMax] input-projection partial outputs, 2 slots, (fp32, epoch)
  float* cpgu;       // [8][2][kColparMax] gate|up partial outputs, 2 slots (flag hand-off)
  uint16_t* hloc;    // [8][hidden] the hidden vector, one copy per XCD (flag hand-off)
  uint32_t* core;    // [8][512] DeltaNet core / merged attention output of the XCD, (bf16 | epoch << 16)
  float* apart;      // split partials: [8][32 splits][2 heads][kApHead] fp32, or in the PAIR
                     // instance [4 XCD pairs][64 records][4 head slots][kApHead] (fp32, u32 epoch)
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
  char* colpar = take((size_t)kXcd * 2 * kColparMax * sizeof(uint64_t));
  char* cpgu = take((size_t)kXcd * 2 * kColparMax * sizeof(float));
  char* hloc = take((size_t)kXcd * hidden * sizeof(uint16_t));
  char* core = take((size_t)kXcd * 512 * sizeof(uint32_t));
  char* apart = take(std::max((size_t)kXcd * kPerXcd * 2 * kApHead * sizeof(float),
                               (size_t)(kXcd / 2) * kSplits * kPairHeads * kApHead * sizeof(uint64_t)));
  char* rowpar = take((size_t)2 * kXcd * hidden * sizeof(uint64_t));
  char* cand = take((size_t)kNwg * sizeof(uint64_t));
  if (w) {
    w->ctl = reinterpret_cast<int*>(ctl);
    w->flags = reinterpret_cast<int*>(flags);
    w->colpar = reinterpret_cast<uint64_t*>(colpar);
    w->cpgu = reinterpret_cast<float*>(cpgu);
    w->hloc = reinterpret_cast<uint16_t*>(hloc);
    w->core = reinterpret_cast<uint32_t*>(core);
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
// Write-through store. The pointer is cast to the global address space: a flat store could
// target LDS, and the compiler would then make every later LDS access wait for it (vmcnt).
template <class T>
DF_DEVICE void st_sys(T* p, T v) {
  __hip_atomic_store((__attribute__((address_space(1))) T*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

DF_DEVICE uint64_t pack_epoch(float v, uint32_t epoch) {
  return (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v);
}
DF_DEVICE uint64_t pack_cand(float v, int index, uint32_t epoch) {
  return (static_cast<uint64_t>(__float_as_uint(v)) << 32) | (static_cast<uint32_t>(index) << 14) | (epoch & 0x3FFFu);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void gbl_void;

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int N>
DF_DEVICE void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wave reductions without LDS round trips (DPP inside 16-lane rows, readlane across rows).
// __shfl_xor compiles to ds_bpermute, an LDS round trip per step, which sits on the
// critical path of every norm and hand-off of this kernel.
template <int CTRL>
DF_DEVICE float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
DF_DEVICE int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
constexpr int kDppRor1 = 0x121, kDppRor2 = 0x122, kDppRor4 = 0x124, kDppRor8 = 0x128;
// Sum over each 16-lane row, in every lane of the row.
DF_DEVICE float row_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}
DF_DEVICE float row_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return v;
}
DF_DEVICE float lane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
// Whole-wave sum / max (same value in every lane).
DF_DEVICE float dsum(float v) {
  v = row_sum(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
DF_DEVICE float dmax(float v) {
  v = row_max(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
// (max value, lowest index among maxima) over each 16-lane row, in every lane of the row.
DF_DEVICE void argmax_step(float& bv, int& bi, float ov, int oi) {
  if (ov > bv || (ov == bv && oi < bi)) {
    bv = ov;
    bi = oi;
  }
}
DF_DEVICE void row_argmax(float& bv, int& bi) {
  argmax_step(bv, bi, dpp<kDppRor8>(bv), dpp_i<kDppRor8>(bi));
  argmax_step(bv, bi, dpp<kDppRor4>(bv), dpp_i<kDppRor4>(bi));
  argmax_step(bv, bi, dpp<kDppRor2>(bv), dpp_i<kDppRor2>(bi));
  argmax_step(bv, bi, dpp<kDppRor1>(bv), dpp_i<kDppRor1>(bi));
}
// Sum over the lanes of a row that share lane % 4 (rotations by 4 and 8 inside the row).
DF_DEVICE float row_sum_mod4(float v) {
  v += dpp<kDppRor4>(v);
  v += dpp<kDppRor8>(v);
  return v;
}

// ---------------------------------------------------------------------------------------
// LDS. The weight ring and the GEMV input row are objects of their own: the compiler then
// knows that reads of the input row and of the workgroup struct cannot alias a ring DMA.
// ---------------------------------------------------------------------------------------

__shared__ __align__(16) uint4 g_ring_w[kCompute][kRing][64];     // 1 KB blocks
__shared__ __align__(16) uint32_t g_ring_s[kCompute][kRing][16];  // scale dword of lane i < 16: columns (i & 14), +1
__shared__ __align__(16) uint16_t g_x[kMaxHidden + 8];            // the staged core (bf16), GatedRMSNorm's input
__shared__ __align__(16) uint16_t g_xh[kMaxHidden + 8];           // GEMV input row (bf16)

struct Lds {
  __align__(16) uint16_t h[kMaxHidden];          // the hidden vector (bf16)
  __align__(16) uint16_t nw[kMaxHidden];         // the next RMSNorm's weight (LDS DMA, a phase ahead)
  __align__(16) uint16_t gnw[kDk];               // GatedRMSNorm weight (LDS DMA, a phase ahead)
  __align__(16) float zs[512];                   // out_proj: SiLU inputs of the GatedRMSNorm (staged during delta)
  float ss;                                      // sum of squares of h (for the next RMSNorm)
  __align__(16) float part[kMaxWgTiles][16][kCompute];  // per-wave tile partials (a column's 8 adjacent)
  float red[64];
  int ok;
  int token;
  int nbw;                                       // compute waves' barrier count at the head's last barrier
  struct {                                       // head
    __align__(16) uint16_t logit[kMaxHeadTiles * 16];
    float bv[kCompute];
    int bi[kCompute];
  } hd;
  union {
    struct {                                     // Gated DeltaNet step
      __align__(16) float4 S[kDk / 16][64];      // state slice by DMA: [row block][lane]
      float qkv_in[kDnCh];                       // pre-conv inputs: q 128, k 128, v 16
      __align__(16) uint2 cw[kDnCh];             // their conv taps (bf16 x 4)
      __align__(16) uint2 hist[kDnCh];           // their conv history ring (bf16 x 4)
      float y[kDnCh];                            // conv + SiLU outputs
      float core[16];                            // the unit's 16 outputs
      float ab8[8];                              // a of the XCD's 4 value heads, then b
      float gp[2];                               // A_log, dt_bias of the unit's value head
      float gates[2];                            // beta, exp(g) (dn_conv's spare lane)
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
      uint32_t rope[kRot / 2];                   // this position's RoPE row (cos | sin << 16)
      float sc[2][kTileKeys + kCompute];         // + the waves' extra keys (at_ext)
      float alpha[2];
      float ml[2][2];
      float red[kCompute][2][kHd];               // 16 KB
    } at;
    struct {                                     // split merge (control wave)
      float m[kPerXcd], l[kPerXcd], wgt[kPerXcd];
      float acc[kPerXcd][16];
      float gate[16];
    } mg;
    struct {                                     // attention split, keys split over the XCD
                                                 // pair: the KV head's 4 query heads (the
                                                 // decode_kernel<., true> instance)
      __align__(16) uint16_t q[kPairHeads][kHd];
      __align__(16) uint16_t knew[kHd];
      __align__(16) uint16_t vnew[kHd];
      float qraw[kPairHeads][kHd];
      float kraw[kHd];                           // kraw and vraw adjacent: one staged segment
      float vraw[kHd];
      __align__(16) uint16_t qn_w[kHd];
      __align__(16) uint16_t kn_w[kHd];
      uint32_t rope[kRot / 2];                   // this position's RoPE row (cos | sin << 16)
      float sc[kPairHeads][kTileKeys + kCompute];  // + the waves' extra keys (at_ext)
      float alpha[kPairHeads];
      float ml[kPairHeads][2];
      __align__(16) float red[kPairHeads][kHd];  // the split's PV sums (the per-wave partials
                                                 // are summed from the drained weight ring)
    } at4;
    struct {                                     // its split merge (control wave)
      float wgt[kSplits];
      __align__(16) float acc[kSplits][16];
      float gate[16];
    } mg4;
    struct {                                     // down: the XCD's gate|up column sums
      __align__(16) float gu[kColparMax];
    } ac;
  } u;
};

// The layer table, copied into LDS when the launch starts. Read through the scalar cache
// instead, each phase's first access missed (the weight stream evicts the table from L2
// between layers) and stalled the wave for about a microsecond, in the middle of the weight
// stream's issue loop. Fields are read with LF(), which makes them wave-uniform (SGPRs).
constexpr int kMaxLayers = 32;
static_assert(sizeof(DfPersistLayer) % 8 == 0, "layer table copied in 8-byte words");
__shared__ __align__(16) DfPersistLayer g_layers[kMaxLayers];

constexpr size_t kLdsBytes = sizeof(Lds) + sizeof(g_ring_w) + sizeof(g_ring_s) + sizeof(g_x) + sizeof(g_xh) + sizeof(g_layers);
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");

typedef const DfPersistLayer* LayerPtr;  // points into g_layers
DF_DEVICE LayerPtr layer_at(const DfPersistModel&, int li) { return &g_layers[li]; }
template <class T>
DF_DEVICE T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}
DF_DEVICE int uniform_int(int v) { return __builtin_amdgcn_readfirstlane(v); }
#define LF(Lp, field) uniform_ptr((Lp)->field)
#define LKIND(Lp) uniform_int((Lp)->kind)

DF_DEVICE uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
// 16 bytes from LDS through an LDS pointer (a ds_read whatever the compiler knows of p).
DF_DEVICE uint4 lds_ld16(const void* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((const __attribute__((address_space(3))) char*)p);
  return __builtin_bit_cast(uint4, v);
}

// Workgroup barrier that orders LDS only. __syncthreads() is a workgroup-scope release
// fence, which on gfx950 waits for every outstanding vector memory operation of the wave
// (vmcnt(0)) and so would drain the compute waves' weight rings at every barrier. Nothing
// in this kernel passes data between the waves of a workgroup through global memory.
DF_DEVICE void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------------------
// per-workgroup context
// ---------------------------------------------------------------------------------------

struct Ctx {
  Ws w;
  int tcap;         // trace capacity
  int max_len;      // KV-cache rows per head
  int nb;           // barriers this wave has passed in the current token
  int xcd, r, tid, wave, lane;
  bool control;
  uint32_t epoch;   // last epoch this workgroup reached (all workgroups agree on the sequence)
  int ar;           // row-parallel all-reduce counter (selects the rowpar buffer)
  int pos;          // position of the token being decoded
  uint64_t* tr;     // phase trace of the traced step (workgroup (0, 0), control wave), or null
  int tn;
};

// Per-workgroup geometry of the phases.
struct Geo {
  int hidden, Gh, inter, inter_x, gu_tiles, rp_lo, rp_hi, ngx, t_lo, t_hi;
};

// Phase trace of the traced step: s_memrealtime << 8 | tag (tags: 1-15 phase starts, 20
// staged after the hand-off, 30 signalled).
enum Tag : int { kTProj = 1, kTDelta, kTOut, kTAttn, kTMerge, kTOProj, kTGateUp, kTDown, kTHead, kTEmbed,
                 kTReduce, kTStaged = 20, kTSignal = 30,
                 // finer points: control wave (delta step, all-reduce, down's hand-off)
                 kTDnLanded = 21, kTDnState = 22, kTDnDone = 23, kTArLanded = 31, kTArLocal = 32, kTGuLanded = 34,
                 kTHeadConsumed = 35, kTHeadDone = 36,
                 // compute waves (their own trace rows): GEMV consume, delta step, attention split
                 kTConsume = 40, kTConsumed = 42, kTDnIn = 43, kTDnConv = 44, kTDnMath = 45, kTAtStaged = 60, kTAtRoped = 61, kTAtQk = 62, kTAtSoftmax = 63,
                 kTAtPv = 64, kTAtDone = 65 };
// Compiled in only with DF_TRACE defined (a separate build of the library): the stamps' code sits
// between the phases of every token, in the instruction cache the decode depends on.
DF_DEVICE void stamp(Ctx& c, int tag) {
#ifdef DF_TRACE
  if (__builtin_expect(c.tr != nullptr, 0)) {  // only workgroup (0, 0)'s control wave, traced step
    if (c.lane == 0 && c.tn < c.tcap) c.tr[c.tn] = (now() << 8) | static_cast<uint64_t>(tag);
    c.tn += 1;
  }
#else
  (void)c;
  (void)tag;
#endif
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

// The control wave and the compute waves run separate code (so neither role's registers or
// pending loads burden the other) and meet only at these barriers, in the same order; each
// counts them and the counts are compared once per token.
DF_DEVICE void sync(Ctx& c) {
  bar();
  c.nb += 1;
}

DF_DEVICE void raise_abort(const Ctx& c, int err) {
  st_sys(c.w.ctl + 2, err);
  st_sys(c.w.ctl + 1, 1);
}

// Control wave: wait until the 32 workgroups of this XCD have reached `epoch`.
DF_DEVICE bool wait_local(const Ctx& c, uint32_t epoch) {
  const int* f = c.w.flags + c.xcd * kPerXcd;
  const uint64_t t0 = now();
  for (int it = 1;; ++it) {
    const int v = c.lane < kPerXcd ? ld_agent(f + c.lane) : static_cast<int>(epoch);
    if (__all(v >= static_cast<int>(epoch))) return true;
    // the abort word is read through to memory: only every 32nd poll pays for that
    if ((it & 31) == 0 && ld_sys(c.w.ctl + 1)) return false;
    if (now() - t0 > kTimeout) {
      raise_abort(c, kErrTimeout);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Control wave: make its stores complete, then publish `epoch` for this workgroup. Every
// store another workgroup reads is made by the control wave, so only it waits.
DF_DEVICE void signal_local(Ctx& c, uint32_t epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  stamp(c, kTSignal);
  if (c.lane == 0) {
    // a plain store (relaxed, workgroup scope: no cache bits and no wait after it) lands in
    // this XCD's L2, where the agent-scope polls of the other workgroups of the XCD read it; a
    // volatile or wider-scope store would write through to memory and wait for that
    __hip_atomic_store((__attribute__((address_space(1))) int*)(c.w.flags + c.xcd * kPerXcd + c.r),
                       static_cast<int>(epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Tagged hand-off data. Most hand-offs carry their epoch in every word, so the consumer polls
// the data itself (one L2 round trip after the producer's stores) and the producer never waits
// for its stores: (fp32 value, u32 epoch) pairs for fp32 data, bf16 | (epoch & 0xFFFF) << 16
// for bf16 data (a slot is rewritten every token, so a stale word's epoch differs from the one
// awaited). Single-copy atomicity of aligned 4- and 8-byte stores is all they rely on.
DF_DEVICE uint32_t tag_bf16(uint16_t v, uint32_t epoch) { return static_cast<uint32_t>(v) | (epoch << 16); }
DF_DEVICE bool tag_ok(uint32_t w, uint32_t epoch) { return (w >> 16) == (epoch & 0xFFFFu); }
DF_DEVICE bool tags_ok(const uint4& v, uint32_t epoch) {
  return tag_ok(v.x, epoch) && tag_ok(v.y, epoch) && tag_ok(v.z, epoch) && tag_ok(v.w, epoch);
}
DF_DEVICE bool pairs_ok(const uint4& v, uint32_t epoch) { return v.y == epoch && v.w == epoch; }

// Control wave: repeat `load` (fills the wave's registers, returns whether every tag it read
// is the awaited one) until every lane's is; false on abort or timeout.
template <class F>
DF_DEVICE bool poll_tagged(const Ctx& c, F&& load) {
  const uint64_t t0 = now();
  for (int it = 1;; ++it) {
    if (__all(load())) return true;
    if ((it & 31) == 0 && ld_sys(c.w.ctl + 1)) return false;
    if (now() - t0 > kTimeout) {
      raise_abort(c, kErrTimeout);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// ---------------------------------------------------------------------------------------
// GEMV input rows
// ---------------------------------------------------------------------------------------

// Compute waves (1 barrier; the control wave passes 1): x = bf16(RMSNorm(h) * (1 + w)) over
// `hidden` (w staged in L.nw) as the bf16 row g_xh. Every wave sums the squares of all of h itself (identical code and order in every wave, so all agree on the factor), which
// saves the cross-wave exchange and its barrier; a wave then produces whole 128-groups
// (2 elements per lane).
constexpr int kNormBars = 1;
DF_DEVICE void norm_w(Lds& L, Ctx& c, int hidden, float eps) {
  const float r = 1.0f / sqrtf(L.ss / static_cast<float>(hidden) + eps);
  const int G = hidden / kGroup;
  for (int g = c.wave; g < G; g += kCompute) {
    const int k = g * kGroup + 2 * c.lane;
    const uint32_t hv = *reinterpret_cast<const uint32_t*>(&L.h[k]);
    const uint32_t wv = *reinterpret_cast<const uint32_t*>(&L.nw[k]);
    const float x0 = round_bf(__uint_as_float(hv << 16) * r * (1.0f + __uint_as_float(wv << 16)));
    const float x1 = round_bf(__uint_as_float(hv & 0xFFFF0000u) * r * (1.0f + __uint_as_float(wv & 0xFFFF0000u)));
    *reinterpret_cast<uint32_t*>(&g_xh[k]) = pack_x2(x0, x1);
  }
  sync(c);
}

// ---------------------------------------------------------------------------------------
// GEMV phases and the weight stream
// ---------------------------------------------------------------------------------------

struct Gemv {
  const uint8_t* w;
  const uint16_t* s;
  int G;           // groups per tile in the stored matrix
  int tile0;       // first tile of the XCD slice
  int g0, ng;      // group slice
  int b_lo, b_hi;  // this workgroup's block range (relative to the slice, tile-major)
  int k;           // phase: 0 input projection, 1 out_proj / o_proj, 2 gate|up, 3 down
};

// Phase k of a layer of kind `kind` (phases: 0 input projection, 1 out_proj / o_proj,
// 2 gate|up, 3 down) for workgroup (xcd, r), without its weight pointers.
DF_DEVICE Gemv gemv_geom(int kind, const Geo& q, int k, int xcd, int r) {
  Gemv g;
  if (k == 0) {
    const int nt = (kind == 0 ? kLinCols : kAttnCols) / kTileCols;
    const int B = nt * q.Gh;
    g = Gemv{nullptr, nullptr, q.Gh, xcd * nt, 0, q.Gh, (r * B) / kPerXcd, ((r + 1) * B) / kPerXcd, 0};
  } else if (k == 1) {
    g = Gemv{nullptr, nullptr, 4096 / kGroup, 0, xcd * 4, 4, q.rp_lo * 4, q.rp_hi * 4, 1};
  } else if (k == 2) {
    const int B = q.gu_tiles * q.Gh;
    g = Gemv{nullptr, nullptr, q.Gh, xcd * q.gu_tiles, 0, q.Gh, (r * B) / kPerXcd, ((r + 1) * B) / kPerXcd, 2};
  } else {
    g = Gemv{nullptr, nullptr, q.inter / kGroup, 0, xcd * q.ngx, q.ngx, q.rp_lo * q.ngx, q.rp_hi * q.ngx, 3};
  }
  return g;
}

// The weight and scale pointers of phase k are adjacent in the layer table (checked below),
// so one LDS read fetches both.
static_assert(offsetof(DfPersistLayer, proj_s) == offsetof(DfPersistLayer, proj_w) + 8 &&
                  offsetof(DfPersistLayer, out_w) == offsetof(DfPersistLayer, proj_w) + 16 &&
                  offsetof(DfPersistLayer, out_s) == offsetof(DfPersistLayer, proj_w) + 24 &&
                  offsetof(DfPersistLayer, gu_w) == offsetof(DfPersistLayer, proj_w) + 32 &&
                  offsetof(DfPersistLayer, gu_s) == offsetof(DfPersistLayer, proj_w) + 40 &&
                  offsetof(DfPersistLayer, down_w) == offsetof(DfPersistLayer, proj_w) + 48 &&
                  offsetof(DfPersistLayer, down_s) == offsetof(DfPersistLayer, proj_w) + 56 &&
                  offsetof(DfPersistLayer, proj_w) % 8 == 0,
              "phase weight/scale pointers are consecutive pairs in DfPersistLayer");
DF_DEVICE void phase_ptrs(int li, int k, const uint8_t*& w, const uint16_t*& s) {
  const uint64_t* p = reinterpret_cast<const uint64_t*>(reinterpret_cast<const char*>(&g_layers[li]) +
                                                        offsetof(DfPersistLayer, proj_w)) + 2 * k;
  const uint64_t a = p[0], b = p[1];
  w = uniform_ptr(reinterpret_cast<const uint8_t*>(a));
  s = uniform_ptr(reinterpret_cast<const uint16_t*>(b));
}

DF_DEVICE Gemv gemv_of(LayerPtr Lp, const Geo& q, int k, int xcd, int r) {
  Gemv g = gemv_geom(LKIND(Lp), q, k, xcd, r);
  const int li = static_cast<int>(Lp - g_layers);
  phase_ptrs(li, k, g.w, g.s);
  return g;
}

// A compute wave's share of a workgroup's blocks. Wave w runs on SIMD w % 4, so waves 4..7
// share their SIMD with the older waves 0..3, which win the issue arbitration: with equal
// shares the younger waves finished 15-25 % later and the phase waited for them while each
// SIMD ran one wave. One ratio for every phase, 3 : 2 (waves 0..3 : 4..7), decoded fastest of
// 1 : 1, 6 : 5, 5 : 4, 3 : 2, 7 : 4 and 2 : 1; the traced finish stamps then showed the older
// waves last in the input projection and the younger ones last in down, so the older wave's
// share of its SIMD pair is set per phase, in 40ths: input projection 22 (11 : 9), out_proj /
// o_proj 24 (3 : 2), gate|up 25 (5 : 3), down 26 (13 : 7); 0.6 % per token over one ratio
// (same-box A/Bs of 12 settings). The head's tiles go 7 : 3 (28; 0.3 % over 3 : 2, and 3 : 1
// or 4 : 1 lost 1.1 %).
constexpr int kSharePair = 40, kShares = 4 * kSharePair, kShareHead = 28;
static_assert(kCompute == 8, "two waves per SIMD");
DF_DEVICE int share_old(int k) { return k == 0 ? 22 : k == 1 ? 24 : k == 2 ? 25 : 26; }
DF_DEVICE int share_before(int a, int wave) {
  return wave <= 4 ? a * wave : 4 * a + (kSharePair - a) * (wave - 4);
}
DF_DEVICE void wave_range(const Gemv& g, int wave, int& lo, int& n) {
  const int len = g.b_hi - g.b_lo;
  const int a = share_old(g.k);
  lo = g.b_lo + (len * share_before(a, wave)) / kShares;
  n = g.b_lo + (len * share_before(a, wave + 1)) / kShares - lo;
}

// The head's vocabulary tiles t_lo .. t_hi of the workgroup, in weighted shares: wave w takes
// the contiguous tiles head_tile(w) .. head_tile(w + 1), one run of its stream.
DF_DEVICE int head_tile(const Geo& q, int wave) {
  return q.t_lo + ((q.t_hi - q.t_lo) * share_before(kShareHead, wave)) / kShares;
}

// A compute wave's weight stream: the wave's 1 KB blocks of every GEMV phase of every layer
// and then of the head, in consumption order, as a list of runs (blocks contiguous in HBM)
// built once per launch in LDS. The same list serves every token of the launch.
//
// Run descriptor: w = weights of the first block | (blocks << 48), s = its scales | hold << 63
// (hold: the stream stops before this run until the attention layer's KV-cache loads are
// consumed, because they share the wave's in-order vmcnt). The hold is a zero-block marker run
// of its own right after each attention layer's input projection: the attention borrows the
// ring there (the per-XCD split's K rows, the pair split's PV partials), so it must be drained
// for every wave, and a flag carried by the next real run would leave a wave with no blocks
// between two attention layers' input projections with its ring full at the second.
struct RunDesc {
  uint64_t w, s;
};
// per wave and token: 6 per layer (<= 2 per row-parallel phase), a marker per attention layer
// and the head's tiles
constexpr int kMaxRuns = 225;
constexpr uint64_t kPtrMask = (1ull << 48) - 1;
__shared__ __align__(16) RunDesc g_runs[kCompute][kMaxRuns];

struct Stream {
  const uint8_t* wp;     // weights of the next block to issue (lane 0's 16 bytes)
  const uint16_t* sp;    // its 16 scales
  int left;              // blocks left in the current run
  int ri, nruns;         // next run to open, runs per token
  int issued, consumed;  // blocks, since the launch began
  int wslot, rslot;      // ring slots of the next issue / the next consume
  int state;             // 0 streaming, 1 held after an attention layer's input projection,
                         // 2 released, 3 past the launch's last block
  int istep;             // token of the cursor
};

enum StreamState : int { kStreaming = 0, kHeld = 1, kReleased = 2, kDone = 3 };

// Compute waves, once per launch: this wave's run list (lane 0 writes it; the wave's LDS
// accesses complete in order, so its own later reads see it). Returns the runs per token.
template <bool PAIR>
DF_DEVICE int build_runs(const DfPersistModel& M, const Geo& q, const Ctx& c) {
  int n = 0;
  auto put = [&](const uint8_t* w, const uint16_t* sc, int blocks, bool hold) {
    if (c.lane == 0 && n < kMaxRuns)
      g_runs[c.wave][n] = RunDesc{reinterpret_cast<uint64_t>(w) | (static_cast<uint64_t>(blocks) << 48),
                                  reinterpret_cast<uint64_t>(sc) | (hold ? 1ull << 63 : 0ull)};
    n += 1;
  };
  for (int li = 0; li < M.num_layers; ++li) {
    const int kind = LKIND(&g_layers[li]) & 1;
    for (int k = 0; k < 4; ++k) {
      const Gemv g = gemv_of(&g_layers[li], q, k, c.xcd, c.r);
      int lo, cnt;
      wave_range(g, c.wave, lo, cnt);
      // blocks lo .. lo + cnt of the slice (tile-major, ng groups per tile): a tile's run is
      // contiguous, and so are consecutive tiles when the slice spans every group
      while (cnt > 0) {
        const int t = lo / g.ng, gi = lo % g.ng;
        const int len = g.ng == g.G ? cnt : min(cnt, g.ng - gi);
        const size_t blk = (size_t)(g.tile0 + t) * g.G + g.g0 + gi;
        put(g.w + blk * kBlockBytes, g.s + blk * kTileCols, len, false);
        lo += len;
        cnt -= len;
      }
      if (kind == 1 && k == 0) put(nullptr, nullptr, 0, true);
    }
  }
  const int t0 = head_tile(q, c.wave), ntw = head_tile(q, c.wave + 1) - t0;
  if (ntw > 0) {  // consecutive tiles are contiguous (tile-major, Gh groups per tile)
    const size_t blk = (size_t)t0 * q.Gh;
    put(M.head_w + blk * kBlockBytes, M.head_s + blk * kTileCols, ntw * q.Gh, false);
  }
  // Every geometry the launcher accepts fits: per layer at most 1 run each for the
  // column-parallel phases and 2 for each row-parallel one (a wave's share of out_proj /
  // o_proj is at most 3 blocks of 4-group runs, of down at most 5/8 of a run of ngx blocks),
  // a marker per attention layer, and one run of head tiles, so 7 x 32 + 1 = kMaxRuns.
  static_assert(kMaxRuns == 7 * kMaxLayers + 1, "run list capacity");
  return min(n, kMaxRuns);
}

// Open the next run (the cursor's run is exhausted): stop at a hold run unless released,
// wrap to the next token's first run, stop after the launch's last token.
DF_DEVICE void open_run(Stream& st, int steps) {
  if (st.ri == st.nruns) {
    st.istep += 1;
    if (st.istep >= steps) {
      st.state = kDone;
      return;
    }
    st.ri = 0;
  }
  const uint4 d = *reinterpret_cast<const uint4*>(&g_runs[__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)][st.ri]);
  const uint64_t w = (static_cast<uint64_t>(uniform_int(static_cast<int>(d.y))) << 32) | static_cast<uint32_t>(uniform_int(static_cast<int>(d.x)));
  const uint64_t sc = (static_cast<uint64_t>(uniform_int(static_cast<int>(d.w))) << 32) | static_cast<uint32_t>(uniform_int(static_cast<int>(d.z)));
  if ((sc >> 63) && st.state == kStreaming) {
    st.state = kHeld;
    return;
  }
  st.state = kStreaming;
  st.wp = reinterpret_cast<const uint8_t*>(w & kPtrMask);
  st.sp = reinterpret_cast<const uint16_t*>(sc & kPtrMask);
  st.left = static_cast<int>(w >> 48);
  st.ri += 1;
}

// LDS DMA of 16 (or 4) bytes per lane: lane i's bytes land at lds_base + 16 i (4 i). The loads
// are non-temporal (nt): each weight byte is used once per token, and streaming it through L2
// as evict-first keeps the hand-off data, activations and cache rows resident. Written
// as inline asm so the compiler does not track these loads: it would otherwise treat every
// later LDS access of the wave as possibly aliasing a pending DMA and wait for all of them
// (vmcnt(0)), draining the ring. The kernel orders ring reads itself (wait_blocks); the
// compiler's own vmcnt waits only get stricter, never wrong, for loads it does not count.
DF_DEVICE void dma16(const void* gaddr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gaddr), "s"(lds_base)
               : "memory", "m0");
}
DF_DEVICE void dma4(const void* gaddr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt" ::"v"(gaddr), "s"(lds_base)
               : "memory", "m0");
}
// The scale DMA runs on lanes 0..15 only (the lanes that apply scales), 64 bytes per block.
DF_DEVICE void dma4_16(const void* gaddr, uint32_t lds_base) {
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %0, exec\n\t"
      "s_mov_b32 exec_lo, 0xffff\n\t"
      "s_mov_b32 exec_hi, 0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off nt\n\t"
      "s_mov_b64 exec, %0"
      : "=&s"(saved)
      : "v"(gaddr), "s"(lds_base)
      : "memory", "m0");
}

// Issue the cursor's block into the next ring slot (scales, then weights) and advance. A block
// issued alone is two vector memory operations, scales then weights; a pair issued by refill2
// is three, both blocks' scales then the two weight blocks. Every block's scales are issued
// before its weights, so a completed weight DMA implies its scales; the consumer's vmcnt
// waits count on these groupings (wait_oldest).
DF_DEVICE void issue_one(Stream& st, const Ctx& c) {
  dma4_16(st.sp + (c.lane & 14), lds_addr(&g_ring_s[c.wave][st.wslot][0]));
  dma16(st.wp + c.lane * 16, lds_addr(&g_ring_w[c.wave][st.wslot][0]));
  st.issued += 1;
  st.wslot = (st.wslot + 1) & (kRing - 1);
  st.wp += kBlockBytes;
  st.sp += kTileCols;
  st.left -= 1;
}

DF_DEVICE void fill(Stream& st, int steps, const Ctx& c, int upto = kRing) {
  while (st.state == kStreaming && st.issued - st.consumed < upto) {
    if (st.left == 0) {
      open_run(st, steps);
      continue;
    }
    issue_one(st, c);
  }
}

// The same DMAs with the global address as a scalar base plus the lane's offset (no vector
// address arithmetic per block).
DF_DEVICE void dma16s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase),
               "s"(lds_base)
               : "memory", "m0");
}
// Both blocks' scale dwords of a pair on lanes 0..31 (lane i < 16: block 0's, i >= 16: block
// 1's), landing in the pair's two adjacent ring slots.
DF_DEVICE void dma4_32s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %0, exec\n\t"
      "s_mov_b32 exec_hi, 0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, %2 nt\n\t"
      "s_mov_b64 exec, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(lds_base)
      : "memory", "m0");
}

// After the consumer took two blocks from a full ring: refill both slots. The common case
// (two more blocks in the current run, landing in two adjacent slots: not the ring's last and
// first) is straight-line code of three DMAs; anything else goes through fill.
DF_DEVICE void refill2(Stream& st, int steps, const Ctx& c) {
  if (__builtin_expect(st.state == kStreaming && st.left >= 2 && st.wslot != kRing - 1 &&
                           st.issued - st.consumed == kRing - 2,
                       1)) {
    const uint32_t voff = c.lane * 16, soff = ((c.lane >> 4) * kTileCols + (c.lane & 14)) * 2;
    const int s0 = st.wslot;
    dma4_32s(st.sp, soff, lds_addr(&g_ring_s[c.wave][s0][0]));
    dma16s(st.wp, voff, lds_addr(&g_ring_w[c.wave][s0][0]));
    dma16s(st.wp, voff + kBlockBytes, lds_addr(&g_ring_w[c.wave][s0 + 1][0]));  // same base, next 1 KB
    st.issued += 2;
    st.wslot = (st.wslot + 2) & (kRing - 1);
    st.wp += 2 * kBlockBytes;
    st.sp += 2 * kTileCols;
    st.left -= 2;
    return;
  }
  fill(st, steps, c);
}

// Wait for the oldest `need` pending blocks (need = 1 or 2). The ring is full except while
// it drains before an attention layer's hold or at the end of a launch, where waiting for
// every block in flight costs nothing extra. With the ring full (blocks i .. i + 7 issued,
// as groups of (scales, weights) singles and (scales, weights, weights) pairs), at least 9
// operations were issued after block i + 1's weights and at least 10 after block i's: the
// fewest come from pairs, and a pair that starts at the awaited block adds its second
// weight DMA. Waiting until no more than that many are outstanding completes the awaited
// blocks and, issued before them, their scales.
template <int NEED>
DF_DEVICE void wait_oldest(const Stream& st) {
  static_assert(kRing == 8, "wait counts derived for an 8-slot ring");
  if (st.issued - st.consumed == kRing) wait_vm<NEED == 2 ? 9 : 10>();
  else wait_vm<0>();
}

DF_DEVICE int next_slot(int s) { return (s + 1) & (kRing - 1); }

// One block's weights and scale dword from ring slot `slot` of this wave.
DF_DEVICE void ring_read1(int slot, const Ctx& c, uint4& wv, uint32_t& sd) {
  const uint32_t wa = lds_addr(&g_ring_w[c.wave][slot][c.lane]);
  const uint32_t sa = lds_addr(&g_ring_s[c.wave][slot][c.lane & 15]);
  asm volatile("ds_read_b128 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(wv), "=&v"(sd)
               : "v"(wa), "v"(sa)
               : "memory");
}

// Everything a pair of blocks needs from LDS, with one wait: both ring slots (weights,
// scale dword) and the two groups' input chunks of this lane's k slot. Only row 0 of each
// product is used: its A operand comes from lanes 0, 16, 32 and 48, and its results live in
// lanes 0..15. The input chunks are read by those four lanes only (exec masked inside the
// asm and restored before it ends), which cuts the LDS traffic of a pair from 11 KB to under
// 4 KB; the other lanes' copies hold stale values that only feed rows 1..15. Every lane reads
// its column's scale dword (16 distinct per slot, broadcasts): the B operand of every lane is
// dequantised with it.
struct PairIn {
  uint4 w0, w1;
  uint32_t s0, s1;
  uint4 x0[4], x1[4];
};
DF_DEVICE void pair_read(int slot, const Ctx& c, const uint16_t* xg0, const uint16_t* xg1, PairIn& in) {
  const int slot1 = next_slot(slot);
  const uint32_t wa0 = lds_addr(&g_ring_w[c.wave][slot][c.lane]);
  const uint32_t sa0 = lds_addr(&g_ring_s[c.wave][slot][c.lane & 15]);
  const uint32_t wa1 = lds_addr(&g_ring_w[c.wave][slot1][c.lane]);
  const uint32_t sa1 = lds_addr(&g_ring_s[c.wave][slot1][c.lane & 15]);
  const uint32_t xa0 = lds_addr(xg0), xa1 = lds_addr(xg1);
  uint64_t saved;
  asm volatile(
      "ds_read_b128 %0, %13\n\t"
      "ds_read_b128 %1, %15\n\t"
      "ds_read_b32 %2, %14\n\t"
      "ds_read_b32 %3, %16\n\t"
      "s_mov_b64 %12, exec\n\t"
      "s_mov_b32 exec_lo, 0x10001\n\t"
      "s_mov_b32 exec_hi, 0x10001\n\t"
      "s_nop 0\n\t"
      "ds_read_b128 %4, %17\n\t"
      "ds_read_b128 %5, %17 offset:16\n\t"
      "ds_read_b128 %6, %17 offset:32\n\t"
      "ds_read_b128 %7, %17 offset:48\n\t"
      "ds_read_b128 %8, %18\n\t"
      "ds_read_b128 %9, %18 offset:16\n\t"
      "ds_read_b128 %10, %18 offset:32\n\t"
      "ds_read_b128 %11, %18 offset:48\n\t"
      "s_mov_b64 exec, %12\n\t"
      "s_nop 0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(in.w0), "=&v"(in.w1), "=&v"(in.s0), "=&v"(in.s1), "=&v"(in.x0[0]), "=&v"(in.x0[1]), "=&v"(in.x0[2]),
        "=&v"(in.x0[3]), "=&v"(in.x1[0]), "=&v"(in.x1[1]), "=&v"(in.x1[2]), "=&v"(in.x1[3]), "=&s"(saved)
      : "v"(wa0), "v"(sa0), "v"(wa1), "v"(sa1), "v"(xa0), "v"(xa1)
      : "memory");
}

// The two groups' input chunks of this lane's k slot alone (the pair_read layout): lanes 0,
// 16, 32 and 48 read, the others keep stale values that only feed rows 1..15.
DF_DEVICE void x_read(const uint16_t* xg0, const uint16_t* xg1, uint4 (&x0)[4], uint4 (&x1)[4]) {
  const uint32_t xa0 = lds_addr(xg0), xa1 = lds_addr(xg1);
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %8, exec\n\t"
      "s_mov_b32 exec_lo, 0x10001\n\t"
      "s_mov_b32 exec_hi, 0x10001\n\t"
      "s_nop 0\n\t"
      "ds_read_b128 %0, %9\n\t"
      "ds_read_b128 %1, %9 offset:16\n\t"
      "ds_read_b128 %2, %9 offset:32\n\t"
      "ds_read_b128 %3, %9 offset:48\n\t"
      "ds_read_b128 %4, %10\n\t"
      "ds_read_b128 %5, %10 offset:16\n\t"
      "ds_read_b128 %6, %10 offset:32\n\t"
      "ds_read_b128 %7, %10 offset:48\n\t"
      "s_mov_b64 exec, %8\n\t"
      "s_nop 0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0[0]), "=&v"(x0[1]), "=&v"(x0[2]), "=&v"(x0[3]), "=&v"(x1[0]), "=&v"(x1[1]), "=&v"(x1[2]),
        "=&v"(x1[3]), "=&s"(saved)
      : "v"(xa0), "v"(xa1)
      : "memory");
}

// Wait for the oldest pending block and read it.
DF_DEVICE void take_block(Stream& st, const Ctx& c, uint4& wv, uint32_t& sd) {
  wait_oldest<1>(st);
  ring_read1(st.rslot, c, wv, sd);
  st.consumed += 1;
  st.rslot = next_slot(st.rslot);
}

DF_DEVICE void take_pair(Stream& st, const Ctx& c, const uint16_t* xg0, const uint16_t* xg1, PairIn& in) {
  wait_oldest<2>(st);
  pair_read(st.rslot, c, xg0, xg1, in);
  st.consumed += 2;
  st.rslot = next_slot(next_slot(st.rslot));
}

// One block's B operands: this lane's 32 weights dequantised with dequant8 (int4_block.h), the
// reference's bf16((n - 8) s) bit for bit (sh = 16 * (lane & 1) selects the lane's column scale
// in the scale dword).
DF_DEVICE void dequant_block(const uint4& wv, uint32_t sd, uint32_t sh, const DqK& K, uint4 (&b)[4]) {
  const GroupScale gs = group_scale(static_cast<uint16_t>(sd >> sh));
  b[0] = dequant8(wv.x, gs, K);
  b[1] = dequant8(wv.y, gs, K);
  b[2] = dequant8(wv.z, gs, K);
  b[3] = dequant8(wv.w, gs, K);
}

// Row 0 of one block's product from its dequantised weights: lanes 0..15 return
// sum_k x_k w_k over the block's 128 k (x = the group's bf16 input chunks at this lane's k
// slot), the four bf16 MFMAs summing the products in fp32.
DF_DEVICE float block_dot_b(const uint4 (&b)[4], const uint4 (&x)[4]) {
  df_f32x4 d4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < 4; ++d)
    d4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, x[d]), __builtin_bit_cast(df_bf16x8, b[d]),
                                                 d4, 0, 0, 0);
  return d4[0];
}

// Both steps for a block whose weights were just read from the ring.
DF_DEVICE float block_dot_r(const uint4& wv, uint32_t sd, const uint4 (&x)[4], uint32_t sh, const DqK& K) {
  uint4 b[4];
  dequant_block(wv, sd, sh, K, b);
  return block_dot_b(b, x);
}

// Single-block form reading its input from LDS.
DF_DEVICE float block_dot(const uint4& wv, uint32_t sd, const uint16_t* x, int lane) {
  uint4 xv[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) xv[d] = *reinterpret_cast<const uint4*>(x + d * 8);
  return block_dot_r(wv, sd, xv, 16u * (lane & 1), dq_consts());
}

// Compute waves: consume this wave's blocks of GEMV phase g (input row g_xh); per-tile
// partials of row 0 go to L.part[tile - first tile of the workgroup][wave].
// Blocks are taken two at a time (two independent MFMA chains per iteration).
// A phase's first block pair, taken from the ring and dequantised while the workgroup waited
// for the phase's input (predequant), and whether it holds them.
struct PreDq {
  uint4 b0[4], b1[4];
  bool ok;
};

// Compute waves, while the control wave runs a hand-off (the stream does not hold there): take
// this wave's first two blocks of GEMV phase g from the ring, refill their slots and
// dequantise them, so the phase starts at its MFMAs. Skipped when the wave has fewer than two
// blocks in the phase or fewer than two are in flight.
DF_DEVICE void predequant(const Gemv& g, const Ctx& c, Stream& st, int steps, PreDq& pre) {
  int lo, n;
  wave_range(g, c.wave, lo, n);
  pre.ok = n >= 2 && st.issued - st.consumed >= 2;
  if (!pre.ok) return;
  wait_oldest<2>(st);
  uint4 w0, w1;
  uint32_t s0, s1;
  ring_read1(st.rslot, c, w0, s0);
  ring_read1(next_slot(st.rslot), c, w1, s1);
  st.consumed += 2;
  st.rslot = next_slot(next_slot(st.rslot));
  refill2(st, steps, c);
  const uint32_t sh = 16u * (c.lane & 1);
  const DqK K = dq_consts();
  dequant_block(w0, s0, sh, K, pre.b0);
  dequant_block(w1, s1, sh, K, pre.b1);
}

DF_DEVICE void gemv_consume(const Gemv& g, const Ctx& c, Stream& st, const DfPersistModel& M, const Geo& q,
                            int steps, Lds& L, PreDq& pre) {
  stamp(const_cast<Ctx&>(c), kTConsume);
  int lo, n;
  wave_range(g, c.wave, lo, n);
  // this wave's partial of every tile starts at zero (only this wave writes its column, and
  // the control wave read the previous phase's partials before the barrier that began this one)
  for (int e = c.lane; e < kMaxWgTiles * 16; e += 64) L.part[e / 16][e % 16][c.wave] = 0.0f;
  const uint16_t* xb = g_xh + (c.lane >> 4) * 32;
  int tr = lo / g.ng - g.b_lo / g.ng;
  int gl = lo % g.ng;
  float acc = 0.0f;
  auto add = [&](float v) {
    acc += v;
    if (++gl == g.ng) {
      if (c.lane < 16) L.part[tr][c.lane][c.wave] = acc;
      acc = 0.0f;
      gl = 0;
      ++tr;
    }
  };
  const uint32_t sh = 16u * (c.lane & 1);
  const DqK K = dq_consts();
  int i = 0;
  if (pre.ok) {  // the first two blocks, dequantised ahead (n >= 2)
    const int gl1 = gl + 1 == g.ng ? 0 : gl + 1;
    uint4 x0[4], x1[4];
    x_read(xb + gl * kGroup, xb + gl1 * kGroup, x0, x1);
    const float v0 = block_dot_b(pre.b0, x0);
    const float v1 = block_dot_b(pre.b1, x1);
    add(v0);
    add(v1);
    pre.ok = false;
    i = 2;
  }
#pragma unroll 1
  for (; i + 1 < n; i += 2) {
    const int gl1 = gl + 1 == g.ng ? 0 : gl + 1;
    PairIn in;
    take_pair(st, c, xb + gl * kGroup, xb + gl1 * kGroup, in);
    const float v0 = block_dot_r(in.w0, in.s0, in.x0, sh, K);
    const float v1 = block_dot_r(in.w1, in.s1, in.x1, sh, K);
    refill2(st, steps, c);
    add(v0);
    add(v1);
  }
  if (i < n) {
    uint4 w0;
    uint32_t s0;
    take_block(st, c, w0, s0);
    add(block_dot(w0, s0, xb + gl * kGroup, c.lane));
    fill(st, steps, c);
  }
  if (n > 0 && gl != 0 && c.lane < 16) L.part[tr][c.lane][c.wave] = acc;
  stamp(const_cast<Ctx&>(c), kTConsumed);
}

// Sum of the waves' partials for relative tile t (fixed wave order).
DF_DEVICE float part_sum(const Lds& L, int t, int col) {
  static_assert(kCompute == 8, "two 16-byte reads per column");
  const float4 a = *reinterpret_cast<const float4*>(&L.part[t][col][0]);
  const float4 b = *reinterpret_cast<const float4*>(&L.part[t][col][4]);
  return ((((((a.x + a.y) + a.z) + a.w) + b.x) + b.y) + b.z) + b.w;  // wave order
}

// ---- control-wave staging: every load of a hand-off is issued before any is used -------

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int df_i4;
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
// 16-byte store; with kCpSystem it writes through (sc0 sc1), like st_sys.
template <int CP>
DF_DEVICE void st16(__amdgpu_buffer_rsrc_t r, int byte_off, uint4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(df_i4, v), r, byte_off, 0, CP);
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

// Control wave: parameter rows copied into LDS by DMA a phase ahead of their use, issued
// while the compute waves consume so the loads are done before the next hand-off wait (the
// wave's vector memory operations complete in order). Their consumers run after a later
// vmcnt(0) of the control wave (a hand-off poll) and a barrier.
DF_DEVICE void dma4(const void* gaddr, uint32_t lds_base);
// n bf16 (n % 512 == 0), 16 bytes per lane per DMA.
DF_DEVICE void dma_row(const uint16_t* src, uint16_t* dst, int n, int lane) {
  for (int k = 0; k * 512 < n; ++k) dma16(src + k * 512 + lane * 8, lds_addr(dst + k * 512));
}
// 128 bf16 (256 bytes), 4 bytes per lane.
DF_DEVICE void dma_row128(const uint16_t* src, uint16_t* dst, int lane) {
  dma4(src + lane * 2, lds_addr(dst));
}

// A run of XCD-local columns [j0, j0 + n) (j0, n even) of the column-parallel outputs,
// delivered as bf16-rounded slot sums into dst.
struct Seg {
  int j0, n;
  float* dst;
};

// Up to NS segments, K 16-byte chunks (2 columns) per lane and slot; polls until every pair
// carries epoch `want`.
template <int NS, int K>
DF_DEVICE bool gather_colpar(const Ctx& c, const Seg (&seg)[NS], uint32_t want) {
  const auto r = rsrc(c.w.colpar + (size_t)c.xcd * 2 * kColparMax);
  int start[NS + 1];
  start[0] = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) start[s + 1] = start[s] + seg[s].n / 2;
  int col[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = c.lane + 64 * k;
    col[k] = -1;
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (ch >= start[s] && ch < start[s + 1]) col[k] = seg[s].j0 + 2 * (ch - start[s]);
  }
  uint4 a[K], b[K];
  const bool ok = poll_tagged(c, [&]() {
    bool t = true;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (col[k] >= 0) {
        a[k] = ld16<kCpAgent>(r, col[k] * 8);
        b[k] = ld16<kCpAgent>(r, (kColparMax + col[k]) * 8);
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (col[k] >= 0) t = t && pairs_ok(a[k], want) && pairs_ok(b[k], want);
    return t;
  });
  if (!ok) return false;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = c.lane + 64 * k;
    if (col[k] >= 0) {
      float* d = nullptr;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        if (ch >= start[s] && ch < start[s + 1]) d = seg[s].dst + 2 * (ch - start[s]);
      d[0] = round_bf(__uint_as_float(a[k].x) + __uint_as_float(b[k].x));
      d[1] = round_bf(__uint_as_float(a[k].z) + __uint_as_float(b[k].z));
    }
  }
  return true;
}

// Control wave: an attention layer's inputs, polled together, as bf16-rounded slot sums: this
// XCD's two query heads (columns 0 and 512) into slots 0, 1, its k | v columns (1024 ..1535)
// and, when the keys are split over the pair, the other XCD's two query heads into slots 2, 3
// (that XCD wrote them through to memory; read at system scope).
DF_DEVICE bool gather_attn(const Ctx& c, float (*qraw)[kHd], float* kvraw, uint32_t want, bool pair) {
  const auto rl = rsrc(c.w.colpar + (size_t)c.xcd * 2 * kColparMax);
  const auto rp = rsrc(c.w.colpar + (size_t)(c.xcd ^ 1) * 2 * kColparMax);
  // chunk k of a lane: 2 columns at col(k); partner chunks 0..3, own chunks 0..7
  auto pcol = [&](int k) { return (k < 2 ? 0 : 512) + 2 * (c.lane + 64 * (k & 1)); };
  auto lcol = [&](int k) { return (k < 2 ? 0 : k < 4 ? 512 : 1024) + 2 * (c.lane + 64 * (k < 4 ? (k & 1) : k - 4)); };
  uint4 pa[4], pb[4], la[8], lb[8];
  const bool ok = poll_tagged(c, [&]() {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (pair) {
        pa[k] = ld16<kCpSystem>(rp, pcol(k) * 8);
        pb[k] = ld16<kCpSystem>(rp, (kColparMax + pcol(k)) * 8);
      } else {  // not used
        pa[k] = pb[k] = make_uint4(0u, want, 0u, want);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      la[k] = ld16<kCpAgent>(rl, lcol(k) * 8);
      lb[k] = ld16<kCpAgent>(rl, (kColparMax + lcol(k)) * 8);
    }
    bool t = true;
#pragma unroll
    for (int k = 0; k < 4; ++k) t = t && pairs_ok(pa[k], want) && pairs_ok(pb[k], want);
#pragma unroll
    for (int k = 0; k < 8; ++k) t = t && pairs_ok(la[k], want) && pairs_ok(lb[k], want);
    return t;
  });
  if (!ok) return false;
  if (pair) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float* d = qraw[2 + (k >> 1)] + 2 * (c.lane + 64 * (k & 1));
      d[0] = round_bf(__uint_as_float(pa[k].x) + __uint_as_float(pb[k].x));
      d[1] = round_bf(__uint_as_float(pa[k].z) + __uint_as_float(pb[k].z));
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float* d = k < 4 ? qraw[k >> 1] + 2 * (c.lane + 64 * (k & 1)) : kvraw + 2 * (c.lane + 64 * (k - 4));
    d[0] = round_bf(__uint_as_float(la[k].x) + __uint_as_float(lb[k].x));
    d[1] = round_bf(__uint_as_float(la[k].z) + __uint_as_float(lb[k].z));
  }
  return true;
}

// Control wave, after the flag hand-off: the XCD's 2 inter_x gate|up columns as (unrounded)
// sums of the two column-parallel slots, into gu. This hand-off keeps flags and untagged
// fp32: polling its data tagged would mean twice the bytes (37 KB per workgroup), more than
// the flag's round trip costs.
template <int K>
DF_DEVICE void stage_gu(const Ctx& c, int inter_x, float* gu) {
  const auto r = rsrc(c.w.cpgu + (size_t)c.xcd * 2 * kColparMax);
  const int chunks = inter_x / 2;  // 4 columns each
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
    if (ch < chunks) {
      float4 v;
      v.x = __uint_as_float(a[k].x) + __uint_as_float(b[k].x);
      v.y = __uint_as_float(a[k].y) + __uint_as_float(b[k].y);
      v.z = __uint_as_float(a[k].z) + __uint_as_float(b[k].z);
      v.w = __uint_as_float(a[k].w) + __uint_as_float(b[k].w);
      *reinterpret_cast<float4*>(gu + 4 * ch) = v;
    }
  }
}

// Compute waves (1 barrier; the control wave passes 1): the down projection's input
// act = bf16(bf16(silu(g)) * u) as the bf16 row g_xh. The gate|up columns come
// in 32-column pairs (16 gate columns, then their 16 up columns), so act j reads gate
// column 32 (j / 16) + j % 16 and the up column 16 further. A wave produces whole
// 128-groups (2 elements per lane).
constexpr int kActBars = 1;
DF_DEVICE void swiglu_act(Lds& L, Ctx& c, int inter_x) {
  const float* gu = L.u.ac.gu;
  for (int g = c.wave; g < inter_x / kGroup; g += kCompute) {
    const int j = g * kGroup + 2 * c.lane;      // even: j and j + 1 share a 16-run
    const int col = (j >> 4) * 32 + (j & 15);
    const float2 gv = *reinterpret_cast<const float2*>(gu + col);
    const float2 uv = *reinterpret_cast<const float2*>(gu + col + 16);
    const float x0 = round_bf(round_bf(silu(round_bf(gv.x))) * round_bf(uv.x));
    const float x1 = round_bf(round_bf(silu(round_bf(gv.y))) * round_bf(uv.y));
    *reinterpret_cast<uint32_t*>(&g_xh[j]) = pack_x2(x0, x1);
  }
  sync(c);
}

// Control wave: the XCD's 512 merged attention / delta outputs (tagged bf16, published by the
// workgroups of the XCD at epoch `want`) into g_x (the GatedRMSNorm's input) or, as the GEMV
// input itself (`direct`), into g_xh.
DF_DEVICE bool stage_core(Lds& L, const Ctx& c, uint32_t want, bool direct) {
  const auto r = rsrc(c.w.core + (size_t)c.xcd * 512);
  uint4 v0, v1;
  if (!poll_tagged(c, [&]() {
        v0 = ld16<kCpAgent>(r, c.lane * 32);
        v1 = ld16<kCpAgent>(r, c.lane * 32 + 16);
        return tags_ok(v0, want) && tags_ok(v1, want);
      }))
    return false;
  const uint4 v = make_uint4((v0.x & 0xFFFFu) | (v0.y << 16), (v0.z & 0xFFFFu) | (v0.w << 16),
                             (v1.x & 0xFFFFu) | (v1.y << 16), (v1.z & 0xFFFFu) | (v1.w << 16));
  *reinterpret_cast<uint4*>(direct ? &g_xh[c.lane * 8] : &g_x[c.lane * 8]) = v;
  return true;
}

// Control wave, column-parallel epilogue: this workgroup's partial of each tile it touched
// into its slot (r & 1); tiles wholly inside its range also zero the other slot.
// TAGGED: the input projection's (fp32, epoch) pairs; else gate|up's plain fp32.
template <bool TAGGED>
DF_DEVICE void colpar_epilogue(const Gemv& g, const Ctx& c, const Lds& L, bool through = false) {
  const int t_first = g.b_lo / g.ng, t_last = (g.b_hi - 1) / g.ng;
  const int nt = t_last - t_first + 1;
  uint64_t* cp = c.w.colpar + (size_t)c.xcd * 2 * kColparMax;
  float* cg = c.w.cpgu + (size_t)c.xcd * 2 * kColparMax;
  const int mine = c.r & 1;
  for (int e = c.lane; e < nt * 16; e += 64) {
    const int tr = e / 16, col = e % 16;
    const int t = t_first + tr;
    const float v = part_sum(L, tr, col);
    const int j = t * 16 + col;
    const bool whole = t * g.ng >= g.b_lo && (t + 1) * g.ng <= g.b_hi;
    if (TAGGED && through && ((j >> 8) & 1) == 0 && j < kAttnK) {  // query columns: read by the pair's other XCD too
      st_sys(&cp[mine * kColparMax + j], pack_epoch(v, c.epoch));
      if (whole) st_sys(&cp[(mine ^ 1) * kColparMax + j], pack_epoch(0.0f, c.epoch));
    } else if (TAGGED) {
      cp[mine * kColparMax + j] = pack_epoch(v, c.epoch);
      if (whole) cp[(mine ^ 1) * kColparMax + j] = pack_epoch(0.0f, c.epoch);
    } else {
      cg[mine * kColparMax + j] = v;
      if (whole) cg[(mine ^ 1) * kColparMax + j] = 0.0f;
    }
  }
}

// Control wave, row-parallel epilogue: the XCD's partial of hidden columns [16 t_first, ...)
// with epoch.
DF_DEVICE void rowpar_epilogue(const Gemv& g, const Ctx& c, const Lds& L, int hidden) {
  const int t_first = g.b_lo / g.ng, nt = (g.b_hi - g.b_lo) / g.ng;
  uint64_t* rp = c.w.rowpar + ((size_t)(c.ar & 1) * kXcd + c.xcd) * hidden;
  for (int e = c.lane; e < nt * 16; e += 64) {
    const int tr = e / 16, col = e % 16;
    st_sys(rp + (t_first + tr) * 16 + col, pack_epoch(part_sum(L, tr, col), c.epoch));
  }
}

// Control wave, the all-reduce after a row-parallel phase: slice [sl0, sl0 + ns) of y = sum
// over XCDs (in order); h = bf16(h + bf16(y)); publish the slice to this XCD's copy of h;
// wait for the XCD; read all of h back into LDS. The caller's next barrier hands h to the
// compute waves.
DF_DEVICE bool allreduce_residual(Ctx& c, Lds& L, int hidden) {
  fence(c, kTReduce);
  const int ns = hidden / kPerXcd;  // columns of this workgroup's slice: even, <= 80
  const int sl0 = c.r * ns;
  const auto r = rsrc(c.w.rowpar + (size_t)(c.ar & 1) * kXcd * hidden);
  const uint32_t want = c.epoch;
  c.ar += 1;
  c.epoch += 1;
  // lane l < ns / 2 owns columns sl0 + 2 l, + 1: one 16-byte load per XCD holds both
  // (value, epoch) pairs, so the sum over XCDs stays in registers
  const bool mine = 2 * c.lane < ns;
  const int off = (sl0 + 2 * c.lane) * 8;
  uint4 v[kXcd];
  bool ok = true;
  const uint64_t t0 = now();
  for (int it = 1;; ++it) {
    bool ready = true;
    if (mine) {
#pragma unroll
      for (int x = 0; x < kXcd; ++x) v[x] = ld16<kCpSystem>(r, x * hidden * 8 + off);
#pragma unroll
      for (int x = 0; x < kXcd; ++x) ready = ready && v[x].y == want && v[x].w == want;
    }
    if (__all(ready)) break;
    if ((it & 31) == 0 && ld_sys(c.w.ctl + 1)) { ok = false; break; }
    if (now() - t0 > kTimeout) { raise_abort(c, kErrTimeout); ok = false; break; }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!ok) return false;
  stamp(c, kTArLanded);
  uint16_t* hx = c.w.hloc + (size_t)c.xcd * hidden;
  if (mine) {
    float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
    for (int x = 0; x < kXcd; ++x) {  // XCD order
      y0 += __uint_as_float(v[x].x);
      y1 += __uint_as_float(v[x].z);
    }
    const int k = sl0 + 2 * c.lane;
    const uint32_t hv = *reinterpret_cast<const uint32_t*>(&L.h[k]);
    const uint16_t b0 = f2bf(__uint_as_float(hv << 16) + round_bf(y0));
    const uint16_t b1 = f2bf(__uint_as_float(hv & 0xFFFF0000u) + round_bf(y1));
    *reinterpret_cast<uint32_t*>(hx + k) = static_cast<uint32_t>(b0) | (static_cast<uint32_t>(b1) << 16);
  }
  // the XCD's copy of h by flags: polling its 32 slices tagged measured slower (twice the
  // bytes, re-read by every workgroup of the XCD while the slices arrive)
  signal_local(c, c.epoch);
  if (!wait_local(c, c.epoch)) return false;
  stamp(c, kTArLocal);
  // h into LDS with its sum of squares for the next RMSNorm (the same order in every
  // workgroup, so all agree)
  const auto rh = rsrc(hx);
  uint4 hv[kHidChunks];
#pragma unroll
  for (int k = 0; k < kHidChunks; ++k) {
    const int ch = c.lane + 64 * k;
    if (ch * 8 < hidden) hv[k] = ld16<kCpAgent>(rh, ch * 16);
  }
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < kHidChunks; ++k) {
    const int ch = c.lane + 64 * k;
    if (ch * 8 < hidden) {
      *reinterpret_cast<uint4*>(&L.h[ch * 8]) = hv[k];
      const uint32_t w[4] = {hv[k].x, hv[k].y, hv[k].z, hv[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xFFFF0000u);
        sq += lo * lo;
        sq += hi * hi;
      }
    }
  }
  sq = dsum(sq);
  if (c.lane == 0) L.ss = sq;
  return true;
}

// ---------------------------------------------------------------------------------------
// Gated DeltaNet step for (value head 4x + r/8, value columns 16 (r%8) ..+15)
// ---------------------------------------------------------------------------------------

DF_DEVICE int dn_channel(const Ctx& c, int i) {
  // i in 0..271: q (128), k (128), v slice (16) of this workgroup's unit -> global channel
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int kh = 2 * c.xcd + (hvl >> 1), hv = 4 * c.xcd + hvl;
  if (i < 128) return kh * kDk + i;
  if (i < 256) return kKeyDim + kh * kDk + (i - 128);
  return 2 * kKeyDim + hv * kDk + vs * 16 + (i - 256);
}

// Control wave, at the start of a Gated DeltaNet layer's input projection: this workgroup's
// 128 x 16 fp32 state slice into LDS (L.u.dn.S) by DMA, lane l's 16 bytes of row l / 4 + 16 j
// into S[j][l]. Issued a whole GEMV phase before the delta step reads it, so its HBM round trip
// is off the step's critical path; the hand-off poll the step begins with waits for every
// earlier memory operation of the wave (in-order vmcnt), this DMA included.
DF_DEVICE void dn_state_prefetch(const Ctx& c, LayerPtr Lp, Lds& L) {
  auto& D = L.u.dn;
  const int hv = 4 * c.xcd + (c.r >> 3), vs = c.r & 7;
  const int row0 = c.lane >> 2, col4 = (c.lane & 3) * 4;
  const float* sbase = LF(Lp, state) + ((size_t)hv * kDk + row0) * kDk + vs * 16 + col4;
#pragma unroll
  for (int i = 0; i < kDk / 16; ++i) dma16(sbase + (size_t)16 * i * kDk, lds_addr(&D.S[i][0]));
}

// The Gated DeltaNet step of this workgroup's unit (value head hv = 4 x + r / 8, value columns
// 16 (r % 8) .. + 15), in three parts around two barriers, so that the eight compute waves (idle
// at out_proj's first barrier otherwise) carry the arithmetic:
//   dn_stage    control wave: the in_proj hand-off (q, k of the key head, the unit's 16 v, a/b)
//               and the unit's conv taps and history into LDS (the XCD's z follows while the
//               compute waves run the conv);                                     | barrier
//   dn_conv     compute waves: the 4-tap conv + SiLU of the 272 channels, 34 per wave, and
//               the gates on a spare lane;                                       | barrier
//   dn_math     compute waves: q/k L2 norms (each wave, identically), then wave w
//               runs the delta rule on value columns 2 w, 2 w + 1 over all 128 state rows (two
//               rows per lane), so each column's recall and output are one wave's sums; the
//               updated slice goes back to the LDS copy, the outputs to LDS;   | barrier
//   dn_publish  control wave: the 16 outputs (tagged with their epoch), to memory; the new
//               state slice and this position's conv history slots follow during out_proj's
//               consume (dn_store_state).
// The arithmetic and rounding points are the reference's (reference.py:407-461, 496-545); fp32
// sums over the state rows run in a fixed order of their own.
constexpr int kDnBars = 3;
constexpr int kDnConvPerWave = (kDnCh + kCompute - 1) / kCompute;  // 34
static_assert(kDnConvPerWave <= 64, "one channel per lane");

DF_DEVICE bool dn_stage(Ctx& c, LayerPtr Lp, Lds& L, uint32_t epoch_in) {
  auto& D = L.u.dn;
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int hv = 4 * c.xcd + hvl;
  constexpr int kCh = (kDnCh + 63) / 64;     // channels per lane
  // loads that do not depend on the hand-off go out first
  uint2 tp[kCh];
  uint64_t hs[kCh];
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int ch = c.lane + 64 * i;
    if (ch < kDnCh) {
      const int gc = dn_channel(c, ch);
      tp[i] = *reinterpret_cast<const uint2*>(LF(Lp, conv_w) + (size_t)gc * 4);
      // another workgroup of the XCD writes the q/k history slots: read at agent scope
      hs[i] = ld_agent(reinterpret_cast<const uint64_t*>(LF(Lp, conv_ring) + (size_t)gc * 4));
    }
  }
  const float alog = bf2f(LF(Lp, A_log)[hv]), dtb = bf2f(LF(Lp, dt_bias)[hv]);
  const int khl = hvl >> 1;
  // (z, the out_proj GatedRMSNorm's gate, is gathered while the compute waves run the conv:
  // the delta step's own poll stays 6 loads per lane instead of 14)
  const Seg seg[4] = {{kLinQ + khl * 128, 128, D.qkv_in},
                      {kLinK + khl * 128, 128, D.qkv_in + 128},
                      {kLinV + hvl * 128 + vs * 16, 16, D.qkv_in + 256},
                      {kLinA, 8, D.ab8}};
  // the state slice is in LDS: its DMA (dn_state_prefetch) preceded this poll
  if (!gather_colpar<4, 3>(c, seg, epoch_in)) return false;
  stamp(c, kTDnLanded);
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int ch = c.lane + 64 * i;
    if (ch < kDnCh) {
      D.cw[ch] = tp[i];
      D.hist[ch] = __builtin_bit_cast(uint2, hs[i]);
    }
  }
  if (c.lane == 0) {
    D.gp[0] = alog;
    D.gp[1] = dtb;
  }
  return true;
}

// Compute waves: conv + SiLU (fp32 sum in tap order, bf16, SiLU, bf16) of channels
// 34 w .. 34 w + 33. History slots (pos+1)&3, (pos+2)&3, (pos+3)&3 hold positions pos-3, pos-2,
// pos-1 (slot pos&3 is written by dn_publish). The last wave's spare lane 63 computes the unit's
// gates, beta = bf16(sigmoid(b)) and exp(g) = exp(-exp(A_log) softplus(a + dt_bias)), for dn_math.
DF_DEVICE void dn_conv(const Ctx& c, Lds& L) {
#pragma clang fp contract(off)
  auto& D = L.u.dn;
  const int ch = c.wave * kDnConvPerWave + c.lane;
  if (c.lane < kDnConvPerWave && ch < kDnCh) {
    const uint2 wt = D.cw[ch];
    const uint2 hr = D.hist[ch];
    const float w0 = __uint_as_float(wt.x << 16), w1 = __uint_as_float(wt.x & 0xFFFF0000u);
    const float w2 = __uint_as_float(wt.y << 16), w3 = __uint_as_float(wt.y & 0xFFFF0000u);
    const uint16_t sl[4] = {static_cast<uint16_t>(hr.x), static_cast<uint16_t>(hr.x >> 16),
                            static_cast<uint16_t>(hr.y), static_cast<uint16_t>(hr.y >> 16)};
    const float h0 = bf2f(sl[(c.pos + 1) & 3]), h1 = bf2f(sl[(c.pos + 2) & 3]), h2 = bf2f(sl[(c.pos + 3) & 3]);
    float acc = h0 * w0;
    acc = acc + h1 * w1;
    acc = acc + h2 * w2;
    acc = acc + D.qkv_in[ch] * w3;
    D.y[ch] = round_bf(silu(round_bf(acc)));
  } else if (c.wave == kCompute - 1 && c.lane == 63) {  // a spare lane: the unit's gates
    const int hvl = c.r >> 3;
    const float a = D.ab8[hvl], b = D.ab8[4 + hvl];
    D.gates[0] = round_bf(sigmoid(b));
    D.gates[1] = expf(-expf(D.gp[0]) * softplus(a + D.gp[1]));
  }
}

// Compute waves: the norms, the gates and the delta rule on value columns 2 w, 2 w + 1 of the
// unit (rows lane and lane + 64 in each lane). The state slice in LDS is S[j][l] = row l / 4 +
// 16 j, columns 4 (l % 4) .. + 3.
DF_DEVICE void dn_math(const Ctx& c, Lds& L) {
#pragma clang fp contract(off)
  auto& D = L.u.dn;
  // L2 norms of q (then scaled by dk^-1/2) and k, in every wave alike
  const float q0 = D.y[c.lane], q1 = D.y[c.lane + 64];
  const float k0 = D.y[kDk + c.lane], k1 = D.y[kDk + c.lane + 64];
  const float rq = 1.0f / sqrtf(dsum(q0 * q0 + q1 * q1) + 1e-6f);
  const float rk = 1.0f / sqrtf(dsum(k0 * k0 + k1 * k1) + 1e-6f);
  const float scale = sqrtf(static_cast<float>(kDk));
  const float qn0 = (q0 * rq) / scale, qn1 = (q1 * rq) / scale;
  const float kn0 = k0 * rk, kn1 = k1 * rk;
  // gates (dn_conv's spare lane computed them, off the reductions' path)
  const float beta = D.gates[0];
  const float eg = D.gates[1];
  // this wave's two columns of rows lane and lane + 64
  const int c0 = 2 * c.wave;
  float* s0 = reinterpret_cast<float*>(&D.S[c.lane / 16][(c.lane % 16) * 4 + c0 / 4]) + (c0 % 4);
  float* s1 = reinterpret_cast<float*>(&D.S[(c.lane + 64) / 16][(c.lane % 16) * 4 + c0 / 4]) + (c0 % 4);
  float2 r0 = *reinterpret_cast<const float2*>(s0), r1 = *reinterpret_cast<const float2*>(s1);
  r0.x = r0.x * eg;
  r0.y = r0.y * eg;
  r1.x = r1.x * eg;
  r1.y = r1.y * eg;
  const float p0 = dsum(r0.x * kn0 + r1.x * kn1), p1 = dsum(r0.y * kn0 + r1.y * kn1);
  const float d0 = (D.y[2 * kDk + c0] - p0) * beta;
  const float d1 = (D.y[2 * kDk + c0 + 1] - p1) * beta;
  r0.x = r0.x + kn0 * d0;
  r0.y = r0.y + kn0 * d1;
  r1.x = r1.x + kn1 * d0;
  r1.y = r1.y + kn1 * d1;
  const float o0 = dsum(r0.x * qn0 + r1.x * qn1), o1 = dsum(r0.y * qn0 + r1.y * qn1);
  *reinterpret_cast<float2*>(s0) = r0;
  *reinterpret_cast<float2*>(s1) = r1;
  if (c.lane == 0) {
    D.core[c0] = o0;
    D.core[c0 + 1] = o1;
  }
}

// Control wave, after the compute waves' delta rule: the 16 outputs tagged with `epoch_out`.
// The stores nobody waits for follow in dn_store_state: the new state slice, and this
// position's conv history slot of the channels this unit owns (its v slice; the key head's q/k
// for the (even value head, slice 0) unit).
DF_DEVICE void dn_publish(Ctx& c, LayerPtr Lp, Lds& L, uint32_t epoch_out) {
  auto& D = L.u.dn;
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int hv = 4 * c.xcd + hvl;
  if (c.lane < 16) c.w.core[(size_t)c.xcd * 512 + hvl * kDk + vs * 16 + c.lane] = tag_bf16(f2bf(D.core[c.lane]), epoch_out);
  stamp(c, kTDnDone);
}

// Control wave, during out_proj's consume (off the hand-off path; the union's delta-step data
// stays untouched until the MLP): the new state slice and this position's conv history slots
// to memory. Read again only by the next token's same layer; the all-reduce's signal waits for
// these stores with the rest.
DF_DEVICE void dn_store_state(Ctx& c, LayerPtr Lp, Lds& L) {
  auto& D = L.u.dn;
  const int hvl = c.r >> 3, vs = c.r & 7;
  const int hv = 4 * c.xcd + hvl;
  const int row0 = c.lane >> 2, col4 = (c.lane & 3) * 4;
  // global-address stores: a flat store (the layer table's pointers are generic) would count
  // on the LDS counter too, and the next barrier's lgkmcnt(0) would wait for its write
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  auto* sbase = (__attribute__((address_space(1))) float*)(LF(Lp, state) + ((size_t)hv * kDk + row0) * kDk + vs * 16 + col4);
#pragma unroll
  for (int i = 0; i < kDk / 16; ++i)
    *(__attribute__((address_space(1))) f32x4*)(sbase + (size_t)16 * i * kDk) = __builtin_bit_cast(f32x4, D.S[i][c.lane]);
  auto* ring = (__attribute__((address_space(1))) uint16_t*)LF(Lp, conv_ring);
  constexpr int kCh = (kDnCh + 63) / 64;
#pragma unroll
  for (int i = 0; i < kCh; ++i) {
    const int ch = c.lane + 64 * i;
    const bool owner = ch >= 2 * kDk || ((hvl & 1) == 0 && vs == 0);
    if (ch < kDnCh && owner) ring[(size_t)dn_channel(c, ch) * 4 + (c.pos & 3)] = f2bf(D.qkv_in[ch]);
  }
}

// ---------------------------------------------------------------------------------------
// attention split r of [0, pos] for query heads 2x, 2x+1
// ---------------------------------------------------------------------------------------

// RMSNorm(1+w) over 256 dims held 4 per lane, then partial RoPE (attention.hip's order).
// rope: this position's row of the RoPE table in LDS, rotary pair j as bf16 cos | bf16 sin << 16.
DF_DEVICE void norm_rope4_lds(float x[4], const uint16_t* nw, float eps, const uint32_t* rope, int lane) {
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
  ss = dsum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(kHd) + eps);
  float n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) n[i] = round_bf((x[i] * r) * (1.0f + bf2f(nw[lane * 4 + i])));
  constexpr int half = kRot / 2;
  float partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = dpp<kDppRor8>(n[i]);  // lane ^ 8 = (lane + 8) mod 16 in a row
  static_assert(half / 4 == 8, "the partner of a rotary dim is 8 lanes away");
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dim = lane * 4 + i;
    const uint32_t cw = rope[dim & (half - 1)];
    const float cs = bf2f(static_cast<uint16_t>(cw)), sn = bf2f(static_cast<uint16_t>(cw >> 16));
    if (dim < kRot) {
      const float rotated = dim < half ? -partner[i] : partner[i];
      x[i] = round_bf(round_bf(n[i] * cs) + round_bf(rotated * sn));
    } else {
      x[i] = n[i];
    }
  }
}

struct AtPre {
  uint4 kb[8];   // K rows: this lane's key (t0 + 16 wave + col), dims d*32 + slot*8 ..+7
  uint2 ke;      // the wave's extra key t0 + 128 + wave (at_ext), K dims 4 lane ..+3
};
// A tile's V rows in registers (the per-XCD key split; its K rows come by DMA into the ring).
struct AtPreKV {
  uint2 vb[16];  // V rows: keys t0 + 16 wave + j, dims 4 lane ..+3
  uint2 ke, ve;  // the wave's extra key t0 + 128 + wave (at_ext), K and V dims 4 lane ..+3
};

DF_DEVICE void at_keys(const Ctx& c, int& j0, int& j1) {
  const int nkeys = c.pos + 1;
  const int per = (nkeys + kPerXcd - 1) / kPerXcd;
  j0 = min(c.r * per, nkeys);
  j1 = min(j0 + per, nkeys);
}

// Whether the tile at t0 is the split's last and runs past 128 keys by at most one key per
// wave: wave w then takes key t0 + 128 + w besides its 16 (a lane-parallel dot product and
// one more PV term) instead of a second, near-empty tile. A split of 4097..4352 keys over 32
// workgroups (129..136 keys each) is one tile so, and one of 32769..33280 keys over the 64
// workgroups of an XCD pair (513..520 each) four tiles instead of five.
__host__ __device__ inline bool at_ext(int t0, int j1) {
  return j1 - t0 > kTileKeys && j1 - t0 <= kTileKeys + kCompute;
}

typedef const __attribute__((address_space(1))) uint16_t* GlobalBf16;
typedef uint32_t df_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t df_u32x2 __attribute__((ext_vector_type(2)));
// Loads through global-address-space pointers (never flat: see st_sys).
DF_DEVICE uint4 gload16(GlobalBf16 p) {
  const df_u32x4 v = *(const __attribute__((address_space(1))) df_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
DF_DEVICE uint2 gload8(GlobalBf16 p) {
  const df_u32x2 v = *(const __attribute__((address_space(1))) df_u32x2*)p;
  return make_uint2(v.x, v.y);
}

// Compute waves: load the K rows of one 128-key tile of the split (not the new position).
DF_DEVICE void at_issue_k(const Ctx& c, LayerPtr Lp, int t0, int j1, AtPre& P) {
  const int col = c.lane & 15, slot = c.lane >> 4;
  const size_t base = (size_t)(c.xcd >> 1) * c.max_len;
  const int key = t0 + c.wave * 16 + col;
  // defined on every path: a conditionally-set register array is a value the compiler carries
  // around the whole layer loop (spilled across every other phase)
#pragma unroll
  for (int d = 0; d < 8; ++d) P.kb[d] = make_uint4(0u, 0u, 0u, 0u);
  if (key < j1 && key != c.pos) {
    GlobalBf16 kp = (GlobalBf16)LF(Lp, k_cache) + (base + key) * kHd + slot * 8;
#pragma unroll
    for (int d = 0; d < 8; ++d) P.kb[d] = gload16(kp + d * 32);
  }
  const int ek = t0 + kTileKeys + c.wave;
  P.ke = make_uint2(0u, 0u);
  if (at_ext(t0, j1) && ek < j1 && ek != c.pos) P.ke = gload8((GlobalBf16)LF(Lp, k_cache) + (base + ek) * kHd + c.lane * 4);
}

// Compute waves: the K rows of one 128-key tile by LDS DMA into the wave's weight ring, which
// is idle through the attention (the stream holds at the marker run after the input projection
// with every block consumed), so they go out before the q/k staging without holding registers.
// Chunk d (16 bytes) of this lane's key lands in ring slot d at the lane's position: the QK
// reads of one d are one contiguous 1 KB. Rows past the split clamp into it (the tile ignores
// them; the new position's row is taken from LDS).
constexpr int kAtVLoads = 18;  // vector loads at_issue_v issues after the K DMAs
static_assert(kRing >= 8, "a wave's ring holds its 16 keys' K rows (8 KB)");
DF_DEVICE void at_dma_k(const Ctx& c, LayerPtr Lp, int t0, int j1) {
  const int col = c.lane & 15, slot = c.lane >> 4;
  const size_t base = (size_t)(c.xcd >> 1) * c.max_len;
  const int key = min(t0 + c.wave * 16 + col, j1 - 1);
  const uint16_t* kp = LF(Lp, k_cache) + (base + key) * kHd + slot * 8;
#pragma unroll
  for (int d = 0; d < 8; ++d) dma16(kp + d * 32, lds_addr(&g_ring_w[c.wave][d][0]));
}

// Compute waves: the V rows of one 128-key tile and the wave's extra key's K and V rows
// (at_ext): kAtVLoads loads on every path (rows clamp into the split), so a wait for the older
// K DMAs can count them.
DF_DEVICE void at_issue_v(const Ctx& c, LayerPtr Lp, int t0, int j1, AtPreKV& P) {
  const size_t base = (size_t)(c.xcd >> 1) * c.max_len;
  GlobalBf16 vc = (GlobalBf16)LF(Lp, v_cache);
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    const int kk = min(t0 + c.wave * 16 + jj, j1 - 1);
    P.vb[jj] = gload8(vc + (base + kk) * kHd + c.lane * 4);
  }
  const int ek = min(t0 + kTileKeys + c.wave, j1 - 1);
  P.ke = gload8((GlobalBf16)LF(Lp, k_cache) + (base + ek) * kHd + c.lane * 4);
  P.ve = gload8(vc + (base + ek) * kHd + c.lane * 4);
}

// Compute waves (kTileBars barriers): one 128-key tile whose K and V rows are in flight in P
// (plus up to one extra key per wave, at_ext): QK (MFMA), the online softmax (waves 0 / 1 for
// heads 0 / 1), then PV.
constexpr int kTileBars = 3;
DF_DEVICE void at_tile(Ctx& c, LayerPtr Lp, int t0, int j1, const AtPreKV& P, float acc[2][4], Lds& L) {
  auto& A = L.u.at;
  const int col = c.lane & 15, slot = c.lane >> 4;
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  asm volatile("" ::: "memory");  // at_issue_v's loads stay ahead of the wait
  wait_vm<kAtVLoads>();           // the tile's K DMAs (older than at_issue_v's loads)
  asm volatile("" ::: "memory");
  {
    const int key = t0 + c.wave * 16 + col;
    const bool live = key < j1;
    df_f32x4 d4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      // both rows by LDS loads (a generic pointer on one side would make the select a flat load
      // that waits for every outstanding vector memory operation, the tile's V rows included)
      const uint4 kn = lds_ld16(A.knew + d * 32 + slot * 8);
      const uint4 kr = lds_ld16(&g_ring_w[c.wave][d][c.lane]);
      uint4 bw = make_uint4(0u, 0u, 0u, 0u);
      if (live) bw = key == c.pos ? kn : kr;
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
  const bool ext = at_ext(t0, j1);
  const int ek = t0 + kTileKeys + c.wave;
  if (ext) {  // this wave's extra key: q . k over the 64 lanes' 4 dims each
    float se[2] = {-INFINITY, -INFINITY};
    if (ek < j1) {
      uint2 kr = P.ke;
      if (ek == c.pos) kr = *reinterpret_cast<const uint2*>(A.knew + c.lane * 4);
      const float k4[4] = {__uint_as_float(kr.x << 16), __uint_as_float(kr.x & 0xFFFF0000u),
                           __uint_as_float(kr.y << 16), __uint_as_float(kr.y & 0xFFFF0000u)};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint2 qr = *reinterpret_cast<const uint2*>(&A.q[h][c.lane * 4]);
        float p = __uint_as_float(qr.x << 16) * k4[0];
        p += __uint_as_float(qr.x & 0xFFFF0000u) * k4[1];
        p += __uint_as_float(qr.y << 16) * k4[2];
        p += __uint_as_float(qr.y & 0xFFFF0000u) * k4[3];
        se[h] = dsum(p) * scale;
      }
    }
    if (c.lane == 0) {
      A.sc[0][kTileKeys + c.wave] = se[0];
      A.sc[1][kTileKeys + c.wave] = se[1];
    }
  }
  stamp(c, kTAtQk);
  sync(c);
  if (c.wave < 2) {
    const int h = c.wave;
    const float s0 = A.sc[h][c.lane], s1 = A.sc[h][c.lane + 64];
    const float s2 = ext && c.lane < kCompute ? A.sc[h][kTileKeys + c.lane] : -INFINITY;
    const float tmax = dmax(fmaxf(fmaxf(s0, s1), s2));
    const float mo = A.ml[h][0];
    const float m_new = fmaxf(mo, tmax);
    float p0 = 0.f, p1 = 0.f, p2 = 0.f, alpha = 1.0f;
    if (m_new != -INFINITY) {
      p0 = s0 == -INFINITY ? 0.0f : expf(s0 - m_new);
      p1 = s1 == -INFINITY ? 0.0f : expf(s1 - m_new);
      p2 = s2 == -INFINITY ? 0.0f : expf(s2 - m_new);
      alpha = mo == -INFINITY ? 0.0f : expf(mo - m_new);
    }
    const float lsum = dsum((p0 + p1) + p2);
    A.sc[h][c.lane] = p0;
    A.sc[h][c.lane + 64] = p1;
    if (ext && c.lane < kCompute) A.sc[h][kTileKeys + c.lane] = p2;
    if (c.lane == 0) {
      A.ml[h][0] = m_new;
      A.ml[h][1] = A.ml[h][1] * alpha + lsum;
      A.alpha[h] = alpha;
    }
  }
  sync(c);
  stamp(c, kTAtSoftmax);
  {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float a = A.alpha[h];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[h][i] *= a;
    }
    uint2 vn = *reinterpret_cast<const uint2*>(A.vnew + c.lane * 4);
    asm volatile("" : "+v"(vn.x), "+v"(vn.y));
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int kk = t0 + c.wave * 16 + jj;
      if (kk < j1) {
        const uint2 raw = kk == c.pos ? vn : P.vb[jj];
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
    if (ext && ek < j1) {
      const uint2 raw = ek == c.pos ? vn : P.ve;
      const float v0 = __uint_as_float(raw.x << 16), v1 = __uint_as_float(raw.x & 0xFFFF0000u);
      const float v2 = __uint_as_float(raw.y << 16), v3 = __uint_as_float(raw.y & 0xFFFF0000u);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float pr = A.sc[h][kTileKeys + c.wave];
        acc[h][0] += pr * v0;
        acc[h][1] += pr * v1;
        acc[h][2] += pr * v2;
        acc[h][3] += pr * v3;
      }
    }
  }
  stamp(c, kTAtPv);
  sync(c);
}

// Two ways to split the keys of KV head x / 2, chosen per step from the context length:
// - per XCD: each XCD of the pair splits all keys over its 32 workgroups for its own two
//   query heads (both XCDs stream every key);
// - over the pair: the 64 workgroups of XCDs x & ~1 and x | 1 split the keys once, each
//   split serving all four query heads, so every key and value row leaves HBM once per layer.
//   It costs two cross-XCD hand-offs (the partner's queries, the merge over 64 splits), about
//   one 128-key tile of time, so it is used when it saves at least two tiles per workgroup.
__host__ __device__ inline bool at_pair(int nkeys) {
  const int t32 = (nkeys + kPerXcd * kTileKeys - 1) / (kPerXcd * kTileKeys);
  const int t64 = (nkeys + kSplits * kTileKeys - 1) / (kSplits * kTileKeys);
  return t32 - t64 >= 2;
}
// Split of this workgroup: keys [j0, j1). Its record index in the pair's partials is
// (x & 1) * 32 + r in both modes.
DF_DEVICE void at_keys4(const Ctx& c, int& j0, int& j1) {
  const int nkeys = c.pos + 1;
  const bool pair = at_pair(nkeys);
  const int nsplit = pair ? kSplits : kPerXcd;
  const int per = (nkeys + nsplit - 1) / nsplit;
  const int split = pair ? (c.xcd & 1) * kPerXcd + c.r : c.r;
  j0 = min(split * per, nkeys);
  j1 = min(j0 + per, nkeys);
}

// Compute waves (kTileBars barriers): one 128-key tile for nh query heads (2: this XCD's, 4:
// the KV head's, split over the pair): QK (MFMA, row h = head slot h), then the V rows are
// loaded while the online softmax runs (wave h for head h), then PV.
DF_DEVICE void at_tile4(Ctx& c, LayerPtr Lp, int t0, int j1, const AtPre& P, float acc[kPairHeads][4], int nh,
                        Lds& L) {
  auto& A = L.u.at4;
  const int col = c.lane & 15, slot = c.lane >> 4;
  const float scale = 1.0f / sqrtf(static_cast<float>(kHd));
  // the tile's K loads are the only vector loads in flight (the weight stream is held):
  // waiting for all of them here also tells the compiler that none is pending afterwards
  wait_vm<0>();
  {
    const int key = t0 + c.wave * 16 + col;
    const bool live = key < j1;
    df_f32x4 d4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      uint4 kn = *reinterpret_cast<const uint4*>(A.knew + d * 32 + slot * 8);
      asm volatile("" : "+v"(kn.x), "+v"(kn.y), "+v"(kn.z), "+v"(kn.w));  // a value, not a pointer select into P
      uint4 bw = make_uint4(0u, 0u, 0u, 0u);
      if (live) bw = key == c.pos ? kn : P.kb[d];
      uint4 aw = make_uint4(0u, 0u, 0u, 0u);
      if (col < nh) aw = *reinterpret_cast<const uint4*>(&A.q[col][d * 32 + slot * 8]);
      d4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(df_bf16x8, aw), __builtin_bit_cast(df_bf16x8, bw),
                                                   d4, 0, 0, 0);
    }
    if (slot == 0) {
#pragma unroll
      for (int h = 0; h < kPairHeads; ++h)
        if (h < nh) A.sc[h][c.wave * 16 + col] = live ? d4[h] * scale : -INFINITY;
    }
  }
  const bool ext = at_ext(t0, j1);
  const int ek = t0 + kTileKeys + c.wave;
  if (ext) {  // this wave's extra key: q . k over the 64 lanes' 4 dims each, per head
    uint2 kr = P.ke;
    if (ek == c.pos) kr = *reinterpret_cast<const uint2*>(A.knew + c.lane * 4);
    const float k4[4] = {__uint_as_float(kr.x << 16), __uint_as_float(kr.x & 0xFFFF0000u),
                         __uint_as_float(kr.y << 16), __uint_as_float(kr.y & 0xFFFF0000u)};
#pragma unroll
    for (int h = 0; h < kPairHeads; ++h) {
      if (h >= nh) break;
      float se = -INFINITY;
      if (ek < j1) {
        const uint2 qr = *reinterpret_cast<const uint2*>(&A.q[h][c.lane * 4]);
        float p = __uint_as_float(qr.x << 16) * k4[0];
        p += __uint_as_float(qr.x & 0xFFFF0000u) * k4[1];
        p += __uint_as_float(qr.y << 16) * k4[2];
        p += __uint_as_float(qr.y & 0xFFFF0000u) * k4[3];
        se = dsum(p) * scale;
      }
      if (c.lane == 0) A.sc[h][kTileKeys + c.wave] = se;
    }
  }
  // V rows: keys t0 + 16 wave + j, dims 4 lane ..+3 (and the extra key's)
  uint2 vb[16], ve = make_uint2(0u, 0u);
  {
    const size_t base = (size_t)(c.xcd >> 1) * c.max_len;
    GlobalBf16 vc = (GlobalBf16)LF(Lp, v_cache);
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int kk = t0 + c.wave * 16 + jj;
      vb[jj] = make_uint2(0u, 0u);
      if (kk < j1 && kk != c.pos) vb[jj] = gload8(vc + (base + kk) * kHd + c.lane * 4);
    }
    if (ext && ek < j1 && ek != c.pos) ve = gload8(vc + (base + ek) * kHd + c.lane * 4);
  }
  sync(c);
  if (c.wave < nh) {
    const int h = c.wave;
    const float s0 = A.sc[h][c.lane], s1 = A.sc[h][c.lane + 64];
    const float s2 = ext && c.lane < kCompute ? A.sc[h][kTileKeys + c.lane] : -INFINITY;
    const float tmax = dmax(fmaxf(fmaxf(s0, s1), s2));
    const float mo = A.ml[h][0];
    const float m_new = fmaxf(mo, tmax);
    float p0 = 0.f, p1 = 0.f, p2 = 0.f, alpha = 1.0f;
    if (m_new != -INFINITY) {
      p0 = s0 == -INFINITY ? 0.0f : expf(s0 - m_new);
      p1 = s1 == -INFINITY ? 0.0f : expf(s1 - m_new);
      p2 = s2 == -INFINITY ? 0.0f : expf(s2 - m_new);
      alpha = mo == -INFINITY ? 0.0f : expf(mo - m_new);
    }
    const float lsum = dsum((p0 + p1) + p2);
    A.sc[h][c.lane] = p0;
    A.sc[h][c.lane + 64] = p1;
    if (ext && c.lane < kCompute) A.sc[h][kTileKeys + c.lane] = p2;
    if (c.lane == 0) {
      A.ml[h][0] = m_new;
      A.ml[h][1] = A.ml[h][1] * alpha + lsum;
      A.alpha[h] = alpha;
    }
  }
  sync(c);
  wait_vm<0>();  // the V rows (nothing else is in flight)
  {
#pragma unroll
    for (int h = 0; h < kPairHeads; ++h) {
      if (h >= nh) break;
      const float a = A.alpha[h];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[h][i] *= a;
    }
    uint2 vn = *reinterpret_cast<const uint2*>(A.vnew + c.lane * 4);
    asm volatile("" : "+v"(vn.x), "+v"(vn.y));
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int kk = t0 + c.wave * 16 + jj;
      if (kk < j1) {
        const uint2 raw = kk == c.pos ? vn : vb[jj];
        const float v0 = __uint_as_float(raw.x << 16), v1 = __uint_as_float(raw.x & 0xFFFF0000u);
        const float v2 = __uint_as_float(raw.y << 16), v3 = __uint_as_float(raw.y & 0xFFFF0000u);
#pragma unroll
        for (int h = 0; h < kPairHeads; ++h) {
          if (h >= nh) break;
          const float pr = A.sc[h][c.wave * 16 + jj];
          acc[h][0] += pr * v0;
          acc[h][1] += pr * v1;
          acc[h][2] += pr * v2;
          acc[h][3] += pr * v3;
        }
      }
    }
    if (ext && ek < j1) {
      const uint2 raw = ek == c.pos ? vn : ve;
      const float v0 = __uint_as_float(raw.x << 16), v1 = __uint_as_float(raw.x & 0xFFFF0000u);
      const float v2 = __uint_as_float(raw.y << 16), v3 = __uint_as_float(raw.y & 0xFFFF0000u);
#pragma unroll
      for (int h = 0; h < kPairHeads; ++h) {
        if (h >= nh) break;
        const float pr = A.sc[h][kTileKeys + c.wave];
        acc[h][0] += pr * v0;
        acc[h][1] += pr * v1;
        acc[h][2] += pr * v2;
        acc[h][3] += pr * v3;
      }
    }
  }
  sync(c);
}

// ---------------------------------------------------------------------------------------
// the two roles
//
// Barrier schedule per token (C = control wave, W = compute waves; every step below ends
// at one barrier that both pass):
//   embed      C: token row into L.h                                   | 1
//   in_proj    W: RMSNorm -> g_x, group sums (h, its sum of squares and| kNormBars
//                 the norm weight are in LDS since the last barrier)
//              W: consume blocks                                       | 1, then C: epilogue (tagged)
//   delta      C: hand-off, conv inputs                                 | 1
//              W: conv + SiLU                                          | 1
//              W: norms, gates, delta rule                             | 1, then C: core (tagged), state
//   out_proj   C: hand-off, core                                       | 1
//              W: GatedRMSNorm -> g_x, group sums                      | 1
//              W: consume                                              | 1
//              C: row-parallel partials, all-reduce, h into LDS        | 1
//   attention  C: hand-off, q/k/v / norm weights; W: first KV tile     | 1
//              W: q/k norm + RoPE                                      | 1
//              W: tiles                                                | kTileBars per tile
//              W: PV partials; sum                                     | 2, then C: publish split
//   merge      C only
//   o_proj     C: hand-off, core -> g_x, group sums                    | 1
//              W: consume                                              | 1
//              C: row-parallel partials, all-reduce                    | 1
//   gate|up    as in_proj
//   down       C: hand-off, gate|up column sums                        | 1
//              W: SwiGLU -> g_x, group sums                            | kActBars
//              then as o_proj
//   head       W: RMSNorm                                              | kNormBars
//              W: consume head blocks, argmax per wave                 | 1
//              C: logits, candidate, global argmax                     | 1
// The control wave works on a phase's outputs (partials, logits) after that phase's last
// barrier, so the compute waves write shared LDS only after the next barrier.
// ---------------------------------------------------------------------------------------

// The compute waves' whole launch.
template <bool PAIR>
DF_DEVICE void compute_main(const DfPersistModel& M, const Geo& q, Ctx& c, int steps, Lds& L) {
  const int hidden = M.hidden;
  const int G = q.Gh;
  const int pos0 = *M.position;
  wait_vm<0>();
  // the weight stream starts with layer 0's input projection
  Stream st;
  st.wp = nullptr;
  st.sp = nullptr;
  st.left = 0;
  st.issued = st.consumed = st.wslot = st.rslot = 0;
  st.ri = st.istep = 0;
  st.state = kStreaming;
  st.nruns = build_runs<PAIR>(M, q, c);
  fill(st, steps, c);
  auto stop = [&]() { __builtin_amdgcn_s_waitcnt(0); };

  for (int step = 0; step < steps; ++step) {
    c.pos = pos0 + step;
    c.nb = 0;
#ifdef DF_TRACE
    // each compute wave of workgroup (0, 0) stamps into its own row after the control wave's
    const bool traced = M.trace && step == M.trace_step && c.xcd == 0 && c.r == 0 && M.trace_capacity >= 4096;
    c.tr = traced ? M.trace + 2048 + c.wave * 240 : nullptr;
    c.tn = 0;
    c.tcap = 240;
#endif
    fence(c);
    sync(c);  // embed
    if (!L.ok) return stop();
    // a GEMV phase's first block pair, dequantised while the control wave runs the hand-off
    // before it (after out_proj / o_proj for gate|up, after gate|up for down, after down for the
    // next input projection, after the delta step for out_proj)
    PreDq pre;
    pre.ok = false;
    for (int li = 0; li < M.num_layers; ++li) {
      LayerPtr Lp = layer_at(M, li);
      const int kind = LKIND(Lp);
      {  // input projection
        fence(c);
        const Gemv g = gemv_of(Lp, q, 0, c.xcd, c.r);
        norm_w(L, c, hidden, M.eps);
        gemv_consume(g, c, st, M, q, steps, L, pre);
        sync(c);
      }
      if (kind == 0) {
        {  // the Gated DeltaNet step's arithmetic (dn_conv, dn_math); the control wave stages it
          sync(c);  // inputs in LDS
          if (!L.ok) return stop();
          stamp(c, kTDnIn);
          dn_conv(c, L);
          sync(c);
          stamp(c, kTDnConv);
          dn_math(c, L);
          stamp(c, kTDnMath);
          sync(c);
          static_assert(kDnBars == 3, "the control wave passes the same barriers");
        }
        {  // gated norm + out_proj
          fence(c);
          const Gemv g = gemv_of(Lp, q, 1, c.xcd, c.r);
          predequant(g, c, st, steps, pre);
          sync(c);
          if (!L.ok) return stop();
          // GatedRMSNorm: wave h < 4 takes head h whole (elements 128 h + lane and + 64), so
          // no partial crosses waves; each sum is the two 64-lane halves added in order
          if (c.wave < 4) {
            const int i0 = 128 * c.wave + c.lane, i1 = i0 + 64;
            const float v0 = bf2f(g_x[i0]), v1 = bf2f(g_x[i1]);
            const float tot = dsum(v0 * v0) + dsum(v1 * v1);
            const float rr = 1.0f / sqrtf(tot / 128.0f + M.eps);
            const float t0 = round_bf(bf2f(L.gnw[c.lane]) * round_bf(v0 * rr));
            const float t1 = round_bf(bf2f(L.gnw[64 + c.lane]) * round_bf(v1 * rr));
            const float xv0 = round_bf(t0 * silu(L.zs[i0]));
            const float xv1 = round_bf(t1 * silu(L.zs[i1]));
            g_xh[i0] = f2bf(xv0);
            g_xh[i1] = f2bf(xv1);
          }
          sync(c);
          gemv_consume(g, c, st, M, q, steps, L, pre);
          sync(c);
          predequant(gemv_of(Lp, q, 2, c.xcd, c.r), c, st, steps, pre);
          sync(c);  // all-reduce done, h in LDS
          if (!L.ok) return stop();
        }
      } else {
        // attention split
        if constexpr (PAIR) {
          fence(c);
          int j0, j1;
          at_keys4(c, j0, j1);
          auto& A = L.u.at4;
          sync(c);  // q/k/v staged
          if (!L.ok) return stop();
          const int nh = at_pair(c.pos + 1) ? kPairHeads : 2;  // head slots in use
          if (c.wave < nh || c.wave == kPairHeads) {  // waves 0..nh-1: the query heads, wave 4: the new key
            const bool qw = c.wave < kPairHeads;
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = qw ? A.qraw[c.wave][c.lane * 4 + i] : A.kraw[c.lane * 4 + i];
            norm_rope4_lds(x, qw ? A.qn_w : A.kn_w, M.eps, A.rope, c.lane);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (qw) A.q[c.wave][c.lane * 4 + i] = f2bf(x[i]);
              else A.knew[c.lane * 4 + i] = f2bf(x[i]);
            }
          } else if (c.wave == kPairHeads + 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) A.vnew[c.lane * 4 + i] = f2bf(A.vraw[c.lane * 4 + i]);
          }
          sync(c);
          // the split that holds the new position writes its key/value row (write-through: any
          // workgroup of either XCD of the pair reads the row in later steps); split per XCD,
          // the even XCD's
          if (c.pos >= j0 && c.pos < j1 && c.tid < kHd / 2 && (at_pair(c.pos + 1) || (c.xcd & 1) == 0)) {
            const size_t row = ((size_t)(c.xcd >> 1) * M.max_len + c.pos) * kHd;
            const uint32_t kw = static_cast<uint32_t>(A.knew[2 * c.tid]) | (static_cast<uint32_t>(A.knew[2 * c.tid + 1]) << 16);
            const uint32_t vw = static_cast<uint32_t>(A.vnew[2 * c.tid]) | (static_cast<uint32_t>(A.vnew[2 * c.tid + 1]) << 16);
            st_sys(reinterpret_cast<uint32_t*>(LF(Lp, k_cache) + row) + c.tid, kw);
            st_sys(reinterpret_cast<uint32_t*>(LF(Lp, v_cache) + row) + c.tid, vw);
          }
          float acc[kPairHeads][4];
#pragma unroll
          for (int h = 0; h < kPairHeads; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[h][i] = 0.0f;
          for (int t0 = j0; t0 < j1; t0 += kTileKeys) {
            // K rows are loaded here, in straight-line code with their use (a prefetch across
            // the staging barrier leaves the compiler unsure they completed, and it then makes
            // the weight-stream loops wait for them)
            AtPre P;
            at_issue_k(c, Lp, t0, j1, P);
            at_tile4(c, Lp, t0, j1, P, acc, nh, L);
            if (at_ext(t0, j1)) break;  // its extra keys were the split's last
          }
          // the split's KV loads are consumed (wait unconditionally: the compiler cannot pair
          // the first tile's prefetch with the loop, and the held stream has nothing in flight)
          wait_vm<0>();
          // combine the waves' PV partials into A.red. The partials (32 KB) go to the weight
          // ring, which is drained here: the stream holds at this layer's marker run, right after
          // its input projection, so every block it issued was consumed and no DMA is in flight;
          // the ring is refilled only after the second barrier below.
          {
            float(*prt)[kPairHeads][kHd] = reinterpret_cast<float(*)[kPairHeads][kHd]>(&g_ring_w[0][0][0]);
            static_assert(sizeof(float) * kCompute * kPairHeads * kHd <= sizeof(g_ring_w), "partials fit the ring");
#pragma unroll
            for (int hh = 0; hh < kPairHeads; ++hh)
              if (hh < nh)
                *reinterpret_cast<float4*>(&prt[c.wave][hh][c.lane * 4]) = make_float4(acc[hh][0], acc[hh][1], acc[hh][2], acc[hh][3]);
            sync(c);
#pragma unroll
            for (int e = c.tid; e < nh * kHd; e += kCompute * 64) {
              const int hh = e / kHd, d = e % kHd;
              float sum = 0.0f;
#pragma unroll
              for (int wv = 0; wv < kCompute; ++wv) sum += prt[wv][hh][d];
              A.red[hh][d] = sum;
            }
          }
          sync(c);
          // the weight stream resumes with o_proj while the control wave merges the splits: two
          // blocks per wave at a time, spaced out, so the refill (64 KB per CU) does not hold up
          // the control wave's hand-off loads, which share the CU's memory pipeline
          if (st.state == kHeld) {
            st.state = kReleased;
            open_run(st, steps);
#pragma unroll 1
            for (int k = 2; k <= kRing; k += 2) {
              fill(st, steps, c, k);
              if (k < kRing) __builtin_amdgcn_s_sleep(10);
            }
          }
          {  // o_proj (the merge runs on the control wave meanwhile)
            fence(c);
            const Gemv g = gemv_of(Lp, q, 1, c.xcd, c.r);
              sync(c);
            if (!L.ok) return stop();
            gemv_consume(g, c, st, M, q, steps, L, pre);
            sync(c);
            predequant(gemv_of(Lp, q, 2, c.xcd, c.r), c, st, steps, pre);
            sync(c);  // all-reduce done
            if (!L.ok) return stop();
          }
        } else {
          fence(c);
          int j0, j1;
          at_keys(c, j0, j1);
          auto& A = L.u.at;
          if (j0 < j1) at_dma_k(c, Lp, j0, j1);  // the first tile's K rows, ahead of the staging
          sync(c);  // q/k/v staged
          if (!L.ok) return stop();
          stamp(c, kTAtStaged);
          if (c.wave < 3) {
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = c.wave < 2 ? A.qraw[c.wave][c.lane * 4 + i] : A.kraw[c.lane * 4 + i];
            norm_rope4_lds(x, c.wave < 2 ? A.qn_w : A.kn_w, M.eps, A.rope, c.lane);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (c.wave < 2) A.q[c.wave][c.lane * 4 + i] = f2bf(x[i]);
              else A.knew[c.lane * 4 + i] = f2bf(x[i]);
            }
          } else if (c.wave == 3) {
#pragma unroll
            for (int i = 0; i < 4; ++i) A.vnew[c.lane * 4 + i] = f2bf(A.vraw[c.lane * 4 + i]);
          }
          sync(c);
          stamp(c, kTAtRoped);
          // the even XCD of the pair writes the new key/value (write-through: the odd XCD
          // reads this row in later steps)
          if ((c.xcd & 1) == 0 && c.pos >= j0 && c.pos < j1 && c.tid < kHd / 2) {
            const size_t row = ((size_t)(c.xcd >> 1) * M.max_len + c.pos) * kHd;
            const uint32_t kw = static_cast<uint32_t>(A.knew[2 * c.tid]) | (static_cast<uint32_t>(A.knew[2 * c.tid + 1]) << 16);
            const uint32_t vw = static_cast<uint32_t>(A.vnew[2 * c.tid]) | (static_cast<uint32_t>(A.vnew[2 * c.tid + 1]) << 16);
            st_sys(reinterpret_cast<uint32_t*>(LF(Lp, k_cache) + row) + c.tid, kw);
            st_sys(reinterpret_cast<uint32_t*>(LF(Lp, v_cache) + row) + c.tid, vw);
          }
          float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
          for (int t0 = j0; t0 < j1; t0 += kTileKeys) {
            // V rows are loaded here, in straight-line code with their use (loads held across
            // the staging code raise the register pressure of the whole kernel, which then
            // spills around the GEMV phases); K rows go by DMA, the first tile's before the staging
            if (t0 != j0) at_dma_k(c, Lp, t0, j1);  // the previous tile's QK is past its barriers
            AtPreKV P;
            at_issue_v(c, Lp, t0, j1, P);
            at_tile(c, Lp, t0, j1, P, acc, L);
            if (at_ext(t0, j1)) break;  // its extra keys were the split's last
          }
          // the split's KV loads are consumed (wait unconditionally: the compiler cannot pair
          // the first tile's prefetch with the loop, and the held stream has nothing in flight)
          wait_vm<0>();
          // combine the waves' PV partials (into wave 0's row)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 4; ++i) A.red[c.wave][hh][c.lane * 4 + i] = acc[hh][i];
          sync(c);
          {
            const int e = c.tid;  // 512 = 2 heads x 256 dims
            const int hh = e / kHd, d = e % kHd;
            float sum = 0.0f;
#pragma unroll
            for (int wv = 0; wv < kCompute; ++wv) sum += A.red[wv][hh][d];
            A.red[0][hh][d] = sum;
          }
          sync(c);
          stamp(c, kTAtDone);
          // the weight stream resumes with o_proj while the control wave merges the splits: two
          // blocks per wave at a time, spaced out, so the refill (64 KB per CU) does not hold up
          // the control wave's hand-off loads, which share the CU's memory pipeline
          if (st.state == kHeld) {
            st.state = kReleased;
            open_run(st, steps);
#pragma unroll 1
            for (int k = 2; k <= kRing; k += 2) {
              fill(st, steps, c, k);
              if (k < kRing) __builtin_amdgcn_s_sleep(10);
            }
          }
          {  // o_proj (the merge runs on the control wave meanwhile)
            fence(c);
            const Gemv g = gemv_of(Lp, q, 1, c.xcd, c.r);
              sync(c);
            if (!L.ok) return stop();
            gemv_consume(g, c, st, M, q, steps, L, pre);
            sync(c);
            predequant(gemv_of(Lp, q, 2, c.xcd, c.r), c, st, steps, pre);
            sync(c);  // all-reduce done
            if (!L.ok) return stop();
          }
        }
      }
      {  // gate|up + SwiGLU
        fence(c);
        const Gemv g = gemv_of(Lp, q, 2, c.xcd, c.r);
        norm_w(L, c, hidden, M.eps);
        gemv_consume(g, c, st, M, q, steps, L, pre);
        sync(c);
      }
      {  // down
        fence(c);
        const Gemv g = gemv_of(Lp, q, 3, c.xcd, c.r);
        predequant(g, c, st, steps, pre);
        sync(c);
        if (!L.ok) return stop();
        swiglu_act(L, c, q.inter_x);
        gemv_consume(g, c, st, M, q, steps, L, pre);
        sync(c);
        if (li + 1 < M.num_layers) predequant(gemv_of(layer_at(M, li + 1), q, 0, c.xcd, c.r), c, st, steps, pre);
        sync(c);  // all-reduce done
        if (!L.ok) return stop();
      }
    }
    {  // final norm + tied head
      fence(c);
      auto& H = L.hd;
      norm_w(L, c, hidden, M.eps);
      // tiles t0 .. t0 + ntw, all groups, from the weight stream
      const int t0 = head_tile(q, c.wave), ntw = head_tile(q, c.wave + 1) - t0;
      const uint16_t* xb = g_xh + (c.lane >> 4) * 32;
      const uint32_t sh = 16u * (c.lane & 1);
      const DqK K = dq_consts();
      float bv = -INFINITY;
      int bi = 0x7FFFFFFF;
      float acc = 0.0f;
      int gl = 0, j = 0;
      // G is a multiple of 4 (hidden % 512 == 0), so a pair never straddles two tiles
#pragma unroll 1
      for (int i = 0; i < ntw * G; i += 2) {
        PairIn in;
        take_pair(st, c, xb + gl * kGroup, xb + (gl + 1) * kGroup, in);
        const float v0 = block_dot_r(in.w0, in.s0, in.x0, sh, K);
        const float v1 = block_dot_r(in.w1, in.s1, in.x1, sh, K);
        refill2(st, steps, c);
        acc += v0;
        acc += v1;
        gl += 2;
        if (gl == G) {  // tile complete: logits of 16 columns in lanes 0..15
          const int t = t0 + j;
          const uint16_t lb = f2bf(acc);
          if (c.lane < 16) {
            H.logit[(t - q.t_lo) * 16 + c.lane] = lb;
            const float lv = bf2f(lb);
            const int lix = t * 16 + c.lane;
            if (lv > bv || (lv == bv && lix < bi)) {
              bv = lv;
              bi = lix;
            }
          }
          acc = 0.0f;
          gl = 0;
          ++j;
        }
      }
      row_argmax(bv, bi);
      if (c.lane == 0) {
        H.bv[c.wave] = bv;
        H.bi[c.wave] = bi;
      }
      if (c.tid == 0) L.nbw = c.nb + 2;
      sync(c);
      sync(c);  // global argmax done
      if (!L.ok) return stop();
    }
  }
  stop();
}

// The control wave's whole launch.
template <bool TABLE, bool PAIR>
DF_DEVICE void control_main(const DfPersistModel& M, const Geo& q, Ctx& c, int steps, int teacher_forced, Lds& L) {
  // The control wave shares SIMD 0 with compute waves 0 and 4, which dequantise a phase's
  // first blocks (predequant) while it runs the hand-off: at equal priority its epilogue,
  // polls and staging got about a third of that SIMD's issue slots. It issues little
  // (polls sleep between tries), so letting it win the arbitration costs the compute waves
  // little and shortens the serial chain (1.4 % per token, same-box A/B).
  __builtin_amdgcn_s_setprio(3);
  const int hidden = M.hidden;
  const int G = q.Gh;
  const int pos0 = *M.position;
  const int step0 = M.step ? *M.step : 0;
  int64_t token = M.tokens[0];
  dma_row(LF(layer_at(M, 0), in_norm), L.nw, hidden, c.lane);
  uint32_t pre_rope = 0;  // the next attention layer's RoPE row entry of this lane
  auto fail = [&](int nbars) {  // pass the barriers the compute waves still wait at, then stop
    if (c.lane == 0) L.ok = 0;
    for (int i = 0; i < nbars; ++i) bar();
  };

  for (int step = 0; step < steps; ++step) {
    c.pos = pos0 + step;
    c.tr = (M.trace && step == M.trace_step && c.xcd == 0 && c.r == 0) ? M.trace : nullptr;
    c.tn = 0;
    c.nb = 0;
    // ---- embedding of the step's token into L.h ---------------------------------------
    fence(c, kTEmbed);
    if (teacher_forced) token = M.prompt[c.pos];
    if (token < 0 || token >= M.vocab) {
      if (c.lane == 0 && c.xcd == 0 && c.r == 0) raise_abort(c, kErrToken);
      return fail(1);
    }
    if constexpr (TABLE) {
      // the checkpoint's bf16 row, 16 bytes per lane per chunk, and its sum of squares (the
      // same order in every workgroup)
      const auto rt = rsrc(M.embed_table + (size_t)token * hidden);
      uint4 hv[kHidChunks];
#pragma unroll
      for (int k = 0; k < kHidChunks; ++k) {
        const int ch = c.lane + 64 * k;
        if (ch * 8 < hidden) hv[k] = ld16<kCpPlain>(rt, ch * 16);
      }
      float sq = 0.0f;
#pragma unroll
      for (int k = 0; k < kHidChunks; ++k) {
        const int ch = c.lane + 64 * k;
        if (ch * 8 < hidden) {
          *reinterpret_cast<uint4*>(&L.h[ch * 8]) = hv[k];
          const uint32_t w[4] = {hv[k].x, hv[k].y, hv[k].z, hv[k].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xFFFF0000u);
            sq += lo * lo;
            sq += hi * hi;
          }
        }
      }
      sq = dsum(sq);
      if (c.lane == 0) L.ss = sq;
    } else {
      const int tt = static_cast<int>(token / 16), cc = static_cast<int>(token % 16);
      const uint32_t* wt = reinterpret_cast<const uint32_t*>(M.head_w);
      constexpr int K = (kMaxHidden / kGroup * 16 + 63) / 64;
      uint32_t wd[K];
      uint16_t sc[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int idx = c.lane + 64 * k;  // idx = g*16 + s*4 + d
        if (idx < G * 16) {
          const size_t block = (size_t)tt * G + idx / 16;
          wd[k] = wt[block * 256 + (((idx / 4) & 3) * 16 + cc) * 4 + (idx & 3)];
          sc[k] = M.head_s[block * 16 + cc];
        }
      }
      float sq = 0.0f;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int idx = c.lane + 64 * k;
        if (idx < G * 16) {
          const int g = idx / 16, s = (idx / 4) & 3, d = idx & 3;
          const float scv = bf2f(sc[k]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int sh = (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
            const int qv = static_cast<int>((wd[k] >> sh) & 15u) - 8;
            const uint16_t hb = f2bf(static_cast<float>(qv) * scv);
            L.h[g * 128 + s * 32 + d * 8 + e] = hb;
            sq += bf2f(hb) * bf2f(hb);
          }
        }
      }
      sq = dsum(sq);
      if (c.lane == 0) L.ss = sq;
    }
    if (c.lane == 0) L.ok = 1;
    sync(c);

    for (int li = 0; li < M.num_layers; ++li) {
      LayerPtr Lp = layer_at(M, li);
      const int kind = LKIND(Lp);
      // ================= input projection (column-parallel) =========================
      {
        fence(c, kTProj);
        const Gemv g = gemv_of(Lp, q, 0, c.xcd, c.r);
        // in_norm is in L.nw: its DMA was issued before the previous all-reduce's polls (or
        // the embedding's loads), whose waits it completed by (in-order vmcnt)
        for (int i = 0; i < kNormBars; ++i) sync(c);
        // the next phase's small parameters, while the compute waves consume
        if (kind == 0) {
          dn_state_prefetch(c, Lp, L);
          dma_row128(LF(Lp, gnorm_w), L.gnw, c.lane);
        } else {
          uint16_t* qn_w = PAIR ? L.u.at4.qn_w : L.u.at.qn_w;
          uint16_t* kn_w = PAIR ? L.u.at4.kn_w : L.u.at.kn_w;
          dma_row128(LF(Lp, q_norm), qn_w, c.lane);
          dma_row128(LF(Lp, q_norm) + 128, qn_w + 128, c.lane);
          dma_row128(LF(Lp, k_norm), kn_w, c.lane);
          dma_row128(LF(Lp, k_norm) + 128, kn_w + 128, c.lane);
          pre_rope = c.lane < kRot / 2 ? M.rope[(size_t)c.pos * (kRot / 2) + c.lane] : 0u;
        }
        sync(c);  // blocks consumed
        c.epoch += 1;
        // with the keys split over the pair, an attention layer's query columns (j < 1024,
        // (j / 256) even) are also read by the pair's other XCD
        colpar_epilogue<true>(g, c, L, PAIR && kind != 0 && at_pair(c.pos + 1));
      }
      if (kind == 0) {
        // ================= conv + gated delta step ===================================
        fence(c, kTDelta);
        c.epoch += 1;
        // the compute waves run the conv and the delta rule between these barriers
        if (!dn_stage(c, Lp, L, c.epoch - 1)) return fail(1);
        sync(c);  // the step's inputs in LDS: the compute waves run the conv
        // meanwhile z (the out_proj GatedRMSNorm's gate, from the same input projection); a
        // failed poll passes the step's barriers and stops where the compute waves next check
        const Seg zseg[1] = {{kLinZ, 512, L.zs}};
        const bool zok = gather_colpar<1, 4>(c, zseg, c.epoch - 1);
        for (int i = 1; i < kDnBars; ++i) sync(c);
        if (!zok) return fail(1);
        dn_publish(c, Lp, L, c.epoch);
        // ================= gated norm + out_proj (row-parallel) ======================
        {
          fence(c, kTOut);
          const Gemv g = gemv_of(Lp, q, 1, c.xcd, c.r);
          // core (512) of the XCD's four value heads
          if (!stage_core(L, c, c.epoch, false)) return fail(1);
          sync(c);
          stamp(c, kTStaged);
          dma_row(LF(Lp, post_norm), L.nw, hidden, c.lane);
          sync(c);  // g_x, group sums
          dn_store_state(c, Lp, L);
          sync(c);  // blocks consumed
          rowpar_epilogue(g, c, L, hidden);
          if (!allreduce_residual(c, L, hidden)) return fail(1);
          sync(c);
        }
      } else {
        // ================= attention split ===========================================
        if constexpr (PAIR) {
          fence(c, kTAttn);
          auto& A = L.u.at4;
          {
            if (!gather_attn(c, A.qraw, A.kraw, c.epoch, at_pair(c.pos + 1))) return fail(1);  // kraw, vraw adjacent
            if (c.lane < kRot / 2) A.rope[c.lane] = pre_rope;
            if (c.lane < kPairHeads) {
              A.ml[c.lane][0] = -INFINITY;
              A.ml[c.lane][1] = 0.0f;
            }
          }
          sync(c);
          stamp(c, kTStaged);
          sync(c);  // q/k normed and roped
          int j0, j1;
          at_keys4(c, j0, j1);
          for (int t0 = j0; t0 < j1; t0 += kTileKeys) {
            for (int i = 0; i < kTileBars; ++i) sync(c);
            if (at_ext(t0, j1)) break;  // the compute waves' last tile took the extra keys
          }
          sync(c);
          sync(c);  // PV partials summed into A.red
          c.epoch += 1;
          {
            // the split's nh heads (acc, m, l) as (fp32, epoch) pairs into record (x & 1) * 32 + r
            // of the pair: written through when the keys are split over the pair (each XCD merges
            // its two heads over all 64 splits), else plain (only this XCD reads it, from L2)
            const bool pair = at_pair(c.pos + 1);
            const int nh = pair ? kPairHeads : 2;
            const int split = (c.xcd & 1) * kPerXcd + c.r;
            const auto ra = rsrc(reinterpret_cast<const uint64_t*>(c.w.apart) + ((size_t)(c.xcd >> 1) * kSplits + split) * kPairHeads * kApHead);
            const uint32_t ep = c.epoch;
#pragma unroll
            for (int k = 0; k < kPairHeads * kHd / 128; ++k) {
              const int e = 2 * (c.lane + 64 * k);  // dims e, e + 1 of head e / kHd
              const int hh = e / kHd, d = e % kHd;
              if (hh >= nh) break;  // (uniform: hh = k / 2)
              const float2 v = *reinterpret_cast<const float2*>(&A.red[hh][d]);
              const uint4 w = make_uint4(__float_as_uint(v.x), ep, __float_as_uint(v.y), ep);
              if (pair) st16<kCpSystem>(ra, (hh * kApHead + d) * 8, w);
              else st16<kCpPlain>(ra, (hh * kApHead + d) * 8, w);
            }
            if (c.lane < nh) {
              const uint4 w = make_uint4(__float_as_uint(A.ml[c.lane][0]), ep, __float_as_uint(A.ml[c.lane][1]), ep);
              if (pair) st16<kCpSystem>(ra, (c.lane * kApHead + kHd) * 8, w);
              else st16<kCpPlain>(ra, (c.lane * kApHead + kHd) * 8, w);
            }
          }
          // ================= merge the splits: head r/16, dims 16 (r%16) ..+15 ============
          {
            fence(c, kTMerge);
            auto& Mg = L.u.mg4;
            const int hl = c.r >> 4, d0 = (c.r & 15) * 16;
            const uint32_t want = c.epoch;
            c.epoch += 1;
            // lane s reads a split's (m, l) of this XCD's head hl and its accumulator dims d0 ..
            // d0+15, polling every (value, epoch) pair (the buffer descriptor is wave-uniform:
            // the lane's record goes into the offset). Split over the pair, lane s reads record s
            // at system scope, where the head is slot hl if this XCD wrote the record and slot
            // 2 + hl if the other XCD did; split per XCD, lane s < 32 reads this XCD's record
            // (x & 1) * 32 + s, slot hl, at agent scope, and lanes 32.. stand for empty splits.
            const bool pair = at_pair(c.pos + 1);
            const bool live = pair || c.lane < kPerXcd;
            const auto r = rsrc(reinterpret_cast<const uint64_t*>(c.w.apart) + (size_t)(c.xcd >> 1) * kSplits * kPairHeads * kApHead);
            const int rec = pair ? c.lane : (c.xcd & 1) * kPerXcd + (c.lane & (kPerXcd - 1));
            const int slot = (rec / kPerXcd) == (c.xcd & 1) ? hl : 2 + hl;
            const int so = ((rec * kPairHeads + slot) * kApHead) * 8;
            static_assert(kSplits == 64, "one split per lane");
            // (m, l) first: one 16-byte poll per lane while the splits finish; the accumulators
            // are then read once (and re-polled only if some are not visible yet)
            uint4 mlv = make_uint4(0xFF800000u, want, 0u, want), av[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) av[k] = make_uint4(0u, want, 0u, want);
            auto ld = [&](int off) { return pair ? ld16<kCpSystem>(r, off) : ld16<kCpAgent>(r, off); };
            if (!poll_tagged(c, [&]() {
                  if (live) mlv = ld(so + kHd * 8);
                  return pairs_ok(mlv, want);
                }))
              return fail(1);
            if (!poll_tagged(c, [&]() {
                  if (live) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) av[k] = ld(so + (d0 + 2 * k) * 8);
                  }
                  bool t = true;
#pragma unroll
                  for (int k = 0; k < 8; ++k) t = t && pairs_ok(av[k], want);
                  return t;
                }))
              return fail(1);
            const Seg seg[1] = {{hl * 512 + kHd + d0, 16, Mg.gate}};
            if (!gather_colpar<1, 1>(c, seg, c.epoch - 2)) return fail(1);  // the input projection's
#pragma unroll
            for (int k = 0; k < 8; ++k)
              *reinterpret_cast<float2*>(&Mg.acc[c.lane][2 * k]) = make_float2(__uint_as_float(av[k].x), __uint_as_float(av[k].z));
            stamp(c, kTStaged);
            const float m = __uint_as_float(mlv.x);
            const float l = __uint_as_float(mlv.z);
            const float mm = l > 0.0f ? m : -INFINITY;
            const float mstar = dmax(mm);
            const float wgt = mm == -INFINITY ? 0.0f : expf(mm - mstar);
            const float den = dsum(wgt * l);
            Mg.wgt[c.lane] = wgt;
            // lane l sums splits 16 (l / 16) .. +15 of dim l % 16; the four quarters are added
            // pairwise across lanes (fixed order)
            float num = 0.0f;
            {
              const int dd = c.lane & 15, s0 = (c.lane >> 4) * 16;
#pragma unroll
              for (int j = 0; j < 16; ++j) num += Mg.wgt[s0 + j] * Mg.acc[s0 + j][dd];
              num += __shfl_xor(num, 16, 64);
              num += __shfl_xor(num, 32, 64);
            }
            if (c.lane < 16) {
              const float o = round_bf(num / den);
              const float gx = Mg.gate[c.lane];
              const float gate = round_bf(M.gate_kind == 0 ? sigmoid(gx) : silu(gx));
              c.w.core[(size_t)c.xcd * 512 + hl * kHd + d0 + c.lane] = tag_bf16(f2bf(o * gate), c.epoch);
            }
          }
          // ================= o_proj (row-parallel) =====================================
          {
            fence(c, kTOProj);
            const Gemv g = gemv_of(Lp, q, 1, c.xcd, c.r);
            if (!stage_core(L, c, c.epoch, true)) return fail(1);
            sync(c);
            stamp(c, kTStaged);
            dma_row(LF(Lp, post_norm), L.nw, hidden, c.lane);
            sync(c);  // blocks consumed
            rowpar_epilogue(g, c, L, hidden);
            if (!allreduce_residual(c, L, hidden)) return fail(1);
            sync(c);
          }
        } else {
          fence(c, kTAttn);
          auto& A = L.u.at;
          {
            const Seg seg[3] = {{0, kHd, A.qraw[0]}, {512, kHd, A.qraw[1]}, {kAttnK, 2 * kHd, A.kraw}};
            if (!gather_colpar<3, 8>(c, seg, c.epoch)) return fail(1);  // kraw and vraw are adjacent in LDS
            if (c.lane < kRot / 2) A.rope[c.lane] = pre_rope;
            if (c.lane < 2) {
              A.ml[c.lane][0] = -INFINITY;
              A.ml[c.lane][1] = 0.0f;
            }
          }
          sync(c);
          stamp(c, kTStaged);
          sync(c);  // q/k normed and roped
          int j0, j1;
          at_keys(c, j0, j1);
          for (int t0 = j0; t0 < j1; t0 += kTileKeys) {
            for (int i = 0; i < kTileBars; ++i) sync(c);
            if (at_ext(t0, j1)) break;  // the compute waves' last tile took the extra keys
          }
          sync(c);
          sync(c);  // PV partials summed into A.red[0]
          c.epoch += 1;
          {
            float* ap = c.w.apart + ((size_t)c.xcd * kPerXcd + c.r) * 2 * kApHead;
            for (int e = c.lane; e < 2 * kHd; e += 64) ap[(e / kHd) * kApHead + e % kHd] = A.red[0][e / kHd][e % kHd];
            if (c.lane < 2) {
              ap[c.lane * kApHead + kHd] = A.ml[c.lane][0];
              ap[c.lane * kApHead + kHd + 1] = A.ml[c.lane][1];
            }
          }
          signal_local(c, c.epoch);
          // ================= merge the 32 splits: head r/16, dims 16 (r%16) ..+15 =======
          {
            fence(c, kTMerge);
            auto& Mg = L.u.mg;
            const int hl = c.r >> 4, d0 = (c.r & 15) * 16;
            if (!wait_local(c, c.epoch)) return fail(1);
            c.epoch += 1;
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
            const Seg seg[1] = {{hl * 512 + kHd + d0, 16, Mg.gate}};
            if (!gather_colpar<1, 1>(c, seg, c.epoch - 2)) return fail(1);  // the input projection's
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const int ch = c.lane + 64 * k;
              *reinterpret_cast<uint4*>(&Mg.acc[ch / 4][4 * (ch % 4)]) = av[k];
            }
            stamp(c, kTStaged);
            const float m = __uint_as_float(static_cast<uint32_t>(ml));
            const float l = __uint_as_float(static_cast<uint32_t>(ml >> 32));
            const float mm = c.lane < kPerXcd && l > 0.0f ? m : -INFINITY;
            const float mstar = dmax(mm);
            const float wgt = mm == -INFINITY ? 0.0f : expf(mm - mstar);
            const float den = dsum(c.lane < kPerXcd ? wgt * l : 0.0f);
            if (c.lane < kPerXcd) Mg.wgt[c.lane] = wgt;
            if (c.lane < 16) {
              float num = 0.0f;
              for (int sp = 0; sp < kPerXcd; ++sp) num += Mg.wgt[sp] * Mg.acc[sp][c.lane];
              const float o = round_bf(num / den);
              const float gx = Mg.gate[c.lane];
              const float gate = round_bf(M.gate_kind == 0 ? sigmoid(gx) : silu(gx));
              c.w.core[(size_t)c.xcd * 512 + hl * kHd + d0 + c.lane] = tag_bf16(f2bf(o * gate), c.epoch);
            }
          }
          // ================= o_proj (row-parallel) =====================================
          {
            fence(c, kTOProj);
            const Gemv g = gemv_of(Lp, q, 1, c.xcd, c.r);
            if (!stage_core(L, c, c.epoch, true)) return fail(1);
            sync(c);
            stamp(c, kTStaged);
            dma_row(LF(Lp, post_norm), L.nw, hidden, c.lane);
            sync(c);  // blocks consumed
            rowpar_epilogue(g, c, L, hidden);
            if (!allreduce_residual(c, L, hidden)) return fail(1);
            sync(c);
          }
        }
      }
      // ================= gate|up + SwiGLU (column-parallel) ============================
      {
        fence(c, kTGateUp);
        const Gemv g = gemv_of(Lp, q, 2, c.xcd, c.r);
        // post_norm is in L.nw (its DMA preceded the all-reduce's polls)
        for (int i = 0; i < kNormBars; ++i) sync(c);
        sync(c);  // blocks consumed
        c.epoch += 1;
        colpar_epilogue<false>(g, c, L);
        signal_local(c, c.epoch);
      }
      // ================= down (row-parallel) ===========================================
      {
        fence(c, kTDown);
        const Gemv g = gemv_of(Lp, q, 3, c.xcd, c.r);
        if (!wait_local(c, c.epoch)) return fail(1);
        stamp(c, kTGuLanded);
        stage_gu<(kColparMax / 4 + 63) / 64>(c, q.inter_x, L.u.ac.gu);
        sync(c);
        stamp(c, kTStaged);
        dma_row(li + 1 < M.num_layers ? LF(layer_at(M, li + 1), in_norm) : M.final_norm, L.nw, hidden, c.lane);
        for (int i = 0; i < kActBars; ++i) sync(c);
        sync(c);  // blocks consumed
        rowpar_epilogue(g, c, L, hidden);
        if (!allreduce_residual(c, L, hidden)) return fail(1);
        sync(c);
      }
    }

    // ================= final norm + tied head + argmax =================================
    {
      fence(c, kTHead);
      auto& H = L.hd;
      // final_norm is in L.nw (its DMA preceded the last all-reduce's polls)
      for (int i = 0; i < kNormBars; ++i) sync(c);
      sync(c);  // head blocks consumed, per-wave candidates in LDS
      stamp(c, kTHeadConsumed);
      c.epoch += 1;
      // logits out (this workgroup's columns, 32 B per tile)
      if (M.logits) {
        const int chunks = (q.t_hi - q.t_lo) * 2;
        for (int e = c.lane; e < chunks; e += 64)
          *reinterpret_cast<uint4*>(M.logits + (size_t)q.t_lo * 16 + e * 8) = *reinterpret_cast<const uint4*>(&H.logit[e * 8]);
      }
      // this workgroup's candidate: one atomic word of value, 18-bit index and the epoch's
      // low 14 bits (a slot is rewritten once per token, so its previous epoch differs by
      // the phases per token)
      if (c.lane == 0) {
        float v = H.bv[0];
        int i = H.bi[0];
        for (int wv = 1; wv < kCompute; ++wv) {
          if (H.bv[wv] > v || (H.bv[wv] == v && H.bi[wv] < i)) {
            v = H.bv[wv];
            i = H.bi[wv];
          }
        }
        st_sys(reinterpret_cast<uint64_t*>(c.w.cand) + blockIdx.x, pack_cand(v, i, c.epoch));
      }
      __builtin_amdgcn_s_waitcnt(0);
      // every workgroup reduces the 256 candidates
      const auto r = rsrc(c.w.cand);
      uint64_t v[kNwg / 64];
      bool ok = true;
      const uint64_t t0 = now();
      for (int it = 1;; ++it) {
#pragma unroll
        for (int k = 0; k < kNwg / 64; ++k) v[k] = ld8<kCpSystem>(r, (c.lane + 64 * k) * 8);
        bool ready = true;
#pragma unroll
        for (int k = 0; k < kNwg / 64; ++k) ready = ready && (static_cast<uint32_t>(v[k]) & 0x3FFFu) == (c.epoch & 0x3FFFu);
        if (__all(ready)) break;
        if ((it & 31) == 0 && ld_sys(c.w.ctl + 1)) { ok = false; break; }
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
      // the barrier schedules of the two roles must agree (compute waves recorded theirs)
      if (ok && L.nbw != c.nb + 1) {
        raise_abort(c, kErrSchedule);
        ok = false;
      }
      stamp(c, kTHeadDone);
      if (c.lane == 0) L.ok = ok;
      sync(c);
      if (!ok) return;
      token = bi;
      if (c.lane == 0 && c.xcd == 0 && c.r == 0 && !teacher_forced && M.token_log) M.token_log[step0 + step] = token;
      dma_row(LF(layer_at(M, 0), in_norm), L.nw, hidden, c.lane);  // the next token's first norm
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (c.lane == 0 && c.xcd == 0 && c.r == 0) {
    M.tokens[0] = token;
    *M.position = pos0 + steps;
    if (M.step && !teacher_forced) *M.step = step0 + steps;
    c.w.ctl[0] = static_cast<int>(c.epoch);
  }
}

// TABLE: embed from the checkpoint's bf16 table (M.embed_table) instead of the tied int4
// head. Two instances, so the tied build carries no code for the other path (the decode is
// sensitive to the kernel's code layout).
// TABLE: the embedding reads a bf16 table (else it dequantises the tied head's row). PAIR: the
// KV cache can hold enough keys for attention to split them over the XCD pair (chosen per step
// by at_pair); the other instance keeps the per-XCD split and its code layout.
template <bool TABLE, bool PAIR>
__global__ __launch_bounds__(kThreads) void decode_kernel(DfPersistModel M, Ws w, int steps, int teacher_forced) {
  __shared__ Lds L;
  Ctx c;
  c.w = w;
  c.ar = 0;
  c.nb = 0;
  c.tcap = M.trace_capacity;
  c.max_len = M.max_len;
  c.tr = nullptr;
  c.tn = 0;

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
  {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(M.layers);
    uint64_t* dst = reinterpret_cast<uint64_t*>(g_layers);
    const int words = M.num_layers * static_cast<int>(sizeof(DfPersistLayer) / 8);
    for (int i = threadIdx.x; i < words; i += kThreads) dst[i] = src[i];
  }
  __syncthreads();
  if (!L.ok) return;
  c.xcd = L.token / kPerXcd;
  c.r = L.token % kPerXcd;
  fence(c);
  c.epoch = static_cast<uint32_t>(w.ctl[0]);
  const int pos0 = *M.position;
  const int step0 = M.step ? *M.step : 0;
  if (pos0 < 0 || pos0 + steps > M.max_len || (teacher_forced && pos0 + steps > M.prompt_len) ||
      (!teacher_forced && M.token_log && step0 + steps > M.log_capacity)) {
    if (c.tid == 0 && c.xcd == 0 && c.r == 0) raise_abort(c, kErrPosition);
    return;
  }

  Geo q;
  q.hidden = M.hidden;
  q.Gh = M.hidden / kGroup;
  q.inter = M.inter;
  q.inter_x = M.inter / kXcd;
  q.gu_tiles = 2 * q.inter_x / kTileCols;
  const int row_tiles = M.hidden / kTileCols;
  q.rp_lo = (c.r * row_tiles) / kPerXcd;
  q.rp_hi = ((c.r + 1) * row_tiles) / kPerXcd;
  q.ngx = q.inter_x / kGroup;
  const int vocab_tiles = M.vocab / kTileCols / kXcd;
  q.t_lo = c.xcd * vocab_tiles + (c.r * vocab_tiles) / kPerXcd;
  q.t_hi = c.xcd * vocab_tiles + ((c.r + 1) * vocab_tiles) / kPerXcd;
  __syncthreads();  // everyone has read the registration before L.token is reused

  if (c.control) control_main<TABLE, PAIR>(M, q, c, steps, teacher_forced, L);
  else compute_main<PAIR>(M, q, c, steps, L);
}

__global__ void register_reset_kernel(int* ctl) {
  if (threadIdx.x < kXcd) ctl[kRegBase + threadIdx.x] = 0;
}

// DF_PERSISTENT_PLAIN_LAUNCH=1 launches the decode kernel as an ordinary dispatch instead of a
// cooperative one (read once per process). rocprofv3 cannot finish its trace of a process
// that made cooperative launches (it faults at process exit before writing results), so
// profiles of the decode kernel are taken with this set.
inline bool plain_launch() {
  static const bool v = [] {
    const char* e = std::getenv("DF_PERSISTENT_PLAIN_LAUNCH");
    return e && e[0] == '1';
  }();
  return v;
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
      m.vocab <= 0 || m.vocab % 128 || m.vocab > (1 << 18) || m.num_layers < 1 || m.num_layers > kMaxLayers || m.max_len < 1 || !m.layers ||
      !m.head_w || !m.head_s || !m.final_norm || !m.rope || !m.position || !m.tokens)
    return DF_BAD_ARGUMENT;
  if (2 * (m.inter / kXcd) > kColparMax) return DF_BAD_ARGUMENT;
  if (m.inter / kXcd / kGroup > kMaxGroups || m.hidden / kGroup > kMaxGroups) return DF_BAD_ARGUMENT;
  if ((m.vocab / kTileCols / kXcd + kPerXcd - 1) / kPerXcd > kMaxHeadTiles) return DF_BAD_ARGUMENT;
  if (teacher_forced && !m.prompt) return DF_BAD_ARGUMENT;
  // a workgroup's block range of every GEMV phase spans at most kMaxWgTiles output tiles
  const int G = m.hidden / kGroup;
  auto fits = [&](int blocks, int ng) { return (blocks + kPerXcd - 1) / kPerXcd / ng + 2 <= kMaxWgTiles; };
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
  // the launch's positions are on the device; the cache length bounds them. (The table lists
  // the tied-head, per-XCD instance first, which places its code first in the code object.)
  static const void* const kernels[4] = {
      reinterpret_cast<const void*>(decode_kernel<false, false>), reinterpret_cast<const void*>(decode_kernel<true, false>),
      reinterpret_cast<const void*>(decode_kernel<false, true>), reinterpret_cast<const void*>(decode_kernel<true, true>)};
  const void* kernel = kernels[(m.embed_table ? 1 : 0) + (at_pair(m.max_len) ? 2 : 0)];
  if (plain_launch()) {
    // an ordinary dispatch of the same grid: co-residency is checked here instead of by the
    // cooperative launch (one workgroup per CU, every CU of the device), and a workgroup that
    // never starts makes the others' hand-off waits time out into the abort word
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess ||
        cus * per_cu < kNwg)
      return DF_LAUNCH_FAILED;
    void* args[] = {&m, &w, &steps, &teacher_forced};
    if (hipLaunchKernel(kernel, dim3(kNwg), dim3(kThreads), args, 0, stream) != hipSuccess) return DF_LAUNCH_FAILED;
    return hipGetLastError() == hipSuccess ? DF_OK : DF_LAUNCH_FAILED;
  }
  void* args[] = {&m, &w, &steps, &teacher_forced};
  const hipError_t e = hipLaunchCooperativeKernel(kernel, dim3(kNwg), dim3(kThreads), args, 0, stream);
  return e == hipSuccess ? DF_OK : DF_LAUNCH_FAILED;
}
