// Persistent whole-token decode for batch 1: one kernel launch runs every layer of a Qwen3 decode
// step -- per layer the fused QKV head (RMSNorm, QKV GEMV, QK-norm, RoPE, KV append), split-K
// decode attention and its merge, and the fused MLP (Wo, residual, RMSNorm, gate/up, SiLU*mul,
// down, residual) -- with the arithmetic of the standalone kernels (exact fp64 accumulation, the
// reference's bf16 / fp32 boundaries), so its results equal theirs.
//
// Reference: the per-token runlist of Qwen3NPU (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:
// 249-281), which the reference runs as one NPU dispatch (iron/common/sequence.py:270-559); the
// operators are QKVHeadDataParallelOurs (qkv_head_dp/op_ours.py:31-262), DecodeAttention
// (decode_attn/op.py:20-181) and SwiGLUMLPDataParallelOurs with fuse_o (swiglu_mlp_dp/
// op_ours.py:46-582). Goldens: qkv_head_dp/reference.py:13-33, decode_attn/reference.py:26-38,
// swiglu_mlp_dp/reference.py:8-67.
//
// Why one kernel: at batch 1 every operator is a short dependent chain (a 2-26 KiB weight slice
// per CU, then a reduction), so kernel boundaries and the activation round trip behind each launch
// dominate the token. Here the grid stays resident and hands activations from phase to phase
// through device memory, and each phase's weights (or K/V tile) are loaded before its input is
// awaited, so the weight stream overlaps the hand-off instead of following it.
//
// Grid: 256 workgroups of 256 threads, one per CU (the whole register file per wavefront). Each
// runs the six phases of every layer in order: QKV (A), attention (B), split merge (C), Wo (D),
// gate/up (E), down (F). A phase first issues its weight (or K/V) loads, then waits for its input
// words, so the weight stream overlaps the hand-off from the previous phase.
//
// Hand-off: every activation word is a 64-bit {tag, payload} pair written with one agent-scope
// atomic store and read with agent-scope atomic loads; a consumer waits until the tag of each
// word it needs equals the producing phase's tag (epoch, layer, phase). No counter, fence or
// cache flush is involved: a 64-bit atomic is seen whole or not at all. The epoch (control word
// 0 of the workspace) advances once per launch, so words of an earlier token never match.
// Every wait is bounded: a word that does not arrive within kSpinLimit polls sets control word 1
// and the workgroup stops; waiting workgroups also stop once they see that word set, so the grid
// drains within about one spin limit (the caller then reports the error).
//
// Buffer reuse: a hand-off buffer is rewritten by the same phase of the next layer (gh: four
// layers later). Its producers reach that phase only after they have consumed a later phase's
// words, which every workgroup produces only after it has read this buffer -- provided every
// workgroup that reads the buffer also produces in a phase that the producers wait on. For the
// Qwen3-0.6B shape every workgroup produces in every phase; in smaller shapes workgroups that own
// no rows of the Wo, gate/up or down phase read nothing in that phase (skip_gather).
#include <type_traits>

#include "attn_core.h"
#include "common.h"
#include "gemv_core.h"
#include "internal.h"

namespace {

using namespace iron::dev;

constexpr int kNT = 256;                     // workgroups (one per CU of an MI355X)
constexpr int kPhases = 7;                   // tag slots per layer: six phases + the input row
constexpr int kMaxLayers = 128;              // tag slots per launch: kPhases * kMaxLayers
constexpr long long kSpinLimit = 1ll << 18;  // polls of one word before a wait fails (~0.3 s)

constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// Attention tile: 16 * kRows tokens (4 wavefronts x 4 lane rows x kRows). Each split covers a
// contiguous ceil(ctx / NS) tokens, so up to 80 * NS tokens (2560 for the 0.6B shape) every split
// finishes in one tile.
constexpr int kRows = 5;
constexpr int kTileTokens = 16 * kRows;

// gh, the widest hand-off (every workgroup reads all FF fp32 values), travels in packed words: a
// 16-bit tag over a 48-bit payload, so one gate/up workgroup's 12 values fill 8 words, one
// 64-byte sector at the start of its block of kGhBlock words, and a consumer polls every word of
// the block in one round trip. (With a 32-bit tag per 32-bit value, a consumer polled one
// sentinel word and then read the block: two round trips, 4.7 us against 3.0 us in isolation.)
// Blocks 256 bytes apart spread the 256 polled sectors over more memory channels than 128 bytes
// apart (-2.7 us per token; 512 bytes measured the same as 256). Layers rotate over kGhBuffers
// buffers: one buffer for every layer measured 43 us per token slower than four (the polled
// sectors are then the ones the previous layer's producers wrote). A launch with fewer layers than
// buffers clears the blocks of the buffers it leaves unused, which the short tags rely on.
constexpr int kGhBuffers = 4;
// Every hand-off buffer that many workgroups poll (x, raw qkv, the attention output, a, gh) is
// written in kCopies copies kCopyWords words (32 KiB) apart, and the workgroups of XCD c (wg % 8)
// read copy c. One copy concentrates every workgroup's polls on the one or two memory channels
// that hold a few KiB; spread over copies, a poll's round trip is shorter (measured: 0.4 us per
// layer for the attention output alone, 53 us per token for all five). 4 or 16 copies, or copies
// 16 or 64 KiB apart, measured slower; copies not 256-byte aligned, much slower.
constexpr int kCopies = 8;
constexpr size_t kCopyWords = 4096;
constexpr int kGhBlock = 32;
// Word j of the x, a and attention-output hand-off buffers: 16 words (one 128-byte line) per
// 256 bytes, which spreads each copy's polled lines over twice the memory channels.
IRON_DEV constexpr size_t spread_word(int j) { return (size_t)(j >> 4) * 32 + (j & 15); }

constexpr int cmax(int a, int b) { return a > b ? a : b; }

template <int D_, int FF_, int HQ_, int HKV_>
struct Shape {
  static constexpr int D = D_, FF = FF_, HQ = HQ_, HKV = HKV_, HD = kAttnD;
  static constexpr int QD = HQ * HD, KVD = HKV * HD, MQKV = QD + 2 * KVD;
  static constexpr int WAVES = kNT * 4;             // wavefronts in the grid
  static constexpr int HB = HQ / HKV;               // query heads per KV head
  static constexpr int NS = kNT / HKV;              // attention splits per KV head
  static constexpr int MERGE_PER = HQ * HD / kNT;   // attention outputs merged per workgroup
  // rows per wavefront (R*) and 1024-wide chunks per row (C*) of each GEMV phase
  static constexpr int RA = cdiv(MQKV, WAVES), CA = cdiv(D, 1024);
  static constexpr int RD = cdiv(D, WAVES), CD = cdiv(QD, 1024);
  static constexpr int RE = cdiv(FF, WAVES), CE = cdiv(D, 1024);
  static constexpr int RF = cdiv(D, WAVES), CF = cdiv(FF, 1024);
  static constexpr int MERGE_WPS = 2 * MERGE_PER + 4;  // words per split: o[PER], m, l as fp64
  static constexpr size_t PART_WORDS = (size_t)HQ * NS * (HD + 2) * 2;  // all split partials
  // LDS words of the widest phase input
  static constexpr int LDS_WORDS =
      cmax(cmax(D, QD / 2), cmax(FF, cmax(NS * MERGE_WPS, (HB + 2) * 64)));
  static constexpr int RMAX = cmax(cmax(RA, RD), RF);
  static constexpr int GH_ROWS = 4 * RE;               // gh rows one workgroup produces
  static constexpr int GH_PROD = cdiv(FF, GH_ROWS);    // gate/up workgroups with rows
  static constexpr int GH_WORDS = GH_PROD * kGhBlock;  // one gh buffer, blocked per producer
  static constexpr int GH_PACKED = cdiv(2 * GH_ROWS, 3);  // 48-bit words of one producer's block
  static constexpr int XW = 2 * RF;  // words of x (and of a) one down (Wo) workgroup writes
  // Whether every workgroup owns rows of the Wo / down phases (RD == RF) and of gate/up. Where
  // they do, the skip branch is compiled out: its second call site of the phase's `issue` hook
  // measured 31 us per token slower for the Qwen3-0.6B shape although it never runs.
  static constexpr bool WO_ALL = (kNT - 1) * 4 * RD < D;
  static constexpr bool GU_ALL = (kNT - 1) * 4 * RE < FF;
  // words between the replicated copies of the kGhBuffers gh buffers (a multiple of kCopyWords)
  static constexpr size_t GH_COPY =
      (((size_t)kGhBuffers * GH_WORDS + kCopyWords - 1) / kCopyWords) * kCopyWords;
  // One KV head per XCD: the 32 workgroups of XCD x (wg % 8 == x) compute KV head x's QKV rows
  // (its two query heads, its key and value: 512 rows, 16 per workgroup), run its 32 attention
  // splits and merge its two query heads' outputs, so the raw q/k/v and the split partials
  // travel through that XCD's L2 (xcd_local_*), never through the fabric.
  static constexpr bool TRACE = false;  // phase timestamps (Traced<>)
  static constexpr bool XCD_LOCAL = HKV == kCopies && NS * HKV == kNT &&
                                    (HB + 2) * HD == 4 * RA * NS && RA == 4 &&
                                    MERGE_PER * NS == HB * HD;

  static_assert(HQ % HKV == 0 && HB == 2, "the attention phase handles GQA pairs");
  static_assert(kNT % HKV == 0 && NS <= 256, "splits per KV head");
  static_assert(kNT * MERGE_PER == HQ * HD && MERGE_PER >= 2 && MERGE_PER % 2 == 0 &&
                    HD % MERGE_PER == 0, "merge slices");
  static_assert(NS * MERGE_PER == 256 && (NS == 32 || NS == 64 || NS == 128),
                "one merge thread per (split, dim)");
  static_assert(D % 16 == 0 && FF % 16 == 0 && MQKV % 2 == 0, "GEMV widths");
  static_assert(GH_PACKED <= kGhBlock && GH_PROD <= kNT, "gh blocks");
  static_assert(RD == RF, "the Wo and down phases own the same rows");
  static_assert(spread_word(D / 2 - 1) < kCopyWords && spread_word(QD / 2 - 1) < kCopyWords,
                "spread x, a and attention-output words in one copy");
  static_assert(D / 2 <= (int)kCopyWords && MQKV / 2 <= (int)kCopyWords &&
                    QD / 2 <= (int)kCopyWords, "hand-off copies");
};

using ShapeQwen3_0_6B = Shape<1024, 3072, 16, 8>;
using ShapeTiny = Shape<256, 768, 4, 2>;

// A shape whose kernel also records phase timestamps (iron_decode_persistent_set_trace).
template <class S>
struct Traced : S {
  static constexpr bool TRACE = true;
};

struct WireGeom {
  int gshift, tile_m;
  FastDiv tdiv;
  uint32_t blk_bytes, xor_mask;
};

struct PParams {
  const iron_layer_desc* layers;
  int n_layers, max_seq;
  WireGeom g_qkv, g_o, g_gu, g_d;
  const uint16_t* x_in;   // bf16 [D]: the current token's embedding row
  uint16_t* x_out;        // bf16 [D]: the last layer's output
  const int32_t* pos;     // device int32: the current position
  const uint16_t* ang;    // bf16 [HD]: the position's interleaved (cos, sin) row
  long long kv_sh, kv_st;
  float eps;
  double scale;
  unsigned long long *X, *RAW, *PART, *ATT, *AO, *GH;  // tagged hand-off buffers
  uint32_t* ctrl;         // [0] epoch, [1] error flags
  // device-resident greedy loop (iron_decode_persistent_gen); key is null otherwise
  unsigned long long* key;     // argmax key of the previous token: read first, reset last
  const uint16_t* emb;         // bf16 [vocab][D] embedding table
  int vocab, log_len;
  int32_t *token, *token_log, *step, *pos_next, *ctx;
  const uint16_t* rope_table;  // bf16 [max_seq][HD] RoPE rows
  uint16_t* ang_next;          // the buffer `ang` points to, given the next position's row
  // the final RMSNorm + bf16 LM head + argmax folded into the launch (lm_w null: not folded).
  // The argmax keys then alternate between two slots by epoch: launch e reads the previous
  // token from key[e & 1] and accumulates its own argmax into key[(e + 1) & 1], which workgroup 0
  // clears at the start of the launch.
  const uint16_t* lm_w;        // bf16 [vocab][D]
  const uint16_t* lm_norm;     // bf16 [D]
  uint16_t* logits;            // bf16 [vocab], or null
  // Traced<> kernels: kStampMarks realtime-clock stamps per (layer, workgroup)
  unsigned long long* stamps;
};

// Phase stamps of a traced launch: stamps[(layer * kNT + wg) * kStampMarks + mark], the 100 MHz
// constant clock (s_memrealtime) read by thread 0 of the workgroup at: 0 QKV phase entry, 1 its
// input gathered, 2 its rows stored; 3 attention input gathered, 4 QK-norm/RoPE done, 15 tiles
// done, 5 partials stored; 6 merge input gathered, 7 outputs stored; 8 Wo input gathered, 9 rows
// stored; 10 gate/up input gathered, 11 prologue done, 12 gh stored; 13 down input gathered,
// 14 rows stored.
constexpr int kStampMarks = 16;

template <class S>
IRON_DEV void stamp(const PParams& p, int wg, int l, int mark) {
  if constexpr (S::TRACE)
    if (threadIdx.x == 0)
      p.stamps[((size_t)l * kNT + wg) * kStampMarks + mark] = __builtin_amdgcn_s_memrealtime();
}

IRON_DEV GemvParams gemv_of(const WireGeom& g, const void* w, int M, int K) {
  GemvParams p = {};
  p.w = (const uint8_t*)w;
  p.M = M;
  p.K = K;
  p.gshift = g.gshift;
  p.tile_m = g.tile_m;
  p.tdiv = g.tdiv;
  p.blk_bytes = g.blk_bytes;
  p.xor_mask = g.xor_mask;
  return p;
}

// ---------------------------------------------------------------------------------------------
// Tagged words
// ---------------------------------------------------------------------------------------------
// A launch's tags take the fixed range [epoch * kPhases * kMaxLayers, +kPhases * kMaxLayers), so
// launches with different layer counts on one workspace never expect a tag an earlier launch left
// in a word (a stride of kPhases * n_layers would let epoch e with n layers overlap epoch e - 1
// with more layers).
IRON_DEV uint32_t phase_tag(uint32_t epoch, int n_layers, int layer, int phase) {
  (void)n_layers;
  const unsigned long long v = (unsigned long long)epoch * (unsigned long long)(kPhases * kMaxLayers) +
                               (unsigned long long)(kPhases * layer + phase);
  return (uint32_t)(v % 0xffffffffull) + 1u;  // never 0, the value of a cleared word
}

// The tag x carries into layer l: the previous layer's down phase, or for layer 0 the embedding
// row the grid publishes at its start (slot 6 of layer 0, used by nothing else).
IRON_DEV uint32_t x_tag(uint32_t epoch, int n_layers, int layer) {
  return layer == 0 ? phase_tag(epoch, n_layers, 0, 6) : phase_tag(epoch, n_layers, layer - 1, 5);
}

IRON_DEV void put_word(unsigned long long* dst, uint32_t payload, uint32_t tag) {
  __hip_atomic_store(dst, ((unsigned long long)tag << 32) | payload, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// A word of a replicated hand-off buffer: the same word in every copy, `stride` words apart.
IRON_DEV void put_word_copies(unsigned long long* dst, size_t stride, uint32_t payload,
                              uint32_t tag) {
#pragma unroll
  for (int c = 0; c < kCopies; ++c) put_word(dst + c * stride, payload, tag);
}

// The copy of a replicated buffer that workgroup wg reads.
IRON_DEV unsigned long long* copy_for(unsigned long long* base, size_t stride, int wg) {
  return base + (size_t)(wg % kCopies) * stride;
}

IRON_DEV double word_double(uint32_t lo, uint32_t hi) {
  return __hiloint2double((int)hi, (int)lo);
}

// XCD-local hand-off (the raw q/k/v rows and the attention split partials of shapes with
// Shape::XCD_LOCAL): producer and consumers are workgroups of one XCD, which share its L2. The
// producer's store carries sc0 (written through the CU's L1 into the L2); a consumer polls with nt
// loads (gather_pairs_local), whose L1 policy is hit-evict, so a line its L1 held from an earlier
// read is dropped after one read and the next poll is served by the L2. A 64-bit word is written and read whole, as
// with the device-scope words. Both need the workgroups of one hand-off on one XCD, which the
// kernel's mapping gives when workgroups with equal wg % 8 share an XCD (checked every launch).
// Measured alone (32 workgroups per XCD, 2000 phases): 0.70 against 0.80 us per phase for 256
// words, 1.15 against 1.44 us for 640, with device-scope words; sc0 polls returned stale words.
constexpr int kCpolSc0 = 1;

IRON_DEV __amdgpu_buffer_rsrc_t xcd_local_rsrc(unsigned long long* base, size_t words) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)(words * 8), kBufferDword3);
}

IRON_DEV void put_word_local(__amdgpu_buffer_rsrc_t rs, size_t word, uint32_t payload,
                             uint32_t tag) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = {payload, tag};  // the low dword is the payload, the high one the tag
  __builtin_amdgcn_raw_buffer_store_b64(v, rs, (int)(word * 8), 0, kCpolSc0);
}

// Words `word` and `word` + 1 (16-byte aligned) in one 16-byte store: {p0, tag, p1, tag}. Each
// 64-bit word is written whole, as put_word_local writes it.
IRON_DEV void put_pair_local(__amdgpu_buffer_rsrc_t rs, size_t word, uint32_t p0, uint32_t p1,
                             uint32_t tag) {
  const iron_u32x4 v = {p0, tag, p1, tag};
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, (int)(word * 8), 0, kCpolSc0);
}

// The hardware XCC id of the executing workgroup (HW_REG_XCC_ID, bits 3:0).
IRON_DEV uint32_t xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xfu; }

// Packed words (gh): tag in bits 48..63, payload in bits 0..47. The 16-bit tag is the full tag
// reduced to 1..65535 (never 0, the value of a cleared word). Every launch rewrites or clears every
// gh block, so a stale word is at most one completed launch old (plus launches that failed before
// their layer), i.e. a few multiples of kPhases * kMaxLayers full tags behind, never 65535.
IRON_DEV uint32_t short_tag(uint32_t tag) { return tag % 0xffffu + 1u; }

IRON_DEV void put_packed_copies(unsigned long long* dst, size_t stride, unsigned long long payload,
                                uint32_t stag) {
  const unsigned long long w = ((unsigned long long)stag << 48) | (payload & 0xffffffffffffull);
#pragma unroll
  for (int c = 0; c < kCopies; ++c)
    __hip_atomic_store(dst + c * stride, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Word i (bits [48 i, 48 i + 48)) of the little-endian concatenation of n 32-bit values.
IRON_DEV unsigned long long pack48(const uint32_t* v, int n, int i) {
  const int v0 = (3 * i) >> 1;
  const unsigned long long a = v0 < n ? v[v0] : 0u, b = v0 + 1 < n ? v[v0 + 1] : 0u;
  return (i & 1) ? ((a >> 16) | (b << 16)) : (a | ((b & 0xffffull) << 32));
}

// Waits for n tagged words and puts their payloads in LDS. Thread t owns slots j = t + 256 k < n;
// src(j, tag) names slot j's word and the tag it must carry; the payload goes to dst[j]. A thread
// re-reads its pending words together each round.
//
// `issue` runs once in every thread when the wait is over (also when it failed): the caller
// issues the weight loads of a later phase there, and they stream during this phase's compute
// and the next phase's wait. Issued earlier, they would sit ahead of the later poll loads, which
// complete in issue order behind them.
//
// Returns false (workgroup-uniform) if a word did not arrive within kSpinLimit rounds (or another
// workgroup has already failed), after raising the error flag. Starts and ends with a workgroup
// barrier.
IRON_DEV void retire_loads() {
  // Every load issued so far (this phase's weights, issued a phase or two ago) completes here,
  // before the poll and the `issue` loads: the compiler then knows those registers are ready and
  // places no wait on them in this phase's compute, which would otherwise also wait for the
  // younger `issue` loads (vector loads complete in order).
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

// True in every thread if `flag` is set in any thread of the workgroup: one barrier (where
// __syncthreads_or takes three). The flags are rewritten only after the next wait's opening
// barrier, which every wavefront reaches after reading these.
IRON_DEV bool workgroup_any(bool flag) {
  __shared__ uint32_t s_flag[4];
  const bool w = __ballot(flag) != 0ull;
  if ((threadIdx.x & 63) == 0) s_flag[threadIdx.x >> 6] = w ? 1u : 0u;
  __syncthreads();
  return (s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3]) != 0u;
}

// A wait's first poll is issued ~0.27 us after the phase starts (s_sleep counts 64 clocks). Its
// producers are other workgroups finishing the same previous phase, so an immediate poll almost
// never finds the words; it only adds to the poll traffic that lengthens every hand-off's round
// trip. Measured per step: sleep 4 / 6 / 8 / 10 / 12 / 16 / 32 units -> -6 / -10 / -18 / -21 /
// -18 / -5 / +47 us against no sleep.
constexpr int kFirstPollDelay = 10;
// The XCD-local waits (raw q/k/v, split partials) poll first after 4 units: their round trip is
// shorter (measured per step against 10 units: 4 / 2: -5 / -4 us; 16: +5 us).
constexpr int kLocalFirstPollDelay = 4;
// The QKV phase's x wait and the down phase's gh wait, retuned after the XCD-local mapping (per
// token against 10 and 18 units: 4 and 12 -5 us; 6 and 14 -4.5 us; 6 and 10 -1 us; QKV 14 +3 us,
// down 22 +3 us; the Wo and gate/up waits at 6 or 14 units measured no better than 10).
constexpr int kQkvFirstPollDelay = 4, kDownFirstPollDelay = 12;
template <int UNITS>
IRON_DEV void first_poll_delay() { __builtin_amdgcn_s_sleep(UNITS); }

IRON_DEV bool gave_up(long long spins, uint32_t* err) {
  return spins >= kSpinLimit ||
         ((spins & 255) == 255 &&
          __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u);
}

IRON_DEV unsigned long long poll_word(unsigned long long* w) {
  return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class Issue>
IRON_DEV void issue_fenced(Issue issue) {
  __builtin_amdgcn_sched_barrier(0);
  issue();
  __builtin_amdgcn_sched_barrier(0);
}

// A workgroup that owns no rows of a phase reads none of its input: it only keeps the phase
// structure (the opening barrier and the retired loads of gather_words) and issues the later
// phase's loads. Not reading words it does not need also keeps it from waiting on a word whose
// buffer a faster workgroup may already have rewritten for the next layer.
template <class Issue>
IRON_DEV bool skip_gather(Issue issue) {
  __syncthreads();
  retire_loads();
  issue_fenced(issue);
  return true;
}

template <int NPT, int DELAY = kFirstPollDelay, class Src, class Issue>
IRON_DEV bool gather_words(int n, Src src, Issue issue, uint32_t* dst, uint32_t* err) {
  __syncthreads();  // the previous phase's LDS reads are done before dst is rewritten
  retire_loads();
  first_poll_delay<DELAY>();
  bool pending[NPT];
  unsigned long long* ptr[NPT];
  uint32_t want[NPT];
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int j = threadIdx.x + 256 * k;
    pending[k] = j < n;
    ptr[k] = pending[k] ? src(j, want[k]) : nullptr;
  }
  bool missing = false;
  for (long long spins = 0;; ++spins) {
    unsigned long long w[NPT];
#pragma unroll
    for (int k = 0; k < NPT; ++k)
      if (pending[k]) w[k] = poll_word(ptr[k]);
    missing = false;
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
      if (!pending[k]) continue;
      if ((uint32_t)(w[k] >> 32) == want[k]) {
        dst[threadIdx.x + 256 * k] = (uint32_t)w[k];
        pending[k] = false;
      } else {
        missing = true;
      }
    }
    if (!missing || gave_up(spins, err)) break;
  }
  if (missing) atomicOr(err, 1u);
  const bool ok = !workgroup_any(missing);
  issue_fenced(issue);
  return ok;
}

// gather_words for XCD-local words (put_word_local), taken two at a time: thread t polls the word
// pairs (2p, 2p + 1), p = t + 256 k, with one 16-byte nt load (src(2p) is 16-byte aligned and
// src(2p + 1) follows it), and checks each word of a pair against its own tag. nt loads are
// plain loads to the compiler (a volatile one would be issued past every cache), so a compiler
// memory barrier before each round keeps them in the loop. Polling pairs instead of single words
// measured -2.5 us per token.
template <int NPP, int DELAY, class Src, class Issue>
IRON_DEV bool gather_pairs_local(int n, Src src, Issue issue, uint32_t* dst, uint32_t* err) {
  __syncthreads();  // the previous phase's LDS reads are done before dst is rewritten
  retire_loads();
  first_poll_delay<DELAY>();
  bool pending[NPP];
  unsigned long long* ptr[NPP];
  uint32_t want0[NPP], want1[NPP];
#pragma unroll
  for (int k = 0; k < NPP; ++k) {
    const int j = 2 * ((int)threadIdx.x + 256 * k);
    pending[k] = j < n;
    ptr[k] = pending[k] ? src(j, want0[k]) : nullptr;
    if (pending[k]) (void)src(j + 1, want1[k]);
  }
  bool missing = false;
  for (long long spins = 0;; ++spins) {
    iron_u32x4 w[NPP];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < NPP; ++k)
      if (pending[k])
        w[k] = __builtin_nontemporal_load(
            (const __attribute__((address_space(1))) iron_u32x4*)ptr[k]);
    missing = false;
#pragma unroll
    for (int k = 0; k < NPP; ++k) {
      if (!pending[k]) continue;
      if (w[k].y == want0[k] && w[k].w == want1[k]) {  // {payload, tag} of words 2p and 2p + 1
        *(uint2*)&dst[2 * ((int)threadIdx.x + 256 * k)] = make_uint2(w[k].x, w[k].z);
        pending[k] = false;
      } else {
        missing = true;
      }
    }
    if (!missing || gave_up(spins, err)) break;
  }
  if (missing) atomicOr(err, 1u);
  const bool ok = !workgroup_any(missing);
  issue_fenced(issue);
  return ok;
}

// gather_words for device-scope words taken two at a time: 16-byte sc1 buffer loads of the word
// pairs (2p, 2p + 1) of the region at `base` (src(2p) 16-byte aligned, src(2p + 1) next to it),
// each word checked against its own tag (a pair is read in one transaction and each 64-bit word
// was stored whole). Half the poll instructions of gather_words: -19 us per token for the x,
// attention-output and a waits (the packed gh words measured +2 us this way, so gather_gh keeps
// single words). A compiler memory barrier before each round keeps the loads in the loop.
template <int NPP, int DELAY = kFirstPollDelay, class Src, class Issue>
IRON_DEV bool gather_pairs_dev(int n, unsigned long long* base, Src src, Issue issue,
                               uint32_t* dst, uint32_t* err) {
  __syncthreads();  // the previous phase's LDS reads are done before dst is rewritten
  retire_loads();
  first_poll_delay<DELAY>();
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)(kCopyWords * 8), kBufferDword3);
  bool pending[NPP];
  int off[NPP];
  uint32_t want0[NPP], want1[NPP];
#pragma unroll
  for (int k = 0; k < NPP; ++k) {
    const int j = 2 * ((int)threadIdx.x + 256 * k);
    pending[k] = j < n;
    off[k] = 0;
    if (pending[k]) {
      off[k] = (int)((src(j, want0[k]) - base) * 8);
      (void)src(j + 1, want1[k]);
    }
  }
  bool missing = false;
  for (long long spins = 0;; ++spins) {
    iron_u32x4 w[NPP];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < NPP; ++k)
      if (pending[k])
        w[k] = __builtin_bit_cast(iron_u32x4,
                                  __builtin_amdgcn_raw_buffer_load_b128(rs, off[k], 0, kCpolSc1));
    missing = false;
#pragma unroll
    for (int k = 0; k < NPP; ++k) {
      if (!pending[k]) continue;
      if (w[k].y == want0[k] && w[k].w == want1[k]) {  // {payload, tag} of words 2p and 2p + 1
        *(uint2*)&dst[2 * ((int)threadIdx.x + 256 * k)] = make_uint2(w[k].x, w[k].z);
        pending[k] = false;
      } else {
        missing = true;
      }
    }
    if (!missing || gave_up(spins, err)) break;
  }
  if (missing) atomicOr(err, 1u);
  const bool ok = !workgroup_any(missing);
  issue_fenced(issue);
  return ok;
}

// Waits for the gh blocks of n_blk producers and puts their values in LDS. Producer q's ROWS
// 32-bit values travel as the first W = ceil(2 ROWS / 3) packed words (put_packed_copies) of the
// block at blk + q kGhBlock, word i holding bits [48 i, 48 i + 48) of their little-endian
// concatenation; they land as dst32[ROWS q + r]. Every pending word is polled each round (8 per
// thread for the Qwen3-0.6B shape: 2048 words, 64 contiguous bytes per producer). Same contract
// as gather_words otherwise, with one short tag for all words.
template <int ROWS, int NPT, int DELAY = kFirstPollDelay, class Issue>
IRON_DEV bool gather_gh(int n_blk, unsigned long long* blk, uint32_t stag, Issue issue,
                        uint32_t* dst32, uint32_t* err) {
  constexpr int W = cdiv(2 * ROWS, 3);
  __syncthreads();
  retire_loads();
  first_poll_delay<DELAY>();
  uint16_t* const dst = (uint16_t*)dst32;
  const int n = n_blk * W;
  bool pending[NPT];
  unsigned long long* ptr[NPT];
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int j = threadIdx.x + 256 * k;
    pending[k] = j < n;
    ptr[k] = pending[k] ? blk + (j / W) * kGhBlock + j % W : nullptr;
  }
  bool missing = false;
  for (long long spins = 0;; ++spins) {
    unsigned long long w[NPT];
#pragma unroll
    for (int k = 0; k < NPT; ++k)
      if (pending[k]) w[k] = poll_word(ptr[k]);
    missing = false;
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
      if (!pending[k]) continue;
      if ((uint32_t)(w[k] >> 48) == stag) {
        // 16-bit half c of word i is half 3 i + c of the block (2 ROWS halves; the last word of a
        // block may carry fewer than three)
        const int j = threadIdx.x + 256 * k, q = j / W, i = j % W;
        uint16_t* d = dst + q * 2 * ROWS + 3 * i;
#pragma unroll
        for (int c = 0; c < 3; ++c)
          if (3 * W == 2 * ROWS || 3 * i + c < 2 * ROWS) d[c] = (uint16_t)(w[k] >> (16 * c));
        pending[k] = false;
      } else {
        missing = true;
      }
    }
    if (!missing || gave_up(spins, err)) break;
  }
  if (missing) atomicOr(err, 1u);
  const bool ok = !workgroup_any(missing);
  issue_fenced(issue);
  return ok;
}

// This lane's activation slices from LDS, in the layout load_x_lane produces from global memory:
// bf16 elements [c*1024 + 16 lane, +16) as two uint4, or fp32 ones as four.
template <int NCH>
IRON_DEV void lane_bf16(const uint32_t* s, int K, int lane, uint4 (&xl)[NCH][4]) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 1024 + lane * 16;
#pragma unroll
    for (int u = 0; u < 4; ++u) xl[c][u] = make_uint4(0u, 0u, 0u, 0u);
    if (e < K) {
      xl[c][0] = ((const uint4*)s)[e / 8];
      xl[c][1] = ((const uint4*)s)[e / 8 + 1];
    }
  }
}

template <int NCH>
IRON_DEV void lane_f32(const uint32_t* s, int K, int lane, uint4 (&xl)[NCH][4]) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 1024 + lane * 16;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      xl[c][u] = e < K ? ((const uint4*)s)[e / 4 + u] : make_uint4(0u, 0u, 0u, 0u);
  }
}

// A norm weight's slices for this lane (bf16 [K], elements [c*1024 + 16 lane, +16)).
template <int NCH>
IRON_DEV void lane_weight(const uint16_t* w, int K, int lane, uint4 (&nw)[NCH][2]) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 1024 + lane * 16;
    const int ec = e < K ? e : 0;
    nw[c][0] = ld_global((const uint4*)(w + ec));
    nw[c][1] = ld_global((const uint4*)(w + ec + 8));
  }
}

// bf16 outputs of R rows per wavefront: the workgroup's 4R consecutive rows go out as tagged
// pairs (rows 4R wg + 2t, +1), at word spread_word(row / 2) when SPREAD. `plain` (optional):
// also written as plain bf16 pairs.
template <int R, bool SPREAD = false>
IRON_DEV void store_bf16_pairs(const uint16_t (&h)[R], int wg, int M, unsigned long long* dst,
                               uint32_t tag, uint16_t* s_out, uint16_t* plain) {
  // dst: copy 0 of a replicated buffer (put_word_copies)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (R % 2 == 0) {
    // a wavefront's rows pair up within it: lane k < R/2 stores rows 2k, 2k+1 (every lane holds
    // every row's value)
    const int row0 = (wg * 4 + wave) * R;
    uint32_t pair = 0u;
#pragma unroll
    for (int k = 0; k < R / 2; ++k)
      if (lane == k) pair = (uint32_t)h[2 * k] | ((uint32_t)h[2 * k + 1] << 16);
    const int row = row0 + 2 * lane;
    if (lane < R / 2 && row < M) {
      put_word_copies(dst + (SPREAD ? spread_word(row / 2) : (size_t)(row / 2)), kCopyWords,
                      pair, tag);
      if (plain) ((uint32_t*)plain)[row / 2] = pair;
    }
    return;
  }
  if (lane < R) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lane == r) s_out[wave * R + r] = h[r];
  }
  __syncthreads();
  // thread c (2R) + t stores word t of copy c: one store instruction for all copies (-1 us per
  // token against eight stores from each of 2R threads)
  const int t = threadIdx.x % (2 * R), c = threadIdx.x / (2 * R);
  if (c < kCopies) {
    const int row = wg * 4 * R + 2 * t;
    if (row < M) {
      const uint32_t pair = (uint32_t)s_out[2 * t] | ((uint32_t)s_out[2 * t + 1] << 16);
      put_word(dst + (size_t)c * kCopyWords +
                   (SPREAD ? spread_word(row / 2) : (size_t)(row / 2)), pair, tag);
      if (plain && c == 0) ((uint32_t*)plain)[row / 2] = pair;
    }
  }
}

// The 2R words store_bf16_pairs (odd R) just published for this workgroup, kept in LDS for a later
// phase of the same workgroup: word t = rows 2t, 2t+1 of its 4R rows. It reads s_out after the
// store's barrier, so it needs no barrier of its own.
template <int R>
IRON_DEV void keep_own_words(const uint16_t* s_out, uint32_t* own) {
  static_assert(R % 2 == 1, "the odd-R store stages its rows in s_out");
  const int t = threadIdx.x;
  if (t < 2 * R) own[t] = (uint32_t)s_out[2 * t] | ((uint32_t)s_out[2 * t + 1] << 16);
}

// Max / sum over the G consecutive threads of a group (G = 32 or 64 within a wavefront, G = 128
// over two wavefronts through LDS); every thread of the group receives the result. All 256 threads
// call it together. Sums add in a fixed tree order.
// Lane n's value, in every lane.
// x and y exchange lanes: v_permlane32_swap (ROWS32) swaps x's lanes 32..63 with y's lanes 0..31,
// v_permlane16_swap swaps x's 16-lane rows 1 and 3 with y's rows 0 and 2; each half of a double
// moves with one instruction.
template <bool ROWS32>
IRON_DEV void swap_lanes_d(double& x, double& y) {
  const uint32_t xl = (uint32_t)__double2loint(x), xh = (uint32_t)__double2hiint(x);
  const uint32_t yl = (uint32_t)__double2loint(y), yh = (uint32_t)__double2hiint(y);
  if constexpr (ROWS32) {
    const auto lo = __builtin_amdgcn_permlane32_swap(xl, yl, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(xh, yh, false, false);
    x = __hiloint2double((int)hi[0], (int)lo[0]);
    y = __hiloint2double((int)hi[1], (int)lo[1]);
  } else {
    const auto lo = __builtin_amdgcn_permlane16_swap(xl, yl, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap(xh, yh, false, false);
    x = __hiloint2double((int)hi[0], (int)lo[0]);
    y = __hiloint2double((int)hi[1], (int)lo[1]);
  }
}


// Maximum / sum over groups of G consecutive lanes, in every lane of the group. G = 32: the four
// 16-lane DPP steps, then the two rows of each half-wavefront meet through v_permlane16_swap --
// the same pairings as an xor butterfly (lane l with l ^ 1, 2, 4, 8, 16), so the same values,
// without an LDS round trip (readlanes of rows 0, 16, 32 and 48 measured 1.4 us per token
// slower, with the tile maximum's). Other G: xor shuffles, and for G > 64 the wavefronts through
// LDS.
template <int G>
IRON_DEV double group_max(double v, double (&s_red)[4][2]) {
  if constexpr (G == 32) {
    v = row16_max_d(v);
    double w = v;
    swap_lanes_d<false>(v, w);  // rows 0 | 1 and 2 | 3 meet
    return fmax(v, w);
  }
#pragma unroll
  for (int k = 1; k < (G < 64 ? G : 64); k <<= 1) v = fmax(v, __shfl_xor(v, k));
  if constexpr (G > 64) {
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_red[wave][0] = v;
    __syncthreads();
    v = fmax(s_red[wave & ~1][0], s_red[wave | 1][0]);
  }
  return v;
}

template <int G>
IRON_DEV double group_sum(double v, double (&s_red)[4][2]) {
  if constexpr (G == 32) {
    v = row16_sum_d(v);
    double w = v;
    swap_lanes_d<false>(v, w);
    return v + w;
  }
#pragma unroll
  for (int k = 1; k < (G < 64 ? G : 64); k <<= 1) v += __shfl_xor(v, k);
  if constexpr (G > 64) {
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_red[wave][1] = v;
    __syncthreads();
    v = s_red[wave & ~1][1] + s_red[wave | 1][1];
  }
  return v;
}

// ---------------------------------------------------------------------------------------------
// Register-resident prefetches: the weight slices (or first K/V tile) a phase multiplies, loaded
// one or two phases before the phase runs.
// ---------------------------------------------------------------------------------------------
template <int R, int NCH>
struct W8 {
  uint4 w[R][NCH];
  uint32_t sc[R][NCH];
};

template <class S>
IRON_DEV int row0_of(int wg, int R) {
  return (wg * 4 + (int)(threadIdx.x >> 6)) * R;
}

// The QKV phase's block of 4 RA consecutive rows that workgroup wg computes. With XCD_LOCAL,
// XCD x = wg % 8 computes KV head x's rows: i = wg / 8 < 16 the rows of query heads 2x, 2x + 1,
// then 8 blocks of key head x and 8 of value head x; otherwise block wg.
template <class S>
IRON_DEV int qkv_block(int wg) {
  if constexpr (S::XCD_LOCAL) {
    constexpr int BR = 4 * S::RA, QB = S::HB * S::HD / BR, KB = S::HD / BR;
    const int x = wg % S::HKV, i = wg / S::HKV;
    return i < QB ? x * QB + i
                  : (i < QB + KB ? (S::QD + x * S::HD) / BR + (i - QB)
                                 : (S::QD + S::KVD + x * S::HD) / BR + (i - QB - KB));
  } else {
    return wg;
  }
}

// The attention phase's KV head and split of workgroup wg (XCD_LOCAL: head wg % 8, so a head's
// splits share the XCD that computed its raw rows).
template <class S>
IRON_DEV int attn_head(int wg) {
  return S::XCD_LOCAL ? wg % S::HKV : wg / S::NS;
}
template <class S>
IRON_DEV int attn_split(int wg) {
  return S::XCD_LOCAL ? wg / S::HKV : wg % S::NS;
}

// The first of the MERGE_PER attention outputs (query head h, dim d at h * HD + d) that
// workgroup wg merges (XCD_LOCAL: outputs of KV head wg % 8's query heads, on that XCD).
template <class S>
IRON_DEV int merge_o0(int wg) {
  return S::XCD_LOCAL ? (wg % S::HKV) * S::HB * S::HD + (wg / S::HKV) * S::MERGE_PER
                      : wg * S::MERGE_PER;
}

template <class S>
IRON_DEV void prefetch_qkv(const PParams& p, const iron_layer_desc& L, int wg,
                           W8<S::RA, S::CA>& W, uint4 (&nw)[S::CA][2]) {
  const GemvParams g = gemv_of(p.g_qkv, L.wqkv, S::MQKV, S::D);
  fetch_w8<S::RA, S::CA>(g, g.w, row0_of<S>(qkv_block<S>(wg), S::RA), threadIdx.x & 63, W.w,
                         W.sc);
  lane_weight<S::CA>(L.n_in, S::D, threadIdx.x & 63, nw);
}

// The first K/V tile of this workgroup's split and the QKV epilogue's constants.
// nq / nk: the q / k norm weights of dims lane and lane + 64 (bf16 pair, low half first); cs: the
// (cos, sin) bf16 pair of rotary index lane.
struct KVPrefetch {
  uint4 kr[kRows], vr[kRows];
  uint32_t nq, nk, cs;
};

// Rows t0 + 16u + 4 wave + lane/16 of a tile; rows at or past `bound` repeat row bound - 1 (and
// row 0 when bound is 0: the cache always has it), so every load is issued unconditionally.
IRON_DEV void load_kv_rows(const PParams& p, const iron_layer_desc& L, int kv, int t0, int bound,
                           uint4 (&kr)[kRows], uint4 (&vr)[kRows]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, row = lane >> 4, dl = lane & 15;
  const size_t base = (size_t)kv * p.kv_sh + dl * 8;
  const int last = bound > 0 ? bound - 1 : 0;
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    int t = t0 + u * 16 + wave * 4 + row;
    t = t <= last ? t : last;  // rows past the split are masked where they are used
    kr[u] = ld_global((const uint4*)(L.k_cache + base + (size_t)t * p.kv_st));
    vr[u] = ld_global((const uint4*)(L.v_cache + base + (size_t)t * p.kv_st));
  }
}

IRON_DEV int context_of(const PParams& p, int pos) {
  const int ctx = pos + 1;
  return ctx < 0 ? 0 : (ctx > p.max_seq ? p.max_seq : ctx);
}

// Split s of NS covers positions [s * chunk, min(ctx, (s + 1) * chunk)).
struct SplitRange {
  int begin, end;
};

template <class S>
IRON_DEV SplitRange split_range(int ctx, int split) {
  const int chunk = (ctx + S::NS - 1) / S::NS;
  const int b = split * chunk;
  const int e = b + chunk < ctx ? b + chunk : ctx;
  return {b < ctx ? b : ctx, e};
}

template <class S>
IRON_DEV void prefetch_attn(const PParams& p, const iron_layer_desc& L, int wg, int pos,
                            KVPrefetch& kv) {
  const int head = attn_head<S>(wg), split = attn_split<S>(wg), lane = threadIdx.x & 63;
  const SplitRange r = split_range<S>(context_of(p, pos), split);
  load_kv_rows(p, L, head, r.begin, r.end, kv.kr, kv.vr);
  kv.nq = (uint32_t)ld_global(L.n_qn + lane) | ((uint32_t)ld_global(L.n_qn + lane + 64) << 16);
  kv.nk = (uint32_t)ld_global(L.n_kn + lane) | ((uint32_t)ld_global(L.n_kn + lane + 64) << 16);
  kv.cs = ld_global((const uint32_t*)p.ang + lane);
}

template <class S>
IRON_DEV void prefetch_wo(const PParams& p, const iron_layer_desc& L, int wg, W8<S::RD, S::CD>& W) {
  const GemvParams g = gemv_of(p.g_o, L.wo, S::D, S::QD);
  fetch_w8<S::RD, S::CD>(g, g.w, row0_of<S>(wg, S::RD), threadIdx.x & 63, W.w, W.sc);
}

template <class S>
IRON_DEV void prefetch_gateup(const PParams& p, const iron_layer_desc& L, int wg,
                              W8<S::RE, S::CE>& Wg, W8<S::RE, S::CE>& Wu,
                              uint4 (&nw)[S::CE][2]) {
  const GemvParams g = gemv_of(p.g_gu, L.wg, S::FF, S::D);
  const int row0 = row0_of<S>(wg, S::RE), lane = threadIdx.x & 63;
  fetch_w8<S::RE, S::CE>(g, (const uint8_t*)L.wg, row0, lane, Wg.w, Wg.sc);
  fetch_w8<S::RE, S::CE>(g, (const uint8_t*)L.wu, row0, lane, Wu.w, Wu.sc);
  lane_weight<S::CE>(L.n_post, S::D, lane, nw);
}

template <class S>
IRON_DEV void prefetch_down(const PParams& p, const iron_layer_desc& L, int wg,
                            W8<S::RF, S::CF>& W) {
  const GemvParams g = gemv_of(p.g_d, L.wd, S::D, S::FF);
  fetch_w8<S::RF, S::CF>(g, g.w, row0_of<S>(wg, S::RF), threadIdx.x & 63, W.w, W.sc);
}

// Wavefront totals of R rows of per-lane partials, in exactly wave_sum_d's order (a balanced tree
// over the 64 lanes in lane order, so bit-identical to it) with the work shared: the partials go
// through this wavefront's LDS rows s[R][64]; lane j of group r (lanes 8r..8r+7) adds lanes
// 8j..8j+7 of row r (the tree's first three levels), and the group combines its eight sums with
// three DPP steps (the last three). R separate wave_sum_d calls cost ~22 instructions a row.
// Returns row (lane / 8)'s total in every lane of that group; lanes from 8R on return garbage.
template <int R>
IRON_DEV double rows_sum_d(const double (&v)[R], double (*s)[64]) {
  static_assert(R >= 1 && R <= 8, "one 8-lane group per row");
  const int lane = threadIdx.x & 63, grp = lane >> 3, j = lane & 7;
#pragma unroll
  for (int r = 0; r < R; ++r) s[r][lane] = v[r];
  // one wavefront's LDS accesses complete in order: its reads below see its writes
  double t = 0.0;
  if (grp < R) {
    const double2* q = (const double2*)&s[grp][8 * j];
    const double2 a = q[0], b = q[1], c = q[2], d = q[3];
    t = ((a.x + a.y) + (b.x + b.y)) + ((c.x + c.y) + (d.x + d.y));
  }
  t += dpp_d<0xb1>(t);   // quad_perm [1,0,3,2]: lane groups 2i, 2i+1 (16-lane rows)
  t += dpp_d<0x4e>(t);   // quad_perm [2,3,0,1]: rows 0+1, 2+3
  t += dpp_d<0x141>(t);  // row_half_mirror: (0+1) + (2+3)
  return t;
}

// ---------------------------------------------------------------------------------------------
// Phase A: raw = bf16(Wqkv . bf16(RMSNorm(x) * n_in))                [MQKV rows x D]
// ---------------------------------------------------------------------------------------------
template <class S, class Issue>
IRON_DEV bool phase_qkv(const PParams& p, int l, int wg, uint32_t ep, uint32_t* s_in,
                        uint16_t* s_out, const W8<S::RA, S::CA>& W,
                        const uint4 (&nwl)[S::CA][2], Issue issue) {
  constexpr int R = S::RA, NCH = S::CA;
  const int lane = threadIdx.x & 63;
  stamp<S>(p, wg, l, 0);
  const int blk = qkv_block<S>(wg);
  const int row0 = row0_of<S>(blk, R);
  GemvParams g = gemv_of(p.g_qkv, nullptr, S::MQKV, S::D);
  g.pro = PRO_RMS_BF16;
  g.eps = p.eps;
  {
    const uint32_t tx = x_tag(ep, p.n_layers, l);
    unsigned long long* const xs = copy_for(p.X, kCopyWords, wg);
    auto src = [&](int j, uint32_t& t) { t = tx; return xs + spread_word(j); };
    if (!gather_pairs_dev<cdiv(S::D / 2, 512), kQkvFirstPollDelay>(S::D / 2, xs, src, issue,
                                                                    s_in, p.ctrl + 1))
      return false;
  }
  stamp<S>(p, wg, l, 1);
  uint4 xl[NCH][4], x2l[NCH][2] = {};
  lane_bf16<NCH>(s_in, S::D, lane, xl);
  float xf[NCH][16];
  prologue_lane<NCH, 16>(g, lane, xl, x2l, nwl, xf);
  double acc[R][1];
  const uint32_t tag = phase_tag(ep, p.n_layers, l, 0);
  if constexpr (R % 2 == 0 && R <= 8) {
    // a wavefront's rows pair up within it
    dot_w8_lane<R, NCH, false>(g, W.w, W.sc, xf, row0, lane, acc);
    __shared__ double s_rows[4][R][64];
    double v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = acc[r][0];
    // row r's total is in lanes 8r..8r+7; lane 16k pairs rows 2k and 2k+1 (row_ror:8)
    const uint32_t hb = f64_to_bf16(rows_sum_d<R>(v, s_rows[threadIdx.x >> 6]));
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)hb, 0x128, 0xf, 0xf, false);
    const int k = lane >> 4, wave = threadIdx.x >> 6;
    // the workgroup's 4R rows leave as 2R consecutive words from one store instruction
    __shared__ uint32_t s_pairs[4 * R / 2];
    if ((lane & 15) == 0 && k < R / 2) s_pairs[wave * (R / 2) + k] = (hb & 0xffffu) | (hi << 16);
    __syncthreads();
    const int t = threadIdx.x, row = blk * 4 * R + 2 * t;
    if (t < 2 * R && row < S::MQKV) {
      if constexpr (S::XCD_LOCAL)  // read only by this XCD's attention workgroups: one copy
        put_word_local(xcd_local_rsrc(p.RAW, S::MQKV / 2), row / 2, s_pairs[t], tag);
      else
        put_word_copies(p.RAW + row / 2, kCopyWords, s_pairs[t], tag);
    }
  } else {
    dot_w8_lane<R, NCH>(g, W.w, W.sc, xf, row0, lane, acc);
    uint16_t h[R];
#pragma unroll
    for (int r = 0; r < R; ++r) h[r] = f64_to_bf16(acc[r][0]);
    static_assert(!S::XCD_LOCAL, "the XCD-local raw rows leave from the even-R branch");
    store_bf16_pairs<R>(h, blk, S::MQKV, p.RAW, tag, s_out, nullptr);
  }
  stamp<S>(p, wg, l, 2);
  return true;
}

// The QKV head epilogue (qkv_head_dp/reference.py:13-33) for one head by one wavefront:
//   y = bf16(RMSNorm(x) * w), r = bf16(RoPE(y)), r[i] = y[i] c_i - y[i+64] s_i,
//   r[i+64] = y[i+64] c_i + y[i] s_i (i < 64).
// Lane a owns dims a and a + 64, the two halves of one rotation, so no lane exchange is needed.
// The operations and roundings are those of norm_rope8 and of the epilogue kernel in qkv.hip; the
// sum of squares is exact in fp64, so its order does not matter.
IRON_DEV void norm_rope_pair(const uint16_t* raw, uint32_t w2, uint32_t cs, int lane, double eps,
                             uint16_t* out) {
  const double x0 = bf16_to_f32(raw[lane]), x1 = bf16_to_f32(raw[lane + 64]);
  const double inv = inv_rms(wave_sum_d(x0 * x0 + x1 * x1), kAttnD, eps);
  const double y0 = round_bf16((float)((x0 * inv) * (double)bf16lo_to_f32(w2)));
  const double y1 = round_bf16((float)((x1 * inv) * (double)bf16hi_to_f32(w2)));
  const double c = bf16lo_to_f32(cs), s = bf16hi_to_f32(cs);
  out[lane] = f64_to_bf16(y0 * c - y1 * s);
  out[lane + 64] = f64_to_bf16(y1 * c + y0 * s);
}

// One tile of kTileTokens positions of the exact (fp64) core for a GQA pair (two query heads).
// Lane (wave, row, dl) holds K/V rows t0 + tt, tt = 16u + 4 wave + row, head dims 8 dl..+8; rows
// at or past t_end are masked, and the row at `pos` is the current token's (s_new) when has_new
// (this split then ends at pos).
//  1. each lane's 8-dim partial products go to LDS ([head][token][dl]);
//  2. lane (wave, row, i) of a reducing row sums the 16 partials of one (token, head) pair:
//     token 32 wave + 16 (row / 2) + i, head row % 2 -- 160 pairs on wavefronts 0..2 -- and the
//     pair maxima give the tile maximum per head (a row maximum, then rows r and r ^ 2, then
//     the four wavefronts through LDS);
//  3. the pair lanes write e^(s - m) to LDS, and every lane reads back the U probabilities of its
//     rows for the P.V products.
// The q.k sums are exact in fp64 (bf16 products), so summing them by a tree over lanes gives the
// values of a sequential sum; the exponential and the P.V order are those of attn_tile_f64.
// Updates the running maximum m, sum l and unnormalised output o of the two heads; `it` is the
// tile's index within this workgroup's sequence (0 = the first tile, which starts from zero).
template <int U>
IRON_DEV void attn_tile_pairs(uint4 (&kr)[U], uint4 (&vr)[U], int t0, int t_end, bool has_new,
                              int pos, const uint4 (&s_new)[2][16], const double (&qf)[2][8],
                              double scale, int it, double (&m)[2], double (&l)[2],
                              double (&o)[2][8], int wave, int lane, int row, int dl) {
  constexpr int NT = 16 * U;
  static_assert(NT <= 96, "three wavefronts of pair lanes");
  // row stride 18 doubles: 16 consecutive tokens of one head fall in distinct LDS bank groups
  __shared__ __align__(16) double s_ps[2][NT][18];
  __shared__ __align__(16) double s_p[NT][2];
  __shared__ double s_mx[4][2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tt = u * 16 + wave * 4 + row;
    // rows past the split repeat its last row (load_kv_rows); when that row is the current
    // token's, the cache still holds stale data there, so all of them take the new rows: every
    // masked V row is then finite, and its zero probability adds exact zeros
    if (has_new && t0 + tt >= pos) {
      kr[u] = s_new[0][dl];
      vr[u] = s_new[1][dl];
    }
    double kf[8];
    unpack8d(kr[u], kf);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      double a = 0.0;
#pragma unroll
      for (int j = 0; j < 8; ++j) a = fma(qf[h][j], kf[j], a);
      s_ps[h][tt][dl] = a;
    }
  }
  __syncthreads();
  const int ph = row & 1, pt = wave * 32 + (row >> 1) * 16 + dl;
  double s = -INFINITY;
  if (pt < NT) {
    double v[16];
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
      const double2 d = *(const double2*)&s_ps[ph][pt][k];
      v[k] = d.x;
      v[k + 1] = d.y;
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int k = 0; k < w; ++k) v[k] += v[k + w];
    if (t0 + pt < t_end) s = v[0] * scale;
  }
  // row maxima; rows r and r + 2 hold the same head (a lane exchange: no LDS shuffle)
  double wm = row16_max_d(s), wm2 = wm;
  swap_lanes_d<true>(wm, wm2);  // rows r and r + 2 meet: row 0 holds head 0's maximum, row 1 head 1's
  const double mh = fmax(wm, wm2);
  if ((lane & 47) == 0) s_mx[wave][ph] = mh;  // lanes 0 and 16: heads 0 and 1
  __syncthreads();
  double mn[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const double t = fmax(fmax(s_mx[0][h], s_mx[1][h]), fmax(s_mx[2][h], s_mx[3][h]));
    mn[h] = fmax(m[h], t);
  }
  // every tile of the loop holds at least one valid token, so mn is finite here
  if (pt < NT) s_p[pt][ph] = s == -INFINITY ? 0.0 : exp(s - (ph ? mn[1] : mn[0]));
  __syncthreads();
  double pe[U][2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const double2 d = *(const double2*)&s_p[u * 16 + wave * 4 + row][0];
    pe[u][0] = d.x;
    pe[u][1] = d.y;
  }
  if (it > 0) {  // rescale the running sums (the first tile starts from zero)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const double c = m[h] == -INFINITY ? 0.0 : exp(m[h] - mn[h]);
      l[h] *= c;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] *= c;
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    l[h] += tile_sum<U>(pe, h);
    m[h] = mn[h];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double vf[8];
    unpack8d(vr[u], vf);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] = fma(pe[u][h], vf[j], o[h][j]);
  }
}

// Sums of four values over the four 16-lane rows of the wavefront, one value's sum per row: row 0
// gets the sum of a, row 1 of c, row 2 of b, row 3 of d (lane i of a row: the sum of lane i of
// every row). Two exchange steps, each halving what a lane holds: rows (r, r + 2), then (r, r + 1).
IRON_DEV double rows4_sum(double a, double b, double c, double d) {
  swap_lanes_d<true>(a, b);
  swap_lanes_d<true>(c, d);
  double u = a + b, v = c + d;
  swap_lanes_d<false>(u, v);
  return u + v;
}

// The end of the exact core for a GQA pair (attn_finish_f64 with HB = 2): the 16 token rows of
// the workgroup (4 per wavefront) hold partial sums under the same offsets m, so they add. The
// four rows of a wavefront add by lane exchanges (rows4_sum), which leaves each lane 5 of its 18
// values (o of two heads x 8 dims, l of two heads) summed over its wavefront; the four wavefronts
// add through LDS (10 KB written, where a 16-row LDS tree wrote 32 KB and read 64 KB: -7 us per
// token). Thread (oh, od) emits head oh, dim od: emit(oh, od, O, L, M).
template <class Emit>
IRON_DEV void attn_finish_pairs(const double (&m)[2], const double (&l)[2],
                                const double (&o)[2][8], int wave, int row, int dl, Emit emit) {
  constexpr int kSlots = 5;
  __shared__ double s_w[4][kSlots][64];
  const int lane = row * 16 + dl;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q)  // slot 2h + q: dims 4q..4q+3 of head h
      s_w[wave][2 * h + q][lane] =
          rows4_sum(o[h][4 * q], o[h][4 * q + 1], o[h][4 * q + 2], o[h][4 * q + 3]);
  s_w[wave][4][lane] = rows4_sum(l[0], l[1], 0.0, 0.0);
  __syncthreads();
  // value p of a quad lands in row ((p & 1) << 1) | (p >> 1)
  const int oh = threadIdx.x >> 7, od = threadIdx.x & 127, j = od & 7, p = j & 3;
  const int at = (((p & 1) << 1) | (p >> 1)) * 16 + (od >> 3);
  const int slot = 2 * oh + (j >> 2), lat = (oh ? 2 : 0) * 16 + (od >> 3);
  const double O = (s_w[0][slot][at] + s_w[1][slot][at]) + (s_w[2][slot][at] + s_w[3][slot][at]);
  const double L = (s_w[0][4][lat] + s_w[1][4][lat]) + (s_w[2][4][lat] + s_w[3][4][lat]);
  emit(oh, od, O, L, oh ? m[1] : m[0]);
}

// ---------------------------------------------------------------------------------------------
// Phase B: the QKV epilogue and the exact attention core over this split's positions. Workgroup
// (kv, split) handles a contiguous 1/NS of the context of KV head kv and writes its partial
// (o unnormalised, m, l) of the HB query heads as tagged fp64 words.
// ---------------------------------------------------------------------------------------------
template <class S, class Issue>
IRON_DEV bool phase_attn(const PParams& p, const iron_layer_desc& L, int l, int wg, uint32_t ep,
                         int pos, uint32_t* s_in, KVPrefetch& kv, Issue issue) {
  constexpr int HB = S::HB, NS = S::NS;
  const int head = attn_head<S>(wg), split = attn_split<S>(wg);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, row = lane >> 4, dl = lane & 15;
  const bool pos_ok = pos >= 0 && pos < p.max_seq;
  const SplitRange range = split_range<S>(context_of(p, pos), split);

  // the raw q rows of heads head*HB.., and the raw k and v rows of KV head `head`
  {
    constexpr int n = (HB + 2) * 64;
    const uint32_t tr = phase_tag(ep, p.n_layers, l, 0);
    unsigned long long* const raw = S::XCD_LOCAL ? p.RAW : copy_for(p.RAW, kCopyWords, wg);
    auto src = [&](int j, uint32_t& t) {
      t = tr;
      const int seg = j >> 6, off = j & 63;
      const int base = seg < HB ? (head * HB + seg) * 64
                                : (seg == HB ? (S::QD + head * S::HD) / 2
                                             : (S::QD + S::KVD + head * S::HD) / 2);
      return raw + base + off;
    };
    bool ok;
    if constexpr (S::XCD_LOCAL)
      ok = gather_pairs_local<cdiv(n, 512), kLocalFirstPollDelay>(n, src, issue, s_in,
                                                                  p.ctrl + 1);
    else
      ok = gather_words<cdiv(n, 256)>(n, src, issue, s_in, p.ctrl + 1);
    if (!ok) return false;
  }
  stamp<S>(p, wg, l, 3);
  const uint16_t* s_raw = (const uint16_t*)s_in;  // segment seg: 128 bf16

  // QK RMSNorm + RoPE: wave h < HB rotates query head h; wave HB % 4 builds the current token's
  // K row (V unchanged) when this split owns its tile, and appends both to the caches
  __shared__ __align__(16) uint16_t s_q[HB][kAttnD];
  __shared__ uint4 s_new[2][16];
  const bool has_new = pos_ok && pos >= range.begin && pos < range.end;
  const bool new_wave = has_new && wave == HB % 4;
  if (wave < HB)
    norm_rope_pair(s_raw + wave * kAttnD, kv.nq, kv.cs, lane, (double)p.eps, s_q[wave]);
  if (new_wave) {
    norm_rope_pair(s_raw + HB * kAttnD, kv.nk, kv.cs, lane, (double)p.eps, (uint16_t*)s_new[0]);
    if (lane < 16) s_new[1][lane] = ((const uint4*)s_raw)[(HB + 1) * 16 + lane];
  }
  __syncthreads();
  if (new_wave && lane < 16) {
    const size_t at = (size_t)head * p.kv_sh + (size_t)pos * p.kv_st + lane * 8;
    st_global((uint4*)(L.k_cache + at), s_new[0][lane]);
    st_global((uint4*)(L.v_cache + at), s_new[1][lane]);
  }

  double qf[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) unpack8d(((const uint4*)s_q[h])[dl], qf[h]);
  double m[HB], lsum[HB], o[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    m[h] = -INFINITY;
    lsum[h] = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[h][j] = 0.0;
  }
  stamp<S>(p, wg, l, 4);
  int it = 0;
  for (int t0 = range.begin; t0 < range.end; t0 += kTileTokens, ++it) {
    if (it > 0) load_kv_rows(p, L, head, t0, range.end, kv.kr, kv.vr);
    attn_tile_pairs<kRows>(kv.kr, kv.vr, t0, range.end, has_new, pos, s_new, qf, p.scale, it, m,
                           lsum, o, wave, lane, row, dl);
  }
  stamp<S>(p, wg, l, 15);
  const uint32_t tp = phase_tag(ep, p.n_layers, l, 1);
  // Word 2 d + k of a partial holds half k of dim d. XCD-local: thread (oh, od) writes dim od's
  // two words with one 16-byte store (a wavefront's store covers 1 KB contiguously; against two
  // lane-exchanged 8-byte stores, -4 us per token). Device-wide:
  // each store instruction writes 64 consecutive words (the wavefront's 64 dims, exchanged so lane
  // j holds word j): those stores write through the L2, which merges nothing, so a store per half
  // would write every sector twice.
  attn_finish_pairs(m, lsum, o, wave, row, dl,
                    [&](int oh, int od, double O, double Ls, double M) {
    const size_t part = ((size_t)(head * HB + oh) * NS + split) * (2 * (kAttnD + 2));
    const double v = od < 2 ? M : Ls;       // m and l (the same in every thread of the head)
    const uint32_t v32 = (uint32_t)(od & 1 ? __double2hiint(v) : __double2loint(v));
    if constexpr (S::XCD_LOCAL) {  // read only by this XCD's merge workgroups
      const __amdgpu_buffer_rsrc_t rs = xcd_local_rsrc(p.PART, S::PART_WORDS);
      put_pair_local(rs, part + 2 * od, (uint32_t)__double2loint(O), (uint32_t)__double2hiint(O),
                     tp);
      if (od < 4) put_word_local(rs, part + 2 * kAttnD + od, v32, tp);  // words 2 kAttnD .. + 3
    } else {
      const int j = od & 63;
      const int lo = __double2loint(O), hi = __double2hiint(O);
      const int lo1 = __shfl(lo, j >> 1), hi1 = __shfl(hi, j >> 1);
      const int lo2 = __shfl(lo, 32 + (j >> 1)), hi2 = __shfl(hi, 32 + (j >> 1));
      const size_t w = part + 2 * (od & 64);  // this wavefront's 128 words
      put_word(p.PART + w + j, (uint32_t)(j & 1 ? hi1 : lo1), tp);
      put_word(p.PART + w + 64 + j, (uint32_t)(j & 1 ? hi2 : lo2), tp);
      if (od < 4) put_word(p.PART + part + 2 * kAttnD + od, v32, tp);
    }
  });
  stamp<S>(p, wg, l, 5);
  return true;
}

// ---------------------------------------------------------------------------------------------
// Phase C: merge the NS splits of MERGE_PER attention outputs (one head, consecutive dims):
// o = sum_s f_s O_s / sum_s f_s L_s with f_s = e^(m_s - max m), evaluated in fp64.
// ---------------------------------------------------------------------------------------------
template <class S, class Issue>
IRON_DEV bool phase_merge(const PParams& p, int l, int wg, uint32_t ep, uint32_t* s_in,
                          Issue issue) {
  constexpr int PER = S::MERGE_PER, NS = S::NS, WPS = S::MERGE_WPS;
  const int o0 = merge_o0<S>(wg), h = o0 / kAttnD, d0 = o0 % kAttnD;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  {
    constexpr int n = NS * WPS;
    const uint32_t tp = phase_tag(ep, p.n_layers, l, 1);
    auto part_of = [&](int s) { return p.PART + ((size_t)h * NS + s) * (2 * (kAttnD + 2)); };
    auto src = [&](int j, uint32_t& t) {
      t = tp;
      const int s = j / WPS, k = j % WPS;
      unsigned long long* part = part_of(s);
      return k < 2 * PER ? part + 2 * d0 + k : part + 2 * kAttnD + (k - 2 * PER);
    };
    bool ok;
    if constexpr (S::XCD_LOCAL)
      ok = gather_pairs_local<cdiv(n, 512), kLocalFirstPollDelay>(n, src, issue, s_in,
                                                                  p.ctrl + 1);
    else
      ok = gather_words<cdiv(n, 256)>(n, src, issue, s_in, p.ctrl + 1);
    if (!ok) return false;
  }
  stamp<S>(p, wg, l, 6);
  // thread (split sp, dim d): sp = t % NS, d = t / NS holds o_sp[d0 + d], m_sp and l_sp; the
  // max and the two sums run over the NS threads of one d (a wavefront, or two for NS = 128)
  const int t = threadIdx.x, sp = t % NS, d = t / NS;
  const uint32_t* w = s_in + sp * WPS;
  const double os = word_double(w[2 * d], w[2 * d + 1]);
  const double ms = word_double(w[2 * PER], w[2 * PER + 1]);
  const double ls = word_double(w[2 * PER + 2], w[2 * PER + 3]);
  __shared__ double s_red[4][2];
  const double M = group_max<NS>(ms, s_red);
  const double f = (M == -INFINITY || ms == -INFINITY) ? 0.0 : exp(ms - M);
  const double Lt = group_sum<NS>(f * ls, s_red);
  const double O = group_sum<NS>(f * os, s_red);
  __shared__ uint16_t s_o16[PER];
  if (sp == 0) s_o16[d] = f64_to_bf16(Lt > 0.0 ? O / Lt : 0.0);
  __syncthreads();
  // thread c (PER / 2) + i stores word i of copy c: one store instruction for all copies (-0.7 us
  // per token)
  const int wi = t % (PER / 2), wc = t / (PER / 2);
  if (wc < kCopies)
    put_word(p.ATT + (size_t)wc * kCopyWords + spread_word((h * kAttnD + d0) / 2 + wi),
             (uint32_t)s_o16[2 * wi] | ((uint32_t)s_o16[2 * wi + 1] << 16),
             phase_tag(ep, p.n_layers, l, 2));
  (void)wave;
  (void)lane;
  stamp<S>(p, wg, l, 7);
  return true;
}

// ---------------------------------------------------------------------------------------------
// Phase D: a = bf16(Wo . attn)                                        [D rows x QD]
// ---------------------------------------------------------------------------------------------
template <class S, class Issue>
IRON_DEV bool phase_wo(const PParams& p, int l, int wg, uint32_t ep, uint32_t* s_in,
                       uint16_t* s_out, uint32_t* s_own, const W8<S::RD, S::CD>& W,
                       Issue issue) {
  constexpr int R = S::RD, NCH = S::CD;
  const int lane = threadIdx.x & 63;
  const int row0 = row0_of<S>(wg, R);
  GemvParams g = gemv_of(p.g_o, nullptr, S::D, S::QD);
  g.pro = PRO_BF16;
  if constexpr (!S::WO_ALL)
    if (wg * 4 * R >= S::D) return skip_gather(issue);  // no Wo rows here (small shapes)
  {
    const uint32_t ta = phase_tag(ep, p.n_layers, l, 2);
    unsigned long long* const att = copy_for(p.ATT, kCopyWords, wg);
    auto src = [&](int j, uint32_t& t) { t = ta; return att + spread_word(j); };
    if (!gather_pairs_dev<cdiv(S::QD / 2, 512)>(S::QD / 2, att, src, issue, s_in,
                                            p.ctrl + 1))
      return false;
  }
  stamp<S>(p, wg, l, 8);
  uint4 xl[NCH][4], x2l[NCH][2] = {}, nwl[NCH][2] = {};
  lane_bf16<NCH>(s_in, S::QD, lane, xl);
  float xf[NCH][16];
  prologue_lane<NCH, 16>(g, lane, xl, x2l, nwl, xf);
  double acc[R][1];
  dot_w8_lane<R, NCH>(g, W.w, W.sc, xf, row0, lane, acc);
  uint16_t h[R];
#pragma unroll
  for (int r = 0; r < R; ++r) h[r] = f64_to_bf16(acc[r][0]);
  store_bf16_pairs<R, true>(h, wg, S::D, p.AO, phase_tag(ep, p.n_layers, l, 3), s_out, nullptr);
  keep_own_words<R>(s_out, s_own);  // the down phase's residual a
  stamp<S>(p, wg, l, 9);
  return true;
}

// ---------------------------------------------------------------------------------------------
// Phase E: x1 = f32(x + a); hf = f32(RMSNorm(x1) * n_post);
//          gh = f32(silu(Wg . hf) * (Wu . hf))                        [FF rows x D, two matrices]
// ---------------------------------------------------------------------------------------------
template <class S, class Issue>
IRON_DEV bool phase_gateup(const PParams& p, int l, int wg, uint32_t ep, uint32_t* s_in,
                           const uint32_t* s_x, float* s_gh, const W8<S::RE, S::CE>& Wg,
                           const W8<S::RE, S::CE>& Wu,
                           const uint4 (&nwl)[S::CE][2], Issue issue) {
  constexpr int R = S::RE, NCH = S::CE;
  const int lane = threadIdx.x & 63;
  const int row0 = row0_of<S>(wg, R);
  GemvParams g = gemv_of(p.g_gu, nullptr, S::FF, S::D);
  g.pro = PRO_RES_RMS_F32;
  g.eps = p.eps;
  g.x2 = (const uint16_t*)p.AO;  // marks the residual term (read from LDS here)
  if constexpr (!S::GU_ALL)
    if (wg * 4 * R >= S::FF) return skip_gather(issue);  // no gate/up rows here (small shapes)
  {
    // a only: the layer input x is still in s_x from this workgroup's QKV phase
    const uint32_t ta = phase_tag(ep, p.n_layers, l, 3);
    unsigned long long* const as = copy_for(p.AO, kCopyWords, wg);
    auto src = [&](int j, uint32_t& t) {
      t = ta;
      return as + spread_word(j);
    };
    if (!gather_pairs_dev<cdiv(S::D / 2, 512)>(S::D / 2, as, src, issue, s_in, p.ctrl + 1))
      return false;
  }
  stamp<S>(p, wg, l, 10);
  uint4 xl[NCH][4], al[NCH][4], x2l[NCH][2];
  lane_bf16<NCH>(s_x, S::D, lane, xl);
  lane_bf16<NCH>(s_in, S::D, lane, al);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    x2l[c][0] = al[c][0];
    x2l[c][1] = al[c][1];
  }
  float xf[NCH][16];
  prologue_lane<NCH, 16>(g, lane, xl, x2l, nwl, xf);
  stamp<S>(p, wg, l, 11);
  double acc[R][1], acc2[R][1];
  dot_w8_lane<R, NCH, false>(g, Wg.w, Wg.sc, xf, row0, lane, acc);
  dot_w8_lane<R, NCH, false>(g, Wu.w, Wu.sc, xf, row0, lane, acc2);
  // each wavefront's 2R row totals (rows_sum_d), then SiLU(gate) * up in the lanes of its R rows
  const int wave = threadIdx.x >> 6;
  static_assert(2 * R <= 8, "gate and up rows of a wavefront in 8-lane groups");
  __shared__ double s_rows[4][2 * R][64];
  double v[2 * R];  // gate row r in group 2r, up row r in group 2r + 1 (the same 16-lane row)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    v[2 * r] = acc[r][0];
    v[2 * r + 1] = acc2[r][0];
  }
  const double tot = rows_sum_d<2 * R>(v, s_rows[wave]);
  const double u_r = dpp_d<0x128>(tot);  // row_ror:8: lane 16r gets up row r
  const float gh = (float)silu_mul(tot, u_r);  // lane 16r: SiLU(gate r) * up r
  unsigned long long* const blk = p.GH + (l % kGhBuffers) * S::GH_WORDS + wg * kGhBlock;
  const uint32_t stag = short_tag(phase_tag(ep, p.n_layers, l, 4));
  if constexpr (R == 3) {
    // The wavefront's three values fill packed words 2 wave and 2 wave + 1 of the block (96 bits),
    // so each wavefront publishes its own: no LDS exchange, no barrier (-2.6 us per token). Lanes
    // 0..15 store one (copy, word) each.
    const uint32_t g0 = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(gh), 0);
    const uint32_t g1 = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(gh), 16);
    const uint32_t g2 = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(gh), 32);
    const unsigned long long w0 =
        (unsigned long long)g0 | ((unsigned long long)(g1 & 0xffffu) << 32);
    const unsigned long long w1 =
        (unsigned long long)(g1 >> 16) | ((unsigned long long)g2 << 16);
    if (lane < 2 * kCopies) {
      const int i = lane & 1, c = lane >> 1;
      const unsigned long long w =
          ((unsigned long long)stag << 48) | ((i ? w1 : w0) & 0xffffffffffffull);
      __hip_atomic_store(blk + (size_t)c * S::GH_COPY + 2 * wave + i, w, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    if ((lane & 15) == 0 && (lane >> 4) < R) s_gh[wave * R + (lane >> 4)] = gh;
    __syncthreads();
    // the block's GH_PACKED words: 16-bit halves 3 t .. 3 t + 2 of the GH_ROWS values
    const int t = threadIdx.x;
    if (t < S::GH_PACKED)
      put_packed_copies(blk + t, S::GH_COPY, pack48((const uint32_t*)s_gh, S::GH_ROWS, t), stag);
  }
  stamp<S>(p, wg, l, 12);
  return true;
}

// ---------------------------------------------------------------------------------------------
// Phase F: x' = bf16(f32(x + a) + Wd . gh)                            [D rows x FF]
// ---------------------------------------------------------------------------------------------
template <class S, class Issue>
IRON_DEV bool phase_down(const PParams& p, int l, int wg, uint32_t ep, uint32_t* s_in,
                         uint16_t* s_out, uint32_t* s_own, const W8<S::RF, S::CF>& W,
                         Issue issue) {
  constexpr int R = S::RF, NCH = S::CF;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = row0_of<S>(wg, R);
  GemvParams g = gemv_of(p.g_d, nullptr, S::D, S::FF);
  g.pro = PRO_F32;
  // LDS words [0, FF): gh; the residual (a and x of this workgroup's 4R rows) is in s_own
  unsigned long long* const gh =
      copy_for(p.GH, S::GH_COPY, wg) + (l % kGhBuffers) * S::GH_WORDS;
  if constexpr (!S::WO_ALL)
    if (wg * 4 * R >= S::D) return skip_gather(issue);  // no down rows here (small shapes)
  {
    // gate/up workgroup q publishes rows [GH_ROWS q, GH_ROWS (q + 1)) in block q
    static_assert(S::GH_ROWS * S::GH_PROD == S::FF, "whole gh blocks");
    // first poll after kDownFirstPollDelay units (the gh producers finish last in the layer)
    if (!gather_gh<S::GH_ROWS, cdiv(S::GH_PROD * S::GH_PACKED, 256), kDownFirstPollDelay>(
            S::GH_PROD, gh, short_tag(phase_tag(ep, p.n_layers, l, 4)), issue, s_in, p.ctrl + 1))
      return false;
  }
  stamp<S>(p, wg, l, 13);
  uint4 xl[NCH][4], x2l[NCH][2] = {}, nwl[NCH][2] = {};
  lane_f32<NCH>(s_in, S::FF, lane, xl);
  float xf[NCH][16];
  prologue_lane<NCH, 16>(g, lane, xl, x2l, nwl, xf);
  double acc[R][1];
  dot_w8_lane<R, NCH>(g, W.w, W.sc, xf, row0, lane, acc);
  const uint16_t* s_res = (const uint16_t*)s_own;  // a rows, then x rows (4R each)
  uint16_t h[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = wave * R + r;  // row within the workgroup
    const float x1 = bf16_to_f32(s_res[4 * R + k]) + bf16_to_f32(s_res[k]);
    h[r] = f64_to_bf16((double)x1 + acc[r][0]);
  }
  store_bf16_pairs<R, true>(h, wg, S::D, p.X, phase_tag(ep, p.n_layers, l, 5), s_out,
                      l == p.n_layers - 1 ? p.x_out : nullptr);
  keep_own_words<R>(s_out, s_own + S::XW);  // the next layer's residual x (its reads are done)
  stamp<S>(p, wg, l, 14);
  return true;
}

// ---------------------------------------------------------------------------------------------
// Phase H (folded LM head): logits = bf16(W_head . bf16(RMSNorm(x) * n_final)), argmax key.
// Workgroup wg owns a contiguous range of 16-row blocks; in each block wavefront w takes rows
// 4w..4w+3 (lane l: elements c*512 + 8l .. +8 of each 512-wide chunk, one 16-byte load per row
// and chunk). Blocks stream through a ring of kLmStages register stages, so kLmStages - 1 blocks
// of loads are in flight while one is multiplied; the first two stages are issued as soon as the
// last layer's output has arrived, so they stream while the final RMSNorm is computed.
// Arithmetic of iron_lm_head's bf16 path: exact bf16 products summed in fp64, one bf16 rounding.
// ---------------------------------------------------------------------------------------------
constexpr int kLmRows = 4;     // rows per wavefront per block
constexpr int kLmStages = 3;   // register stages of the block ring (3 or 4; 3 measured faster)

template <class S>
struct LmRing {
  static constexpr int NC = cdiv(S::D, 512);  // 512-wide chunks of a row
  uint4 w[kLmStages][kLmRows][NC];
};

template <class S>
IRON_DEV int lm_blocks(int vocab) { return (vocab + 4 * kLmRows - 1) / (4 * kLmRows); }

template <class S>
IRON_DEV void lm_range(int vocab, int wg, int& b0, int& b1) {
  const int nb = lm_blocks<S>(vocab);
  b0 = (int)(((long long)nb * wg) / kNT);
  b1 = (int)(((long long)nb * (wg + 1)) / kNT);
}

// Loads block b (rows 16b + 4 wave + r; rows past the head clamp to row 0 and are never stored)
// into ring stage st.
template <class S>
IRON_DEV void lm_fetch(const PParams& p, int b, int st, LmRing<S>& ring) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kLmRows; ++r) {
    const int row = b * 4 * kLmRows + wave * kLmRows + r;
    const size_t at = (size_t)(row < p.vocab ? row : 0) * S::D;
#pragma unroll
    for (int c = 0; c < LmRing<S>::NC; ++c) {
      const int e = c * 512 + lane * 8;  // elements past D: a clamped load, multiplied by x = 0
      ring.w[st][r][c] = ld_global((const uint4*)(p.lm_w + at + (e < S::D ? e : 0)));
    }
  }
}

// The first two blocks of this workgroup's range (issued during the last layer).
template <class S>
IRON_DEV void lm_prefetch(const PParams& p, int wg, LmRing<S>& ring) {
  int b0, b1;
  lm_range<S>(p.vocab, wg, b0, b1);
#pragma unroll
  for (int st = 0; st < kLmStages - 1; ++st)
    if (b0 + st < b1) lm_fetch<S>(p, b0 + st, st, ring);
}

template <class S>
IRON_DEV bool phase_lm_head(const PParams& p, int wg, uint32_t ep, uint32_t* s_in,
                            unsigned long long* key_out, LmRing<S>& ring) {
  constexpr int NC = LmRing<S>::NC;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  {
    const uint32_t tx = x_tag(ep, p.n_layers, p.n_layers);
    unsigned long long* const xs = copy_for(p.X, kCopyWords, wg);
    auto src = [&](int j, uint32_t& t) { t = tx; return xs + spread_word(j); };
    if (!gather_pairs_dev<cdiv(S::D / 2, 512)>(S::D / 2, xs, src,
                                               [&]() { lm_prefetch<S>(p, wg, ring); }, s_in,
                                               p.ctrl + 1))
      return false;
  }
  // xn = bf16(RMSNorm(x) * n_final) for this lane's elements c*512 + 8 lane .. +8
  GemvParams g = {};
  g.pro = PRO_RMS_BF16;
  g.K = S::D;
  g.eps = p.eps;
  uint4 xl[NC][2], x2l[NC][1] = {}, nwl[NC][1];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = c * 512 + lane * 8;
    const bool in = e < S::D;  // elements past D are zero (they add nothing to the statistic)
    xl[c][0] = in ? ((const uint4*)s_in)[e / 8] : make_uint4(0u, 0u, 0u, 0u);
    xl[c][1] = make_uint4(0u, 0u, 0u, 0u);
    nwl[c][0] = ld_global((const uint4*)(p.lm_norm + (in ? e : 0)));
  }
  float xf[NC][8];
  prologue_lane<NC, 8>(g, lane, xl, x2l, nwl, xf);
  double xv[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[c][j] = xf[c][j];

  __shared__ double s_lrows[4][kLmRows][64];
  __shared__ unsigned long long s_kbest[4];
  int b0, b1;
  lm_range<S>(p.vocab, wg, b0, b1);
  unsigned long long best = 0ull;
  // block b's products from ring stage ST (a compile-time index, so the ring stays in registers
  // and the compiler waits only for that stage's loads, not for the younger ones in flight)
  auto block = [&](auto st_c, int b) {
    constexpr int ST = decltype(st_c)::value;
    double v[kLmRows];
#pragma unroll
    for (int r = 0; r < kLmRows; ++r) {
      double pa = 0.0, pb = 0.0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 w4 = ring.w[ST][r][c];
        const uint32_t dd[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pa = fma((double)bf16lo_to_f32(dd[j]), xv[c][2 * j], pa);
          pb = fma((double)bf16hi_to_f32(dd[j]), xv[c][2 * j + 1], pb);
        }
      }
      v[r] = pa + pb;
    }
    const double tot = rows_sum_d<kLmRows>(v, s_lrows[wave]);  // row lane/8 in lanes 8r..8r+7
    const int r = lane >> 3, row = b * 4 * kLmRows + wave * kLmRows + r;
    if ((lane & 7) == 0 && r < kLmRows && row < p.vocab) {
      const uint16_t h = f64_to_bf16(tot);
      if (p.logits) p.logits[row] = h;
      const unsigned long long key = ((unsigned long long)bf16_order_key(h) << 32) |
                                     (unsigned long long)(~(uint32_t)row);
      best = key > best ? key : best;
    }
  };
  // stages 0 .. kLmStages - 2 hold blocks b0 .. (lm_prefetch); block b0 + k sits in stage
  // k % kLmStages: before block b + k is multiplied, block b + k + kLmStages - 1 is issued into the
  // stage that block b + k - 1 has just left
  auto step = [&](auto k_c, int b) {
    constexpr int K = decltype(k_c)::value;
    if (b + K + kLmStages - 1 < b1)
      lm_fetch<S>(p, b + K + kLmStages - 1, (K + kLmStages - 1) % kLmStages, ring);
    block(std::integral_constant<int, K>(), b + K);
  };
  for (int b = b0; b < b1; b += kLmStages) {
    step(std::integral_constant<int, 0>(), b);
    if (b + 1 >= b1) break;
    step(std::integral_constant<int, 1>(), b);
    if (b + 2 >= b1) break;
    step(std::integral_constant<int, 2>(), b);
    if constexpr (kLmStages == 4) {
      if (b + 3 >= b1) break;
      step(std::integral_constant<int, 3>(), b);
    }
  }
  // the workgroup's best key, then one atomic
#pragma unroll
  for (int k = 1; k < 64; k <<= 1) {
    const unsigned long long o = __shfl_xor(best, k);
    best = o > best ? o : best;
  }
  if (lane == 0) s_kbest[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = s_kbest[0];
    for (int i = 1; i < 4; ++i) k = s_kbest[i] > k ? s_kbest[i] : k;
    if (k) atomicMax(key_out, k);
  }
  return true;
}

// Each phase's weights are issued from an earlier phase's wait (gather_words' `issue` hook):
//   A waits -> B's first K/V tile;  B waits -> D's Wo;  C waits -> E's Wg/Wu;
//   D waits -> F's Wd;  E waits -> the next layer's Wqkv.
template <class S>
__global__ __launch_bounds__(256, 1) void decode_persistent_kernel(PParams p) {
  __shared__ uint32_t s_in[S::LDS_WORDS];
  __shared__ uint16_t s_out[4 * S::RMAX];
  __shared__ float s_gh[4 * S::RE];
  // this workgroup's own rows of a (words [0, XW), from its Wo phase) and of the layer input x
  // (words [XW, 2 XW), from its previous down phase): the residual of its down phase, kept here
  // rather than polled back from the hand-off buffers
  __shared__ uint32_t s_own[2 * S::XW];
  // the layer input x as the QKV phase gathered it; the gate/up phase reads it back from here
  __shared__ uint32_t s_x[S::D / 2];
  const int wg = blockIdx.x;
  const uint32_t ep = p.ctrl[0];
  const int pos = *p.pos;
  // The XCD-local hand-offs need the workgroups with equal wg % 8 on one XCD. The round-robin
  // dispatch of a one-dimensional grid puts workgroup wg on XCD (wg + o) % 8, where the offset o
  // depends on earlier dispatches (measured: not always 0). Each workgroup records its offset in
  // control word 2 before its first hand-off store; workgroup 0 checks at the end of the launch
  // that they agree (error flag 2 otherwise: a word the mapping strands in another XCD's L2 would
  // make its wait time out, never deliver a stale value).
  if constexpr (S::XCD_LOCAL)
    if (threadIdx.x == 0) {
      __hip_atomic_fetch_or(p.ctrl + 2, 1u << ((xcc_id() - (uint32_t)wg) & 7u), __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    }
  W8<S::RA, S::CA> wqkv;
  uint4 n_in[S::CA][2];
  prefetch_qkv<S>(p, p.layers[0], wg, wqkv, n_in);
  // the previous token's argmax key, and (folded head) the slot this launch's argmax goes to
  unsigned long long* const key_in = p.lm_w ? p.key + (ep & 1u) : p.key;
  unsigned long long* const key_out = p.lm_w ? p.key + ((ep + 1u) & 1u) : nullptr;
  if (p.lm_w && wg == 0) {
    // Clear this launch's argmax slot before workgroup 0 publishes anything: every workgroup's
    // atomicMax into it follows (through the hand-offs) this workgroup's later stores, and the
    // returned value makes the exchange complete before them. The slot was last read at the start
    // of the previous launch.
    __shared__ uint32_t s_cleared;
    if (threadIdx.x == 0)
      s_cleared = (uint32_t)__hip_atomic_exchange(key_out, 0ull, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    (void)s_cleared;
  }
  // the greedy loop's input: the embedding row of the token the previous LM head chose (key =
  // (order(max) << 32) | ~index; a zero key is token 0)
  const uint16_t* x_in = p.x_in;
  int32_t tok = 0;
  if (p.key) {
    const unsigned long long k = *key_in;
    tok = k ? (int32_t)(~(uint32_t)(k & 0xffffffffull)) : 0;
    tok = tok < 0 ? 0 : (tok >= p.vocab ? p.vocab - 1 : tok);
    x_in = p.emb + (size_t)tok * S::D;
  }
  // the embedding row enters the hand-off like any layer's output (x's tag of layer 0)
  if (threadIdx.x < 64)
    for (int j = wg * 64 + threadIdx.x; j < S::D / 2; j += kNT * 64)
      put_word_copies(p.X + spread_word(j), kCopyWords, ((const uint32_t*)x_in)[j],
                      x_tag(ep, p.n_layers, 0));
  if (threadIdx.x < S::XW) {
    const int word = wg * S::XW + threadIdx.x;
    s_own[S::XW + threadIdx.x] = word < S::D / 2 ? ((const uint32_t*)x_in)[word] : 0u;
  }
  // gh buffers no layer of this launch uses: clear this workgroup's block (nothing reads them in
  // this launch; a later launch with more layers then finds zeros there, never an old short tag)
  if (p.n_layers < kGhBuffers && wg < S::GH_PROD && threadIdx.x < S::GH_PACKED)
    for (int b = p.n_layers; b < kGhBuffers; ++b)
      put_packed_copies(p.GH + b * S::GH_WORDS + wg * kGhBlock + threadIdx.x, S::GH_COPY, 0ull, 0u);
  LmRing<S> lm;
  bool ok = true;
  for (int l = 0; l < p.n_layers; ++l) {
    const iron_layer_desc L = p.layers[l];
    KVPrefetch kv;
    W8<S::RD, S::CD> wo;
    W8<S::RE, S::CE> wgate, wup;
    uint4 n_post[S::CE][2];
    W8<S::RF, S::CF> wdown;
    ok =
        phase_qkv<S>(p, l, wg, ep, s_x, s_out, wqkv, n_in,
                     [&]() { prefetch_attn<S>(p, L, wg, pos, kv); }) &&
        phase_attn<S>(p, L, l, wg, ep, pos, s_in, kv, [&]() { prefetch_wo<S>(p, L, wg, wo); }) &&
        phase_merge<S>(p, l, wg, ep, s_in,
                       [&]() { prefetch_gateup<S>(p, L, wg, wgate, wup, n_post); }) &&
        phase_wo<S>(p, l, wg, ep, s_in, s_out, s_own, wo,
                    [&]() { prefetch_down<S>(p, L, wg, wdown); }) &&
        phase_gateup<S>(p, l, wg, ep, s_in, s_x, s_gh, wgate, wup, n_post, [&]() {
          if (l + 1 < p.n_layers) prefetch_qkv<S>(p, p.layers[l + 1], wg, wqkv, n_in);
        }) &&
        phase_down<S>(p, l, wg, ep, s_in, s_out, s_own, wdown, []() {});
    if (!ok) break;
  }
  if (ok && p.lm_w) phase_lm_head<S>(p, wg, ep, s_in, key_out, lm);
  // Advance the epoch for the next launch. Workgroup 0 finishes only after every workgroup has
  // contributed to the last layer, so every workgroup has read `ep`, the key, the position and
  // (in its attention phase) the RoPE row by now: the greedy loop's state advances here too.
  if (wg != 0) return;
  if constexpr (S::XCD_LOCAL)
    if (threadIdx.x == 0) {
      const uint32_t offs = __hip_atomic_exchange(p.ctrl + 2, 0u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if (__popc(offs) != 1) atomicOr(p.ctrl + 1, 2u);
    }
  if (p.key) {
    const int next = pos + 1;
    if (threadIdx.x == 0) {
      if (!p.lm_w) *p.key = 0ull;  // folded: the slot is cleared when it next receives a key
      *p.token = tok;
      if (p.token_log) {
        const int32_t s = *p.step;
        if (s >= 0 && s < p.log_len) p.token_log[s] = tok;
        *p.step = s + 1;
      }
      *p.pos_next = next;
      if (p.ctx) *p.ctx = next + 1;
    }
    if (p.rope_table && next < p.max_seq && threadIdx.x < S::HD / 8)
      ((uint4*)p.ang_next)[threadIdx.x] =
          ((const uint4*)(p.rope_table + (size_t)next * S::HD))[threadIdx.x];
  }
  if (threadIdx.x == 0) p.ctrl[0] = ep + 1u;
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

struct Layout {
  size_t ctrl, X, RAW, PART, ATT, AO, GH, total;
};

template <class S>
Layout layout_of() {
  Layout lo;
  size_t off = 0;
  auto take = [&](size_t words) {
    const size_t at = off;
    off += round256(words * 8);
    return at;
  };
  lo.ctrl = take(32);
  lo.X = take(kCopies * kCopyWords);
  lo.RAW = take(kCopies * kCopyWords);
  lo.PART = take(S::PART_WORDS);
  lo.ATT = take(kCopies * kCopyWords);
  lo.AO = take(kCopies * kCopyWords);
  lo.GH = take((size_t)kCopies * S::GH_COPY);
  lo.total = off;
  return lo;
}

enum ShapeId { SHAPE_NONE = 0, SHAPE_0_6B = 1, SHAPE_TINY = 2 };

ShapeId shape_id(int D, int FF, int Hq, int Hkv, int HD) {
  if (HD != kAttnD) return SHAPE_NONE;
  if (D == ShapeQwen3_0_6B::D && FF == ShapeQwen3_0_6B::FF && Hq == ShapeQwen3_0_6B::HQ &&
      Hkv == ShapeQwen3_0_6B::HKV)
    return SHAPE_0_6B;
  if (D == ShapeTiny::D && FF == ShapeTiny::FF && Hq == ShapeTiny::HQ && Hkv == ShapeTiny::HKV)
    return SHAPE_TINY;
  return SHAPE_NONE;
}

Layout layout_for(ShapeId id) {
  return id == SHAPE_0_6B ? layout_of<ShapeQwen3_0_6B>() : layout_of<ShapeTiny>();
}

// The grid must be resident at once: kNT workgroups, one per CU of a kNT-CU device. Checked once
// per device and shape.
int device_check(ShapeId id, const char* fn) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return iron::fail(IRON_ERR_HIP, "%s: no current HIP device", fn);
  static int cache[64][3];  // 0 unknown, 1 ok, -1 unsupported
  if (dev < 0 || dev >= 64) return iron::fail(IRON_ERR_UNSUPPORTED, "%s: device %d", fn, dev);
  int& c = cache[dev][id];
  if (c == 0) {
    int ncu = 0, nb = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return iron::fail(IRON_ERR_HIP, "%s: cannot query the CU count", fn);
    hipError_t e = id == SHAPE_0_6B
        ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &nb, decode_persistent_kernel<ShapeQwen3_0_6B>, 256, 0)
        : hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, decode_persistent_kernel<ShapeTiny>,
                                                       256, 0);
    if (e == hipSuccess && id == SHAPE_0_6B) {
      int nt = 0;
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &nt, decode_persistent_kernel<Traced<ShapeQwen3_0_6B>>, 256, 0);
      nb = nt < nb ? nt : nb;
    }
    if (e != hipSuccess) return iron::fail(IRON_ERR_HIP, "%s: occupancy query failed", fn);
    c = (ncu == kNT && nb >= 1) ? 1 : -1;
    if (c < 0)
      return iron::fail(IRON_ERR_UNSUPPORTED,
                        "%s: needs %d CUs holding a workgroup each (device has %d CUs, %d per CU)",
                        fn, kNT, ncu, nb);
  }
  return c > 0 ? IRON_OK
               : iron::fail(IRON_ERR_UNSUPPORTED, "%s: grid cannot be resident on device %d", fn,
                            dev);
}

WireGeom geom(int K, int G, int tile_m, int domain) {
  WireGeom g;
  g.gshift = iron::ilog2(G);
  g.tile_m = tile_m;
  g.tdiv = make_fastdiv((uint32_t)tile_m);
  g.blk_bytes = (uint32_t)iron::wire_block_bytes(K, G, tile_m);
  g.xor_mask = domain == IRON_DOMAIN_BIASED ? 0x80808080u : 0u;
  return g;
}

// The tagged-word hand-off of this kernel, alone (iron_handoff_probe, IRON_HANDOFF_TAGGED):
// kNT workgroups, n_phases phases; in each, workgroup w publishes words [w per, (w + 1) per) of
// an n-word vector with put_word_copies (the kCopies copies at the spread_word layout of the x, a
// and attention-output buffers) and waits in gather_words for all n words from its XCD's copy.
// Two buffers alternate by phase, as a buffer here is rewritten by the next layer's phase.
__global__ __launch_bounds__(256, 1) void handoff_probe_tagged_kernel(unsigned long long* vec,
                                                                      uint32_t* err, int n,
                                                                      int n_phases,
                                                                      uint32_t base) {
  constexpr int NPT = iron::kHandoffMaxWords / kNT;
  __shared__ uint32_t s_in[NPT * 256];
  const int wg = blockIdx.x, per = n / kNT;
  for (int ph = 0; ph < n_phases; ++ph) {
    const uint32_t tag = base + (uint32_t)ph + 1u;
    unsigned long long* buf = vec + (size_t)(ph & 1) * kCopies * kCopyWords;
    if ((int)threadIdx.x < per)
      put_word_copies(buf + spread_word(wg * per + threadIdx.x), kCopyWords,
                      (uint32_t)(ph + wg), tag);
    unsigned long long* const mine = copy_for(buf, kCopyWords, wg);
    auto src = [&](int j, uint32_t& t) {
      t = tag;
      return mine + spread_word(j);
    };
    if (!gather_words<NPT>(n, src, [] {}, s_in, err)) return;  // workgroup-uniform
  }
}

static_assert(spread_word(iron::kHandoffMaxWords - 1) < kCopyWords, "probe vector fits a copy");

// The same exchange inside each XCD (iron_handoff_probe, IRON_HANDOFF_XCD_L2 / _XCD_AGENT): the
// kCopies groups of workgroups with equal wg % kCopies (one XCD each, as the decode kernel maps
// its KV heads) exchange n-word vectors in their own region; workgroup wg publishes words
// [(wg / kCopies) per, +per) of its group's vector, per = n * kCopies / kNT, and waits for all n.
// L2 = true: put_word_local stores and gather_pairs_local polls, the raw q/k/v and split-partial
// hand-off of the kernel; false: device-scope words (one copy), for comparison.
template <bool L2>
__global__ __launch_bounds__(256, 1) void handoff_probe_xcd_kernel(unsigned long long* vec,
                                                                   uint32_t* err, int n,
                                                                   int n_phases, uint32_t base) {
  constexpr int NPT = iron::kHandoffMaxWords / kNT;
  __shared__ uint32_t s_in[NPT * 256];
  const int wg = blockIdx.x, grp = wg % kCopies, per = n * kCopies / kNT;
  for (int ph = 0; ph < n_phases; ++ph) {
    const uint32_t tag = base + (uint32_t)ph + 1u;
    unsigned long long* buf = vec + (size_t)(ph & 1) * kCopies * kCopyWords;
    unsigned long long* mine = buf + (size_t)grp * kCopyWords;
    if ((int)threadIdx.x < per) {
      const int j = (wg / kCopies) * per + threadIdx.x;
      if constexpr (L2)
        put_word_local(xcd_local_rsrc(mine, (size_t)n), (size_t)j, (uint32_t)(ph + wg), tag);
      else
        put_word(mine + j, (uint32_t)(ph + wg), tag);
    }
    auto src = [&](int j, uint32_t& t) {
      t = tag;
      return mine + j;
    };
    bool ok;
    if constexpr (L2)
      ok = gather_pairs_local<NPT / 2, kLocalFirstPollDelay>(n, src, [] {}, s_in, err);
    else
      ok = gather_words<NPT, kLocalFirstPollDelay>(n, src, [] {}, s_in, err);
    if (!ok) return;  // workgroup-uniform
  }
}

}  // namespace

namespace iron {

size_t handoff_tagged_bytes() { return (size_t)2 * kCopies * kCopyWords * 8; }

// vec: handoff_tagged_bytes() of zero-filled (or earlier-tagged) words; err: one uint32.
int handoff_tagged_launch(void* vec, uint32_t* err, int n, int n_phases, uint32_t base,
                          hipStream_t s) {
  hipLaunchKernelGGL(handoff_probe_tagged_kernel, dim3(kNT), dim3(256), 0, s,
                     (unsigned long long*)vec, err, n, n_phases, base);
  return check_launch("iron_handoff_probe");
}

int handoff_xcd_launch(bool l2, void* vec, uint32_t* err, int n, int n_phases, uint32_t base,
                       hipStream_t s) {
  if (l2)
    hipLaunchKernelGGL(handoff_probe_xcd_kernel<true>, dim3(kNT), dim3(256), 0, s,
                       (unsigned long long*)vec, err, n, n_phases, base);
  else
    hipLaunchKernelGGL(handoff_probe_xcd_kernel<false>, dim3(kNT), dim3(256), 0, s,
                       (unsigned long long*)vec, err, n, n_phases, base);
  return check_launch("iron_handoff_probe");
}

}  // namespace iron

extern "C" {

size_t iron_decode_persistent_workspace(int D, int FF, int Hq, int Hkv, int HD) {
  const ShapeId id = shape_id(D, FF, Hq, Hkv, HD);
  return id == SHAPE_NONE ? 0 : layout_for(id).total;
}

int iron_decode_persistent_supported(int D, int FF, int Hq, int Hkv, int HD) {
  iron::clear_error();
  const char* fn = "iron_decode_persistent_supported";
  const ShapeId id = shape_id(D, FF, Hq, Hkv, HD);
  if (id == SHAPE_NONE)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: no persistent kernel for D=%d FF=%d Hq=%d "
                      "Hkv=%d HD=%d", fn, D, FF, Hq, Hkv, HD);
  return device_check(id, fn);
}

int iron_decode_persistent_check_layer(const iron_layer_desc* layer, int D, int FF, int Hq,
                                       int Hkv, int HD, int G, int tile_qkv, int tile_o,
                                       int tile_gu, int tile_d, int domain) {
  iron::clear_error();
  const char* fn = "iron_decode_persistent_check_layer";
  if (!layer) return iron::fail(IRON_ERR_NULL, "%s: null descriptor", fn);
  if (shape_id(D, FF, Hq, Hkv, HD) == SHAPE_NONE)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: unsupported shape", fn);
  const int QD = Hq * HD, MQKV = QD + 2 * Hkv * HD;
  int st;
  if ((st = iron::check_wire(fn, layer->wqkv, MQKV, D, G, tile_qkv, domain)) ||
      (st = iron::check_wire(fn, layer->wo, D, QD, G, tile_o, domain)) ||
      (st = iron::check_wire(fn, layer->wg, FF, D, G, tile_gu, domain)) ||
      (st = iron::check_wire(fn, layer->wu, FF, D, G, tile_gu, domain)) ||
      (st = iron::check_wire(fn, layer->wd, D, FF, G, tile_d, domain)))
    return st;
  if (!layer->n_in || !layer->n_post || !layer->n_qn || !layer->n_kn || !layer->k_cache ||
      !layer->v_cache)
    return iron::fail(IRON_ERR_NULL, "%s: null norm weight or cache", fn);
  if (!iron::aligned(layer->n_in, 16) || !iron::aligned(layer->n_post, 16) ||
      !iron::aligned(layer->n_qn, 16) || !iron::aligned(layer->n_kn, 16) ||
      !iron::aligned(layer->k_cache, 16) || !iron::aligned(layer->v_cache, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: norm weights and caches must be 16-byte aligned", fn);
  return IRON_OK;
}

}  // extern "C"

// The phase-stamp buffer of iron_decode_persistent_set_trace (null: launches are not traced).
static unsigned long long* g_stamps = nullptr;
static size_t g_stamp_bytes = 0;

// Both entry points: `gen` null takes the input row from x_in; otherwise from the embedding row
// of gen->keys[0]'s token, and the loop's state advances at the end (pos is then written).
static int decode_persistent(const char* fn, const iron_decode_gen* gen,
                             const iron_layer_desc* layers, int n_layers, int D, int FF, int Hq,
                             int Hkv, int HD, int max_seq, long long kv_sh, long long kv_st,
                             int G, int tile_qkv, int tile_o, int tile_gu, int tile_d, int domain,
                             const uint16_t* x_in, uint16_t* x_out, int32_t* pos,
                             uint16_t* ang, float eps, float scale, void* workspace,
                             size_t workspace_bytes, void* stream) {
  iron::clear_error();
  if (!layers || (!gen && !x_in) || !x_out || !pos || !ang)
    return iron::fail(IRON_ERR_NULL, "%s: null pointer", fn);
  if (gen) {
    if (!gen->keys || !gen->emb || !gen->tokens)
      return iron::fail(IRON_ERR_NULL, "%s: null keys, embedding table or tokens", fn);
    if (gen->vocab <= 0) return iron::fail(IRON_ERR_SHAPE, "%s: vocab=%d", fn, gen->vocab);
    if (gen->token_log && (!gen->step || gen->log_len <= 0))
      return iron::fail(IRON_ERR_NULL, "%s: token_log needs a step counter and a length", fn);
    if (!iron::aligned(gen->emb, 16) || (gen->rope_table && !iron::aligned(gen->rope_table, 16)))
      return iron::fail(IRON_ERR_ALIGN, "%s: emb and rope_table must be 16-byte aligned", fn);
    if (gen->lm_head) {
      if (!gen->lm_norm)
        return iron::fail(IRON_ERR_NULL, "%s: the folded LM head needs its norm weight", fn);
      if (!iron::aligned(gen->lm_head, 16) || !iron::aligned(gen->lm_norm, 16) ||
          !iron::aligned(gen->keys, 16))
        return iron::fail(IRON_ERR_ALIGN, "%s: lm_head, lm_norm and keys must be 16-byte "
                          "aligned", fn);
    }
  }
  const ShapeId id = shape_id(D, FF, Hq, Hkv, HD);
  if (id == SHAPE_NONE)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: no persistent kernel for D=%d FF=%d Hq=%d Hkv=%d "
                      "HD=%d", fn, D, FF, Hq, Hkv, HD);
  if (n_layers <= 0 || n_layers > kMaxLayers || max_seq <= 0)
    return iron::fail(IRON_ERR_SHAPE, "%s: n_layers=%d (at most %d) max_seq=%d", fn, n_layers,
                      kMaxLayers, max_seq);
  if (kv_st % 8 || kv_sh % 8 || kv_st < HD || kv_sh < (long long)max_seq * kv_st / 2)
    return iron::fail(IRON_ERR_SHAPE, "%s: KV strides sh=%lld st=%lld", fn, kv_sh, kv_st);
  const int QD = Hq * HD, MQKV = QD + 2 * Hkv * HD;
  if (!iron::is_pow2(G) || G < 16 || D % G || FF % G || QD % G)
    return iron::fail(IRON_ERR_SHAPE, "%s: group size %d", fn, G);
  if (tile_qkv <= 0 || MQKV % tile_qkv || tile_o <= 0 || D % tile_o || tile_gu <= 0 ||
      FF % tile_gu || tile_d <= 0 || D % tile_d)
    return iron::fail(IRON_ERR_SHAPE, "%s: row-block heights must divide the row counts", fn);
  if (domain != IRON_DOMAIN_SIGNED && domain != IRON_DOMAIN_BIASED)
    return iron::fail(IRON_ERR_SHAPE, "%s: unknown payload domain %d", fn, domain);
  if ((x_in && !iron::aligned(x_in, 16)) || !iron::aligned(x_out, 16) || !iron::aligned(ang, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: x_in, x_out and ang must be 16-byte aligned", fn);
  const Layout lo = layout_for(id);
  if (!workspace || workspace_bytes < lo.total)
    return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                      lo.total);
  if (!iron::aligned(workspace, 256))
    return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
  int st = device_check(id, fn);
  if (st) return st;
  const bool traced = g_stamps != nullptr;
  if (traced) {
    if (id != SHAPE_0_6B)
      return iron::fail(IRON_ERR_UNSUPPORTED, "%s: phase stamps exist for the Qwen3-0.6B shape "
                        "only", fn);
    const size_t need = (size_t)n_layers * kNT * kStampMarks * sizeof(unsigned long long);
    if (g_stamp_bytes < need)
      return iron::fail(IRON_ERR_WORKSPACE, "%s: stamp buffer %zu < %zu bytes for %d layers", fn,
                        g_stamp_bytes, need, n_layers);
  }
  PParams p = {};
  p.stamps = g_stamps;
  p.layers = layers;
  p.n_layers = n_layers;
  p.max_seq = max_seq;
  p.g_qkv = geom(D, G, tile_qkv, domain);
  p.g_o = geom(QD, G, tile_o, domain);
  p.g_gu = geom(D, G, tile_gu, domain);
  p.g_d = geom(FF, G, tile_d, domain);
  p.x_in = x_in;
  p.x_out = x_out;
  p.pos = pos;
  p.ang = ang;
  p.kv_sh = kv_sh;
  p.kv_st = kv_st;
  p.eps = eps;
  p.scale = (double)scale;
  char* base = (char*)workspace;
  p.ctrl = (uint32_t*)(base + lo.ctrl);
  p.X = (unsigned long long*)(base + lo.X);
  p.RAW = (unsigned long long*)(base + lo.RAW);
  p.PART = (unsigned long long*)(base + lo.PART);
  p.ATT = (unsigned long long*)(base + lo.ATT);
  p.AO = (unsigned long long*)(base + lo.AO);
  p.GH = (unsigned long long*)(base + lo.GH);
  if (gen) {
    p.key = gen->keys;
    p.emb = gen->emb;
    p.vocab = gen->vocab;
    p.log_len = gen->log_len;
    p.token = gen->tokens;
    p.token_log = gen->token_log;
    p.step = gen->step;
    p.pos_next = pos;
    p.ctx = gen->ctx;
    p.rope_table = gen->rope_table;
    p.ang_next = ang;
    p.lm_w = gen->lm_head;
    p.lm_norm = gen->lm_norm;
    p.logits = gen->logits;
  }
  hipStream_t s = (hipStream_t)stream;
  if (traced)
    hipLaunchKernelGGL(decode_persistent_kernel<Traced<ShapeQwen3_0_6B>>, dim3(kNT), dim3(256), 0,
                       s, p);
  else if (id == SHAPE_0_6B)
    hipLaunchKernelGGL(decode_persistent_kernel<ShapeQwen3_0_6B>, dim3(kNT), dim3(256), 0, s,
                       p);
  else
    hipLaunchKernelGGL(decode_persistent_kernel<ShapeTiny>, dim3(kNT), dim3(256), 0, s, p);
  return iron::check_launch(fn);
}

extern "C" {

int iron_decode_persistent(const iron_layer_desc* layers, int n_layers, int D, int FF, int Hq,
                           int Hkv, int HD, int max_seq, long long kv_sh, long long kv_st, int G,
                           int tile_qkv, int tile_o, int tile_gu, int tile_d, int domain,
                           const uint16_t* x_in, uint16_t* x_out, const int32_t* pos,
                           const uint16_t* ang, float eps, float scale, void* workspace,
                           size_t workspace_bytes, void* stream) {
  // without `gen` the kernel only reads pos and ang
  return decode_persistent("iron_decode_persistent", nullptr, layers, n_layers, D, FF, Hq, Hkv,
                           HD, max_seq, kv_sh, kv_st, G, tile_qkv, tile_o, tile_gu, tile_d,
                           domain, x_in, x_out, const_cast<int32_t*>(pos),
                           const_cast<uint16_t*>(ang), eps, scale, workspace, workspace_bytes,
                           stream);
}

int iron_decode_persistent_set_trace(unsigned long long* stamps, size_t stamp_bytes) {
  iron::clear_error();
  if (stamps && !iron::aligned(stamps, 8))
    return iron::fail(IRON_ERR_ALIGN, "iron_decode_persistent_set_trace: stamps not 8-byte "
                      "aligned");
  g_stamps = stamps;
  g_stamp_bytes = stamps ? stamp_bytes : 0;
  return IRON_OK;
}

int iron_decode_persistent_gen(const iron_layer_desc* layers, int n_layers, int D, int FF,
                               int Hq, int Hkv, int HD, int max_seq, long long kv_sh,
                               long long kv_st, int G, int tile_qkv, int tile_o, int tile_gu,
                               int tile_d, int domain, const iron_decode_gen* gen,
                               uint16_t* x_out, int32_t* pos, uint16_t* ang, float eps,
                               float scale, void* workspace, size_t workspace_bytes,
                               void* stream) {
  iron::clear_error();
  if (!gen) return iron::fail(IRON_ERR_NULL, "iron_decode_persistent_gen: null gen");
  return decode_persistent("iron_decode_persistent_gen", gen, layers, n_layers, D, FF, Hq, Hkv,
                           HD, max_seq, kv_sh, kv_st, G, tile_qkv, tile_o, tile_gu, tile_d,
                           domain, nullptr, x_out, pos, ang, eps, scale, workspace,
                           workspace_bytes, stream);
}

}  // extern "C"
