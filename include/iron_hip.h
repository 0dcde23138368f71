/* iron_hip.h -- C ABI of the MI355X (gfx950) Qwen3 int8 decode hot path.
 *
 * Every entry point is stream-ordered and asynchronous: it validates its arguments on the host,
 * launches HIP kernels on `stream` (a hipStream_t passed as void*, NULL = the null stream) and
 * returns. Device memory is always owned by the caller; the library never allocates. Entry points
 * that need scratch memory take a caller-provided workspace and export a size query.
 * Workspaces are zero-filled once before their first use. The entry points that can run the
 * batched MFMA GEMM (iron_gemm_w8a16, iron_qkv_head, iron_qkv_attn, iron_swiglu_mlp) keep its
 * split-K arrival counters in the first 16 KiB of their workspace, for every batch size, and
 * leave them zero after each call; a workspace serves one of these entry points (any B), and
 * calls on one workspace are stream-ordered.
 *
 * Return value: IRON_OK (0) or a negative iron_status; iron_last_error() then returns a
 * thread-local message. Validation errors (IRON_ERR_NULL/SHAPE/ALIGN/WORKSPACE/UNSUPPORTED) are
 * raised before any HIP call is made.
 *
 * Data conventions: bf16 tensors are uint16_t bit patterns; int8 weights travel in the reference's
 * row-block wire (iron/operators/gemv_int8/reference.py:59-80): consecutive blocks of `tile_m`
 * rows, each = tile_m*K payload bytes then tile_m*(K/G) bf16 scales. `domain` selects the payload
 * encoding: IRON_DOMAIN_SIGNED (two's-complement q, aie_kernels/aie2p/mv_int8_signed.cc) or
 * IRON_DOMAIN_BIASED (q+128, aie_kernels/aie2p/mv_int8.cc).
 */
#ifndef IRON_HIP_H
#define IRON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IRON_ABI_VERSION 11

enum iron_status {
  IRON_OK = 0,
  IRON_ERR_NULL = -1,        /* a required pointer is NULL */
  IRON_ERR_SHAPE = -2,       /* a shape / geometry constraint is violated */
  IRON_ERR_ALIGN = -3,       /* a pointer or wire block is misaligned */
  IRON_ERR_WORKSPACE = -4,   /* workspace missing or too small */
  IRON_ERR_HIP = -5,         /* a HIP call or kernel launch failed */
  IRON_ERR_UNSUPPORTED = -6  /* valid but not implemented for these sizes */
};

enum iron_domain { IRON_DOMAIN_SIGNED = 0, IRON_DOMAIN_BIASED = 1 };
enum iron_weight_kind { IRON_WEIGHT_INT8 = 0, IRON_WEIGHT_BF16 = 1 };
/* Accumulation of the decode-attention core (scores, softmax, P.V):
 *   IRON_ACCUM_F64 -- the exact value of the golden, evaluated in fp64 and rounded once to bf16
 *                     (bit-identical to the fp64 oracle);
 *   IRON_ACCUM_F32 -- the arithmetic the reference kernel uses: bf16 operands, fp32 dot products,
 *                     exp2-form softmax and accumulation (within 1 bf16 ulp of the exact value on
 *                     the parity cases; the contract is rel/abs 1e-2). */
enum iron_accum { IRON_ACCUM_F64 = 0, IRON_ACCUM_F32 = 1 };
/* RoPE pairing (rope/op.py method_type): dims (i, i + cols/2), or (2i, 2i + 1). */
enum iron_rope_method { IRON_ROPE_TWO_HALVES = 0, IRON_ROPE_INTERLEAVED = 1 };

/* ABI version of the loaded library (IRON_ABI_VERSION). No reference counterpart. */
int iron_abi_version(void);

/* Message of the last failing call on this thread ("" if none). No reference counterpart. */
const char* iron_last_error(void);

/* Host-only: bytes of an int8 wire of M x K with group G and row-block tile_m.
 * Replaces the wire sizing in GEMVInt8.get_arg_spec (iron/operators/gemv_int8/op.py:151-171). */
int iron_wire_bytes(int M, int K, int G, int tile_m, size_t* out_bytes);

/* Bit-exact dequant w[m][k] = bf16(q[m][k] * s[m][k/G]) into a row-major bf16 [M][K].
 * Replaces the host dequant of SwiGLUMLPDataParallelOurs._dequant_tiles
 * (iron/operators/swiglu_mlp_dp/op_ours.py:515-541) and _payload_to_q (op_ours.py:31-43). */
int iron_dequant_w8(const void* wire, uint16_t* w_out, int M, int K, int G, int tile_m,
                    int domain, void* stream);

/* y[b][m] = bf16(sum_k dequant(W)[m][k] * x[b][k]), B in [1,4]. The sum is accumulated in fp64
 * and rounded once, so y is the correctly rounded bf16 of the exact dot product.
 * Replaces GEMVInt8's callable (iron/operators/gemv_int8/op.py:20-178; kernel
 * aie_kernels/aie2p/mv_int8_signed.cc:60-113). x: [B][K] bf16, y: [B][M] bf16. */
int iron_gemv_w8a16(const void* wire, const uint16_t* x, uint16_t* y, int B, int M, int K, int G,
                    int tile_m, int domain, void* stream);

/* y[b][m] = bf16(sum_k W[m][k] * x[b][k]) for bf16 row-major W [M][K], B in [1,4].
 * Replaces the bf16 GEMV (iron/operators/gemv/op.py) used for a bf16 LM head. */
int iron_gemv_bf16(const uint16_t* w, const uint16_t* x, uint16_t* y, int B, int M, int K,
                   void* stream);

/* Workspace bytes for iron_gemm_w8a16 (MFMA split-K partials; 256 when none are needed). */
size_t iron_gemm_w8a16_workspace(int B, int M, int K, int G);

/* Batched decode GEMM on MFMA: y[b][m] = bf16(sum_g s[m][g] * sum_{k in g} q[m][k] x[b][k]) for
 * B in [1,16] (the batch sizes above the GEMV path), M % 64 == 0, K % 128 == 0, G in {32,64,128}.
 * q is exact in bf16, each 32-wide k step is one v_mfma_f32_16x16x32_bf16 (fp32 sums of exact
 * products), and the group scales apply in fp64; x: [B][K] bf16, y: [B][M] bf16. No reference
 * counterpart (the reference has a bf16 GEMM operator, iron/operators/gemm/op.py:23-80, golden
 * gemm/reference.py:8-19, and the int8 GEMV golden gemv_int8/op.py:173-178 it generalises). */
int iron_gemm_w8a16(const void* wire, const uint16_t* x, uint16_t* y, int B, int M, int K, int G,
                    int tile_m, int domain, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Weighted RMSNorm y[r][c] = bf16(x[r][c] * rsqrt(mean_c(x^2) + eps) * w[c]).
 * Replaces RMSNorm (iron/operators/rms_norm/op.py:21-130; kernel rms_norm.cc:83-147). */
int iron_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows, int cols, float eps,
                 void* stream);

/* RoPE of bf16 rows: y = bf16(x_a cos_i - x_b sin_i), bf16(x_b cos_i + x_a sin_i) for each pair
 * (a, b) of `method` (IRON_ROPE_TWO_HALVES: (i, i + cols/2); IRON_ROPE_INTERLEAVED: (2i, 2i + 1)),
 * i < cols/2, each output exact before its one rounding. angles: [angle_rows][cols] interleaved
 * [cos_i, sin_i] rows; row r uses angle row r / (rows / angle_rows). cols even, angle_rows divides
 * rows. Replaces RoPE (iron/operators/rope/op.py:19-96; kernel aie_kernels/generic/rope.cc,
 * golden rope/reference.py:118-154). */
int iron_rope(const uint16_t* x, const uint16_t* angles, uint16_t* y, int rows, int cols,
              int angle_rows, int method, void* stream);

/* Fused QK RMSNorm + RoPE + V copy of one decode QKV vector. qkv_in / qkv_out: bf16
 * [Q (n_qk_heads - n_v_heads) | K (n_v_heads) | V (n_v_heads)] heads of head_dim; scratch: bf16
 * [gamma (n_qk_heads x head_dim) | cos (head_dim) | sin (head_dim)]. Q and K head h:
 * y = bf16(x / sqrt(mean(x^2) + eps) * gamma_h), then out_d = bf16(y_d cos_d - y_{d+m} sin_d)
 * for d < m = head_dim/2 and bf16(y_d cos_d + y_{d-m} sin_d) above; V heads are copied. With
 * kv_cache != NULL (the reference's kv_direct) the K heads' outputs and the V heads also go to
 * the head-major cache [n_v_heads][max_seq][K_t | V_t] at the element offset *kv_offset (device
 * int32, t * 2 * head_dim): head j's K at j * 2 * max_seq * head_dim + *kv_offset, its V
 * head_dim later; an offset outside the cache writes nothing there. head_dim even and <= 1024.
 * Replaces QKNormRoPE (iron/operators/qk_norm_rope/op.py:20-117; kernels
 * aie_kernels/aie2p/qk_norm_rope.cc, qk_norm_rope_kv.cc; golden qk_norm_rope/reference.py:19-40,
 * which rounds once at the end where the kernel rounds the normalised head first, as here). */
int iron_qk_norm_rope(const uint16_t* qkv_in, const uint16_t* scratch, uint16_t* qkv_out,
                      uint16_t* kv_cache, const int32_t* kv_offset, int head_dim, int n_qk_heads,
                      int n_v_heads, int max_seq, float eps, void* stream);

/* LM head: logits[b][v] = bf16(W[v] . xn[b]) with xn = bf16(RMSNorm(x[b]) * norm_w) when
 * norm_w != NULL (else xn = x), W int8 wire (w_kind IRON_WEIGHT_INT8) or bf16 [V][D]
 * (IRON_WEIGHT_BF16). When argmax_keys != NULL it must be zeroed before the call; on return
 * argmax_keys[b] holds (order(bf16 max) << 32) | ~index, the first maximal index on ties.
 * Replaces the final RMSNorm + GEMVInt8 LM head + host argmax of Qwen3NPU
 * (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:278-281, 612-621). */
int iron_lm_head(const void* w, int w_kind, const uint16_t* x, const uint16_t* norm_w, float eps,
                 uint16_t* logits, unsigned long long* argmax_keys, int B, int V, int D, int G,
                 int tile_m, int domain, void* stream);

/* Decode the token id from an argmax key written by iron_lm_head, on the device:
 * tokens[b] = index of keys[b]; then keys[b] = 0 (ready for the next iron_lm_head).
 * If `emb` != NULL also gathers x[b][:] = emb[tokens[b]][:] (bf16 [vocab][D]) and, when
 * `token_log` != NULL, writes tokens[b] to token_log[b * log_stride + *step] if *step < log_len
 * (a row of the log holds log_len entries) and increments *step (device int32) either way.
 * Replaces the host argmax + embedding lookup of the reference decode loop
 * (qwen3_npu_int8.py:612-621; check_cosine_int8.py:41-52). */
int iron_next_token(unsigned long long* keys, int32_t* tokens, const uint16_t* emb, uint16_t* x,
                    int32_t* token_log, int log_stride, int log_len, int32_t* step, int B, int D,
                    int vocab, void* stream);

/* Embedding gather x[b][:] = emb[tokens[b]][:] (tokens device int32 [B]). */
int iron_embed(const int32_t* tokens, const uint16_t* emb, uint16_t* x, int B, int D, int vocab,
               void* stream);

/* Device-side decode position advance, per row b: pos[b] += delta and ctx[b] = pos[b] + 1
 * (either pointer may be NULL; with pos NULL the position is ctx[b] - 1). When `table` is not
 * NULL it also copies the RoPE angle row of the new position, ang_rows[b][:] = table[pos[b]][:]
 * (bf16 [max_pos][HD] -> [B][HD]; positions outside [0, max_pos) leave the row unchanged).
 * Replaces the host writes of k_cache_offset / S_kv_eff and of the angle row before each
 * dispatch (qwen3_npu_int8.py:580-591, 598-610), so a captured per-token HIP graph replays
 * without host work. */
int iron_advance_positions(int32_t* pos, int32_t* ctx, const uint16_t* table,
                           uint16_t* ang_rows, int HD, int max_pos, int B, int delta,
                           void* stream);

/* Workspace bytes for iron_qkv_head (raw QKV staging; for B > 4 also the normalised input and
 * the MFMA split-K partials). */
size_t iron_qkv_head_workspace(int B, int D, int Hq, int Hkv, int HD);

/* Fused decode QKV head, per batch row b:
 *   hn  = bf16(RMSNorm(cur[b]) * n_in)                                (rms_norm.cc:83-147)
 *   raw = bf16(Wqkv . hn)          Wqkv rows = [Hq*HD | Hkv*HD | Hkv*HD] int8 wire, K = D
 *   q   = bf16(RoPE(bf16(RMSNorm_head(raw_q) * n_qn), ang))  -> q_out[b][Hq*HD]
 *   k   = bf16(RoPE(bf16(RMSNorm_head(raw_k) * n_kn), ang))  -> k cache at position pos[b]
 *   v   = raw_v                                              -> v cache at position pos[b]
 * ang: interleaved [cos_i, sin_i] bf16 rows of HD elements; row b is at ang + b*HD, or at
 * ang + pos[b]*HD when ang_by_pos != 0 (a whole angle table). KV cache addressing (elements):
 * k_cache + b*kv_sb + h*kv_sh + pos*kv_st (same for v_cache), so both the separate [B,Hkv,S,HD]
 * layout and the reference's token-interleaved [Hkv][S][K_t|V_t] layout are expressible.
 * Replaces QKVHeadDataParallelOurs (iron/operators/qkv_head_dp/op_ours.py:31-262, op.py:20-231;
 * golden qkv_head_dp/reference.py:13-33). */
int iron_qkv_head(const uint16_t* cur, const uint16_t* n_in, const void* wqkv,
                  const uint16_t* n_qn, const uint16_t* n_kn, const uint16_t* ang, int ang_by_pos,
                  uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, long long kv_sb,
                  long long kv_sh, long long kv_st, const int32_t* pos, int B, int D, int HD,
                  int Hq, int Hkv, int max_seq, int G, int tile_m, int domain, float eps,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for iron_decode_attn (the in-kernel merge's arrival counters, then the split-K
 * partials, sized for either accumulation mode). The first 16 KiB must be zero before the first
 * call (a zero-filled workspace); every call leaves them zero, so one workspace serves every later
 * call on the same stream. */
size_t iron_decode_attn_workspace(int B, int H, int KV, int D, int max_ctx);

/* GQA decode attention, one query token per sequence:
 *   o[b][h] = softmax_j(q[b][h] . K[b][h*KV/H][j] * scale) . V[b][h*KV/H][j],  j < ctx_len[b]
 * with the scores / softmax / accumulation of `acc` (enum iron_accum: exact fp64, or the fp32
 * exp2 form of decode_attn.cc:117-311), rounded once to bf16 output; a sequence
 * with ctx_len 0 yields zeros (decode_attn.cc:300-311). q/o: [B][H][D] bf16; K/V addressed as in
 * iron_qkv_head. ctx_len: device int32 [B] (or NULL: every sequence uses ctx_const).
 * Replaces DecodeAttention (iron/operators/decode_attn/op.py:20-181; golden
 * decode_attn/reference.py:26-38). */
int iron_decode_attn(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                     long long kv_sb, long long kv_sh, long long kv_st, const int32_t* ctx_len,
                     int ctx_const, uint16_t* out, int B, int H, int KV, int D, int max_ctx,
                     float scale, int acc, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Bytes of the library-owned scratch array that iron_decode_attn_noalloc uses on each GPU. */
#define IRON_ATTN_NOALLOC_SCRATCH_BYTES (4u << 20)

/* iron_decode_attn without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, allocator-free serving loops, harnesses that forbid hipMalloc).
 * No reference counterpart. The split-K partials go to a file-scope device array of
 * IRON_ATTN_NOALLOC_SCRATCH_BYTES held by each GPU until the process ends; the entry point calls
 * no allocating routine, and returns IRON_ERR_WORKSPACE when the partials of (B, H, max_ctx) would
 * not fit (iron_decode_attn_workspace() > the scratch). Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, or threads without ordering) race and
 * must be serialised by the caller. Results equal iron_decode_attn's bit for bit. */
int iron_decode_attn_noalloc(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                             long long kv_sb, long long kv_sh, long long kv_st,
                             const int32_t* ctx_len, int ctx_const, uint16_t* out, int B, int H,
                             int KV, int D, int max_ctx, float scale, int acc, void* stream);

/* Workspace bytes for iron_decode_attn_verify (split-K partials, fp32; 256 when none are needed;
 * 0 for an invalid shape). */
size_t iron_decode_attn_verify_workspace(int n_new, int H, int KV, int D, int max_ctx);

/* Batch / verify decode attention (speculative-decode verify): n_new new tokens at positions
 * base .. base + n_new - 1 query ONE KV cache (K/V addressed as in iron_qkv_head, batch 1):
 *   o[t][h] = softmax_j(q[t][h] . K[h*KV/H][j] * scale) . V[h*KV/H][j],
 *             j < min(base + t + 1, max_ctx) when causal, j < max_ctx otherwise.
 * q/o: [n_new][H][D] bf16, token-major (row t * H + h). base: device int32 (the S_kv_base runtime
 * parameter), or NULL to use base_const. Arithmetic of the reference kernel: bf16 operands, fp32
 * scores and exp2-form online softmax, probabilities rounded to bf16 for P.V, fp32 accumulation
 * (MFMA); each staged 64-key K/V block serves up to 64 query rows (64 / (H/KV) tokens).
 * n_new <= 4096. Replaces DecodeAttention's batch mode (iron/operators/decode_attn/op.py:40-48;
 * design.py:243-276, per-query bound S_kv_base + g*M + m + 1; causal=False attends the whole
 * cache). */
int iron_decode_attn_verify(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                            long long kv_sh, long long kv_st, const int32_t* base,
                            int base_const, int causal, uint16_t* out, int n_new, int H, int KV,
                            int D, int max_ctx, float scale, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Workspace bytes for iron_qkv_attn (raw QKV staging + the attention's merge counters and split-K
 * partials). Zero-filled before the first call; every call leaves the counters zero. */
size_t iron_qkv_attn_workspace(int B, int D, int Hq, int Hkv, int HD, int max_seq);

/* Fused QKV head + decode attention for one decode step, per batch row b (ctx = pos[b] + 1):
 *   q, k, v  exactly as iron_qkv_head computes them (the k and v rows are appended to the caches
 *            at pos[b]; q is consumed in registers and not written out)
 *   out[b]   exactly as iron_decode_attn computes it (same `acc`) over positions 0..pos[b] with
 *            ctx_len = pos + 1
 * i.e. the composition of iron_qkv_head and iron_decode_attn with the per-head epilogue moved
 * into the attention kernel (two launches plus the split merge instead of four). out: [B][Hq][HD].
 * ang holds one angle row per batch row ([B][HD], the position's row; no table lookup).
 * Replaces the QKVHeadDataParallelOurs -> DecodeAttention pair of the reference runlist
 * (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:249-281; qkv_head_dp/op_ours.py:31-262,
 * decode_attn/op.py:20-181). */
int iron_qkv_attn(const uint16_t* cur, const uint16_t* n_in, const void* wqkv,
                  const uint16_t* n_qn, const uint16_t* n_kn, const uint16_t* ang,
                  uint16_t* k_cache, uint16_t* v_cache, long long kv_sb, long long kv_sh,
                  long long kv_st, const int32_t* pos, uint16_t* out, int B, int D, int HD, int Hq,
                  int Hkv, int max_seq, int G, int tile_m, int domain, float eps, float scale,
                  int acc, void* workspace, size_t workspace_bytes, void* stream);

/* Causal prefill attention (GQA) on MFMA:
 *   o[b][h][i] = sum_{j <= i} softmax_j(q[b][h][i] . k[b][h*KV/H][j] * scale) v[b][h*KV/H][j]
 * q/o: [B][H][S][D] bf16, k/v: [B][KV][S][D] bf16, D in {64, 128}, S a multiple of 64 (the
 * reference pads to 64), H/KV in {1, 2} or a multiple of 4. Scores, softmax and accumulation in
 * fp32 (bf16 MFMAs), probabilities rounded to bf16 for the P.V product, bf16 output.
 * Replaces MHA (iron/operators/mha/op.py:20-153; golden mha/reference.py:27-94, causal SDPA). */
int iron_prefill_attn(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int B,
                      int H, int KV, int S, int D, float scale, void* stream);

/* Workspace bytes for iron_swiglu_mlp (x1 residual halves + gh, fp32). */
size_t iron_swiglu_mlp_workspace(int B, int D, int FF);

/* Fused decode SwiGLU MLP block, per batch row b:
 *   a   = bf16(Wo . cx[b])   when wo != NULL (fuse_o; cx [B][QD]), else a = a_in[b] ([B][D])
 *   x1  = cur[b] + a                                      (fp32)
 *   hf  = RMSNorm(x1) * n_pf                              (fp32)
 *   gh  = silu(Wg . hf) * (Wu . hf)                       (fp32)
 *   nxt = bf16(x1 + Wd . gh)
 * Wo: [D][QD] wire (tile_m_o rows), Wg/Wu: [FF][D] wires (tile_m_gu), Wd: [D][FF] (tile_m_d).
 * a_out (optional, [B][D] bf16) receives a. B <= 4 runs the fused GEMV kernels; B in [5,16] runs
 * the prologue once per row and the three products on MFMA (fp32 hf and gh enter the MFMA as
 * three exact bf16 planes, hi + mid + lo). Replaces SwiGLUMLPDataParallelOurs
 * (iron/operators/swiglu_mlp_dp/op_ours.py:46-582, op.py:22-227; golden
 * swiglu_mlp_dp/reference.py:8-67). */
int iron_swiglu_mlp(const uint16_t* cur, const uint16_t* cx_or_a, const uint16_t* n_pf,
                    const void* wo, const void* wg, const void* wu, const void* wd,
                    uint16_t* nxt, uint16_t* a_out, int B, int D, int FF, int QD, int G,
                    int tile_m_o, int tile_m_gu, int tile_m_d, int domain, float eps,
                    void* workspace, size_t workspace_bytes, void* stream);

/* One decoder layer's device pointers for iron_decode_persistent (a device array of these, one per
 * layer). Wires as in iron_qkv_attn / iron_swiglu_mlp: wqkv [Hq*HD + 2*Hkv*HD][D], wo [D][Hq*HD],
 * wg and wu [FF][D], wd [D][FF]; norm weights bf16 (n_in, n_post [D]; n_qn, n_kn [HD]); the
 * layer's K and V caches for batch 1 ([Hkv][max_seq][HD] through the kv_sh / kv_st strides).
 * Mirrors the per-layer buffer names of the reference runlist (W_norm1_i, W_qkv_i, W_qn_i, W_kn_i,
 * W_norm2_i, Wo_i, Wg_i, Wu_i, Wd_i and the layer's caches; qwen3_npu_int8.py:249-281). */
typedef struct iron_layer_desc {
  const void* wqkv;
  const void* wo;
  const void* wg;
  const void* wu;
  const void* wd;
  const uint16_t* n_in;
  const uint16_t* n_post;
  const uint16_t* n_qn;
  const uint16_t* n_kn;
  uint16_t* k_cache;
  uint16_t* v_cache;
} iron_layer_desc;

/* Workspace bytes for iron_decode_persistent (0 if no kernel exists for the shape). The workspace
 * holds the tagged hand-off words and two control words: uint32 [0] = epoch, [1] = error flags
 * (nonzero after a hand-off wait timed out). It must be zero-filled once before its first use
 * and then kept for the lifetime of the decode state. */
size_t iron_decode_persistent_workspace(int D, int FF, int Hq, int Hkv, int HD);

/* IRON_OK if iron_decode_persistent has a kernel for this shape and the current device can hold
 * its grid resident (256 CUs, one 256-thread workgroup per CU); else IRON_ERR_UNSUPPORTED. Shapes:
 * D, FF, Hq, Hkv = (1024, 3072, 16, 8) (Qwen3-0.6B) and (256, 768, 4, 2); HD = 128. */
int iron_decode_persistent_supported(int D, int FF, int Hq, int Hkv, int HD);

/* Host-only validation of one layer descriptor (a host copy of what the device array holds): wire
 * geometry and alignment as the standalone entry points check them. */
int iron_decode_persistent_check_layer(const iron_layer_desc* layer, int D, int FF, int Hq,
                                       int Hkv, int HD, int G, int tile_qkv, int tile_o,
                                       int tile_gu, int tile_d, int domain);

/* Whole-token decode of n_layers Qwen3 layers at batch 1 in one persistent kernel:
 *   x = x_in; for each layer i (layers[i], a device array):
 *     out = iron_qkv_attn(x, ...)            (QKV head at position *pos, K/V appended, attention
 *                                              over positions 0..*pos, exact fp64 core)
 *     x   = iron_swiglu_mlp(x, out, ...)     (fuse_o: Wo, residual, RMSNorm, SwiGLU, down)
 *   x_out = x.
 * The results equal those of the per-operator entry points (same arithmetic and roundings).
 * pos: device int32 [1]; ang: the position's RoPE row (bf16 [HD]); kv_sh / kv_st: head and token
 * strides of the caches in elements. Launches 256 workgroups (one per CU) that exchange activations
 * through the workspace: calls on one workspace must be stream-ordered, and the workspace's error word must be
 * checked (and cleared) by the caller after synchronising. Replaces the per-token runlist dispatch
 * of Qwen3NPU (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:249-281, 594-621; one dispatch of
 * iron/common/sequence.py:270-559) for the layers; the final RMSNorm and LM head follow it
 * (iron_lm_head). */
int iron_decode_persistent(const iron_layer_desc* layers, int n_layers, int D, int FF, int Hq,
                           int Hkv, int HD, int max_seq, long long kv_sh, long long kv_st, int G,
                           int tile_qkv, int tile_o, int tile_gu, int tile_d, int domain,
                           const uint16_t* x_in, uint16_t* x_out, const int32_t* pos,
                           const uint16_t* ang, float eps, float scale, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Device state of a greedy decode loop run by iron_decode_persistent_gen. */
typedef struct iron_decode_gen {
  unsigned long long* keys;   /* argmax keys: [1] the previous iron_lm_head's, reset to 0; or,
                                 with lm_head, [2] slots the launches alternate between */
  const uint16_t* emb;        /* bf16 [vocab][D] embedding table (16-byte aligned) */
  int32_t* tokens;            /* [1] receives the decoded token */
  int32_t* token_log;         /* [log_len] token by step, or NULL */
  int32_t* step;              /* [1] step counter, incremented (needed with token_log) */
  int32_t* ctx;               /* [1] receives the new position + 1, or NULL */
  const uint16_t* rope_table; /* bf16 [max_seq][HD] RoPE rows, or NULL */
  int vocab, log_len;
  const uint16_t* lm_head;    /* bf16 [vocab][D]: fold the final RMSNorm, LM head and argmax into
                                 the launch (NULL: the layers only) */
  const uint16_t* lm_norm;    /* bf16 [D] final RMSNorm weight (with lm_head) */
  uint16_t* logits;           /* bf16 [vocab] logits out (with lm_head), or NULL */
} iron_decode_gen;

/* iron_decode_persistent with the greedy loop's per-token work folded in:
 *   token = the index of gen->keys[0] (0 for a zero key, clamped to [0, vocab)); x_in is
 *   emb[token]; the layers run as in iron_decode_persistent; then keys[0] = 0, tokens[0] = token,
 *   token_log[*step] = token (when *step < log_len), *step += 1, *pos += 1, ctx[0] = *pos + 1 and
 *   ang = rope_table[*pos] (when *pos < max_seq).
 * The results equal iron_next_token (emb, log) + iron_decode_persistent + iron_advance_positions
 * (delta 1), the per-token loop of the reference decode (qwen3_npu_int8.py:594-621) in one
 * launch. With gen->lm_head the launch also runs the final RMSNorm (lm_norm), the bf16 LM head
 * (logits) and its argmax, i.e. iron_lm_head as well: a whole greedy step in ONE launch, the
 * reference's single dispatch per token with its host argmax (qwen3_npu_int8.py:249-281,
 * 612-621). The keys then alternate by epoch e (workspace control word 0 at launch): the launch
 * reads the previous token from keys[e & 1], clears keys[(e + 1) & 1] and leaves its argmax there
 * (so after a launch the latest key is keys[epoch & 1] with the advanced epoch). */
int iron_decode_persistent_gen(const iron_layer_desc* layers, int n_layers, int D, int FF,
                               int Hq, int Hkv, int HD, int max_seq, long long kv_sh,
                               long long kv_st, int G, int tile_qkv, int tile_o, int tile_gu,
                               int tile_d, int domain, const iron_decode_gen* gen,
                               uint16_t* x_out, int32_t* pos, uint16_t* ang, float eps,
                               float scale, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Host-only check of the device-side divide used for wire row-blocks: returns n / d computed with
 * the same multiply-shift sequence the kernels use (test hook; no reference counterpart). */
uint32_t iron_test_fastdiv(uint32_t n, uint32_t d);

/* Device check of the bf16 rounding every kernel uses (test hook; no reference counterpart). The
 * caller zero-fills out[0] and out[2] and sets out[1] = 0xffffffff; after the stream synchronises,
 * out[0] = number of fp32 bit patterns whose hardware round-to-nearest-even bf16 differs from the
 * integer form (NaN inputs: a non-NaN result), out[1] = the smallest such pattern, out[2] = the
 * bf16 of the fp64 value 1 + 2^-8 + 2^-40, which is 0x3f80 when fp64 values round to fp32 and
 * then to bf16 (as torch does), 0x3f81 if they were rounded once. */
int iron_test_bf16_round(uint32_t* out, void* stream);

/* Measurement hook (no reference counterpart): streams `bytes` (a multiple of 16, 16-byte aligned)
 * through 16-byte loads, workgroup b of `blocks` (x 256 threads) reading the b-th contiguous
 * 1/blocks of the buffer, and writes one xor word per thread to out[blocks * 256]. Its time is
 * the achievable HBM read rate that the roofline figures are read against. */
int iron_stream_read(const void* p, size_t bytes, uint32_t* out, int blocks, void* stream);

/* Measurement hook (no reference counterpart): phase timestamps of the persistent decode kernel.
 * While a buffer is set, iron_decode_persistent and iron_decode_persistent_gen launch a copy of
 * the Qwen3-0.6B kernel (the other shape is rejected with IRON_ERR_UNSUPPORTED) that writes, per
 * layer l and workgroup w, 16 readings of the 100 MHz constant clock to
 * stamps[(l * 256 + w) * 16 + mark]: 0 QKV phase entry, 1 its input gathered, 2 its rows stored;
 * 3 attention input gathered, 4 QK-norm/RoPE done, 15 attention tiles done, 5 partials stored;
 * 6 merge input gathered, 7 outputs stored; 8 Wo input gathered, 9 rows stored; 10 gate/up input
 * gathered, 11 its RMSNorm prologue done, 12 gh stored; 13 down input gathered, 14 rows stored.
 * stamp_bytes must cover n_layers * 256 * 16 * 8 bytes (IRON_ERR_WORKSPACE otherwise). Results
 * are those of the untraced kernel. NULL stops tracing. Process-wide, not thread-safe. */
int iron_decode_persistent_set_trace(unsigned long long* stamps, size_t stamp_bytes);

/* Measurement hook (no reference counterpart): the grid-wide hand-off a persistent kernel needs
 * between phases, timed alone. 256 workgroups of 256 threads (one per CU; the device needs 256
 * CUs) run n_phases phases; in each, every workgroup publishes its n_words / 256 words of an
 * n_words vector (a multiple of 256, at most 2048; 32 for the XCD modes) and waits until it has
 * every workgroup's:
 *   IRON_HANDOFF_TAGGED  -- the persistent decode kernel's own hand-off code: 64-bit
 *                           {tag, payload} words stored in 8 copies, polled from one copy;
 *   IRON_HANDOFF_COUNTER -- one atomic arrival counter polled to the grid size (no vector);
 *   IRON_HANDOFF_FLAGS   -- plain stores, device-scope fences and one flag per workgroup;
 *   IRON_HANDOFF_XCD_L2  -- the decode kernel's XCD-local hand-off: the 32 workgroups with equal
 *                           index mod 8 (one XCD) exchange their own n_words vector through that
 *                           XCD's L2 (sc0 stores, nt polls), 8 groups at once;
 *   IRON_HANDOFF_XCD_AGENT -- the same groups with device-scope words.
 * Phase p of a launch uses tag base + p + 1: successive launches on one workspace pass distinct
 * bases. The workspace (iron_handoff_probe_workspace bytes) is zero-filled before the first
 * launch, and again before each IRON_HANDOFF_COUNTER launch (its counter starts at zero). Every
 * wait is bounded: after the stream synchronises, a nonzero uint32 at byte
 * iron_handoff_probe_workspace(n_words) - 4096 + 256 of the workspace means a wait gave up. */
enum iron_handoff_mode {
  IRON_HANDOFF_TAGGED = 0,
  IRON_HANDOFF_COUNTER = 1,
  IRON_HANDOFF_FLAGS = 2,
  IRON_HANDOFF_XCD_L2 = 3,
  IRON_HANDOFF_XCD_AGENT = 4
};
size_t iron_handoff_probe_workspace(int n_words);
int iron_handoff_probe(int mode, int n_words, int n_phases, unsigned int base, void* workspace,
                       size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* IRON_HIP_H */
