/* C restatement of the reference's byte/integer arithmetic for the Qwen3 int8 decode path.
 * TEST INFRASTRUCTURE: built into oracle/liboracle.so and used only by tests (as an independent
 * second witness for the torch oracle) -- never by the product.
 *
 *   oracle_wire_unpack  -- row-block wire parse (iron/operators/gemv_int8/reference.py:59-80)
 *   oracle_dequant      -- bf16(q * s), RNE done with integer bit operations
 *                          (qwen3_npu_int8.py:350-379, swiglu_mlp_dp/op_ours.py:31-43)
 *   oracle_gemv_f64     -- sum_g s * sum_k q * x in double (every term exact)
 *                          (iron/operators/gemv_int8/op.py:173-178)
 *   oracle_decode_attn_f64 -- softmax attention in double with explicit loops
 *                          (iron/operators/decode_attn/reference.py:26-38)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

/* wire -> q (int16, row-major M x K) and s (bf16 bits, M x K/G). domain 0 signed, 1 biased. */
int oracle_wire_unpack(const uint8_t* wire, int M, int K, int G, int tile_m, int domain,
                       int16_t* q, uint16_t* s) {
  if (M <= 0 || K <= 0 || G <= 0 || tile_m <= 0 || K % G || M % tile_m) return -1;
  const int ng = K / G;
  const size_t blk = (size_t)tile_m * K + (size_t)tile_m * ng * 2;
  for (int b = 0; b < M / tile_m; ++b) {
    const uint8_t* base = wire + (size_t)b * blk;
    for (int r = 0; r < tile_m; ++r) {
      const int row = b * tile_m + r;
      for (int k = 0; k < K; ++k) {
        uint8_t byte = base[(size_t)r * K + k];
        q[(size_t)row * K + k] = domain ? (int16_t)((int)byte - 128) : (int16_t)(int8_t)byte;
      }
      for (int g = 0; g < ng; ++g) {
        const uint8_t* sp = base + (size_t)tile_m * K + ((size_t)r * ng + g) * 2;
        s[(size_t)row * ng + g] = (uint16_t)(sp[0] | (sp[1] << 8));
      }
    }
  }
  return 0;
}

void oracle_dequant(const int16_t* q, const uint16_t* s, uint16_t* out, int M, int K, int G) {
  const int ng = K / G;
  for (int m = 0; m < M; ++m)
    for (int k = 0; k < K; ++k) {
      const float sv = bf16_to_f32(s[(size_t)m * ng + k / G]);
      out[(size_t)m * K + k] = f32_to_bf16_rne((float)q[(size_t)m * K + k] * sv);
    }
}

/* y[b][m] = sum_g s[m][g] * sum_{k in g} q[m][k] * x[b][k]; x bf16 bits; y double. */
void oracle_gemv_f64(const int16_t* q, const uint16_t* s, const uint16_t* x, double* y, int B,
                     int M, int K, int G) {
  const int ng = K / G;
  for (int b = 0; b < B; ++b)
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int g = 0; g < ng; ++g) {
        double part = 0.0;
        for (int k = g * G; k < (g + 1) * G; ++k)
          part += (double)q[(size_t)m * K + k] * (double)bf16_to_f32(x[(size_t)b * K + k]);
        acc += part * (double)bf16_to_f32(s[(size_t)m * ng + g]);
      }
      y[(size_t)b * M + m] = acc;
    }
}

/* q: [B][H][D], k/v: [B][KV][L][D] bf16 bits; ctx: [B]; out: [B][H][D] double. */
void oracle_decode_attn_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const int32_t* ctx, double* out, int B, int H, int KV, int L, int D,
                            double scale) {
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int kvh = h * KV / H;
      double* o = out + ((size_t)b * H + h) * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      const int n = ctx[b] < 0 ? 0 : (ctx[b] > L ? L : ctx[b]);
      if (n == 0) continue;
      const uint16_t* qh = q + ((size_t)b * H + h) * D;
      const uint16_t* kh = k + ((size_t)b * KV + kvh) * (size_t)L * D;
      const uint16_t* vh = v + ((size_t)b * KV + kvh) * (size_t)L * D;
      double mx = -INFINITY;
      for (int j = 0; j < n; ++j) {
        double sc = 0.0;
        for (int d = 0; d < D; ++d)
          sc += (double)bf16_to_f32(qh[d]) * (double)bf16_to_f32(kh[(size_t)j * D + d]);
        sc *= scale;
        if (sc > mx) mx = sc;
      }
      double den = 0.0;
      for (int j = 0; j < n; ++j) {
        double sc = 0.0;
        for (int d = 0; d < D; ++d)
          sc += (double)bf16_to_f32(qh[d]) * (double)bf16_to_f32(kh[(size_t)j * D + d]);
        const double w = exp(sc * scale - mx);
        den += w;
        for (int d = 0; d < D; ++d) o[d] += w * (double)bf16_to_f32(vh[(size_t)j * D + d]);
      }
      for (int d = 0; d < D; ++d) o[d] /= den;
    }
}
