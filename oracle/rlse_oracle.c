/*
 * rlse_oracle.c -- CPU restatement of the reference's KV-cache hot path, as
 * its Candle CPU backend evaluates it.
 *
 * TEST INFRASTRUCTURE ONLY. The tests compare the HIP kernels with this
 * file, which is also the timed CPU baseline of bench.py; no product code
 * links or calls it.
 *
 * Every function cites the reference code it restates. Arithmetic is f32 in
 * the reference's op order (matmul as a sequential dot product, then the
 * scale; softmax as max, subtract, exp, sum, divide). The reference's own
 * summation order inside the gemm crate is not reproducible without building
 * it, so results agree with Candle to rounding, not to the bit. The data
 * movement functions (KvCache append/narrow, paged layout) are exact.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bf16 (half::bf16::from_f32: round to nearest even, NaN kept quiet) ---- */
float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  /* round bit set and (sticky bits or lsb set) -> round up */
  const uint32_t round_bit = 0x8000u;
  if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0) return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

static float rbf(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

void orc_bf16_to_f32_array(const uint16_t* in, float* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

/* ---- candle_nn::kv_cache::KvCache over dim 2 of [1, Hkv, cap, d] ----
 * (src/backends/qwen2.rs:349-361): the buffer is zero-initialised with cap
 * rows, append does slice_set(src, dim=2, cur_len) and the visible cache is
 * narrow(2, 0, cur_len). Elements are es bytes. Returns the new length, or
 * -1 when cap would be exceeded (the buffer is left unchanged). */
int orc_kvcache_append(uint8_t* buf, int Hkv, int cap, int d, int es, int cur_len,
                       const uint8_t* src, int q) {
  if (cur_len < 0 || q < 0 || cur_len + q > cap) return -1;
  const size_t row = (size_t)d * es;
  for (int h = 0; h < Hkv; ++h)
    for (int t = 0; t < q; ++t)
      memcpy(buf + (((size_t)h * cap) + cur_len + t) * row, src + (((size_t)h * q) + t) * row,
             row);
  return cur_len + q;
}

void orc_kvcache_narrow(const uint8_t* buf, int Hkv, int cap, int d, int es, int len,
                        uint8_t* out) {
  const size_t row = (size_t)d * es;
  for (int h = 0; h < Hkv; ++h)
    memcpy(out + (size_t)h * len * row, buf + (size_t)h * cap * row, (size_t)len * row);
}

/* ---- Paged pool layout of the prototype kernels (mini_serve_kernels.cu:
 * 68-70, 93): pool[block][Hkv][16][d], token t of a sequence in block
 * table[t/16], slot t%16. ---- */
void orc_paged_write_token(uint8_t* pool, int Hkv, int d, int es, const int32_t* table, int pos,
                           const uint8_t* src /* [Hkv][d] */) {
  const size_t row = (size_t)d * es;
  const int blk = table[pos / 16];
  for (int h = 0; h < Hkv; ++h)
    memcpy(pool + ((((size_t)blk * Hkv + h) * 16) + pos % 16) * row, src + (size_t)h * row, row);
}

void orc_paged_to_contiguous(const uint8_t* pool, int Hkv, int d, int es, const int32_t* table,
                             int len, uint8_t* out /* [Hkv][len][d] */) {
  const size_t row = (size_t)d * es;
  for (int h = 0; h < Hkv; ++h)
    for (int t = 0; t < len; ++t) {
      const int blk = table[t / 16];
      memcpy(out + ((size_t)h * len + t) * row,
             pool + ((((size_t)blk * Hkv + h) * 16) + t % 16) * row, row);
    }
}

/* ---- decode_attention_gqa_zero_copy (src/backends/qwen2.rs:177-203) ----
 * q [Hq][d]; k, v [Hkv][cap][d] of which the first len rows are visible.
 * For each KV head h: scores = (q_group . k^T) * scale; softmax over the
 * last dim (candle_nn::ops::softmax: max, sub, exp, sum, div); out = p . v. */
static void decode_one_head(const float* qg, int G, const float* kh, const float* vh, int len,
                            int d, float scale, float* outg, float* scores) {
  for (int g = 0; g < G; ++g) {
    const float* qr = qg + (size_t)g * d;
    float* sc = scores + (size_t)g * len;
    for (int t = 0; t < len; ++t) {
      const float* kr = kh + (size_t)t * d;
      float acc = 0.f;
      for (int e = 0; e < d; ++e) acc += qr[e] * kr[e];
      sc[t] = acc * scale;
    }
    float mx = -INFINITY;
    for (int t = 0; t < len; ++t) mx = sc[t] > mx ? sc[t] : mx;
    float sum = 0.f;
    for (int t = 0; t < len; ++t) {
      sc[t] = expf(sc[t] - mx);
      sum += sc[t];
    }
    for (int t = 0; t < len; ++t) sc[t] = sc[t] / sum;
    float* o = outg + (size_t)g * d;
    for (int e = 0; e < d; ++e) o[e] = 0.f;
    for (int t = 0; t < len; ++t) {
      const float p = sc[t];
      const float* vr = vh + (size_t)t * d;
      for (int e = 0; e < d; ++e) o[e] += p * vr[e];
    }
  }
}

void orc_decode_gqa_f32(const float* q, const float* k, const float* v, int Hq, int Hkv, int cap,
                        int len, int d, float scale, float* out) {
  const int G = Hq / Hkv;
  float* scores = (float*)malloc(sizeof(float) * (size_t)G * (len > 0 ? len : 1));
  for (int h = 0; h < Hkv; ++h)
    decode_one_head(q + (size_t)h * G * d, G, k + (size_t)h * cap * d, v + (size_t)h * cap * d,
                    len, d, scale, out + (size_t)h * G * d, scores);
  free(scores);
}

/* Batched decode over per-sequence contiguous buffers k, v [B][Hkv][cap][d]
 * (the loop at src/backends/qwen2.rs:723-744), parallel over (b, h) with
 * OpenMP like Candle's rayon CPU backend. threads <= 0 uses the default. */
void orc_decode_batch_f32(const float* q, const float* k, const float* v, const int32_t* lens,
                          int B, int Hq, int Hkv, int cap, int d, float scale, float* out,
                          int threads) {
  const int G = Hq / Hkv;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel
  {
    float* scores = (float*)malloc(sizeof(float) * (size_t)G * (cap > 0 ? cap : 1));
#pragma omp for schedule(dynamic, 1)
    for (long long r = 0; r < (long long)B * Hkv; ++r) {
      const int b = (int)(r / Hkv), h = (int)(r % Hkv);
      const size_t kv = (((size_t)b * Hkv) + h) * cap * d;
      decode_one_head(q + ((size_t)b * Hq + (size_t)h * G) * d, G, k + kv, v + kv, lens[b], d,
                      scale, out + ((size_t)b * Hq + (size_t)h * G) * d, scores);
    }
    free(scores);
  }
}

/* ---- Prefill / chunked attention (src/backends/qwen2.rs:329-345) with the
 * causal mask of prepare_causal_attention_mask (:476-503): query i of a
 * q_len chunk that starts after `offset` cached tokens sees keys
 * j <= offset + i. repeat_kv maps query head h to KV head h / G.
 * q, out [Hq][q_len][d]; k, v [Hkv][cap][d], first offset+q_len rows visible. */
void orc_prefill_f32(const float* q, const float* k, const float* v, int Hq, int Hkv, int cap,
                     int q_len, int offset, int d, float scale, float* out, int threads) {
  const int G = Hq / Hkv;
  const int lk = offset + q_len;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)(lk > 0 ? lk : 1));
#pragma omp for schedule(dynamic, 4)
    for (long long r = 0; r < (long long)Hq * q_len; ++r) {
      const int h = (int)(r / q_len), i = (int)(r % q_len);
      const float* qr = q + ((size_t)h * q_len + i) * d;
      const float* kh = k + (size_t)(h / G) * cap * d;
      const float* vh = v + (size_t)(h / G) * cap * d;
      float mx = -INFINITY;
      for (int j = 0; j < lk; ++j) {
        float acc = 0.f;
        for (int e = 0; e < d; ++e) acc += qr[e] * kh[(size_t)j * d + e];
        acc = acc * scale;
        /* mask: 0 for the cached columns, -inf above the diagonal of the chunk */
        if (j >= offset && (j - offset) > i) acc = -INFINITY;
        sc[j] = acc;
        mx = acc > mx ? acc : mx;
      }
      float sum = 0.f;
      for (int j = 0; j < lk; ++j) {
        sc[j] = expf(sc[j] - mx);
        sum += sc[j];
      }
      float* o = out + ((size_t)h * q_len + i) * d;
      for (int e = 0; e < d; ++e) o[e] = 0.f;
      for (int j = 0; j < lk; ++j) {
        const float p = sc[j] / sum;
        for (int e = 0; e < d; ++e) o[e] += p * vh[(size_t)j * d + e];
      }
    }
    free(sc);
  }
}

/* ---- RmsNorm::forward (src/backends/qwen2.rs:68-75) ----
 * x_f32 = x; variance = mean_keepdim(x^2) = sum * (1/n) (candle's mean is a
 * sum scaled by 1/n); norm = sqrt(variance + eps); x_normed = (x / norm) cast
 * to dtype; out = x_normed * weight in dtype.
 *
 * Summation order of sum(x^2). Candle's own order inside its reduction is
 * not reproducible without building it, so this restatement fixes one order,
 * which every RMSNorm kernel of the build that writes cached K follows too:
 * the row is cut into packets of epl consecutive elements (epl = 16 bytes /
 * element size: 4 for f32, 8 for bf16 and f16), each packet's squares are
 * summed in element order starting from 0, and the packet sums are added by
 * a balanced pairwise tree over the next power of two of packets, the missing
 * ones counting as 0 (level k adds the sums of blocks 2j and 2j+1 of 2^k
 * packets). Elements past n in the last packet count as 0. */
float orc_sumsq_tree(const float* x, int n, int epl) {
  const int np = (n + epl - 1) / epl;
  int p2 = 1;
  while (p2 < np) p2 <<= 1;
  float* ps = (float*)calloc((size_t)p2, sizeof(float));
  for (int j = 0; j < np; ++j) {
    float a = 0.f;
    for (int e = 0; e < epl; ++e) {
      const int i = j * epl + e;
      const float v = i < n ? x[i] : 0.f;
      a = a + v * v;
    }
    ps[j] = a;
  }
  for (int span = 1; span < p2; span <<= 1)
    for (int j = 0; j < p2; j += 2 * span) ps[j] = ps[j] + ps[j + span];
  const float ss = ps[0];
  free(ps);
  return ss;
}

void orc_sumsq_tree_rows(const float* x, int rows, int n, int epl, float* out) {
  for (int r = 0; r < rows; ++r) out[r] = orc_sumsq_tree(x + (size_t)r * n, n, epl);
}

void orc_rmsnorm_f32(const float* x, const float* w, float* out, int rows, int n, float eps) {
  const float inv_n = (float)(1.0 / (double)n);
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * n;
    const float ss = orc_sumsq_tree(xr, n, 4);
    const float var = ss * inv_n;
    const float norm = sqrtf(var + eps);
    for (int i = 0; i < n; ++i) out[(size_t)r * n + i] = (xr[i] / norm) * w[i];
  }
}

void orc_rmsnorm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int n,
                      float eps) {
  const float inv_n = (float)(1.0 / (double)n);
  float* xf = (float*)malloc(sizeof(float) * (size_t)n);
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + (size_t)r * n;
    for (int i = 0; i < n; ++i) xf[i] = orc_bf16_to_f32(xr[i]);
    const float ss = orc_sumsq_tree(xf, n, 8);
    const float norm = sqrtf(ss * inv_n + eps);
    for (int i = 0; i < n; ++i) {
      const float xn = rbf(xf[i] / norm);
      out[(size_t)r * n + i] = orc_f32_to_bf16(xn * orc_bf16_to_f32(w[i]));
    }
  }
  free(xf);
}

/* ---- RotaryEmbedding::new (src/backends/qwen2.rs:90-108) ----
 * inv_freq[i] = 1f32 / (theta.powf(2i/d) as f32); freqs[t][i] = (t as f32) *
 * inv_freq[i]; tables are sin/cos of freqs (f32), [max_pos][d/2]. */
void orc_rope_tables_f32(double theta, int d, int max_pos, float* cos_t, float* sin_t) {
  const int half = d / 2;
  float* inv = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; ++i) inv[i] = 1.0f / (float)pow(theta, (double)(2 * i) / (double)d);
  for (int t = 0; t < max_pos; ++t)
    for (int i = 0; i < half; ++i) {
      const float f = (float)t * inv[i];
      cos_t[(size_t)t * half + i] = cosf(f);
      sin_t[(size_t)t * half + i] = sinf(f);
    }
  free(inv);
}

/* ---- apply_rope with rotate_half (src/backends/qwen2.rs:125-142) ----
 * out = x * [cos, cos] + [-x2, x1] * [sin, sin]; each product and the sum
 * are separate ops (rounded to dtype for bf16). Row r is at position pos[r]. */
void orc_apply_rope_f32(float* x, const int32_t* pos, const float* cos_t, const float* sin_t,
                        int rows, int d) {
  const int half = d / 2;
  for (int r = 0; r < rows; ++r) {
    float* xr = x + (size_t)r * d;
    const float* c = cos_t + (size_t)pos[r] * half;
    const float* s = sin_t + (size_t)pos[r] * half;
    for (int i = 0; i < half; ++i) {
      const float x1 = xr[i], x2 = xr[i + half];
      volatile float a = x1 * c[i], b = (-x2) * s[i], e = x2 * c[i], f = x1 * s[i];
      xr[i] = a + b;
      xr[i + half] = e + f;
    }
  }
}

void orc_apply_rope_bf16(uint16_t* x, const int32_t* pos, const uint16_t* cos_t,
                         const uint16_t* sin_t, int rows, int d) {
  const int half = d / 2;
  for (int r = 0; r < rows; ++r) {
    uint16_t* xr = x + (size_t)r * d;
    const uint16_t* c = cos_t + (size_t)pos[r] * half;
    const uint16_t* s = sin_t + (size_t)pos[r] * half;
    for (int i = 0; i < half; ++i) {
      const float x1 = orc_bf16_to_f32(xr[i]), x2 = orc_bf16_to_f32(xr[i + half]);
      const float ci = orc_bf16_to_f32(c[i]), si = orc_bf16_to_f32(s[i]);
      xr[i] = orc_f32_to_bf16(rbf(x1 * ci) + rbf(-x2 * si));
      xr[i + half] = orc_f32_to_bf16(rbf(x2 * ci) + rbf(x1 * si));
    }
  }
}

/* One decode step of the reference CPU path for a batch over per-sequence
 * contiguous buffers: append the new k/v row of every sequence at lens[b]-1
 * (KvCache::append, src/backends/qwen2.rs:728-730) and run the zero-copy GQA
 * decode over lens[b] keys (:735-742). k_new, v_new [B][Hkv][d]. Used as the
 * timed CPU baseline. */
void orc_decode_step_f32(const float* q, const float* k_new, const float* v_new, float* k,
                         float* v, const int32_t* lens, int B, int Hq, int Hkv, int cap, int d,
                         float scale, float* out, int threads) {
  for (int b = 0; b < B; ++b) {
    const int pos = lens[b] - 1;
    if (pos < 0 || pos >= cap) continue;
    for (int h = 0; h < Hkv; ++h) {
      const size_t dst = ((((size_t)b * Hkv) + h) * cap + pos) * d;
      const size_t src = (((size_t)b * Hkv) + h) * d;
      memcpy(k + dst, k_new + src, sizeof(float) * (size_t)d);
      memcpy(v + dst, v_new + src, sizeof(float) * (size_t)d);
    }
  }
  orc_decode_batch_f32(q, k, v, lens, B, Hq, Hkv, cap, d, scale, out, threads);
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
