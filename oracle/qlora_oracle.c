/*
 * qlora_oracle.c -- CPU restatement of stuarch/VkQLoRA.rs `qlora-core`.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing shipped or
 * measured as the product).  Built with -O2 -ffp-contract=off and no
 * fast-math so every f32 operation rounds exactly where the Rust source
 * rounds: Rust never contracts a*b+c into an FMA and never reassociates.
 *
 * Rust semantics reproduced here:
 *   f32::max ignores NaN            -> fmaxf
 *   f32::round is half-away-from-0  -> roundf
 *   `as i32` saturates, NaN -> 0    -> rs_f32_to_i32
 *   f32::powf goes to the C libm    -> powf
 *
 * Parity pins (what checks each function besides restatement) are listed
 * in tests/test_oracle.py; functions without an independent pin say so.
 */
#include "qlora_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* qlora-core/src/quant.rs:27-44.  Each f64 literal is exactly
 * representable in f32, so the f32 constants below are the same values. */
const float OR_NF4_LEVELS[16] = {
    -1.0f,
    -0.6961928009986877f,
    -0.5250730514526367f,
    -0.39491748809814453f,
    -0.28444138169288635f,
    -0.18477343022823334f,
    -0.09105003625154495f,
    0.0f,
    0.07958029955625534f,
    0.16093020141124725f,
    0.24611230194568634f,
    0.33791524171829224f,
    0.44070982933044434f,
    0.5626170039176941f,
    0.7229568362236023f,
    1.0f,
};

static int32_t rs_f32_to_i32(float v) {
  /* Rust `as i32`: saturating, NaN -> 0. */
  if (isnan(v)) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v <= -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}

static int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

/* ---- qlora-core/tests/quant.rs:6-24 ---------------------------------- */
double or_rng_next_f64(or_rng *r) {
  uint64_t x = r->s;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  r->s = x;
  return (double)((x * 0x2545F4914F6CDD1DULL) >> 11) /
         (double)(UINT64_MAX >> 11);
}

float or_rng_next_normal(or_rng *r) {
  double u1 = fmax(or_rng_next_f64(r), 1e-12);
  double u2 = or_rng_next_f64(r);
  return (float)(sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2));
}

void or_fill_normal(uint64_t *state, float *out, size_t n, float scale) {
  or_rng r = {*state};
  for (size_t i = 0; i < n; i++) out[i] = scale * or_rng_next_normal(&r);
  *state = r.s;
}

void or_fill_uniform(uint64_t *state, float *out, size_t n, float lo,
                     float hi) {
  or_rng r = {*state};
  for (size_t i = 0; i < n; i++)
    out[i] = (float)or_rng_next_f64(&r) * (hi - lo) + lo;
  *state = r.s;
}

/* ---- quant.rs:263-278 ------------------------------------------------ */
uint8_t or_nearest_nf4_code(float w, float absmax) {
  if (absmax == 0.0f) return OR_NF4_ZERO_CODE;
  float target = w / absmax;
  uint8_t best = 0;
  float best_dist = INFINITY;
  for (int i = 0; i < 16; i++) {
    float d = fabsf(OR_NF4_LEVELS[i] - target);
    if (d < best_dist) {
      best_dist = d;
      best = (uint8_t)i;
    }
  }
  return best;
}

/* ---- quant.rs:283-299 ------------------------------------------------ */
static void double_quantize_scales(const float *scales, size_t nb,
                                   uint8_t *codes, float *absmax) {
  size_t nsb = (nb + OR_DOUBLE_QUANT_BLOCK - 1) / OR_DOUBLE_QUANT_BLOCK;
  for (size_t c = 0; c < nsb; c++) {
    size_t s0 = c * OR_DOUBLE_QUANT_BLOCK;
    size_t s1 = s0 + OR_DOUBLE_QUANT_BLOCK < nb ? s0 + OR_DOUBLE_QUANT_BLOCK
                                                : nb;
    float amax = 0.0f;
    for (size_t i = s0; i < s1; i++) amax = fmaxf(amax, fabsf(scales[i]));
    absmax[c] = amax;
    for (size_t i = s0; i < s1; i++) {
      int8_t q;
      if (amax == 0.0f) {
        q = 0;
      } else {
        float t = scales[i] / amax * 127.0f;
        q = (int8_t)clamp_i32(rs_f32_to_i32(roundf(t)), -127, 127);
      }
      codes[i] = (uint8_t)q;
    }
  }
}

/* ---- quant.rs:104-154 ------------------------------------------------ */
int or_quantize(const float *w, size_t n, size_t block_size, int double_quant,
                uint8_t *codes, float *scales_f32, uint8_t *scale_codes,
                float *absmax) {
  if (block_size == 0) return -1;
  size_t nb = (n + block_size - 1) / block_size;
  memset(codes, 0, (n + 1) / 2);
  float *sc = scales_f32;
  float *tmp = NULL;
  if (double_quant) {
    tmp = (float *)malloc((nb ? nb : 1) * sizeof(float));
    sc = tmp;
  }
  for (size_t b = 0; b < nb; b++) {
    size_t s = b * block_size;
    size_t e = s + block_size < n ? s + block_size : n;
    float am = 0.0f;
    for (size_t i = s; i < e; i++) am = fmaxf(am, fabsf(w[i]));
    sc[b] = am;
    for (size_t idx = s; idx < e; idx++) {
      uint8_t code = or_nearest_nf4_code(w[idx], am);
      if (idx % 2 == 0)
        codes[idx / 2] |= code;
      else
        codes[idx / 2] |= (uint8_t)(code << 4);
    }
  }
  if (double_quant) {
    double_quantize_scales(sc, nb, scale_codes, absmax);
    free(tmp);
  }
  return 0;
}

/* ---- quant.rs:212-221 ------------------------------------------------ */
void or_block_scales_dq(const uint8_t *scale_codes, const float *absmax,
                        size_t nb, float *out) {
  for (size_t i = 0; i < nb; i++)
    out[i] = (float)(int8_t)scale_codes[i] / 127.0f *
             absmax[i / OR_DOUBLE_QUANT_BLOCK];
}

/* ---- quant.rs:157-167 ------------------------------------------------ */
void or_dequantize(const uint8_t *codes, const float *scales, size_t n,
                   size_t block_size, float *out) {
  for (size_t idx = 0; idx < n; idx++) {
    uint8_t byte = codes[idx / 2];
    uint8_t code = (idx % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
    out[idx] = OR_NF4_LEVELS[code] * scales[idx / block_size];
  }
}

/* ---- lora.rs:129-142 (i, p, j order) -------------------------------- */
void or_matmul(const float *a, const float *b, size_t m, size_t k, size_t n,
               float *c) {
  memset(c, 0, m * n * sizeof(float));
  for (size_t i = 0; i < m; i++)
    for (size_t p = 0; p < k; p++) {
      float a_ip = a[i * k + p];
      for (size_t j = 0; j < n; j++) c[i * n + j] += a_ip * b[p * n + j];
    }
}

/* ---- lora.rs:148-162 ------------------------------------------------- */
void or_matmul_trans_a(const float *a, const float *b, size_t m, size_t k,
                       size_t n, float *c) {
  for (size_t i = 0; i < k; i++)
    for (size_t j = 0; j < n; j++) {
      float acc = 0.0f;
      for (size_t p = 0; p < m; p++) acc += a[p * k + i] * b[p * n + j];
      c[i * n + j] = acc;
    }
}

/* ---- lora.rs:169-183 ------------------------------------------------- */
void or_matmul_trans_b(const float *a, const float *b, size_t m, size_t k,
                       size_t n, float *c) {
  for (size_t i = 0; i < m; i++)
    for (size_t j = 0; j < n; j++) {
      float acc = 0.0f;
      for (size_t p = 0; p < k; p++) acc += a[i * k + p] * b[j * k + p];
      c[i * n + j] = acc;
    }
}

/* ---- qlora.rs:86-107 with lora.rs:86-103 ---------------------------- */
void or_qlora_forward(const float *w_deq, size_t out_dim, size_t in_dim,
                      const float *lora_a, const float *lora_b, size_t r,
                      float alpha, const float *x, size_t batch, float *y) {
  or_matmul_trans_b(x, w_deq, batch, in_dim, out_dim, y);
  if (lora_a && lora_b && r > 0) {
    float *t1 = (float *)malloc(batch * r * sizeof(float) + 4);
    float *t2 = (float *)malloc(batch * out_dim * sizeof(float) + 4);
    or_matmul_trans_b(x, lora_a, batch, in_dim, r, t1);
    or_matmul_trans_b(t1, lora_b, batch, r, out_dim, t2);
    float s = alpha / (float)r; /* lora.rs:64-66 */
    for (size_t i = 0; i < batch * out_dim; i++) t2[i] *= s;
    for (size_t i = 0; i < batch * out_dim; i++) y[i] += t2[i];
    free(t1);
    free(t2);
  }
}

/* ---- qlora.rs:116-165 ------------------------------------------------ */
void or_qlora_backward(const float *w_deq, size_t out_dim, size_t in_dim,
                       const float *lora_a, const float *lora_b, size_t r,
                       float alpha, const float *x, const float *dy,
                       size_t batch, float *grad_x, float *grad_a,
                       float *grad_b) {
  or_matmul(dy, w_deq, batch, out_dim, in_dim, grad_x);
  if (!(lora_a && lora_b && r > 0)) return;
  float s = alpha / (float)r;
  size_t ndy = batch * out_dim;
  float *dys = (float *)malloc(ndy * sizeof(float) + 4);
  for (size_t i = 0; i < ndy; i++) dys[i] = dy[i] * s;
  float *t1 = (float *)malloc(batch * r * sizeof(float) + 4);
  or_matmul_trans_b(x, lora_a, batch, in_dim, r, t1);
  or_matmul_trans_a(dys, t1, batch, out_dim, r, grad_b);
  float *ds = (float *)malloc(batch * r * sizeof(float) + 4);
  or_matmul(dys, lora_b, batch, out_dim, r, ds);
  or_matmul_trans_a(ds, x, batch, r, in_dim, grad_a);
  float *dxl = (float *)malloc(batch * in_dim * sizeof(float) + 4);
  or_matmul(ds, lora_a, batch, r, in_dim, dxl);
  for (size_t i = 0; i < batch * in_dim; i++) grad_x[i] += dxl[i];
  free(dys);
  free(t1);
  free(ds);
  free(dxl);
}

/* ---- optim.rs:84-100 ------------------------------------------------- */
float or_quantize_block_i8(const float *x, size_t len, uint8_t *codes) {
  float absmax = 0.0f;
  for (size_t i = 0; i < len; i++) absmax = fmaxf(absmax, fabsf(x[i]));
  if (absmax == 0.0f) {
    memset(codes, 0, len);
    return 0.0f;
  }
  for (size_t i = 0; i < len; i++) {
    float t = x[i] / absmax * 127.0f;
    codes[i] = (uint8_t)(int8_t)clamp_i32(rs_f32_to_i32(roundf(t)), -127, 127);
  }
  return absmax;
}

void or_dequant_block_i8(const uint8_t *codes, float absmax, size_t len,
                         float *out) {
  for (size_t i = 0; i < len; i++)
    out[i] = (float)(int8_t)codes[i] / 127.0f * absmax;
}

/* ---- optim.rs:103-249 ------------------------------------------------ */
typedef struct {
  size_t numel, num_blocks;
  uint8_t *m_codes, *v_codes;
  float *m_scales, *v_scales;
  uint64_t step;
} or_param_state;

struct or_adam {
  float lr, beta1, beta2, eps;
  size_t block_size, max_resident_pages;
  or_param_state *states;
  size_t nstates, cap;
};

static void state_init(or_param_state *st, size_t numel, size_t bs) {
  st->numel = numel;
  st->num_blocks = (numel + bs - 1) / bs;
  st->m_codes = (uint8_t *)calloc(numel + 1, 1);
  st->v_codes = (uint8_t *)calloc(numel + 1, 1);
  st->m_scales = (float *)calloc(st->num_blocks + 1, sizeof(float));
  st->v_scales = (float *)calloc(st->num_blocks + 1, sizeof(float));
  st->step = 0;
}

static void state_free(or_param_state *st) {
  free(st->m_codes);
  free(st->v_codes);
  free(st->m_scales);
  free(st->v_scales);
}

or_adam *or_adam_create(float lr, float beta1, float beta2, float eps,
                        size_t block_size, size_t max_resident_pages) {
  /* optim.rs:63-80 */
  if (lr <= 0.0f || !isfinite(lr)) return NULL;
  if (!(beta1 >= 0.0f && beta1 < 1.0f) || !(beta2 >= 0.0f && beta2 < 1.0f))
    return NULL;
  if (block_size == 0 || max_resident_pages == 0) return NULL;
  or_adam *o = (or_adam *)calloc(1, sizeof(or_adam));
  o->lr = lr;
  o->beta1 = beta1;
  o->beta2 = beta2;
  o->eps = eps;
  o->block_size = block_size;
  o->max_resident_pages = max_resident_pages;
  return o;
}

void or_adam_destroy(or_adam *o) {
  if (!o) return;
  for (size_t i = 0; i < o->nstates; i++) state_free(&o->states[i]);
  free(o->states);
  free(o);
}

/* optim.rs:206-248 */
static size_t step_param(const or_adam *cfg, or_param_state *st, float *p,
                         const float *g) {
  st->step += 1;
  float t = (float)st->step;
  float b1t = 1.0f - powf(cfg->beta1, t);
  float b2t = 1.0f - powf(cfg->beta2, t);
  size_t window = cfg->max_resident_pages < st->num_blocks
                      ? cfg->max_resident_pages
                      : st->num_blocks;
  if (window < 1) window = 1;
  size_t streamed = 0;
  float *m = (float *)malloc(cfg->block_size * sizeof(float));
  float *v = (float *)malloc(cfg->block_size * sizeof(float));
  for (size_t bstart = 0; bstart < st->num_blocks; bstart += window) {
    size_t bend = bstart + window < st->num_blocks ? bstart + window
                                                   : st->num_blocks;
    for (size_t b = bstart; b < bend; b++) {
      size_t s = b * cfg->block_size;
      size_t e = s + cfg->block_size < st->numel ? s + cfg->block_size
                                                 : st->numel;
      size_t len = e - s;
      or_dequant_block_i8(st->m_codes + s, st->m_scales[b], len, m);
      or_dequant_block_i8(st->v_codes + s, st->v_scales[b], len, v);
      for (size_t j = 0; j < len; j++) {
        float gj = g[s + j];
        m[j] = cfg->beta1 * m[j] + (1.0f - cfg->beta1) * gj;
        float var = cfg->beta2 * v[j] * v[j] + (1.0f - cfg->beta2) * gj * gj;
        v[j] = sqrtf(var);
        float mh = m[j] / b1t;
        float vh = var / b2t;
        p[s + j] -= cfg->lr * mh / (sqrtf(vh) + cfg->eps);
      }
      st->m_scales[b] = or_quantize_block_i8(m, len, st->m_codes + s);
      st->v_scales[b] = or_quantize_block_i8(v, len, st->v_codes + s);
      streamed += 1;
    }
  }
  free(m);
  free(v);
  return streamed;
}

/* optim.rs:164-199 */
size_t or_adam_step(or_adam *o, float **params, const float *const *grads,
                    const size_t *lens, size_t count) {
  size_t pages = 0;
  for (size_t i = 0; i < count; i++) {
    if (o->nstates <= i) {
      if (o->cap <= i) {
        size_t nc = o->cap ? o->cap * 2 : 8;
        while (nc <= i) nc *= 2;
        o->states = (or_param_state *)realloc(o->states,
                                              nc * sizeof(or_param_state));
        o->cap = nc;
      }
      state_init(&o->states[o->nstates], lens[i], o->block_size);
      o->nstates++;
    }
    if (o->states[i].numel != lens[i]) {
      state_free(&o->states[i]);
      state_init(&o->states[i], lens[i], o->block_size);
    }
    pages += step_param(o, &o->states[i], params[i], grads[i]);
  }
  return pages;
}

/* optim.rs:128-131, 201-204 */
size_t or_adam_state_bytes(const or_adam *o) {
  size_t total = 0;
  for (size_t i = 0; i < o->nstates; i++) {
    const or_param_state *st = &o->states[i];
    total += 2 * st->numel + 2 * st->num_blocks * 4;
  }
  return total;
}

int or_adam_get_state(const or_adam *o, size_t idx, uint8_t *m_codes,
                      float *m_scales, uint8_t *v_codes, float *v_scales,
                      uint64_t *step) {
  if (idx >= o->nstates) return -1;
  const or_param_state *st = &o->states[idx];
  memcpy(m_codes, st->m_codes, st->numel);
  memcpy(v_codes, st->v_codes, st->numel);
  memcpy(m_scales, st->m_scales, st->num_blocks * sizeof(float));
  memcpy(v_scales, st->v_scales, st->num_blocks * sizeof(float));
  *step = st->step;
  return 0;
}

/* ===== qlora-model glue around the projections (qlora-model/src/llama.rs) */

/* llama.rs:730-739.  The row sum is Rust's sequential f32 Sum. */
void or_rmsnorm(const float *x, const float *w, size_t rows, size_t h,
                float eps, float *y) {
  for (size_t t = 0; t < rows; t++) {
    const float *xr = x + t * h;
    float *yr = y + t * h;
    float acc = 0.0f;
    for (size_t j = 0; j < h; j++) acc += xr[j] * xr[j];
    float mean_sq = acc / (float)h;
    float scale = 1.0f / sqrtf(mean_sq + eps);
    for (size_t j = 0; j < h; j++) yr[j] = xr[j] * scale * w[j];
  }
}

/* llama.rs:605-628 */
void or_rmsnorm_backward(const float *x, const float *w, const float *dy,
                         size_t rows, size_t h, float eps, float *dx,
                         float *dw) {
  for (size_t j = 0; j < h; j++) dw[j] = 0.0f;
  for (size_t t = 0; t < rows; t++) {
    const float *xr = x + t * h;
    const float *dyr = dy + t * h;
    float acc = 0.0f;
    for (size_t j = 0; j < h; j++) acc += xr[j] * xr[j];
    float mean_sq = acc / (float)h;
    float ss = mean_sq + eps;
    float r = 1.0f / sqrtf(ss);
    float ds = 0.0f;
    for (size_t j = 0; j < h; j++) {
      ds += dyr[j] * xr[j] * w[j];
      dw[j] += dyr[j] * xr[j] * r;
    }
    ds *= -0.5f * (1.0f / ss) * r;
    for (size_t j = 0; j < h; j++)
      dx[t * h + j] = dyr[j] * w[j] * r + 2.0f * xr[j] / (float)h * ds;
  }
}

/* llama.rs:516-527 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

static float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

float or_silu_prime(float x) {
  float s = or_sigmoid(x);
  return s * (1.0f + x * (1.0f - s));
}

/* llama.rs:452-456 */
void or_swiglu(const float *gate, const float *up, size_t n, float *act) {
  for (size_t i = 0; i < n; i++) act[i] = or_silu(gate[i]) * up[i];
}

/* llama.rs:559-562 */
void or_swiglu_backward(const float *gate, const float *up,
                        const float *d_act, size_t n, float *dg, float *du) {
  for (size_t i = 0; i < n; i++) {
    dg[i] = d_act[i] * up[i] * or_silu_prime(gate[i]);
    du[i] = d_act[i] * or_silu(gate[i]);
  }
}

/* llama.rs:487-514.  f32::max ignores NaN (fmaxf); the row max starts at
 * -inf. */
float or_softmax_cross_entropy(const float *logits, const uint32_t *targets,
                               size_t seq, size_t vocab, float *dlogits) {
  float loss = 0.0f;
  for (size_t t = 0; t < seq; t++) {
    const float *row = logits + t * vocab;
    float *d = dlogits + t * vocab;
    float mx = -INFINITY;
    for (size_t j = 0; j < vocab; j++) mx = fmaxf(mx, row[j]);
    float sum = 0.0f;
    for (size_t j = 0; j < vocab; j++) {
      float e = expf(row[j] - mx);
      d[j] = e;
      sum += e;
    }
    loss -= (row[targets[t]] - mx - logf(sum)) / (float)seq;
    for (size_t j = 0; j < vocab; j++) d[j] = d[j] / sum / (float)seq;
    d[targets[t]] -= 1.0f / (float)seq;
  }
  return loss;
}
