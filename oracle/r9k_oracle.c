/* r9k_oracle.c -- CPU restatement of the reference's quantized-MoE hot path, for TESTS ONLY.
 *
 * This is test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker. Nothing in the product (r9700-stack_amd/) links or calls it.
 *
 * Each function cites the reference code it restates. The formulations are deliberately different from the HIP
 * kernels' (table search instead of bit tricks, brute-force exponent search, nearest-value search instead of
 * threshold counting) so a shared mistake is unlikely; tests/test_oracle_*.py pin every function against torch
 * library routines, closed forms and brute force.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: arithmetic exactly as written, SSE fp32/fp64).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ number formats */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float or_bf16_to_f32(uint16_t h) { return f32_from_bits((uint32_t)h << 16); }

/* fp32 -> bf16 round to nearest even: pick the nearer of the two bf16 neighbours (exact in double), ties to the
 * even one. NaN -> 0x7fc0 (torch's c10::BFloat16). */
uint16_t or_f32_to_bf16(float f) {
  if (isnan(f)) return 0x7fc0;
  uint32_t u = bits_from_f32(f);
  uint32_t lo = u & 0xffff0000u;
  if (lo == u) return (uint16_t)(u >> 16);
  uint32_t hi = lo + 0x10000u;                       /* next bf16 away from zero (may step into inf) */
  double dl = fabs((double)f - (double)f32_from_bits(lo));
  double dh = fabs((double)f32_from_bits(hi) - (double)f);
  if (isinf(f32_from_bits(hi)) && !isinf(f)) {
    /* past the largest finite bf16: the IEEE rule rounds to inf iff |f| >= max + half ulp */
    dh = fabs(ldexp(1.0, 128) - fabs((double)f));
  }
  if (dl < dh) return (uint16_t)(lo >> 16);
  if (dh < dl) return (uint16_t)(hi >> 16);
  return (uint16_t)((((lo >> 16) & 1u) == 0u) ? (lo >> 16) : (hi >> 16));
}

/* OCP e4m3fn value of a byte: exponent bias 7, 3 mantissa bits, 0x7f / 0xff NaN, no infinities. */
double or_e4m3_value(uint8_t b) {
  int em = b & 0x7f;
  if (em == 0x7f) return NAN;
  int e = em >> 3, m = em & 7;
  double v = e == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
  return (b & 0x80) ? -v : v;
}

/* fp32 -> e4m3fn, round to nearest even, by search over the 127 finite non-negative codes (values increase with
 * the code). torch's float8_e4m3fn cast semantics: |f| > 464 (= 448 + half the 448..480 step) or NaN -> 0x7f;
 * exactly 464 rounds to the even code 0x7e (448). The sign bit is kept for zero results. */
uint8_t or_f32_to_e4m3(float f) {
  uint8_t sign = signbit(f) ? 0x80 : 0x00;
  if (isnan(f)) return sign | 0x7f;
  double a = fabs((double)f);
  if (a > 464.0) return sign | 0x7f;
  if (a >= 448.0) return sign | 0x7e;
  int lo = 0, hi = 0x7e;                              /* largest code with value <= a */
  while (lo < hi) {
    int mid = (lo + hi + 1) / 2;
    if (or_e4m3_value((uint8_t)mid) <= a) lo = mid; else hi = mid - 1;
  }
  if (or_e4m3_value((uint8_t)lo) == a) return sign | (uint8_t)lo;
  double dl = a - or_e4m3_value((uint8_t)lo), dh = or_e4m3_value((uint8_t)(lo + 1)) - a;
  int c = dl < dh ? lo : (dh < dl ? lo + 1 : ((lo & 1) ? lo + 1 : lo));
  return sign | (uint8_t)c;
}

void or_f32_to_e4m3_array(const float* x, uint8_t* q, long n) {
  for (long i = 0; i < n; i++) q[i] = or_f32_to_e4m3(x[i]);
}

/* -------------------------------------------------------------- per-row fp8 quant (a3)
 * Reference: kernels/r9k_moe_mxfp4a8.hip:1729-1741 (vectorised) / :504-511 (scalar):
 *   amax = fmaxf(max |x|, 1e-12f); inv = 448.f / amax; q = e4m3_rne(x * inv); s = amax / 448.f */
void or_quant_rows_fp8(const uint16_t* x, int M, int K, long ld, uint8_t* q, float* s) {
  for (int r = 0; r < M; r++) {
    const uint16_t* xr = x + (long)r * ld;
    float m = 0.f;
    for (int k = 0; k < K; k++) m = fmaxf(m, fabsf(or_bf16_to_f32(xr[k])));
    float amax = fmaxf(m, 1e-12f);
    float inv = 448.f / amax;
    s[r] = amax / 448.f;
    for (int k = 0; k < K; k++) {
      float p = or_bf16_to_f32(xr[k]) * inv;
      q[(long)r * K + k] = or_f32_to_e4m3(p);
    }
  }
}

/* ---------------------------------------------------------- silu(gate) * up + quant (a5)
 * Reference: kernels/r9k_moe_mxfp4a8.hip:514-548: gate = first I columns, up = last I, both the stored bf16
 * values; v = g / (1 + exp(-g)) * u in fp32; then the per-row quant of a3. */
float or_silu_mul(float g, float u) { return g / (1.f + expf(-g)) * u; }

void or_silu_mul_quant_fp8(const uint16_t* gu, int M, int I, uint8_t* q, float* s, float* act) {
  for (int r = 0; r < M; r++) {
    const uint16_t* g = gu + (long)r * 2 * I;
    const uint16_t* u = g + I;
    float m = 0.f;
    for (int k = 0; k < I; k++) {
      float v = or_silu_mul(or_bf16_to_f32(g[k]), or_bf16_to_f32(u[k]));
      if (act) act[(long)r * I + k] = v;
      m = fmaxf(m, fabsf(v));
    }
    float amax = fmaxf(m, 1e-12f);
    float inv = 448.f / amax;
    s[r] = amax / 448.f;
    for (int k = 0; k < I; k++) {
      float v = or_silu_mul(or_bf16_to_f32(g[k]), or_bf16_to_f32(u[k]));
      q[(long)r * I + k] = or_f32_to_e4m3(v * inv);
    }
  }
}

/* ----------------------------------------------------------------- routing (a1)
 * Reference: kernels/r9k_moe_route.hip:67-124 (and torch.softmax(..).topk in tests/test_moe_mxfp4.py:44-45).
 * p = softmax over the row in fp32; an entry whose exp is not a finite positive number ("dead": NaN logit, a row
 * whose max is +inf, d = x - max below -87) has probability 0. Selection order: live entries by logit descending
 * (softmax is monotone in the logit), ties to the lower index; then dead entries by index. Weights are computed
 * in fp64: p_k = exp(d_k) / sum_live exp(d); renorm: w_k = p_k / sum_selected p. */
typedef struct { int live; float x; int idx; } RouteKey;

static int key_before(const RouteKey* a, const RouteKey* b) {   /* 1 if a ranks before b */
  if (a->live != b->live) return a->live;
  if (a->live && a->x != b->x) return a->x > b->x;
  return a->idx < b->idx;
}

int or_moe_route(const uint16_t* logits, long ldl, int M, int E, int topk, int renorm, float* w, int32_t* ids) {
  if (M < 1 || E < 1 || topk < 1 || topk > E) return 1;
  RouteKey* keys = (RouteKey*)malloc(sizeof(RouteKey) * E);
  double* ex = (double*)malloc(sizeof(double) * E);
  for (int r = 0; r < M; r++) {
    const uint16_t* row = logits + (long)r * ldl;
    float mx = -INFINITY;
    for (int e = 0; e < E; e++) mx = fmaxf(mx, or_bf16_to_f32(row[e]));
    double S = 0.0;
    for (int e = 0; e < E; e++) {
      float x = or_bf16_to_f32(row[e]);
      float d = x - mx;
      int live = d >= -87.f;
      keys[e].live = live;
      keys[e].x = x + 0.0f;
      keys[e].idx = e;
      ex[e] = live ? exp((double)d) : 0.0;
      S += ex[e];
    }
    /* partial selection sort: topk rounds of "best remaining" */
    double psel[64];
    for (int k = 0; k < topk; k++) {
      int b = -1;
      for (int e = 0; e < E; e++) {
        if (keys[e].idx < 0) continue;
        if (b < 0 || key_before(&keys[e], &keys[b])) b = e;
      }
      ids[(long)r * topk + k] = b;
      psel[k] = S > 0.0 ? ex[b] / S : 0.0;
      keys[b].idx = -1;                                   /* taken */
    }
    double tot = 0.0;
    for (int k = 0; k < topk; k++) tot += psel[k];
    for (int k = 0; k < topk; k++) {
      double v = psel[k];
      if (renorm) v = tot > 0.0 ? v / tot : 0.0;
      w[(long)r * topk + k] = (float)v;
    }
  }
  free(keys);
  free(ex);
  return 0;
}

/* ------------------------------------------------------------ compaction tables (a2)
 * Reference: r9700_vllm/kernels/moe.py:574-592 (align_block_size_ref): experts ascending, the expert's flat rows
 * ascending, each expert padded to a multiple of blk with `numel`; expert_ids[b] = expert or -1 past the end;
 * the whole capacity ceil((numel + E*(blk-1)) / blk) * blk is written. Rows with ids outside [0, E) are skipped. */
long or_capacity(long numel, int E, int blk) { return (numel + (long)E * (blk - 1) + blk - 1) / blk * blk; }

int or_moe_align(const int32_t* ids, long numel, int E, int blk, int32_t* sorted_ids, int32_t* expert_ids,
                 int32_t* ntpp) {
  long cap = or_capacity(numel, E, blk);
  for (long i = 0; i < cap; i++) sorted_ids[i] = (int32_t)numel;
  for (long b = 0; b < cap / blk; b++) expert_ids[b] = -1;
  long pos = 0;
  for (int e = 0; e < E; e++) {
    long c = 0;
    for (long t = 0; t < numel; t++)
      if (ids[t] == e) sorted_ids[pos + c++] = (int32_t)t;
    if (!c) continue;
    long n = (c + blk - 1) / blk * blk;
    for (long b = pos / blk; b < (pos + n) / blk; b++) expert_ids[b] = e;
    pos += n;
  }
  ntpp[0] = (int32_t)pos;
  return 0;
}

/* -------------------------------------------------------------------- top-k sum (a7)
 * Reference: kernels/r9k_moe_sum.hip:7-12, 32-56: fp32 sum over j ascending, then the shared term, one bf16 RNE. */
void or_moe_sum(const uint16_t* down, const uint16_t* shared, uint16_t* out, int M, int topk, int N, long ld_shared,
                long ld_out) {
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      float acc = 0.f;
      for (int j = 0; j < topk; j++) acc += or_bf16_to_f32(down[((long)m * topk + j) * N + n]);
      if (shared) acc += or_bf16_to_f32(shared[(long)m * ld_shared + n]);
      out[(long)m * ld_out + n] = or_f32_to_bf16(acc);
    }
}

/* --------------------------------------------------------- NVFP4 -> MXFP4 (a10)
 * Reference: r9700_vllm/quant/nvfp4.py:35-90. E2M1 values and the decision rule are the OCP MX closed forms. */
static const double E2M1[16] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0};

/* nearest E2M1 magnitude of |v| with ties to the smaller magnitude (torch.bucketize right=False on the midpoints
 * 0.25 .. 5.0), found by distance (exact in fp64); sign bit for v < 0 (not for -0.0). An infinite |v| lies past
 * every midpoint, so bucketize gives the last bucket: 6. */
uint8_t or_e2m1_encode(float v) {
  double a = fabs((double)v);
  if (isinf(a)) return (uint8_t)(7 | (v < 0.f ? 8 : 0));
  int best = 0;
  for (int c = 1; c < 8; c++) {
    double dc = fabs(a - E2M1[c]), db = fabs(a - E2M1[best]);
    if (dc < db) best = c;
  }
  return (uint8_t)(best | (v < 0.f ? 8 : 0));
}

/* smallest integer e with amax <= 6 * 2^e (brute force over the exponent range) */
int or_exp_no_clip(float amax) {
  int e = -160;
  while (ldexp(6.0, e) < (double)amax) e++;
  return e;
}

/* one 32-block: codes (32 bytes, one code each) and the chosen exponent e (unbiased) */
static int search_block(const float* x, uint8_t* codes) {
  float amax = 0.f;
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
  amax = fmaxf(amax, ldexpf(1.f, -126));
  int e0 = or_exp_no_clip(amax);
  if (e0 < -126) e0 = -126;
  if (e0 > 127) e0 = 127;
  uint8_t c0[32], c1[32];
  double err[2];
  for (int d = 0; d <= 1; d++) {
    int e = e0 - d;
    if (e < -127) e = -127;
    if (e > 127) e = 127;
    float s = ldexpf(1.f, e);
    uint8_t* c = d ? c1 : c0;
    double acc = 0.0;
    for (int i = 0; i < 32; i++) {
      c[i] = or_e2m1_encode(x[i] / s);
      double dv = E2M1[c[i]] * (double)s - (double)x[i];
      acc += dv * dv;
    }
    err[d] = acc;
  }
  int e = e0;
  const uint8_t* c = c0;
  if (err[1] < err[0]) {
    e = e0 - 1 < -127 ? -127 : e0 - 1;
    c = c1;
  }
  memcpy(codes, c, 32);
  return e;
}

/* exact NVFP4 dequant (nvfp4.py:39-46): v = E2M1[c] * float(s16) (fp32), then / row_div (fp32 division) */
void or_dequant_nvfp4(const uint8_t* packed, const uint8_t* s16, const float* row_div, int N, int K, float* out) {
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      uint8_t p = packed[(long)n * (K / 2) + k / 2];
      int c = (k & 1) ? (p >> 4) : (p & 15);
      float sc = (float)or_e4m3_value(s16[(long)n * (K / 16) + k / 16]);
      float v = (float)E2M1[c] * sc;
      out[(long)n * K + k] = v / row_div[n];
    }
}

/* MSE-searched MXFP4 of fp32 weights [N, K] (nvfp4.py:54-75): packed [N, K/2], e8m0 [N, K/32] */
void or_quantize_mxfp4_search(const float* w, int N, int K, uint8_t* out_p, uint8_t* out_e) {
  uint8_t codes[32];
  for (int n = 0; n < N; n++)
    for (int b = 0; b < K / 32; b++) {
      int e = search_block(w + (long)n * K + b * 32, codes);
      out_e[(long)n * (K / 32) + b] = (uint8_t)(e + 127);
      for (int i = 0; i < 16; i++)
        out_p[(long)n * (K / 2) + b * 16 + i] = (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
    }
}

/* NVFP4 -> MXFP4 (nvfp4.py:78-90): dequant then the search */
void or_nvfp4_to_mxfp4(const uint8_t* packed, const uint8_t* s16, const float* row_div, int N, int K, uint8_t* out_p,
                       uint8_t* out_e) {
  float* row = (float*)malloc(sizeof(float) * K);
  for (int n = 0; n < N; n++) {
    or_dequant_nvfp4(packed + (long)n * (K / 2), s16 + (long)n * (K / 16), row_div + n, 1, K, row);
    or_quantize_mxfp4_search(row, 1, K, out_p + (long)n * (K / 2), out_e + (long)n * (K / 32));
  }
  free(row);
}
