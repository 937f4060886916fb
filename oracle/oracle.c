/*
 * CPU oracle for the quantized-weight hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Loaded by tests/, __graft_entry__.smoke() (as the checker) and bench.py's
 * cpu_baseline leg (as the timed CPU port).  Nothing in the product library
 * links or calls it.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off so
 * that no multiply-add is fused: Rust never contracts, dequant.rs is IEEE
 * mul/sub step by step).
 *
 * Reference citations are /root/reference paths.
 */
#include "oracle.h"

#include "../mlx-llm_amd/csrc/iq_tables.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* SplitMix64 -- src/primitives/sampler.rs:40-60                      */
/* ------------------------------------------------------------------ */
uint64_t orc_splitmix64_next(uint64_t* s) {
  *s += 0x9E3779B97F4A7C15ull; /* sampler.rs:41 INCREMENT */
  uint64_t z = *s;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float orc_splitmix64_next_f32(uint64_t* s) {
  /* sampler.rs:57-59: 24-bit mantissa in [0,1) */
  return (float)(orc_splitmix64_next(s) >> 40) / (float)(1u << 24);
}

void orc_gen_normal_f32(uint64_t seed, float mean, float std, float* out,
                        size_t n) {
  /* Box-Muller in f64 on two 53-bit uniforms; u1 in (0,1]. */
  uint64_t st = seed;
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    double u1 = ((double)(orc_splitmix64_next(&st) >> 11) + 1.0) *
                (1.0 / 9007199254740992.0);
    double u2 = (double)(orc_splitmix64_next(&st) >> 11) *
                (1.0 / 9007199254740992.0);
    double r = sqrt(-2.0 * log(u1));
    double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
    out[i++] = (float)(mean + std * z0);
    if (i < n) out[i++] = (float)(mean + std * z1);
  }
}

/* ------------------------------------------------------------------ */
/* scalar conversions                                                  */
/* ------------------------------------------------------------------ */
static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* Exact IEEE binary16 -> binary32 (`half::f16::to_f32`); NaNs are quieted
 * the way `half` does (quiet bit set, payload kept). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0x1F) {
    if (man == 0) return bits_f32(sign | 0x7F800000u);
    return bits_f32(sign | 0x7FC00000u | (man << 13));
  }
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    /* subnormal: man * 2^-24, exact in f32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t abs = u & 0x7FFFFFFFu;
  if (abs >= 0x7F800000u) /* inf / nan */
    return (uint16_t)(sign | 0x7C00u | (abs > 0x7F800000u ? 0x200u : 0u));
  if (abs >= 0x477FF000u) /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7C00u);
  if (abs < 0x38800000u) { /* result subnormal (or zero) */
    if (abs < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
    uint32_t e = abs >> 23;
    uint32_t m = (abs & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e; /* value = m * 2^(e-150); want units of 2^-24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t r = abs + 0xFFFu + ((abs >> 13) & 1u); /* RNE on the 13 dropped bits */
  return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* ------------------------------------------------------------------ */
/* GGUF geometry -- src/gguf/dequant.rs:85-153                         */
/* ------------------------------------------------------------------ */
int orc_gguf_block(uint32_t tag, int64_t* elems, int64_t* bytes) {
  int64_t e, b;
  switch (tag) {
    case 0: e = 1; b = 4; break;        /* F32 */
    case 1: case 30: e = 1; b = 2; break; /* F16, BF16 */
    case 2: e = 32; b = 18; break;      /* Q4_0 */
    case 3: e = 32; b = 20; break;      /* Q4_1 */
    case 6: e = 32; b = 22; break;      /* Q5_0 */
    case 7: e = 32; b = 24; break;      /* Q5_1 */
    case 8: e = 32; b = 34; break;      /* Q8_0 */
    case 10: e = 256; b = 84; break;    /* Q2_K */
    case 11: e = 256; b = 110; break;   /* Q3_K */
    case 12: e = 256; b = 144; break;   /* Q4_K */
    case 13: e = 256; b = 176; break;   /* Q5_K */
    case 14: e = 256; b = 210; break;   /* Q6_K */
    case 20: e = 32; b = 18; break;     /* IQ4_NL */
    case 23: e = 256; b = 136; break;   /* IQ4_XS */
    case 16: e = 256; b = 66; break;    /* IQ2_XXS */
    case 17: e = 256; b = 74; break;    /* IQ2_XS */
    case 22: e = 256; b = 82; break;    /* IQ2_S */
    case 18: e = 256; b = 98; break;    /* IQ3_XXS */
    case 21: e = 256; b = 110; break;   /* IQ3_S */
    case 19: e = 256; b = 50; break;    /* IQ1_S */
    case 29: e = 256; b = 56; break;    /* IQ1_M */
    default: return 3;                  /* dequant.rs:109-111 Unsupported */
  }
  if (elems) *elems = e;
  if (bytes) *bytes = b;
  return 0;
}

int orc_gguf_tensor_byte_len(uint32_t tag, int64_t n, int64_t* bytes) {
  int64_t be, bb;
  int rc = orc_gguf_block(tag, &be, &bb);
  if (rc) return rc;
  if (n < 0 || n % be) return 2; /* dequant.rs:147-151 */
  *bytes = (n / be) * bb;
  return 0;
}

static const int8_t KV_IQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                    1,    13,   25,  38,  53,  69,  89,  113};

static float rd_f16(const uint8_t* b, int i) { /* dequant.rs:222-225 */
  return orc_f16_to_f32((uint16_t)(b[i] | (b[i + 1] << 8)));
}

static void dq_q4_0(const uint8_t* b, float* y) { /* dequant.rs:228-237 */
  float d = rd_f16(b, 0);
  const uint8_t* qs = b + 2;
  for (int j = 0; j < 16; j++) {
    int x0 = (qs[j] & 0x0F) - 8;
    int x1 = (qs[j] >> 4) - 8;
    y[j] = (float)x0 * d;
    y[j + 16] = (float)x1 * d;
  }
}

static void dq_q4_1(const uint8_t* b, float* y) { /* dequant.rs:239-247 */
  float d = rd_f16(b, 0), m = rd_f16(b, 2);
  const uint8_t* qs = b + 4;
  for (int j = 0; j < 16; j++) {
    y[j] = (float)(qs[j] & 0x0F) * d + m;
    y[j + 16] = (float)(qs[j] >> 4) * d + m;
  }
}

static uint32_t rd_u32(const uint8_t* b) {
  return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) |
         ((uint32_t)b[3] << 24);
}

static void dq_q5_0(const uint8_t* b, float* y) { /* dequant.rs:249-261 */
  float d = rd_f16(b, 0);
  uint32_t qh = rd_u32(b + 2);
  const uint8_t* qs = b + 6;
  for (int j = 0; j < 16; j++) {
    uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10);
    uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
    int x0 = ((qs[j] & 0x0F) | xh0) - 16;
    int x1 = ((qs[j] >> 4) | xh1) - 16;
    y[j] = (float)x0 * d;
    y[j + 16] = (float)x1 * d;
  }
}

static void dq_q5_1(const uint8_t* b, float* y) { /* dequant.rs:263-276 */
  float d = rd_f16(b, 0), m = rd_f16(b, 2);
  uint32_t qh = rd_u32(b + 4);
  const uint8_t* qs = b + 8;
  for (int j = 0; j < 16; j++) {
    uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10);
    uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
    float x0 = (float)((qs[j] & 0x0F) | xh0);
    float x1 = (float)((qs[j] >> 4) | xh1);
    y[j] = x0 * d + m;
    y[j + 16] = x1 * d + m;
  }
}

static void dq_q8_0(const uint8_t* b, float* y) { /* dequant.rs:278-284 */
  float d = rd_f16(b, 0);
  for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

static void dq_q2_k(const uint8_t* b, float* y) { /* dequant.rs:288-318 */
  const uint8_t* scales = b;
  const uint8_t* qs = b + 16;
  float d = rd_f16(b, 80), dmin = rd_f16(b, 82);
  int is = 0, yi = 0;
  for (int n = 0; n < 256; n += 128) {
    const uint8_t* q = qs + n / 4;
    int shift = 0;
    for (int r = 0; r < 4; r++) {
      uint8_t sc = scales[is++];
      float dl = d * (float)(sc & 0xF);
      float ml = dmin * (float)(sc >> 4);
      for (int l = 0; l < 16; l++) y[yi++] = dl * (float)((q[l] >> shift) & 3) - ml;
      sc = scales[is++];
      dl = d * (float)(sc & 0xF);
      ml = dmin * (float)(sc >> 4);
      for (int l = 16; l < 32; l++) y[yi++] = dl * (float)((q[l] >> shift) & 3) - ml;
      shift += 2;
    }
  }
}

static void dq_q3_k(const uint8_t* b, float* y) { /* dequant.rs:320-371 */
  const uint32_t KMASK1 = 0x03030303u, KMASK2 = 0x0f0f0f0fu;
  const uint8_t* hmask = b;
  const uint8_t* qs = b + 32;
  const uint8_t* sr = b + 96;
  float d_all = rd_f16(b, 108);
  uint32_t aux[4] = {rd_u32(sr), rd_u32(sr + 4), rd_u32(sr + 8), 0};
  uint32_t tmp = aux[2];
  aux[2] = ((aux[0] >> 4) & KMASK2) | (((tmp >> 4) & KMASK1) << 4);
  aux[3] = ((aux[1] >> 4) & KMASK2) | (((tmp >> 6) & KMASK1) << 4);
  aux[0] = (aux[0] & KMASK2) | ((tmp & KMASK1) << 4);
  aux[1] = (aux[1] & KMASK2) | (((tmp >> 2) & KMASK1) << 4);
  int8_t scales[16];
  for (int k = 0; k < 16; k++) scales[k] = (int8_t)((aux[k / 4] >> (8 * (k % 4))) & 0xFF);
  int is = 0, yi = 0, q_off = 0;
  uint8_t m = 1;
  for (int n = 0; n < 256; n += 128) {
    int shift = 0;
    for (int r = 0; r < 4; r++) {
      float dl = d_all * (float)(scales[is++] - 32);
      for (int l = 0; l < 16; l++) {
        int hbit = (hmask[l] & m) ? 0 : 4;
        y[yi++] = dl * (float)(((qs[q_off + l] >> shift) & 3) - hbit);
      }
      dl = d_all * (float)(scales[is++] - 32);
      for (int l = 0; l < 16; l++) {
        int hbit = (hmask[l + 16] & m) ? 0 : 4;
        y[yi++] = dl * (float)(((qs[q_off + l + 16] >> shift) & 3) - hbit);
      }
      shift += 2;
      m = (uint8_t)(m << 1);
    }
    q_off += 32;
  }
}

static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  /* dequant.rs:375-383 */
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

static void dq_q4_k(const uint8_t* b, float* y) { /* dequant.rs:385-410 */
  float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
  const uint8_t* scales = b + 4;
  const uint8_t* qs = b + 16;
  int is = 0, yi = 0;
  for (int j = 0; j < 256; j += 64) {
    const uint8_t* q = qs + j / 2;
    uint8_t sc, m;
    scale_min_k4(is, scales, &sc, &m);
    float d1 = d * (float)sc, m1 = dmin * (float)m;
    scale_min_k4(is + 1, scales, &sc, &m);
    float d2 = d * (float)sc, m2 = dmin * (float)m;
    for (int l = 0; l < 32; l++) y[yi++] = d1 * (float)(q[l] & 0xF) - m1;
    for (int l = 0; l < 32; l++) y[yi++] = d2 * (float)(q[l] >> 4) - m2;
    is += 2;
  }
}

static void dq_q5_k(const uint8_t* b, float* y) { /* dequant.rs:412-444 */
  float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
  const uint8_t* scales = b + 4;
  const uint8_t* qh = b + 16;
  const uint8_t* qs = b + 48;
  int is = 0, yi = 0;
  uint8_t u1 = 1, u2 = 2;
  for (int j = 0; j < 256; j += 64) {
    const uint8_t* ql = qs + j / 2;
    uint8_t sc, m;
    scale_min_k4(is, scales, &sc, &m);
    float d1 = d * (float)sc, m1 = dmin * (float)m;
    scale_min_k4(is + 1, scales, &sc, &m);
    float d2 = d * (float)sc, m2 = dmin * (float)m;
    for (int l = 0; l < 32; l++) {
      int hi = (qh[l] & u1) ? 16 : 0;
      y[yi++] = d1 * (float)((ql[l] & 0xF) + hi) - m1;
    }
    for (int l = 0; l < 32; l++) {
      int hi = (qh[l] & u2) ? 16 : 0;
      y[yi++] = d2 * (float)((ql[l] >> 4) + hi) - m2;
    }
    is += 2;
    u1 = (uint8_t)(u1 << 2);
    u2 = (uint8_t)(u2 << 2);
  }
}

static void dq_q6_k(const uint8_t* b, float* y) { /* dequant.rs:446-468 */
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const uint8_t* scales = b + 192;
  float d = rd_f16(b, 208);
  for (int n = 0; n < 256; n += 128) {
    int idx = n / 128;
    const uint8_t* qlp = ql + 64 * idx;
    const uint8_t* qhp = qh + 32 * idx;
    int sco = 8 * idx;
    for (int l = 0; l < 32; l++) {
      int is = l / 16;
      int8_t q1 = (int8_t)((int8_t)((qlp[l] & 0x0F) | ((qhp[l] & 3) << 4)) - 32);
      int8_t q2 = (int8_t)((int8_t)((qlp[l + 32] & 0x0F) | (((qhp[l] >> 2) & 3) << 4)) - 32);
      int8_t q3 = (int8_t)((int8_t)((qlp[l] >> 4) | (((qhp[l] >> 4) & 3) << 4)) - 32);
      int8_t q4 = (int8_t)((int8_t)((qlp[l + 32] >> 4) | (((qhp[l] >> 6) & 3) << 4)) - 32);
      /* left-to-right: (d * scale) * q, dequant.rs:462-465 */
      y[n + l] = d * (float)(int8_t)scales[sco + is] * (float)q1;
      y[n + l + 32] = d * (float)(int8_t)scales[sco + is + 2] * (float)q2;
      y[n + l + 64] = d * (float)(int8_t)scales[sco + is + 4] * (float)q3;
      y[n + l + 96] = d * (float)(int8_t)scales[sco + is + 6] * (float)q4;
    }
  }
}

static void dq_iq4_nl(const uint8_t* b, float* y) { /* dequant.rs:472-479 */
  float d = rd_f16(b, 0);
  const uint8_t* qs = b + 2;
  for (int j = 0; j < 16; j++) {
    y[j] = d * (float)KV_IQ4NL[qs[j] & 0xF];
    y[j + 16] = d * (float)KV_IQ4NL[qs[j] >> 4];
  }
}

static void dq_iq4_xs(const uint8_t* b, float* y) { /* dequant.rs:481-497 */
  float d = rd_f16(b, 0);
  uint16_t sh = (uint16_t)(b[2] | (b[3] << 8));
  const uint8_t* sl = b + 4;
  const uint8_t* qs = b + 8;
  for (int ib = 0; ib < 8; ib++) {
    int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
    float dl = d * (float)(ls - 32);
    const uint8_t* q = qs + ib * 16;
    for (int j = 0; j < 16; j++) {
      y[ib * 32 + j] = dl * (float)KV_IQ4NL[q[j] & 0xF];
      y[ib * 32 + j + 16] = dl * (float)KV_IQ4NL[q[j] >> 4];
    }
  }
}

/* IQ grid types -- dequant.rs:505-723.  The codebooks are the format's
 * fixed tables (mlx-llm_amd/csrc/iq_tables.h, the reference's
 * src/gguf/iq_grids.rs); the sign table ksigns_iq2xs is its closed form:
 * entry i is i with bit 7 set to the parity of i (every sign byte has an
 * even number of set bits). */
static const uint64_t IQ2XXS[256] = {MLXQ_IQ2XXS_GRID};
static const uint64_t IQ2XS[512] = {MLXQ_IQ2XS_GRID};
static const uint64_t IQ2S[1024] = {MLXQ_IQ2S_GRID};
static const uint32_t IQ3XXS[256] = {MLXQ_IQ3XXS_GRID};
static const uint32_t IQ3S[512] = {MLXQ_IQ3S_GRID};
static const uint64_t IQ1S[2048] = {MLXQ_IQ1S_GRID};
#define IQ1S_DELTA 0.125f /* dequant.rs:26-27 */

uint8_t orc_ksigns_iq2xs(int i) {
  int p = __builtin_popcount((unsigned)i & 127u) & 1;
  return (uint8_t)((i & 127) | (p << 7));
}

int orc_iq_grid(int table, int i, uint64_t* entry) {
  static const int sizes[6] = {256, 512, 1024, 256, 512, 2048};
  if (table < 0 || table > 5) return -1;
  if (!entry) return sizes[table];
  if (i < 0 || i >= sizes[table]) return -1;
  switch (table) {
    case 0: *entry = IQ2XXS[i]; break;
    case 1: *entry = IQ2XS[i]; break;
    case 2: *entry = IQ2S[i]; break;
    case 3: *entry = IQ3XXS[i]; break;
    case 4: *entry = IQ3S[i]; break;
    default: *entry = IQ1S[i]; break;
  }
  return sizes[table];
}

/* sign of output lane j for a sign byte: -1 where bit j is set (dequant.rs:508-516) */
static float iq_sign(uint8_t signs, int j) { return (signs >> j) & 1 ? -1.0f : 1.0f; }
static uint8_t grid_byte(uint64_t g, int j) { return (uint8_t)(g >> (8 * j)); }

static void dq_iq2_xxs(const uint8_t* b, float* y) { /* dequant.rs:521-539 */
  float d = rd_f16(b, 0);
  for (int ib32 = 0; ib32 < 8; ib32++) {
    const uint8_t* q = b + 2 + 8 * ib32;
    uint32_t aux0 = rd_u32(q), aux1 = rd_u32(q + 4);
    float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
    for (int l = 0; l < 4; l++) {
      uint64_t g = IQ2XXS[(aux0 >> (8 * l)) & 255];
      uint8_t signs = orc_ksigns_iq2xs((aux1 >> (7 * l)) & 127);
      for (int j = 0; j < 8; j++) y[32 * ib32 + 8 * l + j] = db * (float)grid_byte(g, j) * iq_sign(signs, j);
    }
  }
}

static void dq_iq2_xs(const uint8_t* b, float* y) { /* dequant.rs:543-564 */
  float d = rd_f16(b, 0);
  for (int ib32 = 0; ib32 < 8; ib32++) {
    uint8_t sc = b[66 + ib32];
    float db[2] = {d * (0.5f + (float)(sc & 0xF)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
    for (int l = 0; l < 4; l++) {
      int qo = 2 + 2 * (4 * ib32 + l);
      uint16_t q = (uint16_t)(b[qo] | (b[qo + 1] << 8));
      uint64_t g = IQ2XS[q & 511];
      uint8_t signs = orc_ksigns_iq2xs(q >> 9);
      for (int j = 0; j < 8; j++) y[32 * ib32 + 8 * l + j] = db[l / 2] * (float)grid_byte(g, j) * iq_sign(signs, j);
    }
  }
}

static void dq_iq2_s(const uint8_t* b, float* y) { /* dequant.rs:568-591 */
  float d = rd_f16(b, 0);
  const uint8_t* qs = b + 2;
  const uint8_t* qh = b + 66;
  const uint8_t* scales = b + 74;
  for (int ib32 = 0; ib32 < 8; ib32++) {
    uint8_t sc = scales[ib32];
    float db[2] = {d * (0.5f + (float)(sc & 0xF)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
    for (int l = 0; l < 4; l++) {
      int idx = qs[4 * ib32 + l] | (((int)qh[ib32] << (8 - 2 * l)) & 0x300);
      uint64_t g = IQ2S[idx];
      uint8_t signs = qs[32 + 4 * ib32 + l];
      for (int j = 0; j < 8; j++) y[32 * ib32 + 8 * l + j] = db[l / 2] * (float)grid_byte(g, j) * iq_sign(signs, j);
    }
  }
}

static void dq_iq3_xxs(const uint8_t* b, float* y) { /* dequant.rs:596-615 */
  float d = rd_f16(b, 0);
  const uint8_t* ss = b + 66;
  for (int ib32 = 0; ib32 < 8; ib32++) {
    uint32_t aux = rd_u32(ss + 4 * ib32);
    float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    const uint8_t* q = b + 2 + 8 * ib32;
    for (int l = 0; l < 4; l++) {
      uint32_t g1 = IQ3XXS[q[2 * l]], g2 = IQ3XXS[q[2 * l + 1]];
      uint8_t signs = orc_ksigns_iq2xs((aux >> (7 * l)) & 127);
      for (int j = 0; j < 4; j++) {
        y[32 * ib32 + 8 * l + j] = db * (float)grid_byte(g1, j) * iq_sign(signs, j);
        y[32 * ib32 + 8 * l + j + 4] = db * (float)grid_byte(g2, j) * iq_sign(signs, j + 4);
      }
    }
  }
}

static void dq_iq3_s(const uint8_t* b, float* y) { /* dequant.rs:619-651 */
  float d = rd_f16(b, 0);
  const uint8_t* qh = b + 66;
  const uint8_t* signs = b + 74;
  const uint8_t* scales = b + 106;
  int yi = 0;
  for (int k = 0; k < 4; k++) {
    uint8_t sc = scales[k];
    float dbs[2] = {d * (float)(1 + 2 * (sc & 0xF)), d * (float)(1 + 2 * (sc >> 4))};
    for (int half = 0; half < 2; half++) {
      float db = dbs[half];
      uint32_t qhb = qh[2 * k + half];
      const uint8_t* q = b + 2 + 16 * k + 8 * half;
      const uint8_t* sg = signs + 8 * k + 4 * half;
      for (int l = 0; l < 4; l++) {
        int i1 = q[2 * l] | (int)((qhb << (8 - 2 * l)) & 256);
        int i2 = q[2 * l + 1] | (int)((qhb << (7 - 2 * l)) & 256);
        uint32_t g1 = IQ3S[i1], g2 = IQ3S[i2];
        for (int j = 0; j < 4; j++) {
          y[yi + j] = db * (float)grid_byte(g1, j) * iq_sign(sg[l], j);
          y[yi + j + 4] = db * (float)grid_byte(g2, j) * iq_sign(sg[l], j + 4);
        }
        yi += 8;
      }
    }
  }
}

static void dq_iq1_s(const uint8_t* b, float* y) { /* dequant.rs:655-673 */
  float d = rd_f16(b, 0);
  const uint8_t* qs = b + 2;
  const uint8_t* qh = b + 34;
  for (int ib = 0; ib < 8; ib++) {
    uint16_t h = (uint16_t)(qh[2 * ib] | (qh[2 * ib + 1] << 8));
    float dl = d * (float)(2 * ((h >> 12) & 7) + 1);
    float delta = (h & 0x8000) ? -IQ1S_DELTA : IQ1S_DELTA;
    for (int l = 0; l < 4; l++) {
      int idx = qs[4 * ib + l] | (((h >> (3 * l)) & 7) << 8);
      uint64_t g = IQ1S[idx];
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = dl * ((float)(int8_t)grid_byte(g, j) + delta);
    }
  }
}

static void dq_iq1_m(const uint8_t* b, float* y) { /* dequant.rs:678-719 */
  const uint8_t* qs = b;
  const uint8_t* qh = b + 32;
  uint16_t sc[4];
  for (int i = 0; i < 4; i++) sc[i] = (uint16_t)(b[48 + 2 * i] | (b[49 + 2 * i] << 8));
  uint16_t bits = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0) | ((sc[2] >> 4) & 0x0F00) | (sc[3] & 0xF000));
  float d = orc_f16_to_f32(bits);
  for (int ib = 0; ib < 8; ib++) {
    uint16_t w = sc[ib / 2];
    int shift = 6 * (ib % 2);
    float dl1 = d * (float)(2 * ((w >> shift) & 7) + 1);
    float dl2 = d * (float)(2 * ((w >> (shift + 3)) & 7) + 1);
    int qh0 = qh[2 * ib], qh1 = qh[2 * ib + 1];
    int idx[4] = {qs[4 * ib] | ((qh0 << 8) & 0x700), qs[4 * ib + 1] | ((qh0 << 4) & 0x700),
                  qs[4 * ib + 2] | ((qh1 << 8) & 0x700), qs[4 * ib + 3] | ((qh1 << 4) & 0x700)};
    float delta[4] = {(qh0 & 0x08) ? -IQ1S_DELTA : IQ1S_DELTA, (qh0 & 0x80) ? -IQ1S_DELTA : IQ1S_DELTA,
                      (qh1 & 0x08) ? -IQ1S_DELTA : IQ1S_DELTA, (qh1 & 0x80) ? -IQ1S_DELTA : IQ1S_DELTA};
    for (int l = 0; l < 4; l++) {
      float dl = l < 2 ? dl1 : dl2;
      uint64_t g = IQ1S[idx[l]];
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = dl * ((float)(int8_t)grid_byte(g, j) + delta[l]);
    }
  }
}

typedef void (*dq_fn)(const uint8_t*, float*);
static dq_fn dq_for(uint32_t tag) {
  switch (tag) {
    case 2: return dq_q4_0;
    case 3: return dq_q4_1;
    case 6: return dq_q5_0;
    case 7: return dq_q5_1;
    case 8: return dq_q8_0;
    case 10: return dq_q2_k;
    case 11: return dq_q3_k;
    case 12: return dq_q4_k;
    case 13: return dq_q5_k;
    case 14: return dq_q6_k;
    case 20: return dq_iq4_nl;
    case 23: return dq_iq4_xs;
    case 16: return dq_iq2_xxs;
    case 17: return dq_iq2_xs;
    case 22: return dq_iq2_s;
    case 18: return dq_iq3_xxs;
    case 21: return dq_iq3_s;
    case 19: return dq_iq1_s;
    case 29: return dq_iq1_m;
    default: return NULL;
  }
}

static int dequant_impl(uint32_t tag, const uint8_t* data, int64_t data_len,
                        int64_t n, float* out, int threads) {
  int64_t be, bb;
  int rc = orc_gguf_block(tag, &be, &bb);
  if (rc) return rc;
  if (n < 0 || n % be) return 2;          /* dequant.rs:159-163 */
  int64_t nblocks = n / be;
  if (data_len < nblocks * bb) return 4;  /* dequant.rs:166-171 */
  if (tag == 0) {
    memcpy(out, data, (size_t)n * 4);
    return 0;
  }
  if (tag == 1 || tag == 30) {
    for (int64_t i = 0; i < n; i++) {
      uint16_t h = (uint16_t)(data[2 * i] | (data[2 * i + 1] << 8));
      out[i] = tag == 1 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
    }
    return 0;
  }
  dq_fn f = dq_for(tag);
  if (!f) return 3;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
#endif
  for (int64_t blk = 0; blk < nblocks; blk++) f(data + blk * bb, out + blk * be);
  (void)threads;
  return 0;
}

int orc_gguf_dequantize(uint32_t tag, const uint8_t* data, int64_t data_len,
                        int64_t n, float* out) {
  return dequant_impl(tag, data, data_len, n, out, 1);
}

int orc_gguf_dequantize_mt(uint32_t tag, const uint8_t* data, int64_t data_len,
                           int64_t n, float* out, int threads) {
  return dequant_impl(tag, data, data_len, n, out, threads);
}

/* ------------------------------------------------------------------ */
/* GGUF block producers (llama.cpp public block layouts; not in the    */
/* reference -- only used to make realistic test blocks)               */
/* ------------------------------------------------------------------ */
static void wr_f16(uint8_t* b, float v) {
  uint16_t h = orc_f32_to_f16(v);
  b[0] = (uint8_t)(h & 0xFF);
  b[1] = (uint8_t)(h >> 8);
}

static int nearest_kv(float v) {
  int best = 0;
  float bd = fabsf(v - (float)KV_IQ4NL[0]);
  for (int i = 1; i < 16; i++) {
    float dd = fabsf(v - (float)KV_IQ4NL[i]);
    if (dd < bd) { bd = dd; best = i; }
  }
  return best;
}

static void qz_q4_0(const float* x, uint8_t* b) {
  float amax = 0.f, mx = 0.f;
  for (int j = 0; j < 32; j++)
    if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
  float d = mx / -8.f;
  float id = d != 0.f ? 1.f / d : 0.f;
  wr_f16(b, d);
  for (int j = 0; j < 16; j++) {
    int x0 = (int)(x[j] * id + 8.5f), x1 = (int)(x[j + 16] * id + 8.5f);
    x0 = x0 < 0 ? 0 : x0 > 15 ? 15 : x0;
    x1 = x1 < 0 ? 0 : x1 > 15 ? 15 : x1;
    b[2 + j] = (uint8_t)(x0 | (x1 << 4));
  }
}

static void qz_q8_0(const float* x, uint8_t* b) {
  float amax = 0.f;
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
  float d = amax / 127.f;
  float id = d != 0.f ? 1.f / d : 0.f;
  wr_f16(b, d);
  for (int j = 0; j < 32; j++) {
    float q = roundf(x[j] * id);
    q = q < -128.f ? -128.f : q > 127.f ? 127.f : q;
    b[2 + j] = (uint8_t)(int8_t)q;
  }
}

static void qz_iq4_nl(const float* x, uint8_t* b) {
  float amax = 0.f, mx = 0.f;
  for (int j = 0; j < 32; j++)
    if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); mx = x[j]; }
  float d = mx / -127.f;
  wr_f16(b, d);
  float dq = orc_f16_to_f32(orc_f32_to_f16(d));
  float id = dq != 0.f ? 1.f / dq : 0.f;
  for (int j = 0; j < 16; j++) {
    int i0 = nearest_kv(x[j] * id), i1 = nearest_kv(x[j + 16] * id);
    b[2 + j] = (uint8_t)(i0 | (i1 << 4));
  }
}

static void qz_iq4_xs(const float* x, uint8_t* b) {
  float dsub[8], dmax = 0.f, dmaxs = 0.f;
  for (int ib = 0; ib < 8; ib++) {
    float amax = 0.f, mx = 0.f;
    for (int j = 0; j < 32; j++)
      if (fabsf(x[ib * 32 + j]) > amax) { amax = fabsf(x[ib * 32 + j]); mx = x[ib * 32 + j]; }
    dsub[ib] = mx / -127.f;
    if (fabsf(dsub[ib]) > dmax) { dmax = fabsf(dsub[ib]); dmaxs = dsub[ib]; }
  }
  float d = dmaxs / -32.f;
  wr_f16(b, d);
  float dq = orc_f16_to_f32(orc_f32_to_f16(d));
  float idq = dq != 0.f ? 1.f / dq : 0.f;
  uint16_t sh = 0;
  memset(b + 4, 0, 4);
  for (int ib = 0; ib < 8; ib++) {
    int l = (int)lrintf(dsub[ib] * idq);
    l = l < -32 ? -32 : l > 31 ? 31 : l;
    int ls = l + 32;
    b[4 + ib / 2] |= (uint8_t)((ls & 0xF) << (4 * (ib % 2)));
    sh |= (uint16_t)(((ls >> 4) & 3) << (2 * ib));
    float dl = dq * (float)l;
    float id = dl != 0.f ? 1.f / dl : 0.f;
    for (int j = 0; j < 16; j++) {
      int i0 = nearest_kv(x[ib * 32 + j] * id), i1 = nearest_kv(x[ib * 32 + j + 16] * id);
      b[8 + ib * 16 + j] = (uint8_t)(i0 | (i1 << 4));
    }
  }
  b[2] = (uint8_t)(sh & 0xFF);
  b[3] = (uint8_t)(sh >> 8);
}

static void qz_q4_k(const float* x, uint8_t* b) {
  float sc[8], mn[8], msc = 0.f, mmn = 0.f;
  for (int j = 0; j < 8; j++) {
    float lo = 0.f, hi = -INFINITY;
    for (int l = 0; l < 32; l++) {
      lo = fminf(lo, x[32 * j + l]);
      hi = fmaxf(hi, x[32 * j + l]);
    }
    sc[j] = (hi - lo) / 15.f;
    mn[j] = -lo;
    msc = fmaxf(msc, sc[j]);
    mmn = fmaxf(mmn, mn[j]);
  }
  float d = msc / 63.f, dmin = mmn / 63.f;
  wr_f16(b, d);
  wr_f16(b + 2, dmin);
  float dq = rd_f16(b, 0), dmq = rd_f16(b, 2);
  uint8_t* s = b + 4;
  memset(s, 0, 12);
  uint8_t ls[8], lm[8];
  for (int j = 0; j < 8; j++) {
    int a = dq > 0.f ? (int)lrintf(sc[j] / dq) : 0;
    int c = dmq > 0.f ? (int)lrintf(mn[j] / dmq) : 0;
    ls[j] = (uint8_t)(a < 0 ? 0 : a > 63 ? 63 : a);
    lm[j] = (uint8_t)(c < 0 ? 0 : c > 63 ? 63 : c);
  }
  for (int j = 0; j < 8; j++) { /* inverse of dequant.rs:375-383 */
    if (j < 4) {
      s[j] |= ls[j];
      s[j + 4] |= lm[j];
    } else {
      s[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
      s[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
      s[j] |= (uint8_t)((lm[j] >> 4) << 6);
    }
  }
  uint8_t q[256];
  for (int j = 0; j < 8; j++) {
    float dl = dq * (float)ls[j], ml = dmq * (float)lm[j];
    for (int l = 0; l < 32; l++) {
      int v = dl > 0.f ? (int)lrintf((x[32 * j + l] + ml) / dl) : 0;
      q[32 * j + l] = (uint8_t)(v < 0 ? 0 : v > 15 ? 15 : v);
    }
  }
  for (int j = 0; j < 4; j++)
    for (int l = 0; l < 32; l++)
      b[16 + 32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
}

static void qz_q6_k(const float* x, uint8_t* b) {
  float s[16], amx = 0.f;
  for (int sb = 0; sb < 16; sb++) {
    float amax = 0.f, mx = 0.f;
    for (int l = 0; l < 16; l++)
      if (fabsf(x[16 * sb + l]) > amax) { amax = fabsf(x[16 * sb + l]); mx = x[16 * sb + l]; }
    s[sb] = mx / -32.f;
    amx = fmaxf(amx, fabsf(s[sb]));
  }
  float d = amx / 127.f;
  wr_f16(b + 208, d);
  float dq = rd_f16(b, 208);
  uint8_t q[256];
  for (int sb = 0; sb < 16; sb++) {
    int sc = dq > 0.f ? (int)lrintf(s[sb] / dq) : 0;
    sc = sc < -128 ? -128 : sc > 127 ? 127 : sc;
    b[192 + sb] = (uint8_t)(int8_t)sc;
    float dl = dq * (float)sc;
    for (int l = 0; l < 16; l++) {
      int v = dl != 0.f ? (int)lrintf(x[16 * sb + l] / dl) : 0;
      v = v < -32 ? -32 : v > 31 ? 31 : v;
      q[16 * sb + l] = (uint8_t)(v + 32);
    }
  }
  for (int n = 0; n < 256; n += 128) { /* inverse of dequant.rs:451-467 */
    int idx = n / 128;
    for (int l = 0; l < 32; l++) {
      uint8_t q1 = q[n + l], q2 = q[n + l + 32], q3 = q[n + l + 64], q4 = q[n + l + 96];
      b[64 * idx + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      b[64 * idx + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      b[128 + 32 * idx + l] =
          (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  }
}

int orc_gguf_quantize(uint32_t tag, const float* x, int64_t n, uint8_t* out) {
  int64_t be, bb;
  int rc = orc_gguf_block(tag, &be, &bb);
  if (rc) return rc;
  if (n % be) return 2;
  void (*f)(const float*, uint8_t*) = NULL;
  switch (tag) {
    case 2: f = qz_q4_0; break;
    case 8: f = qz_q8_0; break;
    case 12: f = qz_q4_k; break;
    case 14: f = qz_q6_k; break;
    case 20: f = qz_iq4_nl; break;
    case 23: f = qz_iq4_xs; break;
    default: return 3;
  }
  int64_t nb = n / be;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < nb; i++) f(x + i * be, out + i * bb);
  return 0;
}

/* ------------------------------------------------------------------ */
/* MLX group-wise affine quantization                                  */
/* quant.rs:38-53 -> mlx_rs::ops::quantize(w, group_size, bits); the  */
/* arithmetic is MLX 0.31.2's CPU `quantize` (fp32 min/max, rint).     */
/* ------------------------------------------------------------------ */
static int check_qargs(int64_t rows, int64_t cols, int group_size, int bits) {
  if (bits != 4 && bits != 8) return 3;
  if (group_size != 32 && group_size != 64 && group_size != 128) return 3;
  if (rows < 0 || cols <= 0 || cols % group_size) return 2;
  return 0;
}

static float ld_w(int dtype, const void* w, int64_t i) {
  if (dtype == 0) return ((const float*)w)[i];
  return orc_bf16_to_f32(((const uint16_t*)w)[i]);
}

static void st_w(int dtype, void* w, int64_t i, float v) {
  if (dtype == 0) ((float*)w)[i] = v;
  else ((uint16_t*)w)[i] = orc_f32_to_bf16(v);
}

int orc_affine_quantize(int dtype, const void* w, int64_t rows, int64_t cols,
                        int group_size, int bits, uint32_t* wq, void* scales,
                        void* biases) {
  int rc = check_qargs(rows, cols, group_size, bits);
  if (rc) return rc;
  if (dtype != 0 && dtype != 2) return 3;
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int per_word = 32 / bits;
  int64_t groups = rows * (cols / group_size);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t g = 0; g < groups; g++) {
    int64_t base = g * group_size;
    float w_min = INFINITY, w_max = -INFINITY;
    for (int j = 0; j < group_size; j++) {
      float v = ld_w(dtype, w, base + j);
      w_max = fmaxf(w_max, v);
      w_min = fminf(w_min, v);
    }
    int mask = fabsf(w_min) > fabsf(w_max);
    float scale = fmaxf((w_max - w_min) / n_bins, eps);
    scale = mask ? scale : -scale;
    float edge = mask ? w_min : w_max;
    float q0 = rintf(edge / scale);
    float bias = 0.f;
    if (q0 != 0.f) {
      scale = edge / q0;
      bias = edge;
    }
    int64_t wbase = base / per_word;
    for (int j = 0; j < group_size / per_word; j++) {
      uint32_t word = 0;
      for (int k = 0; k < per_word; k++) {
        float v = ld_w(dtype, w, base + j * per_word + k);
        float q = rintf((v - bias) / scale);
        q = fminf(fmaxf(q, 0.f), n_bins);
        word |= (uint32_t)q << (k * bits);
      }
      wq[wbase + j] = word;
    }
    st_w(dtype, scales, g, scale);
    st_w(dtype, biases, g, bias);
  }
  return 0;
}

int orc_affine_dequantize(int dtype, const uint32_t* wq, const void* scales,
                          const void* biases, int64_t rows, int64_t cols,
                          int group_size, int bits, void* out) {
  int rc = check_qargs(rows, cols, group_size, bits);
  if (rc) return rc;
  if (dtype != 0 && dtype != 2) return 3;
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  int64_t n = rows * cols;
  for (int64_t i = 0; i < n; i++) {
    int64_t g = i / group_size;
    uint32_t q = (wq[i / per_word] >> ((i % per_word) * bits)) & mask;
    float s = ld_w(dtype, scales, g), b = ld_w(dtype, biases, g);
    float v = s * (float)q + b;
    st_w(dtype, out, i, v);
  }
  return 0;
}

static inline uint32_t code_at(const uint32_t* row, int64_t k, int bits) {
  int per_word = 32 / bits;
  return (row[k / per_word] >> ((k % per_word) * bits)) & ((1u << bits) - 1u);
}

int orc_qmatmul_f64(const uint16_t* x, int64_t M, const uint32_t* wq,
                    const uint16_t* scales, const uint16_t* biases,
                    int64_t N, int64_t K, int group_size, int bits,
                    double* y) {
  int rc = check_qargs(N, K, group_size, bits);
  if (rc) return rc;
  int64_t wpr = K * bits / 32, gpr = K / group_size;
  int failed = 0;
  /* each weight row is dequantized once (w = s*q + b in f64, exact) and
   * then dotted with every activation row in k order */
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
    double* w = (double*)malloc(sizeof(double) * (size_t)K);
    if (!w) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
      failed = 1;
    }
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t n = 0; n < N; n++) {
      if (!w) continue;
      const uint32_t* row = wq + n * wpr;
      for (int64_t k = 0; k < K; k++) {
        int64_t g = k / group_size;
        w[k] = (double)orc_bf16_to_f32(scales[n * gpr + g]) * (double)code_at(row, k, bits) +
               (double)orc_bf16_to_f32(biases[n * gpr + g]);
      }
      for (int64_t m = 0; m < M; m++) {
        const uint16_t* xr = x + m * K;
        double acc = 0.0;
        for (int64_t k = 0; k < K; k++) acc += (double)orc_bf16_to_f32(xr[k]) * w[k];
        y[m * N + n] = acc;
      }
    }
    free(w);
  }
  return failed ? 4 : 0;
}


/* ---------------------------------------------------------------- decode layer chain
 * bf16 ops around the projections, at MLX's rounding points. */

static float bf16_round(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* src/primitives/nn.rs:35-37 -> mlx fast::rms_norm: the f32 row statistic,
 * x * inv rounded to bf16, then the weight product rounded to bf16. */
int orc_rms_norm_bf16(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t dim,
                      float eps, uint16_t* y) {
  if (rows < 0 || dim <= 0) return 1;
  for (int64_t r = 0; r < rows; r++) {
    const uint16_t* xr = x + r * dim;
    double ss = 0.0;
    for (int64_t i = 0; i < dim; i++) {
      double v = (double)orc_bf16_to_f32(xr[i]);
      ss += v * v;
    }
    const float inv = (float)(1.0 / sqrt((double)(float)(ss / (double)dim) + (double)eps));
    for (int64_t i = 0; i < dim; i++) {
      float n = bf16_round(orc_bf16_to_f32(xr[i]) * inv);
      y[r * dim + i] = orc_f32_to_bf16(orc_bf16_to_f32(w[i]) * n);
    }
  }
  return 0;
}

/* src/models/llama.rs:1040-1045 (silu at src/primitives/nn.rs:50-52, then
 * multiply): sigmoid, g * sigmoid and the product with up each rounded to bf16. */
int orc_silu_mul_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* y) {
  if (n < 0) return 1;
  for (int64_t i = 0; i < n; i++) {
    float gv = orc_bf16_to_f32(g[i]);
    float s = bf16_round(1.0f / (1.0f + expf(-gv)));
    float a = bf16_round(gv * s);
    y[i] = orc_f32_to_bf16(a * orc_bf16_to_f32(u[i]));
  }
  return 0;
}

/* residual add (src/models/llama.rs:729-733): bf16(a + b). */
int orc_add_bf16(const uint16_t* a, const uint16_t* b, int64_t n, uint16_t* y) {
  if (n < 0) return 1;
  for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_bf16(orc_bf16_to_f32(a[i]) + orc_bf16_to_f32(b[i]));
  return 0;
}

/* repeat_kv (src/primitives/attention.rs:45-55) for one position: output
 * head h = KV head h / groups. */
int orc_repeat_kv(const uint16_t* x, int64_t rows, int kv_heads, int head_dim, int groups, uint16_t* y) {
  if (rows < 0 || kv_heads <= 0 || head_dim <= 0 || groups <= 0) return 1;
  int64_t in_row = (int64_t)kv_heads * head_dim, out_row = in_row * groups;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t h = 0; h < (int64_t)kv_heads * groups; h++)
      memcpy(y + r * out_row + h * head_dim, x + r * in_row + (h / groups) * head_dim, (size_t)head_dim * 2);
  return 0;
}
