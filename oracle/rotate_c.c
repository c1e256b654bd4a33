/*
 * rotate_c.c -- TEST INFRASTRUCTURE ONLY: a plain C restatement of the oracle's K
 * re-rotation (oracle/kvshift_oracle.py: rotate_k_bits), for checking every K row of
 * the full-size shifts, where the numpy formulation takes minutes.
 *
 * What it restates (reference lines as cited there):
 *   - rotate_half(x) = cat(-x[..., h:], x[..., :h])           (kvshift.py:44-46)
 *   - k * emb_cos + rotate_half(k) * emb_sin in fp32, two separate multiplies and one
 *     add, then one round to nearest even into the cache type (shift_kernels.py:153-156)
 *   - dims at or above `rotary` pass through untouched        (shift_kernels.py:74-75)
 *   - fp8 e4m3fn (no reference; the kernels' own rule): x = fl32(decode(code) * s),
 *     rotate, q = fl32(y / s) clamped to +-448 (NaN kept), encoded to the nearest code,
 *     ties to the even code; NaN -> 0x7F
 * NaN results are canonical: bf16 0x7FC0, fp16 0x7E00, fp32 0x7FC00000, fp8 0x7F.
 *
 * Codecs are written from the format definitions, in a formulation different from the
 * numpy oracle's (the fp8 encoder uses frexp/rint, not a search over the code table);
 * tests/test_oracle_c.py holds the two bit-identical on every fp8 code, every midpoint,
 * tie-heavy fp32 inputs and random rows of every element type.
 *
 * Built by __graft_entry__.build() (gcc, -O2 -ffp-contract=off) into
 * oracle/_lib/liborc_rotate.so; only tests load it.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_BF16 0
#define ORC_F16 1
#define ORC_F32 2
#define ORC_FP8 3

static float f_of(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t u_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* ---- bf16 ---------------------------------------------------------------------- */

static float bf16_dec(uint16_t b) { return f_of((uint32_t)b << 16); }

static uint16_t bf16_enc(float y) {
  if (isnan(y)) return 0x7FC0;
  const uint32_t u = u_of(y);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16); /* no overflow: NaNs left above */
}

/* ---- fp16 (IEEE binary16) ------------------------------------------------------ */

static float f16_dec(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  float mag;
  if (e == 0) {
    mag = ldexpf((float)m, -24);
  } else if (e == 31) {
    mag = m ? NAN : INFINITY;
  } else {
    mag = ldexpf((float)(1024u + m), (int)e - 25);
  }
  return f_of(u_of(mag) | s);
}

static uint16_t f16_enc(float y) {
  if (isnan(y)) return 0x7E00;
  const uint32_t u = u_of(y);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x477FF000u) return sign | 0x7C00u; /* >= 65520: rounds to infinity */
  if (a >= 0x38800000u) {                      /* >= 2^-14: a normal half */
    const uint32_t r = a - (112u << 23);       /* rebias the exponent 127 -> 15 */
    return sign | (uint16_t)((r + 0xFFFu + ((r >> 13) & 1u)) >> 13);
  }
  /* subnormal half: units of 2^-24; the scaling is exact and rintf rounds to even */
  const float m = rintf(f_of(a) * 16777216.0f);
  return sign | (uint16_t)m;
}

/* ---- fp32 ---------------------------------------------------------------------- */

static uint32_t f32_enc(float y) { return isnan(y) ? 0x7FC00000u : u_of(y); }

/* ---- fp8 e4m3fn (OCP) ---------------------------------------------------------- */

static float e4m3_dec(uint8_t c) {
  const int e = (c >> 3) & 0xF;
  const int m = c & 7;
  float mag;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) {
    mag = ldexpf((float)m, -9);
  } else {
    mag = ldexpf((float)(8 + m), e - 10);
  }
  return (c & 0x80) ? -mag : mag;
}

/* |q| <= 448 (already clamped), not NaN */
static uint8_t e4m3_enc(float q) {
  const uint8_t sign = signbit(q) ? 0x80 : 0;
  const float a = fabsf(q);
  uint32_t code;
  if (a < 0.015625f) { /* below 2^-6: subnormal codes m * 2^-9, m = 0..8 */
    code = (uint32_t)rintf(a * 512.0f);
  } else {
    int k;
    frexpf(a, &k);              /* a = f * 2^k, f in [0.5, 1) */
    const int E = k - 1;        /* a in [2^E, 2^(E+1)), E in [-6, 8] */
    const float t = ldexpf(a, 3 - E); /* [8, 16): 1.mmm scaled by 8, exact */
    const uint32_t m = (uint32_t)rintf(t);  /* 8..16; 16 carries into the exponent */
    code = ((uint32_t)(E + 7) << 3) + (m - 8);
  }
  return sign | (uint8_t)code;
}

/* ---- the rotation -------------------------------------------------------------- */

static float load_elem(int dt, const void* row, int i, float scale) {
  switch (dt) {
    case ORC_BF16:
      return bf16_dec(((const uint16_t*)row)[i]);
    case ORC_F16:
      return f16_dec(((const uint16_t*)row)[i]);
    case ORC_F32:
      return f_of(((const uint32_t*)row)[i]);
    default:
      return e4m3_dec(((const uint8_t*)row)[i]) * scale;
  }
}

static void store_elem(int dt, void* row, int i, float y, float scale) {
  switch (dt) {
    case ORC_BF16:
      ((uint16_t*)row)[i] = bf16_enc(y);
      break;
    case ORC_F16:
      ((uint16_t*)row)[i] = f16_enc(y);
      break;
    case ORC_F32:
      ((uint32_t*)row)[i] = f32_enc(y);
      break;
    default: {
      uint8_t* r = (uint8_t*)row;
      if (isnan(y)) {
        r[i] = 0x7F;
        break;
      }
      float q = y / scale;
      if (isnan(q)) {
        r[i] = 0x7F;
        break;
      }
      if (q > 448.0f) q = 448.0f;
      if (q < -448.0f) q = -448.0f;
      r[i] = e4m3_enc(q);
    }
  }
}

static int elem_size(int dt) {
  switch (dt) {
    case ORC_BF16:
    case ORC_F16:
      return 2;
    case ORC_F32:
      return 4;
    case ORC_FP8:
      return 1;
    default:
      return 0;
  }
}

/*
 * Re-rotate `rows` K rows of `head_size` elements (cache bit patterns, rows packed
 * back to back) from `in` into `out`.  cos_f / sin_f: fp32 [rotary / 2], one entry per
 * frequency (emb_cos = cat(cos_f, cos_f), emb_sin likewise).  k_scale: fp8 only.
 * Returns 0, or -1 on a bad argument.
 */
int orc_rotate_k(int dtype, const void* in, void* out, int64_t rows, int32_t head_size,
                 int32_t rotary, const float* cos_f, const float* sin_f, float k_scale) {
  const int eb = elem_size(dtype);
  if (eb == 0 || head_size <= 0 || rotary < 0 || rotary > head_size || (rotary & 1) ||
      rows < 0)
    return -1;
  const int h = rotary / 2;
  const size_t row_bytes = (size_t)head_size * (size_t)eb;
  for (int64_t r = 0; r < rows; ++r) {
    const char* src = (const char*)in + (size_t)r * row_bytes;
    char* dst = (char*)out + (size_t)r * row_bytes;
    /* untouched dims first (and the whole row when rotary is 0) */
    memcpy(dst, src, row_bytes);
    for (int i = 0; i < rotary; ++i) {
      const int f = i < h ? i : i - h;
      const float k = load_elem(dtype, src, i, k_scale);
      const float rot = i < h ? -load_elem(dtype, src, i + h, k_scale)
                              : load_elem(dtype, src, i - h, k_scale);
      const float a = k * cos_f[f];
      const float b = rot * sin_f[f];
      store_elem(dtype, dst, i, a + b, k_scale);
    }
  }
  return 0;
}

/* Single-value codecs, exported so the tests can pin them one by one. */
uint16_t orc_bf16_enc(float y) { return bf16_enc(y); }
uint16_t orc_f16_enc(float y) { return f16_enc(y); }
float orc_f16_dec(uint16_t h) { return f16_dec(h); }
float orc_e4m3_dec(uint8_t c) { return e4m3_dec(c); }
uint8_t orc_e4m3_enc_clamped(float q) { return e4m3_enc(q); }
