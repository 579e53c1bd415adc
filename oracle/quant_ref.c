/*
 * Independent C restatement of the int8 warm/cold-tier quantiser (lazykv/quant.py:42-105).
 *
 * TEST INFRASTRUCTURE ONLY: the product library never links this file. It exists so the numpy
 * restatement in oracle/reference.py is checked against code that does its own float16 and
 * bfloat16 rounding (bit manipulation here, numpy's casts there); both are in turn checked
 * against golden vectors written by the reference's own quant.py.
 *
 * Arithmetic follows lazykv/quant.py:59-70 and :90-105 exactly, in IEEE float32:
 *   mn, mx    = min / max over the group (exact)
 *   scale     = max((mx - mn) / 255, FLT_MIN)           (correctly rounded divide)
 *   q         = clamp(rint((x - mn) / scale), 0, 255) - 128  (rint: half to even)
 *   record    = kq[bs*d] | vq[bs*d] | f16(ks)[d] | f16(kz)[d] | f16(vs)[bs] | f16(vz)[bs]
 *   dequant   = ((q + 128) * f32(s16)) + f32(z16), multiply and add rounded separately,
 *               then rounded to the model dtype.
 * Build with -ffp-contract=off so no fused multiply-add appears.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { OQ_F16 = 0, OQ_BF16 = 1 };

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1f) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in float32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

static uint16_t f32_to_f16_rne(float f) {
  uint32_t u = f32_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds past 65504: inf */
  int32_t e = (int32_t)(a >> 23) - 127;
  uint32_t man = (a & 0x7fffffu) | 0x800000u;
  if (e < -25) return sign; /* below half the smallest subnormal */
  if (e < -14) {
    /* subnormal half: value = man * 2^(e-23); units of 2^-24 */
    int shift = -e - 1; /* 14..24: man >> (shift) gives units of 2^-24 */
    uint32_t q = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  /* normal: keep 10 mantissa bits of 23 */
  uint32_t q = ((uint32_t)(e + 15) << 10) | ((man >> 13) & 0x3ffu);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry into the exponent */
  return (uint16_t)(sign | q);
}

static float bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float load(const uint16_t* p, int dtype) { return dtype == OQ_F16 ? f16_to_f32(*p) : bf16_to_f32(*p); }

static uint16_t store(float f, int dtype) { return dtype == OQ_F16 ? f32_to_f16_rne(f) : f32_to_bf16_rne(f); }

int64_t oq_packed_pair_bytes(int bs, int d) { return 2LL * bs * d + 4LL * d + 4LL * bs; }

static int8_t quantise(float x, float mn, float scale) {
  float t = nearbyintf((x - mn) / scale);
  if (t < 0.0f) t = 0.0f;
  if (t > 255.0f) t = 255.0f;
  return (int8_t)(int)(t - 128.0f);
}

/* pairs [m, 2, bs, d] (model-dtype bits) -> records [m, P] */
void oq_pack(const uint16_t* in, int dtype, int64_t m, int bs, int d, uint8_t* out) {
  const int64_t P = oq_packed_pair_bytes(bs, d);
  for (int64_t i = 0; i < m; ++i) {
    const uint16_t* k = in + i * 2LL * bs * d;
    const uint16_t* v = k + (int64_t)bs * d;
    uint8_t* rec = out + i * P;
    int8_t* kq = (int8_t*)rec;
    int8_t* vq = (int8_t*)(rec + (int64_t)bs * d);
    uint16_t scales[4096];
    uint16_t* ks = scales;
    uint16_t* kz = scales + d;
    uint16_t* vs = scales + 2 * d;
    uint16_t* vz = scales + 2 * d + bs;
    for (int c = 0; c < d; ++c) { /* keys: per channel over tokens */
      float mn = load(&k[c], dtype), mx = mn;
      for (int t = 1; t < bs; ++t) {
        float x = load(&k[t * d + c], dtype);
        if (x < mn) mn = x;
        if (x > mx) mx = x;
      }
      float scale = (mx - mn) / 255.0f;
      if (scale < FLT_MIN) scale = FLT_MIN;
      for (int t = 0; t < bs; ++t) kq[t * d + c] = quantise(load(&k[t * d + c], dtype), mn, scale);
      ks[c] = f32_to_f16_rne(scale);
      kz[c] = f32_to_f16_rne(mn);
    }
    for (int t = 0; t < bs; ++t) { /* values: per token over channels */
      float mn = load(&v[t * d], dtype), mx = mn;
      for (int c = 1; c < d; ++c) {
        float x = load(&v[t * d + c], dtype);
        if (x < mn) mn = x;
        if (x > mx) mx = x;
      }
      float scale = (mx - mn) / 255.0f;
      if (scale < FLT_MIN) scale = FLT_MIN;
      for (int c = 0; c < d; ++c) vq[t * d + c] = quantise(load(&v[t * d + c], dtype), mn, scale);
      vs[t] = f32_to_f16_rne(scale);
      vz[t] = f32_to_f16_rne(mn);
    }
    memcpy(rec + 2LL * bs * d, scales, (size_t)(4 * d + 4 * bs));
  }
}

/* records [m, P] -> pairs [m, 2, bs, d] (model-dtype bits) */
void oq_unpack(const uint8_t* rec_all, int64_t m, int bs, int d, int dtype, uint16_t* out) {
  const int64_t P = oq_packed_pair_bytes(bs, d);
  for (int64_t i = 0; i < m; ++i) {
    const uint8_t* rec = rec_all + i * P;
    const int8_t* kq = (const int8_t*)rec;
    const int8_t* vq = (const int8_t*)(rec + (int64_t)bs * d);
    uint16_t scales[4096];
    memcpy(scales, rec + 2LL * bs * d, (size_t)(4 * d + 4 * bs));
    const uint16_t* ks = scales;
    const uint16_t* kz = scales + d;
    const uint16_t* vs = scales + 2 * d;
    const uint16_t* vz = scales + 2 * d + bs;
    uint16_t* k = out + i * 2LL * bs * d;
    uint16_t* v = k + (int64_t)bs * d;
    for (int t = 0; t < bs; ++t) {
      for (int c = 0; c < d; ++c) {
        float prod = ((float)kq[t * d + c] + 128.0f) * f16_to_f32(ks[c]);
        k[t * d + c] = store(prod + f16_to_f32(kz[c]), dtype);
        float pv = ((float)vq[t * d + c] + 128.0f) * f16_to_f32(vs[t]);
        v[t * d + c] = store(pv + f16_to_f32(vz[t]), dtype);
      }
    }
  }
}
