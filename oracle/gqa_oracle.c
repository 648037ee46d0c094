/*
 * C restatement of the paged GQA decode oracle — TEST INFRASTRUCTURE ONLY
 * (only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * use it, as the checker).
 *
 * Follows, per (sequence b, q-head h), reference attention/reference/gqa.py:29-43
 * with the element addressing of csrc/cuda/dense/gqa_decode.cu:31 and :43-47:
 *   kv_head = h / (Hq / Hkv)
 *   token t -> page t / P, slot t % P, phys = table[b][page],
 *   row = ((phys * P + slot) * Hkv + kv_head) * D            (64-bit)
 *   s_t = (sum_d q[d] * k[row + d]) * scale                  (fp32, d ascending)
 *   w_t = exp(s_t - max s) / sum exp(s - max s)              (softmax, gqa.py:41)
 *   out[d] = sum_t w_t * v[row + d]                          (gqa.py:42)
 *   rounded once to the element type, nearest-even           (gqa.py:43)
 * A length <= 0 gives zeros.  Returns 0, or -1 for an out-of-range page id
 * inside the used range (the oracle never clamps).
 *
 * Element conversions are written here from the IEEE 754 binary16 and
 * bfloat16 formats (gcc 11 has no _Float16 on x86).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

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

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 0x1f;
  const uint32_t m = h & 0x3ff;
  if (e == 0) {
    const float mag = ldexpf((float)m, -24);
    return sign ? -mag : mag;
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

static uint16_t f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  x &= 0x7fffffffu;
  if (x >= 0x7f800000u) return sign | (x > 0x7f800000u ? 0x7e00 : 0x7c00);
  if (x >= 0x477ff000u) return sign | 0x7c00; /* >= 65520 rounds to inf */
  if (x < 0x38800000u) {                      /* below 2^-14: subnormal range */
    const float scaled = bits_f32(x) * 16777216.0f; /* exact: times 2^24 */
    return sign | (uint16_t)rintf(scaled);          /* nearest-even */
  }
  uint32_t h = ((((x >> 23) - 127 + 15) & 0x1f) << 10) | ((x & 0x7fffffu) >> 13);
  const uint32_t rest = x & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1;
  return sign | (uint16_t)h;
}

static float bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

static uint16_t f32_to_bf16(float f) {
  const uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static float load_elem(const void* p, int64_t i, int dt) {
  switch (dt) {
    case DT_F32: return ((const float*)p)[i];
    case DT_F16: return f16_to_f32(((const uint16_t*)p)[i]);
    default: return bf16_to_f32(((const uint16_t*)p)[i]);
  }
}

static void store_elem(void* p, int64_t i, int dt, float x) {
  switch (dt) {
    case DT_F32: ((float*)p)[i] = x; break;
    case DT_F16: ((uint16_t*)p)[i] = f32_to_f16(x); break;
    default: ((uint16_t*)p)[i] = f32_to_bf16(x); break;
  }
}

/* Exposed for the conversion tests. */
uint16_t oracle_f32_to_f16(float f) { return f32_to_f16(f); }
float oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }

int oracle_gqa_decode(const void* q, const void* k, const void* v, const int32_t* table,
                      const int32_t* lens, void* out, int B, int Hq, int Hkv, int D, int P,
                      int max_pages, int dtype, int num_blocks, float scale) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || D > 256 || P <= 0) return -2;
  const int g = Hq / Hkv;
  int status = 0;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hq; ++h) {
      const int len = lens[b];
      const int64_t ob = ((int64_t)b * Hq + h) * D;
      if (len <= 0) {
        for (int d = 0; d < D; ++d) store_elem(out, ob + d, dtype, 0.f);
        continue;
      }
      const int kvh = h / g;
      float qf[256];
      for (int d = 0; d < D; ++d) qf[d] = load_elem(q, ob + d, dtype);
      float* s = (float*)malloc(sizeof(float) * (size_t)len);
      int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)len);
      float mx = -INFINITY;
      int bad = 0;
      for (int t = 0; t < len; ++t) {
        const int page = t / P;
        const int slot = t % P;
        if (page >= max_pages) {
          bad = 1;
          break;
        }
        const int32_t phys = table[(int64_t)b * max_pages + page];
        if (phys < 0 || phys >= num_blocks) {
          bad = 1;
          break;
        }
        const int64_t row = (((int64_t)phys * P + slot) * Hkv + kvh) * D;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += qf[d] * load_elem(k, row + d, dtype);
        s[t] = dot * scale;
        rows[t] = row;
        if (s[t] > mx) mx = s[t];
      }
      if (bad) {
#pragma omp atomic write
        status = -1;
        free(s);
        free(rows);
        continue;
      }
      float z = 0.f;
      for (int t = 0; t < len; ++t) {
        s[t] = expf(s[t] - mx);
        z += s[t];
      }
      float acc[256];
      for (int d = 0; d < D; ++d) acc[d] = 0.f;
      for (int t = 0; t < len; ++t) {
        const float w = s[t] / z;
        for (int d = 0; d < D; ++d) acc[d] += w * load_elem(v, rows[t] + d, dtype);
      }
      for (int d = 0; d < D; ++d) store_elem(out, ob + d, dtype, acc[d]);
      free(s);
      free(rows);
    }
  }
  return status;
}
