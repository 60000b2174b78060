/*
 * C restatement of the bit-exact part of the hot path — TEST INFRASTRUCTURE ONLY (the product never links
 * it).  Built by oracle/build.py into oracle/_build/liboracle.so and called from tests/ and bench.py's
 * cpu_baseline leg through ctypes.
 *
 *   oracle_round_bf16   vkrt/shaders/types.glsl:45-50 (f2bf: RNE, NaN -> 0x7FC0)
 *   oracle_round_f16    vkrt/shaders/types.glsl:18-41 (f2h: RNE incl. subnormals, overflow -> inf)
 *   oracle_dequant_int8 vkrt/shaders/dq8.comp.in:39-62, torch_vulkan/__init__.py:203-205
 */
#include <stdint.h>
#include <string.h>

static uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

static uint16_t f2bf(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static uint16_t f2h(float x) {
  uint32_t u = f32_bits(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t e = (u >> 23) & 0xffu;
  uint32_t m = u & 0x7fffffu;
  if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m != 0u ? (0x200u | (m >> 13)) : 0u));
  int ne = (int)e - 127 + 15;
  if (ne >= 31) return (uint16_t)(sign | 0x7c00u);
  if (ne <= 0) {
    if (ne < -10) return (uint16_t)sign;
    m |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - ne);
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (hm & 1u) != 0u)) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = m >> 13;
  uint32_t rem = m & 0x1fffu;
  uint32_t h = sign | ((uint32_t)ne << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u) != 0u)) h++;
  return (uint16_t)h;
}

void oracle_round_bf16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f2bf(x[i]);
}

void oracle_round_f16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f2h(x[i]);
}

/* kind: 0 = f32 (out is uint32 bit patterns), 1 = bf16, 2 = f16 (out is uint16 bit patterns). */
void oracle_dequant_int8(const int8_t* q, const uint16_t* scale, int64_t rows, int64_t cols, int kind, void* out) {
  const int64_t nb = (cols + 63) / 64;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const float s = bits_f32((uint32_t)scale[r * nb + c / 64] << 16);
      const float v = (float)q[r * cols + c] * s;
      const int64_t i = r * cols + c;
      if (kind == 0)
        ((uint32_t*)out)[i] = f32_bits(v);
      else if (kind == 1)
        ((uint16_t*)out)[i] = f2bf(v);
      else
        ((uint16_t*)out)[i] = f2h(v);
    }
  }
}
