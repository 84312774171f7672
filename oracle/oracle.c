/*
 * CPU oracle: plain-C restatement of the onnx-light reference arithmetic for
 * MatMulInteger, QLinearMatMul, DequantizeLinear and the fp16/bf16 MatMul that
 * follows DequantizeLinear.  Test infrastructure only: the shipped HIP library
 * never links or calls it.  Written from the reference's semantics (cited per
 * function); the loop orders that fix rounding are kept, everything else is
 * this file's own.  Build with -ffp-contract=off so no FMA is formed, matching
 * a baseline x86-64 build of the reference (CMakeLists.txt adds no -march).
 */
#include "oracle.h"
#include "../onnx-light_amd/csrc/gguf_codebooks.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-half-to-even of x / 2^s for an unsigned integer x and 1 <= s <= 31. */
static uint32_t shr_rne(uint32_t x, unsigned s) {
  const uint32_t q = x >> s;
  const uint32_t rem = x & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1u);
  return (rem > half || (rem == half && (q & 1u))) ? q + 1u : q;
}

/* FLOAT -> FLOAT16, round-to-nearest-even; NaN -> sign|0x7e00; overflow ->
 * inf; fp32 subnormals -> signed zero.  rk/cast_helper.cc:51-87. */
uint16_t orc_f32_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const int32_t e32 = (int32_t)((u >> 23) & 0xffu);
  const uint32_t m32 = u & 0x7fffffu;
  if (e32 == 0xff) return (uint16_t)(sign | 0x7c00u | (m32 ? 0x0200u : 0u));
  const int32_t e = e32 - 127 + 15; /* fp16 biased exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return sign;
    /* subnormal: significand (with hidden bit) in units of 2^-24 */
    return (uint16_t)(sign | shr_rne(m32 | 0x800000u, (unsigned)(14 - e)));
  }
  /* normal: exponent and mantissa shifted together so a carry bumps e */
  return (uint16_t)(sign | shr_rne(((uint32_t)e << 23) | m32, 13));
}

/* FLOAT16 -> FLOAT, exact; NaN payload kept.  rk/cast_helper.cc:89-122. */
float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  const uint32_t man = (uint32_t)h & 0x3ffu;
  if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in float */
    const float v = ldexpf((float)man, -24);
    return sign ? -v : v;
  }
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* FLOAT -> BFLOAT16 round-to-nearest-even; NaN keeps its upper half with the
 * quiet bit set.  rk/cast_helper.cc:124-134. */
uint16_t orc_f32_to_bf16(float f) {
  const uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  const uint64_t wide = (uint64_t)u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)((uint32_t)wide >> 16);
}

/* rk/cast_helper.cc:136-141. */
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* FLOAT -> FLOAT8E4M3FN, saturating round-to-nearest-even: |v| beyond the
 * largest finite 448 (and +-inf) -> +-448, NaN -> sign|0x7f, magnitudes below
 * half the smallest subnormal 2^-9 -> +-0, fp32 subnormals -> +-0.
 * rk/cast_float8.cc:27-81 (used to generate fp8 weights). */
uint8_t orc_f32_to_f8e4m3fn(float v) {
  const uint32_t u = f2u(v);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  if (a == 0x7f800000u) return (uint8_t)(sign | 0x7eu);
  const int32_t e = (int32_t)(a >> 23);
  const uint32_t m = a & 0x7fffffu;
  if (e == 0 || e < 117) return sign;
  const int32_t E = e - 120; /* fp8 biased exponent when normal */
  uint32_t mag;
  if (E >= 1) {
    mag = shr_rne(((uint32_t)E << 23) | m, 20);
  } else {
    /* subnormal target: value / 2^-9 = (m|2^23) / 2^(21-E) */
    mag = shr_rne(m | 0x800000u, (unsigned)(21 - E));
  }
  if (mag > 0x7eu) mag = 0x7eu;
  return (uint8_t)(sign | mag);
}

/* FLOAT8E4M3FN -> FLOAT, exact; 0x7f/0xff are NaN.  rk/cast_float8.cc:83-118. */
float orc_f8e4m3fn_to_f32(uint8_t c) {
  if (c == 0xffu) return u2f(0xffc00000u);
  if (c == 0x7fu) return u2f(0x7fc00000u);
  const int E = (c >> 3) & 0xf;
  const int M = c & 7;
  const float mag = (E == 0) ? ldexpf((float)M, -9) : ldexpf((float)(8 + M), E - 10);
  return (c & 0x80u) ? -mag : mag;
}

/* Low nibble holds the even flat index.  rk/cast_sub_byte.h:57-60. */
uint8_t orc_read_4bit(const uint8_t *data, int64_t i) {
  const uint8_t byte = data[i >> 1];
  return (uint8_t)((i & 1) ? (byte >> 4) : (byte & 0x0f));
}

/* Two's-complement 4-bit sign extension.  rk/cast_sub_byte.cc:81-88. */
int8_t orc_int4_to_i8(uint8_t nibble) {
  const int v = nibble & 0x0f;
  return (int8_t)(v >= 8 ? v - 16 : v);
}

void orc_f32_to_f16_n(const float *s, int64_t n, uint16_t *d) {
  for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_f16(s[i]);
}
void orc_f16_to_f32_n(const uint16_t *s, int64_t n, float *d) {
  for (int64_t i = 0; i < n; ++i) d[i] = orc_f16_to_f32(s[i]);
}
void orc_f32_to_bf16_n(const float *s, int64_t n, uint16_t *d) {
  for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_bf16(s[i]);
}
void orc_bf16_to_f32_n(const uint16_t *s, int64_t n, float *d) {
  for (int64_t i = 0; i < n; ++i) d[i] = orc_bf16_to_f32(s[i]);
}
void orc_f32_to_f8e4m3fn_n(const float *s, int64_t n, uint8_t *d) {
  for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_f8e4m3fn(s[i]);
}
void orc_f8e4m3fn_to_f32_n(const uint8_t *s, int64_t n, float *d) {
  for (int64_t i = 0; i < n; ++i) d[i] = orc_f8e4m3fn_to_f32(s[i]);
}

/* ------------------------------------------------------------------------ */
/* SplitMix64 and the reference's samplers, rk/random.cc:32-106.             */

uint64_t orc_splitmix64_next(uint64_t *state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double uniform53(uint64_t x) { return (double)(x >> 11) * (1.0 / 9007199254740992.0); }

void orc_rand_uniform(uint64_t seed, int64_t n, double *out) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) out[i] = uniform53(orc_splitmix64_next(&s));
}

/* Uniform integers in [low, high) by rejection of the top partial span. */
int orc_rand_int(int64_t low, int64_t high, uint64_t seed, int64_t n, int64_t *out) {
  if (high <= low) return 1;
  const uint64_t span = (uint64_t)(high - low);
  const uint64_t limit = 0ull - ((0ull - span) % span); /* 2^64 - 2^64 % span (mod 2^64) */
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t x;
    do {
      x = orc_splitmix64_next(&s);
    } while (limit != 0 && x >= limit);
    out[i] = (int64_t)(x % span) + low;
  }
  return 0;
}

/* Irwin-Hall: sum of 12 uniforms minus 6, summed in double in draw order. */
void orc_randn(uint64_t seed, int64_t n, double *out) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) {
    double acc = 0.0;
    for (int j = 0; j < 12; ++j) acc += uniform53(orc_splitmix64_next(&s));
    out[i] = acc - 6.0;
  }
}

/* ------------------------------------------------------------------------ */
/* MatMul shape rules, km/matmul_shape_utils.h:24-106.                       */

#define ORC_MAX_RANK 16

typedef struct {
  int64_t M, K, N;
  int batch_rank;
  int64_t out_prefix[ORC_MAX_RANK];
  int64_t a_bstride[ORC_MAX_RANK]; /* element stride per output batch dim (0 = broadcast) */
  int64_t b_bstride[ORC_MAX_RANK];
  int64_t batch_count;
} mm_plan;

/* Builds the plan; returns 0 or the error code of orc_matmul_output_shape. */
static int mm_make_plan(const int64_t *a_shape, int a_rank, const int64_t *b_shape, int b_rank,
                        mm_plan *p) {
  if (a_rank <= 0 || b_rank <= 0) return 1;
  if (a_rank > ORC_MAX_RANK || b_rank > ORC_MAX_RANK) return 3;
  int64_t a2[ORC_MAX_RANK + 1], b2[ORC_MAX_RANK + 1];
  int ar = a_rank, br = b_rank;
  if (a_rank == 1) {
    a2[0] = 1;
    a2[1] = a_shape[0];
    ar = 2;
  } else {
    memcpy(a2, a_shape, sizeof(int64_t) * (size_t)a_rank);
  }
  if (b_rank == 1) {
    b2[0] = b_shape[0];
    b2[1] = 1;
    br = 2;
  } else {
    memcpy(b2, b_shape, sizeof(int64_t) * (size_t)b_rank);
  }
  p->M = a2[ar - 2];
  p->K = a2[ar - 1];
  p->N = b2[br - 1];
  if (p->K != b2[br - 2]) return 2;
  const int ap = ar - 2, bp = br - 2;
  const int rank = ap > bp ? ap : bp;
  p->batch_rank = rank;
  /* contiguous strides of the promoted operands */
  int64_t as[ORC_MAX_RANK + 1], bs[ORC_MAX_RANK + 1];
  as[ar - 1] = 1;
  for (int i = ar - 2; i >= 0; --i) as[i] = as[i + 1] * a2[i + 1];
  bs[br - 1] = 1;
  for (int i = br - 2; i >= 0; --i) bs[i] = bs[i + 1] * b2[i + 1];
  p->batch_count = 1;
  for (int i = 0; i < rank; ++i) {
    const int ia = i - (rank - ap), ib = i - (rank - bp);
    const int64_t da = ia >= 0 ? a2[ia] : 1;
    const int64_t db = ib >= 0 ? b2[ib] : 1;
    int64_t d;
    if (da == db || da == 1) {
      d = db;
    } else if (db == 1) {
      d = da;
    } else {
      return 3;
    }
    p->out_prefix[i] = d;
    p->a_bstride[i] = (ia >= 0 && a2[ia] != 1) ? as[ia] : 0;
    p->b_bstride[i] = (ib >= 0 && b2[ib] != 1) ? bs[ib] : 0;
    p->batch_count *= d;
  }
  return 0;
}

int orc_matmul_output_shape(const int64_t *a_shape, int a_rank, const int64_t *b_shape,
                            int b_rank, int64_t *out_shape, int *out_rank) {
  mm_plan p;
  const int rc = mm_make_plan(a_shape, a_rank, b_shape, b_rank, &p);
  if (rc) return rc;
  int r = 0;
  for (int i = 0; i < p.batch_rank; ++i) out_shape[r++] = p.out_prefix[i];
  if (a_rank != 1) out_shape[r++] = p.M;
  if (b_rank != 1) out_shape[r++] = p.N;
  *out_rank = r;
  return 0;
}

/* Element offsets of batch `batch` (row-major over out_prefix) in A and B. */
static void mm_batch_base(const mm_plan *p, int64_t batch, int64_t *a_base, int64_t *b_base) {
  int64_t ab = 0, bb = 0, rem = batch;
  for (int d = p->batch_rank - 1; d >= 0; --d) {
    const int64_t c = rem % p->out_prefix[d];
    rem /= p->out_prefix[d];
    ab += c * p->a_bstride[d];
    bb += c * p->b_bstride[d];
  }
  *a_base = ab;
  *b_base = bb;
}

static int32_t read_byte_elem(const void *t, int dtype, int64_t idx) {
  return dtype == ORC_INT8 ? (int32_t)((const int8_t *)t)[idx] : (int32_t)((const uint8_t *)t)[idx];
}

/* km/kernel_matmul_integer.cc:89-176: i, j, k loops; int32 accumulate of
 * (a - za[i]) * (b - zb[j]); the per-row zero point is indexed by i in every
 * batch.  Unsigned arithmetic gives the two's-complement wrap of `acc`. */
int orc_matmul_integer(const void *a, int a_dtype, const int64_t *a_shape, int a_rank,
                       const void *b, int b_dtype, const int64_t *b_shape, int b_rank,
                       const int32_t *a_zp, int64_t a_zp_count, const int32_t *b_zp,
                       int64_t b_zp_count, int32_t *y) {
  mm_plan p;
  const int rc = mm_make_plan(a_shape, a_rank, b_shape, b_rank, &p);
  if (rc) return rc;
  const int64_t M = p.M, K = p.K, N = p.N;
  for (int64_t bt = 0; bt < p.batch_count; ++bt) {
    int64_t ab, bb;
    mm_batch_base(&p, bt, &ab, &bb);
    for (int64_t i = 0; i < M; ++i) {
      const int32_t za = a_zp_count > 1 ? a_zp[i] : a_zp[0];
      for (int64_t j = 0; j < N; ++j) {
        const int32_t zb = b_zp_count > 1 ? b_zp[j] : b_zp[0];
        uint32_t acc = 0;
        for (int64_t k = 0; k < K; ++k) {
          const int32_t av = read_byte_elem(a, a_dtype, ab + i * K + k);
          const int32_t bv = read_byte_elem(b, b_dtype, bb + k * N + j);
          acc += (uint32_t)(av - za) * (uint32_t)(bv - zb);
        }
        y[(bt * M + i) * N + j] = (int32_t)acc;
      }
    }
  }
  return 0;
}

/* kq/kernel_qlinearmatmul.cc:115-217: int64 accumulate, combined scale
 * a_s*b_s/y_s in fp32 (left to right), (float)acc*cs, nearbyint (ties to
 * even, before the zero point), + (float)y_zp, clamp, cast. */
int orc_qlinear_matmul(const void *a, int a_dtype, const int64_t *a_shape, int a_rank,
                       int32_t a_zp, float a_scale, const void *b, int b_dtype,
                       const int64_t *b_shape, int b_rank, int32_t b_zp, float b_scale,
                       float y_scale, int32_t y_zp, int y_dtype, void *y, int64_t row_begin,
                       int64_t row_end) {
  mm_plan p;
  const int rc = mm_make_plan(a_shape, a_rank, b_shape, b_rank, &p);
  if (rc) return rc;
  const int64_t M = p.M, K = p.K, N = p.N;
  if (row_end < 0 || row_end > M) row_end = M;
  const float cs = a_scale * b_scale / y_scale;
  const float zy = (float)y_zp;
  const float lo = y_dtype == ORC_INT8 ? -128.0f : 0.0f;
  const float hi = y_dtype == ORC_INT8 ? 127.0f : 255.0f;
  for (int64_t bt = 0; bt < p.batch_count; ++bt) {
    int64_t ab, bb;
    mm_batch_base(&p, bt, &ab, &bb);
    for (int64_t i = row_begin; i < row_end; ++i) {
      for (int64_t j = 0; j < N; ++j) {
        int64_t acc = 0;
        for (int64_t k = 0; k < K; ++k) {
          const int32_t av = read_byte_elem(a, a_dtype, ab + i * K + k);
          const int32_t bv = read_byte_elem(b, b_dtype, bb + k * N + j);
          acc += (int64_t)(av - a_zp) * (int64_t)(bv - b_zp);
        }
        float v = nearbyintf((float)acc * cs) + zy;
        if (v < lo) {
          v = lo;
        } else if (v > hi) {
          v = hi;
        }
        const int64_t yi = (bt * M + i) * N + j;
        if (y_dtype == ORC_INT8) {
          ((int8_t *)y)[yi] = (int8_t)v;
        } else {
          ((uint8_t *)y)[yi] = (uint8_t)v;
        }
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* DequantizeLinear, kq/kernel_dequantizelinear.cc.                           */

static int64_t numel(const int64_t *s, int r) {
  int64_t n = 1;
  for (int i = 0; i < r; ++i) n *= s[i];
  return n;
}

static float f32_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* FLOAT8E4M3FNUZ (cast_float8.cc:174-215): bias 8, no infinities, 0x80 the
 * only NaN (decoded as 0xffc00000), no negative zero. */
float orc_f8e4m3fnuz_to_f32(uint8_t v) {
  if (v == 0x80) return f32_bits(0xffc00000u);
  const uint32_t sign = (uint32_t)(v & 0x80u) << 24, e = (v >> 3) & 15u, m = v & 7u;
  if (e == 0) {
    if (m == 0) return f32_bits(sign);
    uint32_t ee = 127u - 8u, mm = m;  /* normalise the subnormal: 1.f x 2^(ee - 127) */
    while (!(mm & 4u)) { mm = (mm & 3u) << 1; --ee; }
    return f32_bits(sign | ee << 23 | (mm & 3u) << 21);
  }
  return f32_bits(sign | (e + 127u - 8u) << 23 | m << 20);
}

/* FLOAT8E5M2 (cast_float8.cc:263-300): the fp16 layout's top byte, with
 * 0x7c / 0xfc infinities, 0x7d-0x7f decoded as 0x7fc00000 and 0xfd-0xff as
 * 0xffc00000. */
float orc_f8e5m2_to_f32(uint8_t v) {
  if (v >= 253) return f32_bits(0xffc00000u);
  if (v >= 125 && v <= 127) return f32_bits(0x7fc00000u);
  if (v == 252) return f32_bits(0xff800000u);
  if (v == 124) return f32_bits(0x7f800000u);
  const uint32_t sign = (uint32_t)(v & 0x80u) << 24, e = (v >> 2) & 31u, m = v & 3u;
  if (e == 0) {
    if (m == 0) return f32_bits(sign);
    uint32_t ee = 127u - 15u, mm = m;
    while (!(mm & 2u)) { mm = (mm & 1u) << 1; --ee; }
    return f32_bits(sign | ee << 23 | (mm & 1u) << 22);
  }
  return f32_bits(sign | (e + 127u - 15u) << 23 | m << 21);
}

/* FLOAT8E5M2FNUZ (cast_float8.cc:347-380): bias 16, 0x80 the only NaN. */
float orc_f8e5m2fnuz_to_f32(uint8_t v) {
  if (v == 0x80) return f32_bits(0xffc00000u);
  const uint32_t sign = (uint32_t)(v & 0x80u) << 24, e = (v >> 2) & 31u, m = v & 3u;
  if (e == 0) {
    if (m == 0) return f32_bits(sign);
    uint32_t ee = 127u - 16u, mm = m;
    while (!(mm & 2u)) { mm = (mm & 1u) << 1; --ee; }
    return f32_bits(sign | ee << 23 | (mm & 1u) << 22);
  }
  return f32_bits(sign | (e + 127u - 16u) << 23 | m << 21);
}

/* FLOAT4E2M1 (cast_helper.cc:161-166): +-{0, 0.5, 1, 1.5, 2, 3, 4, 6}. */
float orc_f4e2m1_to_f32(uint8_t nibble) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float v = mag[nibble & 7u];
  return (nibble & 8u) ? -v : v;
}

/* FLOAT6E2M3 / FLOAT6E3M2 (cast_helper.cc:208-219): sign bit 5, bias
 * 2^(E-1) - 1, subnormals at exponent 0, no infinities or NaN. */
float orc_f6_to_f32(uint8_t bits, int dtype) {
  const int mb = dtype == ORC_FLOAT6E2M3 ? 3 : 2, eb = 5 - mb, bias = (1 << (eb - 1)) - 1;
  const int e = (bits >> mb) & ((1 << eb) - 1), m = bits & ((1 << mb) - 1);
  const float v = e == 0 ? ldexpf((float)m, 1 - bias - mb) : ldexpf(1.0f + (float)m / (float)(1 << mb), e - bias);
  return (bits & 0x20u) ? -v : v;
}

/* two-bit elements, four per byte from the low bits (cast_sub_byte.h:71-75) */
uint8_t orc_read_2bit(const uint8_t *data, int64_t i) { return (uint8_t)((data[i / 4] >> (2 * (i % 4))) & 3u); }

/* six-bit elements as a little-endian bit stream (cast_helper.cc:247-256) */
uint8_t orc_read_6bit(const uint8_t *data, int64_t i) {
  const int64_t bit = i * 6, byte = bit / 8;
  const int sh = (int)(bit % 8);
  uint32_t v = (uint32_t)data[byte] >> sh;
  if (sh > 2) v |= (uint32_t)data[byte + 1] << (8 - sh);
  return (uint8_t)(v & 63u);
}

/* Decoded (float) quantized element i of x (kernel_dequantizelinear.cc:
 * 85-155). */
float orc_dq_decode(const void *x, int dtype, int64_t i) {
  const uint8_t *b = (const uint8_t *)x;
  switch (dtype) {
  case ORC_UINT8: return (float)b[i];
  case ORC_INT8: return (float)((const int8_t *)x)[i];
  case ORC_UINT16: return (float)((const uint16_t *)x)[i];
  case ORC_INT16: return (float)((const int16_t *)x)[i];
  case ORC_INT32: return (float)((const int32_t *)x)[i];
  case ORC_FLOAT8E4M3FN: return orc_f8e4m3fn_to_f32(b[i]);
  case ORC_FLOAT8E4M3FNUZ: return orc_f8e4m3fnuz_to_f32(b[i]);
  case ORC_FLOAT8E5M2: return orc_f8e5m2_to_f32(b[i]);
  case ORC_FLOAT8E5M2FNUZ: return orc_f8e5m2fnuz_to_f32(b[i]);
  case ORC_INT4: return (float)orc_int4_to_i8(orc_read_4bit(b, i));
  case ORC_UINT4: return (float)orc_read_4bit(b, i);
  case ORC_FLOAT4E2M1: return orc_f4e2m1_to_f32(orc_read_4bit(b, i));
  case ORC_UINT2: return (float)orc_read_2bit(b, i);
  case ORC_INT2: return (float)(((int)orc_read_2bit(b, i) ^ 2) - 2);
  case ORC_FLOAT6E2M3: case ORC_FLOAT6E3M2: return orc_f6_to_f32(orc_read_6bit(b, i), dtype);
  default: return 0.0f;
  }
}
#define dq_decode orc_dq_decode

void orc_dq_decode_n(const void *x, int dtype, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_dq_decode(x, dtype, i);
}

static int dq_supported(int dtype) {
  switch (dtype) {
  case ORC_UINT8: case ORC_INT8: case ORC_UINT16: case ORC_INT16: case ORC_INT32:
  case ORC_FLOAT8E4M3FN: case ORC_FLOAT8E4M3FNUZ: case ORC_FLOAT8E5M2: case ORC_FLOAT8E5M2FNUZ:
  case ORC_INT4: case ORC_UINT4: case ORC_FLOAT4E2M1: case ORC_UINT2: case ORC_INT2:
  case ORC_FLOAT6E2M3: case ORC_FLOAT6E3M2:
    return 1;
  default:
    return 0;
  }
}

/* Per-tensor: (x - zp) * s (:65-130).  Per-axis: scale index
 * (i / inner) % axis_size (:237-242).  Blocked (scale rank == x rank): scale
 * index sum_d (coord_d / (x_d / s_d)) * s_stride_d (:204-235).  Each value is
 * (decode(x) - decode(zp)) * scale in fp32, then FLOAT16 RNE or kept FLOAT
 * (:57-63, :247-285). */
int orc_dequantize_linear(const void *x, int x_dtype, const int64_t *x_shape, int x_rank,
                          const void *scale, int scale_dtype, const int64_t *s_shape,
                          int s_rank, const void *zp, int64_t axis, void *y) {
  if (!dq_supported(x_dtype)) return 1;
  if (scale_dtype != ORC_FLOAT && scale_dtype != ORC_FLOAT16) return 1;
  const int64_t n = numel(x_shape, x_rank);
  const int64_t ns = numel(s_shape, s_rank);
  float *sc = (float *)malloc(sizeof(float) * (size_t)(ns > 0 ? ns : 1));
  if (!sc) return 2;
  for (int64_t i = 0; i < ns; ++i) {
    sc[i] = scale_dtype == ORC_FLOAT16 ? orc_f16_to_f32(((const uint16_t *)scale)[i])
                                       : ((const float *)scale)[i];
  }
  int64_t repeats[ORC_MAX_RANK], sstr[ORC_MAX_RANK], coord[ORC_MAX_RANK];
  const int blocked = ns != 1 && s_rank == x_rank;
  int64_t inner = 1, axis_size = 1;
  if (ns != 1) {
    if (axis < 0 || axis >= x_rank || x_rank > ORC_MAX_RANK) {
      free(sc);
      return 1;
    }
    if (blocked) {
      int64_t st = 1;
      for (int d = x_rank - 1; d >= 0; --d) {
        sstr[d] = st;
        st *= s_shape[d];
        repeats[d] = s_shape[d] ? x_shape[d] / s_shape[d] : 1;
        coord[d] = 0;
      }
    } else {
      for (int d = (int)axis + 1; d < x_rank; ++d) inner *= x_shape[d];
      axis_size = x_shape[axis];
    }
  }
  for (int64_t i = 0; i < n; ++i) {
    int64_t si = 0;
    if (ns != 1) {
      if (blocked) {
        for (int d = 0; d < x_rank; ++d) si += (coord[d] / repeats[d]) * sstr[d];
        for (int d = x_rank - 1; d >= 0; --d) {
          if (++coord[d] < x_shape[d]) break;
          coord[d] = 0;
        }
      } else {
        si = (i / inner) % axis_size;
      }
    }
    const float zpv = zp ? dq_decode(zp, x_dtype, si) : 0.0f;
    const float v = (dq_decode(x, x_dtype, i) - zpv) * sc[si];
    if (scale_dtype == ORC_FLOAT16) {
      ((uint16_t *)y)[i] = orc_f32_to_f16(v);
    } else {
      ((float *)y)[i] = v;
    }
  }
  free(sc);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* QuantizeLinear, kq/kernel_quantizelinear.cc.                              */

/* fp32 value of x (FLOAT or FLOAT16), FloatValues :33-55. */
static float ql_load(const void *x, int dtype, int64_t i) {
  return dtype == ORC_FLOAT16 ? orc_f16_to_f32(((const uint16_t *)x)[i]) : ((const float *)x)[i];
}

/* Zero point of scale index si as fp32: the integer value (sub-byte codes
 * sign- or zero-extended, :186-188) or the float decode (:93-107). */
static float ql_zero_point(const void *zp, int dtype, int64_t si) {
  if (!zp) return 0.0f;
  return orc_dq_decode(zp, dtype, si);
}

/* The saturating fp8 encoders of rk/cast_float8.cc:124-173 (E4M3FNUZ),
 * :214-262 (E5M2) and :303-346 (E5M2FNUZ), restated: round to nearest even
 * on the fp32 bits; infinities saturate to the largest finite code; NaN is
 * 0x80 for the FNUZ types and sign|0x7e for E5M2; FNUZ results that round to
 * zero are +0 (0x80 is NaN). */
static uint8_t fp8_encode(float v, int mbits, int bias, int fnuz) {
  uint32_t b;
  memcpy(&b, &v, 4);
  const uint8_t sign = (uint8_t)((b >> 24) & 0x80u);
  const uint8_t maxc = fnuz ? 0x7f : 0x7b;  /* E4M3FNUZ 240, E5M2 / E5M2FNUZ 57344 */
  if ((b & 0x7fffffffu) == 0x7f800000u) return (uint8_t)(sign | maxc);
  if ((b & 0x7f800000u) == 0x7f800000u) return fnuz ? 0x80 : (uint8_t)(sign | 0x7e);
  const int e = (int)((b >> 23) & 0xff);
  const uint32_t m = b & 0x7fffffu;
  if (e == 0) return fnuz ? 0 : sign;  /* fp32 zeros and subnormals */
  const int E = e - 127 + bias;         /* biased exponent of a normal result */
  uint32_t mag;
  if (E >= 1) {
    const uint32_t full = ((uint32_t)E << 23) | m, sh = 23 - mbits;
    const uint32_t q = full >> sh, rem = full & ((1u << sh) - 1), half = 1u << (sh - 1);
    mag = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
  } else {
    const int sh = 24 - mbits - E;       /* value / 2^(1 - bias - mbits), a 24-bit significand */
    if (sh > 25) {
      mag = 0;
    } else {
      const uint32_t full = m | 0x800000u;
      const uint32_t q = full >> sh, rem = full & ((1u << sh) - 1), half = 1u << (sh - 1);
      mag = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
    }
  }
  if (mag > maxc) mag = maxc;
  if (fnuz && mag == 0) return 0;
  return (uint8_t)(sign | mag);
}

/* FLOAT4E2M1 nearest code (cast_helper.cc:168-203): NaN -> 0, beyond +-6
 * saturates, distances in fp32 over the same-sign codes, ties to the even
 * code. */
static uint8_t fp4_encode(float v) {
  static const float pos[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  if (isnan(v)) return 0;
  if (v > 6.0f) return 7;
  if (v < -6.0f) return 15;
  if (v == 0.0f) return signbit(v) ? 8 : 0;
  const int neg = !(v > 0.0f);
  uint8_t best = neg ? 8 : 0;
  float bd = fabsf(v - (neg ? -0.0f : 0.0f));
  for (int i = 1; i < 8; ++i) {
    const float d = fabsf(v - (neg ? -pos[i] : pos[i]));
    const uint8_t code = (uint8_t)(neg ? 8 + i : i);
    if (d < bd || (d == bd && !(code & 1u) && (best & 1u))) {
      best = code;
      bd = d;
    }
  }
  return best;
}

/* FLOAT6 nearest code (cast_helper.cc:220-246): NaN -> 0, +-inf -> +-max,
 * the first magnitude code not below |v| and the one before it compared by
 * fp32 distance, ties to the even code; beyond the largest, the largest. */
static uint8_t fp6_encode(float v, int dtype) {
  if (isnan(v)) return 0;
  const uint8_t s = signbit(v) ? 0x20 : 0;
  if (isinf(v)) return (uint8_t)(0x1f | s);
  const float mag = fabsf(v);
  int up = 0;
  while (up < 32 && orc_f6_to_f32((uint8_t)up, dtype) < mag) ++up;
  uint8_t best = up == 32 ? 0x1f : (uint8_t)up;
  if (up != 0 && up != 32) {
    const float ld = mag - orc_f6_to_f32((uint8_t)(up - 1), dtype), ud = orc_f6_to_f32((uint8_t)up, dtype) - mag;
    if (ld < ud || (ld == ud && !((up - 1) & 1))) best = (uint8_t)(up - 1);
  }
  return (uint8_t)(best | s);
}

uint8_t orc_f32_to_float_code(float v, int dtype) {
  switch (dtype) {
  case ORC_FLOAT8E4M3FN: return orc_f32_to_f8e4m3fn(v);
  case ORC_FLOAT8E4M3FNUZ: return fp8_encode(v, 3, 8, 1);
  case ORC_FLOAT8E5M2: return fp8_encode(v, 2, 15, 0);
  case ORC_FLOAT8E5M2FNUZ: return fp8_encode(v, 2, 16, 1);
  case ORC_FLOAT4E2M1: return fp4_encode(v);
  default: return fp6_encode(v, dtype);
  }
}

static void put_bits(uint8_t *y, int64_t i, int bits, uint32_t code) {
  const int64_t bit = i * bits;
  uint32_t v = (code & ((1u << bits) - 1u)) << (bit % 8);
  y[bit / 8] |= (uint8_t)v;
  if ((bit % 8) + bits > 8) y[bit / 8 + 1] |= (uint8_t)(v >> 8);
}

/* Integer result of nearbyint(v) + zp clamped to [lo, hi] by the
 * reference's two comparisons (:75-80); NaN passes both comparisons and the
 * x86-64 float-to-int conversion of the reference build turns it into
 * 0x80000000, whose low bits the narrowing keeps: 0 for every output type. */
static int32_t ql_saturate(float v, float lo, float hi) {
  if (v < lo) v = lo;
  else if (v > hi) v = hi;
  if (isnan(v)) return 0;
  return (int32_t)v;
}

int orc_quantize_linear(const void *x, int x_dtype, const int64_t *x_shape, int x_rank,
                        const void *scale, int scale_dtype, const int64_t *s_shape, int s_rank,
                        const void *zp, int y_dtype, int64_t axis, void *y) {
  if (x_dtype != ORC_FLOAT && x_dtype != ORC_FLOAT16) return 1;
  if (scale_dtype != ORC_FLOAT && scale_dtype != ORC_FLOAT16) return 1;
  float lo, hi;
  switch (y_dtype) {
  case ORC_UINT8: lo = 0.0f; hi = 255.0f; break;
  case ORC_INT8: lo = -128.0f; hi = 127.0f; break;
  case ORC_UINT16: lo = 0.0f; hi = 65535.0f; break;
  case ORC_INT16: lo = -32768.0f; hi = 32767.0f; break;
  case ORC_UINT4: lo = 0.0f; hi = 15.0f; break;
  case ORC_INT4: lo = -8.0f; hi = 7.0f; break;
  case ORC_UINT2: lo = 0.0f; hi = 3.0f; break;
  case ORC_INT2: lo = -2.0f; hi = 1.0f; break;
  case ORC_FLOAT8E4M3FN: case ORC_FLOAT8E4M3FNUZ: case ORC_FLOAT8E5M2: case ORC_FLOAT8E5M2FNUZ:
  case ORC_FLOAT4E2M1: case ORC_FLOAT6E2M3: case ORC_FLOAT6E3M2:
    lo = hi = 0.0f;
    break;
  default: return 1;
  }
  const int sub_bits = y_dtype == ORC_UINT4 || y_dtype == ORC_INT4 || y_dtype == ORC_FLOAT4E2M1 ? 4
                       : y_dtype == ORC_UINT2 || y_dtype == ORC_INT2                          ? 2
                       : y_dtype == ORC_FLOAT6E2M3 || y_dtype == ORC_FLOAT6E3M2              ? 6
                                                                                            : 0;
  const int64_t n = numel(x_shape, x_rank);
  const int64_t ns = numel(s_shape, s_rank);
  int64_t repeats[ORC_MAX_RANK], sstr[ORC_MAX_RANK], coord[ORC_MAX_RANK];
  const int blocked = ns != 1 && s_rank == x_rank;
  int64_t inner = 1, axis_size = 1;
  if (ns != 1) {
    if (axis < 0 || axis >= x_rank || x_rank > ORC_MAX_RANK) return 1;
    if (blocked) {
      int64_t st = 1;
      for (int d = x_rank - 1; d >= 0; --d) {
        sstr[d] = st;
        st *= s_shape[d];
        repeats[d] = s_shape[d] ? x_shape[d] / s_shape[d] : 1;
        coord[d] = 0;
      }
    } else {
      for (int d = (int)axis + 1; d < x_rank; ++d) inner *= x_shape[d];
      axis_size = x_shape[axis];
    }
  }
  if (sub_bits) memset(y, 0, (size_t)((n * sub_bits + 7) / 8));
  for (int64_t i = 0; i < n; ++i) {
    int64_t si = 0;
    if (ns != 1) {
      if (blocked) {
        for (int d = 0; d < x_rank; ++d) si += (coord[d] / repeats[d]) * sstr[d];
        for (int d = x_rank - 1; d >= 0; --d) {
          if (++coord[d] < x_shape[d]) break;
          coord[d] = 0;
        }
      } else {
        si = (i / inner) % axis_size;
      }
    }
    const float q = ql_load(x, x_dtype, i) / ql_load(scale, scale_dtype, si);
    const float z = ql_zero_point(zp, y_dtype, si);
    if (y_dtype == ORC_FLOAT8E4M3FN || y_dtype == ORC_FLOAT8E4M3FNUZ || y_dtype == ORC_FLOAT8E5M2 ||
        y_dtype == ORC_FLOAT8E5M2FNUZ) {
      /* both NaN: x86-64 returns the destination operand, which gcc -O2
       * makes the zero point in the reference's `x / scale + zp`; stated
       * here so that this file's own register choice does not decide it */
      const float v = (isnan(q) && isnan(z)) ? z : q + z;
      ((uint8_t *)y)[i] = orc_f32_to_float_code(v, y_dtype);
      continue;
    }
    if (y_dtype == ORC_FLOAT4E2M1 || y_dtype == ORC_FLOAT6E2M3 || y_dtype == ORC_FLOAT6E3M2) {
      /* no zero point: nothing is added, so -0 stays -0 (:508-511) */
      put_bits((uint8_t *)y, i, sub_bits, orc_f32_to_float_code(zp ? q + z : q, y_dtype));
      continue;
    }
    const int32_t v = ql_saturate(nearbyintf(q) + z, lo, hi);
    if (y_dtype == ORC_UINT2 || y_dtype == ORC_INT2) {
      put_bits((uint8_t *)y, i, 2, (uint32_t)v);
      continue;
    }
    switch (y_dtype) {
    case ORC_UINT8: ((uint8_t *)y)[i] = (uint8_t)v; break;
    case ORC_INT8: ((int8_t *)y)[i] = (int8_t)v; break;
    case ORC_UINT16: ((uint16_t *)y)[i] = (uint16_t)v; break;
    case ORC_INT16: ((int16_t *)y)[i] = (int16_t)v; break;
    default: /* 4-bit, low nibble first on the flat index (rk/cast_sub_byte.h:50-60) */
      ((uint8_t *)y)[i >> 1] |= (uint8_t)(((uint32_t)v & 0x0fu) << ((i & 1) ? 4 : 0));
    }
  }
  return 0;
}

/* kq/kernel_dynamicquantizelinear.cc:57-121: range widened to include 0,
 * scale = range / 255 (1 when the range is 0), zero point
 * saturate(nearbyint(-min / scale)), y = saturate(nearbyint(x / scale) + zp). */
int orc_dynamic_quantize_linear(const float *x, int64_t n, uint8_t *y, float *y_scale,
                                uint8_t *y_zero_point) {
  if (n <= 0) return 1;
  float x_min = 0.0f, x_max = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    if (!isfinite(v)) return 1;
    if (v < x_min) x_min = v;
    if (v > x_max) x_max = v;
  }
  const float range = x_max - x_min;
  const float scale = range == 0.0f ? 1.0f : range / 255.0f;
  float zpf = nearbyintf(-x_min / scale);
  if (zpf < 0.0f) zpf = 0.0f;
  if (zpf > 255.0f) zpf = 255.0f;
  const uint8_t zp = (uint8_t)zpf;
  *y_scale = scale;
  *y_zero_point = zp;
  const float zf = (float)zp;
  for (int64_t i = 0; i < n; ++i) {
    float v = nearbyintf(x[i] / scale) + zf;
    if (v < 0.0f) v = 0.0f;
    if (v > 255.0f) v = 255.0f;
    y[i] = (uint8_t)v;
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* DequantizePacked for the 32-value GGUF block formats and q4_k / q6_k
 * (onnx_core/runtime/dequantize_packed.cc:173-252, the ggml layouts at ggml
 * da8e2a54b919557b816b1c2beb432ccb766f7ce0): an fp16 scale d, and for the
 * affine formats an fp16 minimum m, then the codes.  Every fp32 product and
 * sum is rounded on its own (the reference forces it through volatile). */

static int pk_unpack4(const uint8_t *p, int i) { /* Unpack(p, i, 4, 16) */
  return (p[i % 16] >> (4 * (i / 16))) & 15;
}

static const int pk_iq4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

int orc_packed_block_bytes(int ggml_type) {
  switch (ggml_type) {
  case 2: return 18;  /* q4_0 */
  case 3: return 20;  /* q4_1 */
  case 6: return 22;  /* q5_0 */
  case 7: return 24;  /* q5_1 */
  case 8: return 34;  /* q8_0 */
  case 9: return 36;  /* q8_1 */
  case 20: return 18; /* iq4_nl */
  case 12: return 144; /* q4_k */
  case 14: return 210; /* q6_k */
  case 10: return 84;  /* q2_k */
  case 11: return 110; /* q3_k */
  case 13: return 176; /* q5_k */
  case 15: return 292; /* q8_k */
  case 23: return 136; /* iq4_xs */
  case 34: return 54;  /* tq1_0 */
  case 35: return 66;  /* tq2_0 */
  case 39: return 17;  /* mxfp4 */
  case 40: return 36;  /* nvfp4 */
  case 41: return 18;  /* q1_0 */
  case 42: return 18;  /* q2_0 */
  case 16: return 66;  /* iq2_xxs */
  case 17: return 74;  /* iq2_xs */
  case 22: return 82;  /* iq2_s */
  case 18: return 98;  /* iq3_xxs */
  case 21: return 110; /* iq3_s */
  case 19: return 50;  /* iq1_s */
  case 29: return 56;  /* iq1_m */
  default: return 0;
  }
}

/* values per block (dequantize_packed.cc:27-36) */
int orc_packed_block_values(int ggml_type) {
  switch (ggml_type) {
  case 2: case 3: case 6: case 7: case 8: case 9: case 20: case 39: return 32;
  case 40: case 42: return 64;
  case 41: return 128;
  default: return orc_packed_block_bytes(ggml_type) ? 256 : 0;
  }
}

/* Unpack(p, i, bits, group) of dequantize_packed.cc:64-68: value i of
 * grouped bit planes (8 / bits planes of `group` bytes). */
static int pk_unpack(const uint8_t *p, int i, int bits, int group) {
  const int planes = 8 / bits;
  return (p[(i / (planes * group)) * group + i % group] >> (bits * ((i / group) % planes))) & ((1 << bits) - 1);
}

/* q4_k and q6_k, the 256-value blocks of dequantize_packed.cc:193-208 and
 * :240-252.  q4_k: fp16 d and dmin, 12 bytes of 6-bit sub-block scales and
 * minima, 128 code bytes; value = (d * scale) * q - dmin * minimum.  q6_k:
 * 128 low-nibble bytes, 64 bytes of 2-bit high parts, 16 int8 sub-block
 * scales, fp16 d; value = (d * scale) * (q - 32).  Every fp32 step rounded
 * on its own. */
static void pk_decode_k(int ggml_type, const uint8_t *p, float *out) {
  for (int i = 0; i < 256; ++i) {
    volatile float v;
    if (ggml_type == 12) {
      const float d = orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
      const float dmin = orc_f16_to_f32((uint16_t)(p[2] | (p[3] << 8)));
      const uint8_t *sc = p + 4;
      const int g = i / 32;
      const int scale = g < 4 ? sc[g] & 63 : (sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4);
      const int minimum = g < 4 ? sc[g + 4] & 63 : (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
      const int q = pk_unpack(p + 16, i, 4, 32);
      volatile float ds = d * (float)scale;
      volatile float dq = ds * (float)q;
      volatile float dm = dmin * (float)minimum;
      v = dq - dm;
    } else {
      const float d = orc_f16_to_f32((uint16_t)(p[208] | (p[209] << 8)));
      const int q = (pk_unpack(p, i, 4, 64) | (pk_unpack(p + 128, i, 2, 32) << 4)) - 32;
      volatile float ds = d * (float)(int8_t)p[192 + i / 16];
      v = ds * (float)q;
    }
    out[i] = v;
  }
}

/* The other non-codebook profiles, value by value (dequantize_packed.cc:
 * 199-279 for the decode, :27-36 for the layouts).  Every fp32 product,
 * sum and difference rounded on its own:
 *  q2_k (84 B): 16 scale bytes (low nibble scale, high nibble minimum per 16
 *    values), 64 bytes of 2-bit codes, fp16 d at 80 and dmin at 82;
 *    (d * scale) * q - dmin * minimum;
 *  q3_k (110 B): 32 bytes of high-bit masks, 64 bytes of 2-bit codes, 6-bit
 *    signed scales (low nibbles at 96, high 2 bits at 104), fp16 d at 108;
 *    q loses 4 where its mask bit is clear; (d * (scale - 32)) * q;
 *  q5_k (176 B): q4_k's header, 32 bytes of fifth bits at 16, 128 nibble
 *    bytes at 48;
 *  q8_k (292 B): fp32 d, 256 int8 codes (and 32 bytes of sums, unused);
 *  iq4_xs (136 B): fp16 d, 2 bytes of high scale bits, 4 bytes of low scale
 *    nibbles, 128 nibble bytes into the iq4 table; (d * (scale - 32)) * v;
 *  tq1_0 (54 B): base-3 digits packed five (then four) per byte by
 *    multiplication, fp16 d at 52; d * (digit - 1);
 *  tq2_0 (66 B): 2-bit codes, fp16 d at 64; d * (q - 1);
 *  mxfp4 (17 B, 32 values): an e8m0 scale byte (2^(e - 127), with e = 0, 1
 *    the fp32 subnormals 2^-128, 2^-127 written as 0x00200000 << e), 16 bytes
 *    of e2m1 codes taken as twice their value; scale * 2v;
 *  nvfp4 (36 B, 64 values): 4 ue4m3 scale bytes (0 and 127 give 0) per 16
 *    values, 32 bytes of e2m1 codes; scale * 2v;
 *  q1_0 (18 B, 128 values): fp16 d, a sign bit per value: +d or -d;
 *  q2_0 (18 B, 64 values): fp16 d, 2-bit codes four per byte; d * (q - 1). */
static const int pk_fp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static float pk_half(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static float pk_mul(float a, float b) { volatile float r = a * b; return r; }
static float pk_sub(float a, float b) { volatile float r = a - b; return r; }

static void pk_decode_ext(int t, const uint8_t *p, float *out) {
  const int n = orc_packed_block_values(t);
  for (int i = 0; i < n; ++i) {
    float v = 0.0f;
    if (t == 10) {
      const int g = i / 16, q = pk_unpack(p + 16, i, 2, 32);
      v = pk_sub(pk_mul(pk_mul(pk_half(p + 80), (float)(p[g] & 15)), (float)q),
                 pk_mul(pk_half(p + 82), (float)(p[g] >> 4)));
    } else if (t == 11) {
      const int g = i / 16;
      const int scale = (pk_unpack(p + 96, g, 4, 8) | (pk_unpack(p + 104, g, 2, 4) << 4)) - 32;
      const int q = pk_unpack(p + 32, i, 2, 32) - (1 - pk_unpack(p, i, 1, 32)) * 4;
      v = pk_mul(pk_mul(pk_half(p + 108), (float)scale), (float)q);
    } else if (t == 13) {
      const uint8_t *sc = p + 4;
      const int g = i / 32;
      const int scale = g < 4 ? sc[g] & 63 : (sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4);
      const int minimum = g < 4 ? sc[g + 4] & 63 : (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
      const int q = pk_unpack(p + 48, i, 4, 32) | (pk_unpack(p + 16, i, 1, 32) << 4);
      v = pk_sub(pk_mul(pk_mul(pk_half(p), (float)scale), (float)q), pk_mul(pk_half(p + 2), (float)minimum));
    } else if (t == 15) {
      uint32_t bits = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
      float d;
      memcpy(&d, &bits, 4);
      v = pk_mul(d, (float)(int8_t)p[4 + i]);
    } else if (t == 23) {
      const int g = i / 32;
      const uint32_t high = (uint32_t)p[2] | ((uint32_t)p[3] << 8);
      const int scale = (((p[4 + g / 2] >> (4 * (g % 2))) & 15) | (((high >> (2 * g)) & 3) << 4)) - 32;
      v = pk_mul(pk_mul(pk_half(p), (float)scale), (float)pk_iq4[pk_unpack(p + 8, i, 4, 16)]);
    } else if (t == 34) {
      static const int powers[5] = {1, 3, 9, 27, 81};
      const int start = i < 160 ? 0 : i < 240 ? 32 : 48;
      const int width = i < 160 ? 32 : i < 240 ? 16 : 4;
      const int offset = i < 160 ? i : i < 240 ? i - 160 : i - 240;
      const int q = ((p[start + offset % width] * powers[offset / width]) & 255) * 3 / 256 - 1;
      v = pk_mul(pk_half(p + 52), (float)q);
    } else if (t == 35) {
      v = pk_mul(pk_half(p + 64), (float)(pk_unpack(p, i, 2, 32) - 1));
    } else if (t == 39) {
      const uint32_t e = p[0];
      const uint32_t bits = e <= 1 ? 0x00200000u << e : (e - 1) << 23;
      float scale;
      memcpy(&scale, &bits, 4);
      v = pk_mul(scale, (float)pk_fp4[pk_unpack(p + 1, i, 4, 16)]);
    } else if (t == 40) {
      const int g = i / 16, e = p[g], exponent = (e >> 3) & 15, mantissa = e & 7;
      const float scale = e == 0 || e == 127 ? 0.0f
                          : exponent == 0    ? ldexpf((float)mantissa, -10)
                                             : ldexpf(1.0f + (float)mantissa / 8.0f, exponent - 8);
      v = pk_mul(scale, (float)pk_fp4[pk_unpack(p + 4 + 8 * g, i % 16, 4, 8)]);
    } else if (t == 41) {
      const float d = pk_half(p);
      v = (p[2 + i / 8] >> (i % 8)) & 1 ? d : -d;
    } else if (t == 42) {
      v = pk_mul(pk_half(p), (float)(pk_unpack(p + 2, i, 2, 1) - 1));
    }
    out[i] = v;
  }
}

/* The codebook profiles (dequantize_packed.cc:84-170, profile table :27-36;
 * the lattice grids of ggml src/ggml-common.h, in gguf_codebooks.h).  A
 * 256-value block is 32 octets: octet o = 4 g + l (g the 32-value group, l its
 * lane) holds values 8 o .. 8 o + 7, lane j of one grid row (8-value rows;
 * the iq3 grids have 4-value rows, two per octet), each value signed by one
 * sign bit and scaled.
 *  iq2_xxs (66 B): fp16 d; group g's 8 bytes at 2 + 8 g: four index bytes
 *    (lane l), then a 32-bit word w: lane l's 7 sign bits at 7 l, completed to
 *    even parity by an eighth, and scale (d * (0.5 + (w >> 28))) * 0.25;
 *  iq2_xs (74 B): fp16 d; a 16-bit word per octet at 2 + 2 o: 9-bit index,
 *    7 sign bits (parity as above); scale (d * (0.5 + s)) * 0.25, s nibble
 *    l / 2 of byte 66 + g;
 *  iq2_s (82 B): fp16 d; index byte 2 + o with bits 2 l .. 2 l + 1 of byte
 *    66 + g above it; 8 sign bits at 34 + o; s nibble l / 2 of byte 74 + g;
 *  iq3_xxs (98 B): fp16 d; two index bytes per octet at 2 + 2 o (4-value
 *    rows); group word at 66 + 4 g: signs as iq2_xxs, scale
 *    (d * (0.5 + (w >> 28))) * 0.5;
 *  iq3_s (110 B): fp16 d; index bytes 2 + 2 o, 2 o + 3, each with a ninth bit
 *    (bit 2 l + half of byte 66 + g); 8 sign bits at 74 + o; scale
 *    d * (1 + 2 s), s nibble g % 2 of byte 106 + g / 2;
 *  iq1_s (50 B): fp16 d; index byte 2 + o with 3 bits (3 l) of the 16-bit word
 *    h at 34 + 2 g above it; value (d * (2 s + 1)) * (grid + delta), s bits
 *    12-14 of h, delta -0.125 when bit 15 of h is set, else 0.125;
 *  iq1_m (56 B): index byte o with the low 3 bits of nibble o % 2 of byte
 *    32 + o / 2 above it, that nibble's bit 3 the sign of delta; d the fp16
 *    made of the top nibbles of the four 16-bit words at 48 (word j: bits
 *    4 j .. 4 j + 3); s the 3-bit field 6 (g % 2) + 3 (l / 2) of word g / 2.
 * Sign bits only flip the sign (a multiply by +-1); every other fp32 product
 * and sum is rounded on its own. */
static float pk_add(float a, float b) { volatile float r = a + b; return r; }

static int pk_u16(const uint8_t *p) { return p[0] | (p[1] << 8); }
static uint32_t pk_u32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
/* +-1 for bit j of 7 sign bits completed to even parity (or 8 given bits) */
static float pk_sign(uint32_t bits, int j, int parity) {
  if (parity) {
    uint32_t c = bits, n = 0;
    while (c) { n += c & 1u; c >>= 1; }
    bits |= (n & 1u) << 7;
  }
  return (bits >> j) & 1u ? -1.0f : 1.0f;
}
static int pk_lane8(uint64_t row, int j) { return (int)(int8_t)(uint8_t)(row >> (8 * j)); }
static int pk_lane4(uint32_t row, int j) { return (int)(int8_t)(uint8_t)(row >> (8 * j)); }

static void pk_decode_iq(int t, const uint8_t *p, float *out) {
  float d = orc_f16_to_f32((uint16_t)pk_u16(p));
  int words[4] = {0, 0, 0, 0};
  if (t == 29) {
    int bits = 0;
    for (int j = 0; j < 4; ++j) {
      words[j] = pk_u16(p + 48 + 2 * j);
      bits |= (words[j] >> 12) << (4 * j);
    }
    d = orc_f16_to_f32((uint16_t)bits);
  }
  for (int o = 0; o < 32; ++o) {
    const int g = o / 4, l = o % 4;
    float *v = out + 8 * o;
    if (t == 16 || t == 17 || t == 22) {
      int index;
      uint32_t signs;
      int parity = 1;
      float s;
      if (t == 16) {
        const uint32_t w = pk_u32(p + 6 + 8 * g);
        index = p[2 + 8 * g + l];
        signs = (w >> (7 * l)) & 127u;
        s = (float)(w >> 28);
      } else if (t == 17) {
        const int w = pk_u16(p + 2 + 2 * o);
        index = w & 511;
        signs = (uint32_t)(w >> 9);
        s = (float)((p[66 + g] >> (4 * (l / 2))) & 15);
      } else {
        index = p[2 + o] | (((p[66 + g] >> (2 * l)) & 3) << 8);
        signs = p[34 + o];
        parity = 0;
        s = (float)((p[74 + g] >> (4 * (l / 2))) & 15);
      }
      const float scale = pk_mul(pk_mul(d, 0.5f + s), 0.25f);
      const uint64_t row = t == 16 ? kGgufIq2xxs[index] : t == 17 ? kGgufIq2xs[index] : kGgufIq2s[index];
      for (int j = 0; j < 8; ++j) v[j] = pk_mul(pk_mul(scale, (float)pk_lane8(row, j)), pk_sign(signs, j, parity));
    } else if (t == 18 || t == 21) {
      uint32_t signs;
      int parity;
      float scale;
      if (t == 18) {
        const uint32_t w = pk_u32(p + 66 + 4 * g);
        signs = (w >> (7 * l)) & 127u;
        parity = 1;
        scale = pk_mul(pk_mul(d, 0.5f + (float)(w >> 28)), 0.5f);
      } else {
        signs = p[74 + o];
        parity = 0;
        scale = pk_mul(d, (float)(1 + 2 * ((p[106 + g / 2] >> (4 * (g % 2))) & 15)));
      }
      for (int half = 0; half < 2; ++half) {
        int index = p[2 + 2 * o + half];
        if (t == 21) index |= ((p[66 + g] >> (2 * l + half)) & 1) << 8;
        const uint32_t row = t == 18 ? kGgufIq3xxs[index] : kGgufIq3s[index];
        for (int j = 0; j < 4; ++j)
          v[4 * half + j] = pk_mul(pk_mul(scale, (float)pk_lane4(row, j)), pk_sign(signs, 4 * half + j, parity));
      }
    } else {
      int index, mult;
      float delta;
      if (t == 19) {
        const int h = pk_u16(p + 34 + 2 * g);
        index = p[2 + o] | (((h >> (3 * l)) & 7) << 8);
        mult = 2 * ((h >> 12) & 7) + 1;
        delta = h & 0x8000 ? -0.125f : 0.125f;
      } else {
        const int nib = (p[32 + o / 2] >> (4 * (o % 2))) & 15;
        index = p[o] | ((nib & 7) << 8);
        mult = 2 * ((words[g / 2] >> (6 * (g % 2) + 3 * (l / 2))) & 7) + 1;
        delta = nib & 8 ? -0.125f : 0.125f;
      }
      const float scale = pk_mul(d, (float)mult);
      for (int j = 0; j < 8; ++j) v[j] = pk_mul(scale, pk_add((float)pk_lane8(kGgufIq1s[index], j), delta));
    }
  }
}

int orc_dequantize_packed(int ggml_type, const uint8_t *x, int64_t nblocks, float *out) {
  const int bytes = orc_packed_block_bytes(ggml_type);
  if (!bytes) return 1;
  if (ggml_type == 16 || ggml_type == 17 || ggml_type == 18 || ggml_type == 19 || ggml_type == 21 ||
      ggml_type == 22 || ggml_type == 29) {
    for (int64_t b = 0; b < nblocks; ++b, x += bytes, out += 256) pk_decode_iq(ggml_type, x, out);
    return 0;
  }
  const int ext = ggml_type == 10 || ggml_type == 11 || ggml_type == 13 || ggml_type == 15 || ggml_type == 23 ||
                  (ggml_type >= 34 && ggml_type <= 42);
  if (ext) {
    const int n = orc_packed_block_values(ggml_type);
    for (int64_t b = 0; b < nblocks; ++b, x += bytes, out += n) pk_decode_ext(ggml_type, x, out);
    return 0;
  }
  if (ggml_type == 12 || ggml_type == 14) {
    for (int64_t b = 0; b < nblocks; ++b, x += bytes, out += 256) pk_decode_k(ggml_type, x, out);
    return 0;
  }
  for (int64_t b = 0; b < nblocks; ++b, x += bytes, out += 32) {
    const float d = orc_f16_to_f32((uint16_t)(x[0] | (x[1] << 8)));
    for (int i = 0; i < 32; ++i) {
      volatile float v;
      if (ggml_type == 8 || ggml_type == 9) {
        const int q = (int8_t)x[(ggml_type == 8 ? 2 : 4) + i];
        v = d * (float)q;
      } else {
        const int affine = ggml_type == 3 || ggml_type == 7, five = ggml_type == 6 || ggml_type == 7;
        const int off = affine ? 4 : 2;
        int q = pk_unpack4(x + off + (five ? 4 : 0), i);
        if (five) {
          const uint32_t qh = (uint32_t)x[off] | ((uint32_t)x[off + 1] << 8) | ((uint32_t)x[off + 2] << 16) |
                              ((uint32_t)x[off + 3] << 24);
          q |= (int)((qh >> i) & 1u) << 4;
        }
        if (ggml_type == 20) {
          v = d * (float)pk_iq4[q];
        } else {
          if (!affine) q -= five ? 16 : 8;
          v = d * (float)q;
          if (affine) {
            const float m = orc_f16_to_f32((uint16_t)(x[2] | (x[3] << 8)));
            v = v + m;
          }
        }
      }
      out[i] = v;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* ConvInteger (nn/kernel_conv_integer.cc) and QLinearConv
 * (kq/kernel_qlinearconv.cc): the same attribute resolution and the same
 * direct loops over (n, m, output position) x (input channel of the group,
 * kernel tap); taps that fall into the padding are skipped.               */

/* ResolveAttributes + ComputeOutputSpatial (kernel_conv_integer.cc:24-54,
 * :107-141; kernel_qlinearconv.cc:53-119 are the same).  kernel_shape,
 * strides, dilations and pads may be NULL (defaults); pads_out receives the
 * resolved pads (2 * spatial rank), out_spatial the output sizes.  Returns
 * 0, or 1 for an attribute the reference rejects. */
int orc_conv_geometry(const int64_t *x_shape, int x_rank, const int64_t *w_shape,
                      const int64_t *kernel_shape, const int64_t *strides, const int64_t *pads,
                      const int64_t *dilations, int auto_pad, int64_t *k_out, int64_t *s_out,
                      int64_t *d_out, int64_t *pads_out, int64_t *out_spatial) {
  const int sr = x_rank - 2;
  if (sr < 1 || sr > ORC_MAX_RANK) return 1;
  for (int i = 0; i < sr; ++i) {
    k_out[i] = kernel_shape ? kernel_shape[i] : w_shape[i + 2];
    s_out[i] = strides ? strides[i] : 1;
    d_out[i] = dilations ? dilations[i] : 1;
    pads_out[i] = pads_out[i + sr] = 0;
    if (auto_pad == ORC_AUTO_PAD_NOTSET && pads) {
      pads_out[i] = pads[i];
      pads_out[i + sr] = pads[i + sr];
    }
  }
  if (auto_pad < ORC_AUTO_PAD_NOTSET || auto_pad > ORC_AUTO_PAD_VALID) return 1;
  for (int i = 0; i < sr; ++i) {
    const int64_t in = x_shape[i + 2], s = s_out[i];
    const int64_t eff_k = (k_out[i] - 1) * d_out[i] + 1;
    if (auto_pad == ORC_AUTO_PAD_VALID) {
      out_spatial[i] = (in - eff_k) / s + 1;
    } else if (auto_pad == ORC_AUTO_PAD_NOTSET) {
      out_spatial[i] = (in + pads_out[i] + pads_out[i + sr] - eff_k) / s + 1;
    } else {
      const int64_t out = (in + s - 1) / s;
      int64_t need = (out - 1) * s + eff_k - in;
      if (need < 0) need = 0;
      if (auto_pad == ORC_AUTO_PAD_SAME_UPPER) {
        pads_out[i] = need / 2;
        pads_out[i + sr] = need - need / 2;
      } else {
        pads_out[i + sr] = need / 2;
        pads_out[i] = need - need / 2;
      }
      out_spatial[i] = out;
    }
  }
  return 0;
}

/* Accumulates sum over the group's input channels and the kernel taps of
 * (x - x_zp) * (w - w_zp) for output (n, m, op) in int64 (QLinearConv,
 * kernel_qlinearconv.cc:306-330); ConvInteger truncates it to int32
 * (kernel_conv_integer.cc:269-299 accumulates in int32, which wraps). */
static int64_t conv_point(const void *x, int x_dtype, const int64_t *x_shape, int sr, const void *w,
                          int w_dtype, int64_t cpg, int64_t mpg, int64_t n, int64_t m, const int64_t *oidx,
                          const int64_t *k, const int64_t *s, const int64_t *d, const int64_t *pads,
                          int32_t x_zp, int32_t w_zp) {
  int64_t in_strides[ORC_MAX_RANK], in_size = 1, ks = 1;
  for (int a = sr - 1; a >= 0; --a) {
    in_strides[a] = in_size;
    in_size *= x_shape[a + 2];
    ks *= k[a];
  }
  const int64_t C = x_shape[1], g = m / mpg;
  int64_t acc = 0;
  for (int64_t ic = 0; ic < cpg; ++ic) {
    const int64_t x_base = (n * C + g * cpg + ic) * in_size;
    const int64_t w_base = (m * cpg + ic) * ks;
    int64_t kidx[ORC_MAX_RANK] = {0};
    for (int64_t kp = 0; kp < ks; ++kp) {
      int in_bounds = 1;
      int64_t off = 0;
      for (int a = 0; a < sr; ++a) {
        const int64_t ia = oidx[a] * s[a] + kidx[a] * d[a] - pads[a];
        if (ia < 0 || ia >= x_shape[a + 2]) {
          in_bounds = 0;
          break;
        }
        off += ia * in_strides[a];
      }
      if (in_bounds)
        acc += (int64_t)(read_byte_elem(x, x_dtype, x_base + off) - x_zp) *
               (int64_t)(read_byte_elem(w, w_dtype, w_base + kp) - w_zp);
      for (int a = sr - 1; a >= 0; --a) {
        if (++kidx[a] < k[a]) break;
        kidx[a] = 0;
      }
    }
  }
  return acc;
}

/* Shared driver: y_i32 (ConvInteger) or y_q8 (QLinearConv) for every output.
 * w_zp / w_scale have w_zp_count / w_scale_count values (1 or M). */
static int conv_run(const void *x, int x_dtype, const int64_t *x_shape, int x_rank, const void *w,
                    int w_dtype, const int64_t *w_shape, int32_t x_zp, const void *w_zp,
                    int64_t w_zp_count, int64_t group, const int64_t *kernel_shape,
                    const int64_t *strides, const int64_t *pads, const int64_t *dilations, int auto_pad,
                    int32_t *y_i32, const float *combined, int64_t cs_count, const int32_t *bias,
                    float y_zp, int y_signed, void *y_q8) {
  const int sr = x_rank - 2;
  int64_t k[ORC_MAX_RANK], s[ORC_MAX_RANK], d[ORC_MAX_RANK], pd[2 * ORC_MAX_RANK], od[ORC_MAX_RANK];
  if (orc_conv_geometry(x_shape, x_rank, w_shape, kernel_shape, strides, pads, dilations, auto_pad, k, s,
                        d, pd, od))
    return 1;
  const int64_t N = x_shape[0], M = w_shape[0], cpg = w_shape[1];
  if (group < 1 || x_shape[1] != cpg * group || M % group != 0) return 1;
  const int64_t mpg = M / group;
  int64_t osize = 1;
  for (int a = 0; a < sr; ++a) osize *= od[a];
  for (int64_t n = 0; n < N; ++n)
    for (int64_t m = 0; m < M; ++m) {
      const int32_t wz = w_zp ? read_byte_elem(w_zp, w_dtype, w_zp_count == M ? m : 0) : 0;
      for (int64_t op = 0; op < osize; ++op) {
        int64_t oidx[ORC_MAX_RANK], rem = op;
        for (int a = sr - 1; a >= 0; --a) {
          oidx[a] = rem % od[a];
          rem /= od[a];
        }
        int64_t acc = conv_point(x, x_dtype, x_shape, sr, w, w_dtype, cpg, mpg, n, m, oidx, k, s, d, pd, x_zp,
                                 wz);
        const int64_t o = (n * M + m) * osize + op;
        if (y_i32) {
          y_i32[o] = (int32_t)(uint32_t)(uint64_t)acc;
          continue;
        }
        if (bias) acc += bias[m];
        const float scaled = (float)acc * combined[cs_count == M ? m : 0];
        float v = nearbyintf(scaled) + y_zp;
        const float lo = y_signed ? -128.0f : 0.0f, hi = y_signed ? 127.0f : 255.0f;
        if (v < lo) v = lo;
        else if (v > hi) v = hi;
        const int32_t q = isnan(v) ? 0 : (int32_t)v; /* x86-64 NaN conversion, then the narrowing */
        if (y_signed) ((int8_t *)y_q8)[o] = (int8_t)q;
        else ((uint8_t *)y_q8)[o] = (uint8_t)q;
      }
    }
  return 0;
}

int orc_conv_integer(const void *x, int x_dtype, const int64_t *x_shape, int x_rank, const void *w,
                     int w_dtype, const int64_t *w_shape, const void *x_zp, const void *w_zp,
                     int64_t w_zp_count, int64_t group, const int64_t *kernel_shape,
                     const int64_t *strides, const int64_t *pads, const int64_t *dilations, int auto_pad,
                     int32_t *y) {
  const int32_t xz = x_zp ? read_byte_elem(x_zp, x_dtype, 0) : 0;
  return conv_run(x, x_dtype, x_shape, x_rank, w, w_dtype, w_shape, xz, w_zp, w_zp_count, group, kernel_shape,
                  strides, pads, dilations, auto_pad, y, NULL, 0, NULL, 0.0f, 0, NULL);
}

int orc_qlinear_conv(const void *x, int x_dtype, const int64_t *x_shape, int x_rank, float x_scale,
                     int32_t x_zp, const void *w, int w_dtype, const int64_t *w_shape, const float *w_scale,
                     int64_t w_scale_count, const void *w_zp, int64_t w_zp_count, float y_scale,
                     int32_t y_zp, int y_signed, const int32_t *bias, int64_t group,
                     const int64_t *kernel_shape, const int64_t *strides, const int64_t *pads,
                     const int64_t *dilations, int auto_pad, void *y) {
  const int64_t M = w_shape[0];
  float *cs = (float *)malloc(sizeof(float) * (size_t)(w_scale_count > 0 ? w_scale_count : 1));
  if (!cs) return 1;
  for (int64_t i = 0; i < w_scale_count; ++i) cs[i] = x_scale * w_scale[i] / y_scale; /* :289 */
  const int rc = conv_run(x, x_dtype, x_shape, x_rank, w, w_dtype, w_shape, x_zp, w_zp, w_zp_count, group,
                          kernel_shape, strides, pads, dilations, auto_pad, NULL, cs,
                          w_scale_count == M ? M : 1, bias, (float)y_zp, y_signed, y);
  free(cs);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* MatMul, km/kernel_matmul.cc:61-147 and :206-218.                          */

typedef struct {
  const mm_plan *p;
  const float *a, *b;
  float *y;
  int64_t r0, r1; /* rows of every batch matrix */
  int64_t part, nparts;
} mm_job;

static void *mm_worker(void *arg) {
  const mm_job *j = (const mm_job *)arg;
  const mm_plan *p = j->p;
  const int64_t K = p->K, N = p->N, M = p->M;
  const int64_t rows = j->r1 - j->r0;
  const int64_t total = p->batch_count * rows;
  const int64_t lo = total * j->part / j->nparts, hi = total * (j->part + 1) / j->nparts;
  for (int64_t t = lo; t < hi; ++t) {
    const int64_t bt = t / rows, i = j->r0 + t % rows;
    int64_t ab, bb;
    mm_batch_base(p, bt, &ab, &bb);
    float *yr = j->y + (bt * M + i) * N;
    for (int64_t c = 0; c < N; ++c) yr[c] = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float av = j->a[ab + i * K + k];
      const float *br = j->b + bb + k * N;
      for (int64_t c = 0; c < N; ++c) yr[c] += av * br[c];
    }
  }
  return NULL;
}

int orc_matmul_f32(const float *a, const int64_t *a_shape, int a_rank, const float *b,
                   const int64_t *b_shape, int b_rank, float *y, int64_t row_begin,
                   int64_t row_end, int nthreads) {
  mm_plan p;
  const int rc = mm_make_plan(a_shape, a_rank, b_shape, b_rank, &p);
  if (rc) return rc;
  if (row_end < 0 || row_end > p.M) row_end = p.M;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  mm_job jobs[256];
  pthread_t th[256];
  for (int t = 0; t < nthreads; ++t) {
    jobs[t].p = &p;
    jobs[t].a = a;
    jobs[t].b = b;
    jobs[t].y = y;
    jobs[t].r0 = row_begin;
    jobs[t].r1 = row_end;
    jobs[t].part = t;
    jobs[t].nparts = nthreads;
  }
  for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, mm_worker, &jobs[t]);
  mm_worker(&jobs[0]);
  for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
  return 0;
}

int orc_matmul_half(const uint16_t *a, const int64_t *a_shape, int a_rank, const uint16_t *b,
                    const int64_t *b_shape, int b_rank, int dtype, uint16_t *y,
                    int64_t row_begin, int64_t row_end, int nthreads) {
  mm_plan p;
  const int rc = mm_make_plan(a_shape, a_rank, b_shape, b_rank, &p);
  if (rc) return rc;
  if (dtype != ORC_FLOAT16 && dtype != ORC_BFLOAT16) return 4;
  const int64_t na = numel(a_shape, a_rank), nb = numel(b_shape, b_rank);
  const int64_t ny = p.batch_count * p.M * p.N;
  float *af = (float *)malloc(sizeof(float) * (size_t)(na ? na : 1));
  float *bf = (float *)malloc(sizeof(float) * (size_t)(nb ? nb : 1));
  float *yf = (float *)calloc((size_t)(ny ? ny : 1), sizeof(float));
  if (!af || !bf || !yf) {
    free(af);
    free(bf);
    free(yf);
    return 5;
  }
  if (dtype == ORC_FLOAT16) {
    orc_f16_to_f32_n(a, na, af);
    orc_f16_to_f32_n(b, nb, bf);
  } else {
    orc_bf16_to_f32_n(a, na, af);
    orc_bf16_to_f32_n(b, nb, bf);
  }
  orc_matmul_f32(af, a_shape, a_rank, bf, b_shape, b_rank, yf, row_begin, row_end, nthreads);
  if (row_end < 0 || row_end > p.M) row_end = p.M;
  for (int64_t bt = 0; bt < p.batch_count; ++bt) {
    for (int64_t i = row_begin; i < row_end; ++i) {
      const int64_t o = (bt * p.M + i) * p.N;
      if (dtype == ORC_FLOAT16) {
        orc_f32_to_f16_n(yf + o, p.N, y + o);
      } else {
        orc_f32_to_bf16_n(yf + o, p.N, y + o);
      }
    }
  }
  free(af);
  free(bf);
  free(yf);
  return 0;
}

/* GroupedMatMul (math/kernel_grouped_matmul.cc:22-46, validation :50-90):
 * y[i, :] for pair i = m * S + s is x[m, :] @ W[g], g = idx[i], W[g] the
 * [K, N] slice of w (transB == 0) or the transpose of its [N, K] slice.  The
 * sum over k runs in order from 0 in the compute type: float for FLOAT,
 * FLOAT16 and BFLOAT16 (16-bit values decoded exactly), double for DOUBLE.
 * With a bias the sum is first rounded to the element type, then
 * bias[g, n] added in the compute type and the result rounded (MatMul
 * followed by Add).  dtype: 1 FLOAT, 11 DOUBLE, 10 FLOAT16, 16 BFLOAT16; idx
 * already widened to int64.  Returns 0, 5 for an index outside [0, G), 4
 * for another dtype. */
int orc_grouped_matmul(int dtype, const void *x, int64_t M, int64_t K, const void *w, int64_t G, int64_t N,
                       int transB, const int64_t *idx, int64_t S, const void *bias, void *y) {
  if (dtype != ORC_FLOAT && dtype != 11 && dtype != ORC_FLOAT16 && dtype != ORC_BFLOAT16) return 4;
  for (int64_t i = 0; i < M * S; ++i)
    if (idx[i] < 0 || idx[i] >= G) return 5;
  for (int64_t i = 0; i < M * S; ++i) {
    const int64_t g = idx[i], m = i / S;
    for (int64_t n = 0; n < N; ++n) {
      if (dtype == 11) {
        const double *xd = (const double *)x, *wd = (const double *)w, *bd = (const double *)bias;
        double v = 0.0;
        for (int64_t l = 0; l < K; ++l)
          v += xd[m * K + l] * wd[transB ? (g * N + n) * K + l : (g * K + l) * N + n];
        if (bd) v = v + bd[g * N + n];
        ((double *)y)[i * N + n] = v;
        continue;
      }
      float v = 0.f;
      for (int64_t l = 0; l < K; ++l) {
        const int64_t wo = transB ? (g * N + n) * K + l : (g * K + l) * N + n;
        float a, b;
        if (dtype == ORC_FLOAT) {
          a = ((const float *)x)[m * K + l];
          b = ((const float *)w)[wo];
        } else if (dtype == ORC_FLOAT16) {
          a = orc_f16_to_f32(((const uint16_t *)x)[m * K + l]);
          b = orc_f16_to_f32(((const uint16_t *)w)[wo]);
        } else {
          a = orc_bf16_to_f32(((const uint16_t *)x)[m * K + l]);
          b = orc_bf16_to_f32(((const uint16_t *)w)[wo]);
        }
        v += a * b;
      }
      if (dtype == ORC_FLOAT) {
        if (bias) v = v + ((const float *)bias)[g * N + n];
        ((float *)y)[i * N + n] = v;
      } else if (dtype == ORC_FLOAT16) {
        if (bias) v = orc_f16_to_f32(orc_f32_to_f16(v)) + orc_f16_to_f32(((const uint16_t *)bias)[g * N + n]);
        ((uint16_t *)y)[i * N + n] = orc_f32_to_f16(v);
      } else {
        if (bias) v = orc_bf16_to_f32(orc_f32_to_bf16(v)) + orc_bf16_to_f32(((const uint16_t *)bias)[g * N + n]);
        ((uint16_t *)y)[i * N + n] = orc_f32_to_bf16(v);
      }
    }
  }
  return 0;
}

/* ORT MatMulNBits value -> dense [K, N] (onnx_core/runtime/quantization.cc:
 * 1806-1880, DecodeValues): B [N, groups, blob] holds the `bits`-bit codes of
 * column n, row r = g * block + j at bit ((j % (8 / bits)) * bits) of byte
 * j / (8 / bits) of blob (n, g); scales [N, groups] (already decoded to
 * double); zero points per (n, g): zp_kind 0 absent (2^(bits-1)), 1 packed
 * UINT8 codes [N, ceil(groups / (8 / bits))] (same bit order), 2 float values
 * [N, groups] (decoded to double).  value = (code - zp) * scale in double,
 * written as double (the caller rounds to the reconstruction dtype).
 * Returns 0, 4 for bits outside {2, 4, 8}. */
int orc_ort_nbits_decode(const uint8_t *B, const double *scales, int zp_kind, const uint8_t *zp_codes,
                         const double *zp_values, int64_t K, int64_t N, int bits, int64_t block, double *out) {
  if (bits != 2 && bits != 4 && bits != 8) return 4;
  const int64_t groups = (K + block - 1) / block, per = 8 / bits, blob = block * bits / 8;
  const int64_t zcol = (groups + per - 1) / per;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t r = 0; r < K; ++r) {
      const int64_t g = r / block, j = r % block, idx = n * groups + g;
      const uint32_t code = (B[idx * blob + j / per] >> ((j % per) * bits)) & mask;
      double zp;
      if (zp_kind == 0) zp = (double)(1u << (bits - 1));
      else if (zp_kind == 1) zp = (double)((zp_codes[n * zcol + g / per] >> ((g % per) * bits)) & mask);
      else zp = zp_values[idx];
      out[r * N + n] = ((double)code - zp) * scales[idx];
    }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* AWQ weights (onnx_core/runtime/awq.cc:185-247, Code and Reconstructed).
 * variant 0 "gemm": qweight INT32 [K, N * bits / 32]; 4 bits: column n of
 *   row k at nibble inv[n % 8] of word k * (N / 8) + n / 8 with inv =
 *   {0, 4, 1, 5, 2, 6, 3, 7}; 8 bits: byte n % 4 of word k * (N / 4) + n / 4;
 *   qzeros INT32 [groups, N * bits / 32] the zero of (group, n) the same way;
 *   scales [groups, N].
 * variant 1 "gemv" (4 bits): qweight [N, K / 8], row k at nibble k % 8 of
 *   word n * (K / 8) + k / 8; qzeros [N, padded / 8], group g at nibble g % 8
 *   of word n * (padded / 8) + g / 8; scales [N, padded].
 * variant 2 "gemv_fast" / "llm-awq" (4 bits): qweight INT16 [N / 4, K], the
 *   inverse of the two 32-code permutations and the 4-row / 64-code
 *   interleave of awq.cc:198-206; float zero terms and scales [padded, N].
 * value: variants 0 and 1 (code - zero) * scale in fp32 (exact); variant 2
 * code * scale rounded to fp32, plus the zero term.  Writes codes [N, K],
 * zeros [N, groups] (variants 0 and 1; 0 for variant 2) and the FLOAT values
 * [N, K]; scales and zero terms are decoded fp16 / bf16 values.  Returns 0,
 * or 1 for an unknown variant or bit width. */
int orc_awq_decode(int variant, int bits, const void *qweight, const void *qzeros, const float *zero_terms,
                   const float *scales, int64_t K, int64_t N, int64_t group, int64_t padded, uint8_t *codes,
                   uint8_t *zeros, float *out) {
  static const int inv[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  if (variant < 0 || variant > 2 || !(bits == 4 || (bits == 8 && variant == 0))) return 1;
  const uint32_t *qw = (const uint32_t *)qweight, *qz = (const uint32_t *)qzeros;
  const uint16_t *qh = (const uint16_t *)qweight;
  const int64_t eff = group == -1 ? K : group, groups = K / eff;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t g = 0; g < groups; ++g) {
      uint32_t z = 0;
      if (variant == 0 && bits == 4) z = qz[g * (N / 8) + n / 8] >> (4 * inv[n % 8]);
      else if (variant == 0) z = qz[g * (N / 4) + n / 4] >> (8 * (n % 4));
      else if (variant == 1) z = qz[n * (padded / 8) + g / 8] >> (4 * (g % 8));
      zeros[n * groups + g] = (uint8_t)(z & mask);
    }
    for (int64_t k = 0; k < K; ++k) {
      uint32_t c;
      if (variant == 0 && bits == 4) c = qw[k * (N / 8) + n / 8] >> (4 * inv[n % 8]);
      else if (variant == 0) c = qw[k * (N / 4) + n / 4] >> (8 * (n % 4));
      else if (variant == 1) c = qw[n * (K / 8) + k / 8] >> (4 * (k % 8));
      else {
        const int64_t i = k % 32;
        const int64_t first = ((i / 2) % 4) * 8 + (i / 8) * 2 + i % 2;
        const int64_t second = (first / 8) * 8 + (first % 2) * 4 + (first % 8) / 2;
        const int64_t flat = (n % 4) * 64 + (k % 64) / 32 * 32 + second;
        c = (uint32_t)qh[(n / 4) * K + (k / 64) * 64 + flat / 4] >> (4 * (flat % 4));
      }
      const int64_t g = k / eff;
      const uint8_t code = (uint8_t)(c & mask);
      codes[n * K + k] = code;
      if (variant == 2) {
        volatile float product = (float)code * scales[g * N + n];
        volatile float v = product + zero_terms[g * N + n];
        out[n * K + k] = v;
      } else {
        const float scale = variant == 1 ? scales[n * padded + g] : scales[g * N + n];
        volatile float v = ((float)code - (float)zeros[n * groups + g]) * scale;
        out[n * K + k] = v;
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* GPTQ weights (onnx_core/runtime/gptq.cc:166-228, Pieces, Code, Zero and
 * Reconstructed).  Words of `width` bytes (1, 2, 4, 8; little-endian).
 * Linear layouts (every format but gptq_p at 3 bits and 5-7 bits): logical
 * code `index` occupies bits index * bits .. of a bit stream of words, split
 * across two words where it crosses one.  Planar layouts (32-bit words):
 * each block of 32 codes spans `bits` words, its 4-, 2- and 1-bit planes (the
 * ones the width has, low to high) one after the other, each plane's code i
 * at bits (i % (32 / plane)) * plane of word (i / (32 / plane)).  qweight
 * [rows, N]: code (k, n) is index k of column n's stream (word w at
 * w * N + n); qzeros [groups, zero_columns]: the zero of (group, n) is index
 * n of row group's stream (word w at group * zero_columns + w), plus 1 for
 * format 0 ("gptq"; 1 "gptq_v2", 2 "gptq_p").  value = (code - zero) *
 * scale[g_idx[k] * N + n] in fp32 (exact).  Writes codes [N, K], zeros
 * [N, groups] (INT16, the +1 included) and the FLOAT values [N, K].
 * Returns 0. */
static uint64_t gq_word(const uint8_t *p, int width) {
  uint64_t w = 0;
  for (int i = 0; i < width; ++i) w |= (uint64_t)p[i] << (8 * i);
  return w;
}

static uint32_t gq_code(const uint8_t *data, int width, int bits, int planar, int64_t index, int64_t stride,
                        int64_t other, int zeros) {
  const int wb = 8 * width;
  uint32_t result = 0;
#define GQ_PIECE(word, shift, nb, off)                                                            \
  do {                                                                                            \
    const int64_t pos_ = zeros ? other * stride + (word) : (word) * stride + other;               \
    result |= (uint32_t)((gq_word(data + pos_ * width, width) >> (shift)) & ((1ull << (nb)) - 1)) \
              << (off);                                                                           \
  } while (0)
  if (!planar) {
    const int64_t bit = index * bits;
    const int shift = (int)(bit % wb);
    const int low = bits < wb - shift ? bits : wb - shift;
    GQ_PIECE(bit / wb, shift, low, 0);
    if (low != bits) GQ_PIECE(bit / wb + 1, 0, bits - low, low);
  } else {
    int offset = 0;
    int64_t word = (index / 32) * bits;
    for (int plane = 4; plane >= 1; plane /= 2) {
      if (!(bits & plane)) continue;
      const int factor = 32 / plane;
      GQ_PIECE(word + (index % 32) / factor, (int)((index % 32) % factor) * plane, plane, offset);
      offset += plane;
      word += plane;
    }
  }
#undef GQ_PIECE
  return result;
}

int orc_gptq_decode(int format, int bits, int width, const void *qweight, const void *qzeros, const float *scales,
                    const int32_t *g_idx, int64_t K, int64_t N, int64_t group, uint8_t *codes, int16_t *zeros,
                    float *out) {
  const int planar = bits == 5 || bits == 6 || bits == 7 || (format == 2 && bits == 3);
  const int64_t eff = group == -1 ? K : group, groups = (K + eff - 1) / eff;
  const int64_t zero_columns = (N * bits + 8 * width - 1) / (8 * width);
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t g = 0; g < groups; ++g)
      zeros[n * groups + g] = (int16_t)(gq_code((const uint8_t *)qzeros, width, bits, planar, n, zero_columns, g, 1) +
                                        (format == 0 ? 1 : 0));
    for (int64_t k = 0; k < K; ++k) {
      const uint32_t code = gq_code((const uint8_t *)qweight, width, bits, planar, k, N, n, 0);
      const int64_t g = g_idx[k];
      codes[n * K + k] = (uint8_t)code;
      volatile float v = ((float)code - (float)zeros[n * groups + g]) * scales[g * N + n];
      out[n * K + k] = v;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* bitsandbytes weights (onnx_core/runtime/bitsandbytes.cc), the encoding
 * "onnx_light.bitsandbytes_weights.v1" of ai.rt:Dequantize.  A weight of
 * logical shape [rows, cols], flattened row-major.  format 0 nf4 / 1 fp4:
 * element i is the 4-bit code (codes[i / 2] >> (i % 2 ? 0 : 4)) & 15 (the
 * even element in the high nibble, :495-496), its value the format's table
 * entry (Codebook, :323-337: nf4 from quantization.cc:126-141 as float, fp4
 * bitsandbytes' fp4 table over 12), one scale per `block` consecutive
 * elements: absmax[b] (FLOAT), or with nested blocks of 256 the UINT8 code
 * absmax[b] resolved as fp32(fp32(nested_map[code] * nested_absmax[b / 256])
 * + offset) (Scale, :339-346).  format 2 int8: element (r, c) is the signed
 * byte codes[r * cols + c], its row's scale fp32(absmax[r] / 127)
 * (:519).  value = fp32(code value * scale) (:523-526).
 *
 * orc_bnb_check: CheckParameters (:348-379) on the side tensors: every FLOAT
 * table finite, the maxima (absmax when FLOAT, nested_absmax) >= 0, the
 * quant map equal to the format's table, every nested scale finite.
 * Returns 0, 3 for "bitsandbytes nonfinite table or invalid absmax.", 4 for
 * "bitsandbytes noncanonical NF4/FP4 table.", 2 for a nonfinite nested scale
 * ("bitsandbytes nonfinite reconstruction.").
 * orc_bnb_reconstruct: ReconstructBitsAndBytesWeights (:502-539) into FLOAT
 * (1), FLOAT16 (10) or BFLOAT16 (16) values; returns 0, or 2 when a scale or
 * value is not finite, or its FLOAT16 / BFLOAT16 rounding is (:527-533). */
static const double bnb_nf4[16] = {-1, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                                   -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0,
                                   0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
                                   0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
                                   0.7229568362236023, 1};
static const float bnb_fp4[16] = {0.f, 1.f / 192, 2.f / 3, 1.f,  1.f / 3,  0.5f,  1.f / 6,  0.25f,
                                  0.f, -1.f / 192, -2.f / 3, -1.f, -1.f / 3, -0.5f, -1.f / 6, -0.25f};

float orc_bnb_table(int format, int code) {
  return format == 0 ? (float)bnb_nf4[code & 15] : bnb_fp4[code & 15];
}

static int bnb_scale(int format, int nested, float offset, const void *absmax, const float *nested_absmax,
                     const float *nested_map, int64_t b, float *scale) {
  float maximum;
  if (format == 2 || !nested) {
    maximum = ((const float *)absmax)[b];
  } else {
    volatile float product = nested_map[((const uint8_t *)absmax)[b]] * nested_absmax[b / 256];
    if (!isfinite(product)) return 2;
    volatile float sum = product + offset;
    if (!isfinite(sum)) return 2;
    maximum = sum;
  }
  if (format == 2) {
    volatile float q = maximum / 127.f;
    if (!isfinite(q)) return 2;
    maximum = q;
  }
  *scale = maximum;
  return 0;
}

int orc_bnb_check(int format, int64_t rows, int64_t cols, int64_t block, int nested, float offset,
                  const void *absmax, const float *quant_map, const float *nested_absmax, const float *nested_map) {
  const int64_t count = rows * cols;
  const int64_t blocks = format == 2 ? rows : (count + block - 1) / block;
  if (format == 2 || !nested) {
    for (int64_t b = 0; b < blocks; ++b) {
      const float v = ((const float *)absmax)[b];
      if (!isfinite(v) || v < 0) return 3;
    }
  }
  if (format == 2) return 0;
  for (int j = 0; j < 16; ++j)
    if (!isfinite(quant_map[j])) return 3;
  if (nested) {
    for (int64_t j = 0; j < (blocks + 255) / 256; ++j)
      if (!isfinite(nested_absmax[j]) || nested_absmax[j] < 0) return 3;
    for (int j = 0; j < 256; ++j)
      if (!isfinite(nested_map[j])) return 3;
  }
  for (int j = 0; j < 16; ++j)
    if (quant_map[j] != orc_bnb_table(format, j)) return 4;
  if (nested)
    for (int64_t b = 0; b < blocks; ++b) {
      float s;
      if (bnb_scale(format, nested, offset, absmax, nested_absmax, nested_map, b, &s)) return 2;
    }
  return 0;
}

int orc_bnb_reconstruct(int format, int64_t rows, int64_t cols, int64_t block, int nested, float offset,
                        const uint8_t *codes, const void *absmax, const float *nested_absmax,
                        const float *nested_map, int out_dtype, void *out) {
  const int64_t count = rows * cols;
  const int64_t bs = format == 2 ? cols : block;
  const int64_t blocks = (count + bs - 1) / bs;
  for (int64_t b = 0; b < blocks; ++b) {
    float scale;
    if (bnb_scale(format, nested, offset, absmax, nested_absmax, nested_map, b, &scale)) return 2;
    const int64_t end = count < b * bs + bs ? count : b * bs + bs;
    for (int64_t i = b * bs; i < end; ++i) {
      const float code = format == 2 ? (float)(int8_t)codes[i]
                                     : orc_bnb_table(format, (codes[i / 2] >> (i % 2 ? 0 : 4)) & 15);
      volatile float v = code * scale;
      if (!isfinite(v)) return 2;
      if (out_dtype == 1) {
        ((float *)out)[i] = v;
      } else if (out_dtype == 10) {
        const uint16_t h = orc_f32_to_f16(v);
        if ((h & 0x7c00u) == 0x7c00u) return 2;
        ((uint16_t *)out)[i] = h;
      } else {
        const uint16_t h = orc_f32_to_bf16(v);
        if ((h & 0x7f80u) == 0x7f80u) return 2;
        ((uint16_t *)out)[i] = h;
      }
    }
  }
  return 0;
}

/* ---- QQQ weights, onnx_core/runtime/qqq.cc ----------------------------------
 * TEST INFRASTRUCTURE (the checker of the GPU decode, never the product).
 * Geometry (:38-68): k rows (in_features), n columns (out_features), both
 * multiples of 64; grouped when group == 128 and k != 128.  The packed words
 * B [k / 16, 2n] hold 16x16 tiles of codes, (k / 16, n / 16) in row-major
 * tile order, each tile row-major, and every 1024-code block permuted by
 * _get_perms (:57-67): permutation[i * 32 + j * 8 + lane] = 256 j +
 * 16 (4 (i % 4) + p % 4) + i / 4 + 8 (p / 4) with p = order[lane] (order
 * {0,2,4,6,1,3,5,7} grouped, {4,0,5,1,6,2,7,3} per channel); the code of
 * (n, k) is nibble inverse[tiled % 1024] of its block (Position, :80-85;
 * Code, :166-169: nibble p at bits 4 (p % 2) of byte p / 2).
 * Scales (ScalePosition, :144-149): channel n at storage index (n / 32) 32 +
 * ((n % 32 % 8) / 2) 8 + (n % 32 / 8) 2 + n % 2; group scale (k / 128, n),
 * index i = (k / 128) n_total + n, at (i / 64) 64 + (i % 8) 8 + (i % 64) / 8.
 * Reconstructed (:185-202): grouped, integer = (code - 8) * group scale
 * rounded half to even in double, clamped to [-128, 127], a zero keeping the
 * product's sign; per channel, integer = signed nibble * 16; value =
 * fp32(integer * channel scale) rounded to nearest even (RoundFloat,
 * :162-183, is IEEE double -> float rounding).
 * orc_qqq_reconstruct returns CheckData's first failure (:204-218) -- 1
 * "QQQ nonfinite or negative channel scale.", 2 "... group scale.", 3 "QQQ
 * FLOAT reconstruction overflow." -- or 4 when a value does not fit
 * out_dtype (WriteFloat, quantization.cc:184-201: "Dequantization output
 * dtype overflow."), else 0; values [n, k] in FLOAT (1), FLOAT16 (10),
 * BFLOAT16 (16) or DOUBLE (11); codes [n, k] when not NULL. */
static void qqq_permutation(int grouped, int32_t *perm, int32_t *inverse) {
  static const int channel_order[8] = {4, 0, 5, 1, 6, 2, 7, 3};
  static const int grouped_order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  const int *order = grouped ? grouped_order : channel_order;
  for (int i = 0; i < 32; ++i)
    for (int j = 0; j < 4; ++j)
      for (int lane = 0; lane < 8; ++lane) {
        const int p = order[lane];
        const int index = i * 32 + j * 8 + lane;
        perm[index] = 256 * j + 16 * (4 * (i % 4) + p % 4) + i / 4 + 8 * (p / 4);
        inverse[perm[index]] = index;
      }
}

static int qqq_grouped(int64_t k, int64_t group) { return group == 128 && k != 128; }

int64_t orc_qqq_position(int64_t k, int64_t n, int64_t group, int64_t n_index, int64_t k_index) {
  int32_t perm[1024], inverse[1024];
  qqq_permutation(qqq_grouped(k, group), perm, inverse);
  const int64_t tiled = (k_index / 16) * n * 16 + (n_index / 16) * 256 + (k_index % 16) * 16 + n_index % 16;
  return (tiled / 1024) * 1024 + inverse[tiled % 1024];
}

int64_t orc_qqq_scale_position(int64_t index, int channel) {
  if (!channel) return (index / 64) * 64 + (index % 8) * 8 + (index % 64) / 8;
  const int64_t local = index % 32;
  return (index / 32) * 32 + ((local % 8) / 2) * 8 + (local / 8) * 2 + local % 2;
}

int orc_qqq_reconstruct(int64_t k, int64_t n, int64_t group, const uint8_t *words, const float *s_channel,
                        const uint16_t *s_group, int out_dtype, void *out, uint8_t *codes) {
  const int grouped = qqq_grouped(k, group);
  int32_t perm[1024], inverse[1024];
  qqq_permutation(grouped, perm, inverse);
  for (int64_t c = 0; c < n; ++c) {
    const float s = s_channel[orc_qqq_scale_position(c, 1)];
    if (!isfinite(s) || s < 0) return 1;
  }
  if (grouped)
    for (int64_t i = 0; i < (k / 128) * n; ++i) {
      const float s = orc_f16_to_f32(s_group[i]);
      if (!isfinite(s) || s < 0) return 2;
    }
  int rc = 0;
  for (int64_t c = 0; c < n; ++c)
    for (int64_t r = 0; r < k; ++r) {
      const int64_t tiled = (r / 16) * n * 16 + (c / 16) * 256 + (r % 16) * 16 + c % 16;
      const int64_t pos = (tiled / 1024) * 1024 + inverse[tiled % 1024];
      const int code = (words[pos / 2] >> ((pos % 2) * 4)) & 15;
      if (codes) codes[c * k + r] = (uint8_t)code;
      float integer;
      if (grouped) {
        const double gs = orc_f16_to_f32(s_group[orc_qqq_scale_position((r / 128) * n + c, 0)]);
        const double scaled = (double)(code - 8) * gs;
        const double lower = floor(scaled), fraction = scaled - lower;
        const double rounded = lower + ((fraction > 0.5 || (fraction == 0.5 && fmod(lower, 2) != 0)) ? 1 : 0);
        integer = rounded == 0 ? copysignf(0.0f, (float)scaled)
                               : (float)(rounded < -128 ? -128 : (rounded > 127 ? 127 : rounded));
      } else {
        integer = (float)((code >= 8 ? code - 16 : code) * 16);
      }
      const float v = (float)((double)integer * (double)s_channel[orc_qqq_scale_position(c, 1)]);
      if (!isfinite(v)) return 3;
      const int64_t e = c * k + r;
      if (out_dtype == 1) {
        ((float *)out)[e] = v;
      } else if (out_dtype == 11) {
        ((double *)out)[e] = (double)v;
      } else {
        const uint16_t h = out_dtype == 10 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
        const int inf = out_dtype == 10 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
        if (inf && rc == 0) rc = 4;
        ((uint16_t *)out)[e] = h;
      }
    }
  return rc;
}

/* ---- BitBLAS row-packed weights, onnx_core/runtime/bitblas.cc --------------
 * TEST INFRASTRUCTURE.  Codes (:239-249): row n of qweight INT8 [n, k * bits
 * / 8] holds its k codes as one little-endian bit stream
 * (UnpackQuantizationCodes, compressed_tensor_packing.cc:58-74, masked to
 * the raw unsigned field); Affine (:251-290): codes from symmetric GPTQ
 * XOR the midpoint 2^(bits-1) with zero = the midpoint, otherwise zero (g, n)
 * is field n of qzeros row g; scale (g, n) = scales[n, g] (FP16); the value
 * is GPTQ's (float(code) - float(zero)) * scale (gptq.cc:222-228; exact in
 * fp32 here).  Returns 1 for a scale not finite or not positive (CheckScales,
 * :228-237: "BitBLAS nonfinite or nonpositive scale."), 4 when a value does
 * not fit out_dtype (WriteFloat), else 0; values [n, k] as in
 * orc_qqq_reconstruct; raw codes [n, k] when `codes` is not NULL. */
static uint32_t bitblas_field(const uint8_t *data, int64_t index, int bits) {
  const int64_t bit = index * bits;
  uint32_t v = (uint32_t)data[bit / 8] >> (bit % 8);
  if (bit % 8 + bits > 8) v |= (uint32_t)data[bit / 8 + 1] << (8 - bit % 8);
  return v & ((1u << bits) - 1);
}

int orc_bitblas_reconstruct(int64_t k, int64_t n, int64_t group, int bits, int signed_codes, const uint8_t *qweight,
                            const uint16_t *scales, const uint8_t *qzeros, int out_dtype, void *out, uint8_t *codes) {
  const int64_t eff = group == -1 ? k : group, groups = k / eff;
  for (int64_t i = 0; i < n * groups; ++i) {
    const float s = orc_f16_to_f32(scales[i]);
    if (!isfinite(s) || !(s > 0)) return 1;
  }
  const uint32_t mid = 1u << (bits - 1);
  int rc = 0;
  for (int64_t c = 0; c < n; ++c)
    for (int64_t r = 0; r < k; ++r) {
      const uint32_t raw = bitblas_field(qweight, c * k + r, bits);
      if (codes) codes[c * k + r] = (uint8_t)raw;
      const int64_t g = r / eff;
      const uint32_t code = signed_codes ? raw ^ mid : raw;
      const uint32_t zero = signed_codes ? mid : bitblas_field(qzeros, g * n + c, bits);
      const float v = ((float)code - (float)zero) * orc_f16_to_f32(scales[c * groups + g]);
      const int64_t e = c * k + r;
      if (out_dtype == 1) {
        ((float *)out)[e] = v;
      } else if (out_dtype == 11) {
        ((double *)out)[e] = (double)v;
      } else {
        const uint16_t h = out_dtype == 10 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
        const int inf = out_dtype == 10 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
        if (inf && rc == 0) rc = 4;
        ((uint16_t *)out)[e] = h;
      }
    }
  return rc;
}

/* ---- GPTQModel FP8 weights, onnx_core/runtime/gptqmodel_fp8.cc -----------
 * TEST INFRASTRUCTURE.  Reconstructed (:160-162): float(code) / the inverse
 * scale of the element's tensor / row / (b0 x b1) block (ScaleIndex,
 * :94-103), one IEEE division.  CheckData (:164-173) returns 1 for a scale
 * not finite or not positive, 2 for a value not finite; 4 when a value does
 * not fit out_dtype (WriteFloat); else 0.  E8M0 as cast_float8.cc:451-461:
 * 2^(bits - 127), 0 is 2^-127, 0xFF the quiet NaN. */
float orc_f8e8m0_to_f32(uint8_t v) {
  uint32_t u = v == 0 ? 0x00400000u : (v == 0xFF ? 0x7FC00000u : (uint32_t)v << 23);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float gptq_fp8_decode(uint8_t c, int type) {
  switch (type) {
  case 17: return orc_f8e4m3fn_to_f32(c);
  case 18: return orc_f8e4m3fnuz_to_f32(c);
  case 19: return orc_f8e5m2_to_f32(c);
  case 20: return orc_f8e5m2fnuz_to_f32(c);
  default: return orc_f8e8m0_to_f32(c);
  }
}

int orc_gptq_fp8_reconstruct(int64_t n, int64_t k, int code_type, int method, int64_t b0, int64_t b1,
                             const uint8_t *codes, const float *scales, int out_dtype, void *out) {
  const int64_t cols = method == 2 ? k / b1 : 0;
  const int64_t count = method == 0 ? 1 : (method == 1 ? n : (n / b0) * cols);
  for (int64_t i = 0; i < count; ++i)
    if (!isfinite(scales[i]) || !(scales[i] > 0)) return 1;
  int rc = 0;
  for (int64_t i = 0; i < n * k; ++i) {
    const int64_t r = i / k, c = i % k;
    const int64_t si = method == 0 ? 0 : (method == 1 ? r : (r / b0) * cols + c / b1);
    volatile float v = gptq_fp8_decode(codes[i], code_type) / scales[si];
    if (!isfinite(v)) return 2;
    if (out_dtype == 1) {
      ((float *)out)[i] = v;
    } else if (out_dtype == 11) {
      ((double *)out)[i] = (double)v;
    } else {
      const uint16_t h = out_dtype == 10 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
      const int inf = out_dtype == 10 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
      if (inf && rc == 0) rc = 4;
      ((uint16_t *)out)[i] = h;
    }
  }
  return rc;
}

/* ---- EXL3 weights, onnx_core/runtime/exl3.cc --------------------------------
 * TEST INFRASTRUCTURE.  ReconstructExl3Weights (:309-357) in FLOAT: for
 * every 16 x 16 tile and position, State (:222-231, the words taken at
 * index ^ 1) through Codebook (:205-220, rounded to binary16) into the MMA
 * fragment place (:331-334); then per 128-row block and column the
 * Hadamard butterflies (:233-245, ascending widths, then x fp32(1 / sqrt
 * 128)), per row x suh, the butterflies per 128-column block, x svh; every
 * step one fp32 rounding.  Returns 0, 1 for a nonfinite value (Rounded :36),
 * 4 for a value past out_dtype's range (WriteFloat). */
static float exl3_codebook(uint32_t state, int book) {
  float r;
  if (book < 2) {
    uint32_t raw = book == 0 ? state * 89226354u + 64248484u : state * 0xcbac1fedu;
    raw = 0x3b603b60u ^ (raw & 0x8fff8fffu);
    volatile float sum = orc_f16_to_f32((uint16_t)raw) + orc_f16_to_f32((uint16_t)(raw >> 16));
    r = sum;
  } else {
    const uint32_t raw = state * 0x83dcd12du;
    const uint32_t sum = (raw & 255u) + ((raw >> 8) & 255u) + ((raw >> 16) & 255u) + (raw >> 24);
    r = fmaf(orc_f16_to_f32((uint16_t)(sum + 0x6400u)), orc_f16_to_f32(0x1eee), orc_f16_to_f32(0xc931));
  }
  return orc_f16_to_f32(orc_f32_to_f16(r));
}

static uint16_t exl3_state(const uint16_t *stream, uint32_t bits, uint32_t position) {
  const uint32_t words = 16u * bits, span = 256u * bits;
  const uint32_t start = ((position + 1u) * bits + span - 16u) % span;
  const uint32_t word = start / 16u, shift = start % 16u;
  uint32_t state = stream[word ^ 1u];
  if (shift) state = ((state << shift) | ((uint32_t)stream[((word + 1u) % words) ^ 1u] >> (16u - shift))) & 65535u;
  return (uint16_t)state;
}

static int exl3_hadamard(float *v, int64_t stride) {
  int bad = 0;
  for (int64_t w = 1; w < 128; w *= 2)
    for (int64_t base = 0; base < 128; base += 2 * w)
      for (int64_t j = base; j < base + w; ++j) {
        const float a = v[j * stride], b = v[(j + w) * stride];
        volatile float s = a + b, d = a - b;
        v[j * stride] = s, v[(j + w) * stride] = d;
        bad |= !isfinite(s) || !isfinite(d);
      }
  for (int64_t i = 0; i < 128; ++i) {
    volatile float x = v[i * stride] * 0.08838834764831845f;
    v[i * stride] = x;
    bad |= !isfinite(x);
  }
  return bad;
}

int orc_exl3_reconstruct(int64_t k, int64_t n, int bits, int book, const uint16_t *trellis, const uint16_t *suh,
                         const uint16_t *svh, int out_dtype, void *out) {
  float *v = (float *)malloc((size_t)(k * n) * sizeof(float));
  if (!v) return -1;
  const int64_t words = 16 * bits;
  for (int64_t tile = 0; tile < k * n / 256; ++tile)
    for (uint32_t p = 0; p < 256; ++p) {
      const uint32_t lane = p / 8, item = p % 8;
      const int64_t row = (tile / (n / 16)) * 16 + (lane % 4) * 2 + (item & 1) + ((item & 2) ? 8 : 0);
      const int64_t col = (tile % (n / 16)) * 16 + lane / 4 + ((item & 4) ? 8 : 0);
      v[row * n + col] = exl3_codebook(exl3_state(trellis + tile * words, (uint32_t)bits, p), book);
    }
  int bad = 0;
  for (int64_t r = 0; r < k; r += 128)
    for (int64_t c = 0; c < n; ++c) bad |= exl3_hadamard(v + r * n + c, n);
  for (int64_t r = 0; r < k; ++r) {
    const float s = orc_f16_to_f32(suh[r]);
    for (int64_t c = 0; c < n; ++c) {
      volatile float x = v[r * n + c] * s;
      v[r * n + c] = x;
      bad |= !isfinite(x);
    }
    for (int64_t c = 0; c < n; c += 128) bad |= exl3_hadamard(v + r * n + c, 1);
    for (int64_t c = 0; c < n; ++c) {
      volatile float x = v[r * n + c] * orc_f16_to_f32(svh[c]);
      v[r * n + c] = x;
      bad |= !isfinite(x);
    }
  }
  int rc = bad ? 1 : 0;
  for (int64_t i = 0; i < k * n && !rc; ++i) {
    if (out_dtype == 1) {
      ((float *)out)[i] = v[i];
    } else if (out_dtype == 11) {
      ((double *)out)[i] = (double)v[i];
    } else {
      const uint16_t h = out_dtype == 10 ? orc_f32_to_f16(v[i]) : orc_f32_to_bf16(v[i]);
      if (out_dtype == 10 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u) rc = 4;
      ((uint16_t *)out)[i] = h;
    }
  }
  free(v);
  return rc;
}

/* ---- MX and NVFP4 weights, onnx_core/runtime/quantization.cc ------------
 * TEST INFRASTRUCTURE.  format 0 MXFP4, 1 MXFP6 E2M3, 2 MXFP8, 3 NVFP4; count
 * = rows * cols, groups of 32 (16 for NVFP4) consecutive values, one scale
 * byte each.  Validate*Reconstruction (:1350-1359, :1477-1486, :1608-1613,
 * :1714-1720) walk the groups in order: the scale (Mxfp4Scale :1458,
 * Mxfp8Scale :1591, Mxfp6E2m3Scale :1700: byte 255 rejected, 2^(e - 127)
 * with byte 0 = 2^-127; Nvfp4EffectiveScale :1322: E4M3FN local / global,
 * both finite and positive, the quotient finite and nonzero), then each
 * element (MXFP8: a NaN code rejected first) as one fp32 product, finite.
 * Returns 0, or 1 a bad scale, 2 NVFP4's quotient not finite, 3 it is zero,
 * 4 a NaN code, 5 a value not finite (group / element of the first), 6 a
 * value past out_dtype's range (WriteFloat, after every check). */
int orc_mx_reconstruct(int format, int64_t count, const uint8_t *codes, const uint8_t *scales, float global,
                       int out_dtype, void *out, int64_t *fail_group, int64_t *fail_element) {
  const int64_t g = format == 3 ? 16 : 32;
  int rc = 0;
  *fail_group = *fail_element = -1;
  for (int64_t grp = 0; grp < count / g; ++grp) {
    float scale;
    if (format == 3) {
      const float local = orc_f8e4m3fn_to_f32(scales[grp]);
      if (!(isfinite(global) && global > 0 && isfinite(local) && local > 0)) { *fail_group = grp; return 1; }
      volatile float eff = local / global;
      if (!isfinite(eff)) { *fail_group = grp; return 2; }
      if (!(eff > 0)) { *fail_group = grp; return 3; }
      scale = eff;
    } else {
      if (scales[grp] == 255) { *fail_group = grp; return 1; }
      scale = ldexpf(1.0f, (int)scales[grp] - 127);
    }
    for (int64_t j = 0; j < g; ++j) {
      const int64_t i = grp * g + j;
      float level;
      if (format == 0 || format == 3) {
        level = orc_f4e2m1_to_f32((uint8_t)(j % 2 ? codes[i / 2] >> 4 : codes[i / 2] & 15));
      } else if (format == 1) {
        const int64_t bit = j * 6;
        const uint8_t *b = codes + grp * 24 + bit / 8;
        unsigned v = b[0] >> (bit % 8);
        if (bit % 8 > 2) v |= (unsigned)b[1] << (8 - bit % 8);
        level = orc_f6_to_f32((uint8_t)(v & 63u), ORC_FLOAT6E2M3);
      } else {
        level = orc_f8e4m3fn_to_f32(codes[i]);
        if (!isfinite(level)) { *fail_group = grp, *fail_element = j; return 4; }
      }
      volatile float v = level * scale;
      if (!isfinite(v)) { *fail_group = grp, *fail_element = j; return 5; }
      if (out_dtype == 1) {
        ((float *)out)[i] = v;
      } else if (out_dtype == 11) {
        ((double *)out)[i] = (double)v;
      } else {
        const uint16_t h = out_dtype == 10 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
        const int inf = out_dtype == 10 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
        if (inf) rc = 6;
        ((uint16_t *)out)[i] = h;
      }
    }
  }
  return rc;
}

/* ---- VPTQ weights, onnx_core/runtime/vptq.cc --------------------------------
 * TEST INFRASTRUCTURE.  Layout (:52-129): the outlier columns
 * ceil(npercent / 100 * k) (plus the remainder (k - outliers) % groups with
 * group_num and an outlier codebook), the groups and their columns, index
 * widths bit_width(num_centroids - 1) (+ the residual's), vectors
 * ceil(n / vector_len), words ceil(columns * width / 32).  Index (:194-202):
 * bits [j * width, +width) of row (g, v) of the INT32 words.  CheckData
 * (:203-240): every index of every column (padding included) inside its
 * codebooks (1), outlier indices inside theirs (2), perm a permutation (3).
 * Reconstruct (:401-443) as described for the device decode; Round
 * (:344-351) rounds to the codebook dtype.  Returns -1 for a layout the
 * reference rejects, the CheckData codes above, 5 for a nonfinite value
 * and 4 for a value past out_dtype (WriteFloat), else 0. */
static float vptq_load(const void *p, int dtype, int64_t i) {
  if (dtype == 1) return ((const float *)p)[i];
  const uint16_t h = ((const uint16_t *)p)[i];
  if (dtype == 10) return orc_f16_to_f32(h);
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float vptq_round(float v, int dtype) {
  volatile float r = v;
  if (dtype == 10) return orc_f16_to_f32(orc_f32_to_f16(r));
  if (dtype == 16) {
    uint32_t u = (uint32_t)orc_f32_to_bf16(r) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  return r;
}

static int vptq_bit_width(int64_t entries) {
  int b = 0;
  for (uint64_t v = (uint64_t)(entries - 1); v; v >>= 1) ++b;
  return b;
}

int orc_vptq_reconstruct(const orc_vptq_config *c, const uint32_t *indices, const void *centroids,
                         const void *res_centroids, const void *outlier_centroids, const int32_t *outlier_indices,
                         const void *scale, const void *bias, const int32_t *perm, int out_dtype, void *out) {
  const int64_t k = c->k, n = c->n;
  const int outlier = c->npercent > 0 && c->vector_lens[0] > 0 && c->num_centroids[0] > 1;
  if (c->npercent != 0 && !outlier) return -1;
  const double initial = ceil((c->npercent / 100.0) * (double)k);
  if (!(initial >= 0 && initial < (double)k)) return -1;
  int64_t outliers = outlier ? (int64_t)initial : 0, groups, columns;
  if (c->group_num != -1) {
    groups = c->group_num;
    if (groups > k - outliers) return -1;
    if (outlier) outliers += (k - outliers) % groups;
    columns = outlier ? (k - outliers) / groups : (k + groups - 1) / groups;
  } else {
    columns = c->group_size == -1 ? k - outliers : c->group_size;
    groups = (k - outliers + columns - 1) / columns;
  }
  if (!(groups > 0 && columns > 0 && groups * columns >= k - outliers)) return -1;
  const int mb = vptq_bit_width(c->num_centroids[1]);
  const int rb = c->num_res_centroids[1] > 1 ? vptq_bit_width(c->num_res_centroids[1]) : 0;
  const int width = mb + rb;
  const int64_t len0 = c->vector_lens[0], len1 = c->vector_lens[1];
  const int64_t vectors = (n + len1 - 1) / len1, words = (columns * width + 31) / 32;
  const uint32_t mask = (uint32_t)((1ull << mb) - 1);
#define VPTQ_INDEX(g, v, j)                                                                      \
  ((uint32_t)(((((uint64_t)indices[((g) * vectors + (v)) * words + (j) * width / 32]) |           \
               ((j) * width % 32 + width > 32                                                    \
                    ? (uint64_t)indices[((g) * vectors + (v)) * words + (j) * width / 32 + 1] << 32 \
                    : 0)) >>                                                                     \
              ((j) * width % 32)) &                                                              \
             ((1ull << width) - 1)))
  for (int64_t g = 0; g < groups; ++g)
    for (int64_t v = 0; v < vectors; ++v)
      for (int64_t j = 0; j < columns; ++j) {
        const uint32_t index = VPTQ_INDEX(g, v, j);
        if ((int64_t)(index & mask) >= c->num_centroids[1]) return 1;
        if (rb && (int64_t)(index >> mb) >= c->num_res_centroids[1]) return 1;
      }
  if (outliers)
    for (int64_t i = 0; i < ((n + len0 - 1) / len0) * outliers; ++i)
      if (outlier_indices[i] < 0 || outlier_indices[i] >= c->num_centroids[0]) return 2;
  if (c->enable_perm) {
    unsigned char *seen = (unsigned char *)calloc((size_t)k, 1);
    for (int64_t i = 0; i < k; ++i) {
      if (perm[i] < 0 || perm[i] >= k || seen[perm[i]]) {
        free(seen);
        return 3;
      }
      seen[perm[i]] = 1;
    }
    free(seen);
  }
  float *vals = (float *)malloc((size_t)(n * k) * sizeof(float));
  for (int64_t r = 0; r < n; ++r)
    for (int64_t col = 0; col < k; ++col) {
      float value;
      if (col < outliers) {
        const int64_t index = outlier_indices[(r / len0) * outliers + col];
        value = vptq_load(outlier_centroids, c->dtype, index * len0 + r % len0);
      } else {
        const int64_t g = (col - outliers) / columns, j = (col - outliers) % columns;
        const uint32_t index = VPTQ_INDEX(g, r / len1, j);
        value = vptq_load(centroids, c->dtype, (g * c->num_centroids[1] + (index & mask)) * len1 + r % len1);
        if (rb)
          value = vptq_round(value + vptq_load(res_centroids, c->dtype,
                                               (g * c->num_res_centroids[1] + (index >> mb)) * len1 + r % len1),
                             c->dtype);
      }
      const int64_t dest = c->enable_perm ? perm[col] : col;
      if (c->enable_norm) {
        const int64_t i = c->norm_dim == 0 ? dest : r;
        value = vptq_round(value * vptq_load(scale, c->dtype, i), c->dtype);
        value = vptq_round(value + vptq_load(bias, c->dtype, i), c->dtype);
      }
      vals[r * k + dest] = value;
    }
#undef VPTQ_INDEX
  /* WriteFloat in output order: the first nonfinite or out-of-range value raises */
  int rc = 0;
  for (int64_t e = 0; e < n * k && rc == 0; ++e) {
    const float value = vals[e];
    if (!isfinite(value)) {
      rc = 5;
    } else if (out_dtype == 1) {
      ((float *)out)[e] = value;
    } else if (out_dtype == 11) {
      ((double *)out)[e] = (double)value;
    } else {
      const uint16_t h = out_dtype == 10 ? orc_f32_to_f16(value) : orc_f32_to_bf16(value);
      if (out_dtype == 10 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u) rc = 4;
      ((uint16_t *)out)[e] = h;
    }
  }
  free(vals);
  return rc;
}
