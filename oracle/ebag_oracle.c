/*
 * ORACLE — test infrastructure, not product code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only to check results against (or as the timed CPU baseline); the product path never calls it.
 *
 * CPU restatement of the fused multi-field embedding-bag step:
 *   - online_best/infer.py:805-827  fused_all_slots_embedding_kernel: per (sample b, slot s),
 *     start/end from the slot's local row offsets plus val_offsets[s] (:810-815), acc = 0 in
 *     fp32 (:819), for i in [start, end): idx = clamp(values[i], 0, max_idx) (:822-823),
 *     acc += weight[idx, :D] (:824-825), out[b, s*D:(s+1)*D] = acc cast to out dtype (:826-827).
 *   - baseline/infer.py:256-263     the per-field loop: clamp, embedding, segment_reduce(sum,
 *     initial=0) (empty bag -> 0), cat along dim 1.
 * Generalised as the build's API is: per-field tables (rows, dim, row stride, output column),
 * global offsets[F*B+1] or the reference layout (row offsets + per-field base), int32/int64
 * indices, fp32/bf16/fp16 tables and outputs, sum or mean (mean = fp32 sum / bag length, empty
 * bag -> 0). Accumulation is strictly sequential in element order, as in the reference kernel's
 * loop, so a bag pooled by one lane group on the GPU matches this bit for bit.
 *
 *   - online_best/infer.py:904-942  fused_all_slots_embedding_kernel_int8: the same loop over an
 *     int8 table with one fp32 scale per row, acc += int8_row * scale_val (:934-936). Triton
 *     fuses that multiply-add (its default fp-fusion), so the restatement is acc = fmaf(q, s, acc)
 *     in element order, with C99 fmaf (exact product and sum, one rounding).
 *   - online_best/infer.py:895-901  quantize_embedding_int8 as evaluated by torch on the device:
 *     s = max(max_j |w_j| * RN32(1/127), 1e-8) (a Python-scalar divisor becomes a multiply by its
 *     fp32 reciprocal), q_j = clamp(round_half_even(w_j / s), -128, 127) with IEEE fp32 division.
 *
 * Conversions are written from the IEEE 754 definitions: bf16 = high half of the fp32 word,
 * fp32 -> bf16/fp16 round to nearest, ties to even; NaN stays NaN.
 * Build with -ffp-contract=off (no fused multiply-add anywhere except the explicit fmaf).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define OR_F32 0
#define OR_BF16 1
#define OR_F16 2
#define OR_I8 3 /* int8 table rows times the table's per-row fp32 scale */

typedef struct oracle_table {
  const void* data;
  int64_t rows;
  int64_t row_stride; /* elements */
  int32_t dim;
  int32_t out_col;
  const float* row_scale; /* OR_I8 tables: fp32 [rows] */
} oracle_table;

static float u32_as_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_as_u32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

float oracle_bf16_to_f32(uint16_t h) { return u32_as_f32((uint32_t)h << 16); }

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* NaN: keep quiet NaN */
  /* add half an ulp of bf16 minus one, plus the lsb of the kept part: ties go to even */
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 is exact in fp32 */
    float v = (float)man * u32_as_f32(0x33800000u); /* 2^-24 */
    return (sign ? -v : v);
  }
  if (exp == 31) return u32_as_f32(sign | 0x7f800000u | (man << 13));
  return u32_as_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  const uint32_t u = f32_as_u32(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> Inf */
  if (a < 0x38800000u) {
    /* result is subnormal (or zero) in fp16: value = a_real / 2^-24, round half to even */
    const uint32_t e = a >> 23;
    if (e < 102) return sign; /* below half of the smallest subnormal (2^-25): rounds to 0 */
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e; /* m * 2^(e-150) / 2^-24 = m >> (126 - e) */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
  }
  /* normal: rebias exponent, round 13 dropped bits half to even */
  uint32_t v = a - 0x38000000u; /* exponent 127-15 = 112 -> subtract 112 << 23 */
  v = v + 0xfffu + ((v >> 13) & 1u);
  return (uint16_t)(sign | (v >> 13));
}

static float load_elem(const void* base, int dt, int64_t i) {
  switch (dt) {
    case OR_F32: return ((const float*)base)[i];
    case OR_BF16: return oracle_bf16_to_f32(((const uint16_t*)base)[i]);
    default: return oracle_f16_to_f32(((const uint16_t*)base)[i]);
  }
}

static void store_elem(void* base, int dt, int64_t i, float v) {
  switch (dt) {
    case OR_F32: ((float*)base)[i] = v; break;
    case OR_BF16: ((uint16_t*)base)[i] = oracle_f32_to_bf16(v); break;
    default: ((uint16_t*)base)[i] = oracle_f32_to_f16(v); break;
  }
}

static int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/*
 * Pool every (field, sample) bag.
 *   values:   nnz indices (int64, or int32 when idx32)
 *   offsets:  field f's bag b spans [base_f + offsets[f*stride + b], base_f + offsets[f*stride + b + 1])
 *             with base_f = val_base ? val_base[f] : 0. Global layout: stride = B, val_base NULL.
 *             Reference layout: stride = B + 1, val_base = val_offsets.
 *   Bounds of a bag are clipped into [0, nnz] (and end >= start) — identical to the GPU path
 *   for every well-formed batch, and defined for malformed ones.
 * Returns 0, or -1 for bad arguments. Parallel over samples when built with OpenMP.
 */
int oracle_pool(const void* values, int32_t idx32, int64_t nnz, const int64_t* offsets, const int64_t* val_base,
                int64_t stride, int64_t batch, int32_t num_fields, const oracle_table* tables, int32_t tdt,
                int32_t mean, void* out, int32_t odt, int64_t out_row_stride, float* scratch_acc) {
  if (batch < 0 || num_fields < 0 || nnz < 0 || !tables || (batch > 0 && num_fields > 0 && (!offsets || !out)))
    return -1;
  (void)scratch_acc;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t b = 0; b < batch; ++b) {
    float acc[4096];
    for (int32_t f = 0; f < num_fields; ++f) {
      const oracle_table* t = &tables[f];
      const int64_t base = val_base ? val_base[f] : 0;
      int64_t start = clamp64(base + offsets[(int64_t)f * stride + b], 0, nnz);
      int64_t end = clamp64(base + offsets[(int64_t)f * stride + b + 1], start, nnz);
      for (int32_t c0 = 0; c0 < t->dim; c0 += 4096) {
        const int32_t nc = t->dim - c0 < 4096 ? t->dim - c0 : 4096;
        for (int32_t c = 0; c < nc; ++c) acc[c] = 0.0f;
        for (int64_t i = start; i < end; ++i) {
          int64_t v = idx32 ? (int64_t)((const int32_t*)values)[i] : ((const int64_t*)values)[i];
          int64_t r = clamp64(v, 0, t->rows - 1);
          const int64_t row0 = r * t->row_stride + c0;
          if (tdt == OR_I8) {
            const int8_t* q = (const int8_t*)t->data + row0;
            const float sc = t->row_scale[r];
            for (int32_t c = 0; c < nc; ++c) acc[c] = fmaf((float)q[c], sc, acc[c]);
          } else {
            for (int32_t c = 0; c < nc; ++c) acc[c] = acc[c] + load_elem(t->data, tdt, row0 + c);
          }
        }
        const int64_t L = end - start;
        for (int32_t c = 0; c < nc; ++c) {
          float x = acc[c];
          if (mean && L > 0) x = x / (float)L;
          store_elem(out, odt, b * out_row_stride + t->out_col + c0 + c, x);
        }
      }
    }
  }
  return 0;
}

/*
 * Row quantisation (online_best/infer.py:895-901) of a [rows, row_stride] table of type dt
 * (first dim columns used) into q int8 [rows, dim] and scale fp32 [rows]. Finite inputs.
 */
int oracle_quantize_int8(const void* w, int32_t dt, int64_t rows, int64_t dim, int64_t row_stride, int8_t* q,
                         float* scale) {
  if (rows < 0 || dim < 1 || row_stride < dim || dt < OR_F32 || dt > OR_F16) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    float m = 0.0f;
    for (int64_t c = 0; c < dim; ++c) {
      const float a = fabsf(load_elem(w, dt, r * row_stride + c));
      if (a > m) m = a;
    }
    /* row_max / 127.0 with a Python-scalar divisor: torch's device kernel multiplies by the fp32
     * reciprocal of the scalar (ATen's div_true_kernel_cuda, "a * reciprocal(b)") */
    float s = m * (1.0f / 127.0f);
    if (s < 1e-8f) s = 1e-8f;
    scale[r] = s;
    for (int64_t c = 0; c < dim; ++c) {
      float v = nearbyintf(load_elem(w, dt, r * row_stride + c) / s); /* default mode: ties to even */
      if (v < -128.0f) v = -128.0f;
      if (v > 127.0f) v = 127.0f;
      q[r * dim + c] = (int8_t)v;
    }
  }
  return 0;
}

/* fmaf over arrays, exposed so the tests can pin the C library's fused multiply-add. */
void oracle_fmaf_array(const float* a, const float* b, const float* c, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = fmaf(a[i], b[i], c[i]);
}

/* Elementwise conversions exposed for the tests that pin them against library routines. */
void oracle_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_bf16(x[i]);
}
void oracle_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16(x[i]);
}
void oracle_f16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_f16_to_f32(x[i]);
}

/* Threads OpenMP will use (1 when built without OpenMP). */
#ifdef _OPENMP
#include <omp.h>
int oracle_num_threads(void) { return omp_get_max_threads(); }
void oracle_set_num_threads(int n) { omp_set_num_threads(n); }
#else
int oracle_num_threads(void) { return 1; }
void oracle_set_num_threads(int n) { (void)n; }
#endif
