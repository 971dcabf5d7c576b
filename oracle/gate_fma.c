/* Gate logits in the router's defined order, restated in C for the oracle.
 *
 * Test infrastructure only: the tests compare the device router with this.
 *
 * z[t][e] = x[t] . W[e] over H, in this order (the reference's logit
 * f32(x) @ f32(W).T, src/deepseeker/mlx_forward.py:62-65, evaluated in one
 * fixed order so that routing can be bit-exact): H is cut into 256-element
 * steps m and the steps into 4 segments of S = ceil(steps / 4) consecutive
 * steps.  In segment w, lane partial l (l = 0..63) starts at +0 and takes,
 * for its steps m in order and then v = 0..3, p = fmaf(x[i], W[i], p) with
 * i = 256 m + 4 l + v (one rounding per step: the fused multiply-add of
 * IEEE 754); positions i >= H are skipped (they add +0 on the device).  The
 * 64 partials are combined by the XOR butterfly (s = 32, 16, 8, 4, 2, 1:
 * p[l] = p[l] + p[l ^ s]) into the segment sum p[0], and
 * z = ((s_0 + s_1) + s_2) + s_3.
 *
 * fmaf is the C library's correctly rounded fused multiply-add.  The hot loop
 * has two forms with the same arithmetic: one built for CPUs with the FMA
 * instruction (chosen at run time), one that calls fmaf.  x and W arrive
 * transposed per step as [steps][4][64] (element (m, v, l) = position
 * 256 m + 4 l + v, zero past H), so the 64 lanes are contiguous.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define LANES 64
#define VEC 4
#define SEGMENTS 4

typedef void (*chain_fn)(const float*, const float*, int, int, float*);

/* p[l] = fmaf(x[m][v][l], w[m][v][l], p[l]) for steps m0..m1-1, then v, for every l */
__attribute__((target("avx2,fma"))) static void chain_fma(const float* x, const float* w, int m0, int m1,
                                                          float* p) {
  for (int m = m0; m < m1; ++m)
    for (int v = 0; v < VEC; ++v) {
      const float* xs = x + ((int64_t)m * VEC + v) * LANES;
      const float* ws = w + ((int64_t)m * VEC + v) * LANES;
      for (int l = 0; l < LANES; ++l) p[l] = __builtin_fmaf(xs[l], ws[l], p[l]);
    }
}

static void chain_libm(const float* x, const float* w, int m0, int m1, float* p) {
  for (int m = m0; m < m1; ++m)
    for (int v = 0; v < VEC; ++v) {
      const float* xs = x + ((int64_t)m * VEC + v) * LANES;
      const float* ws = w + ((int64_t)m * VEC + v) * LANES;
      for (int l = 0; l < LANES; ++l) p[l] = fmaf(xs[l], ws[l], p[l]);
    }
}

static chain_fn pick(void) {
  __builtin_cpu_init();
  return (__builtin_cpu_supports("fma") && __builtin_cpu_supports("avx2")) ? chain_fma : chain_libm;
}

/* xt [T][steps][4][64], wt [E][steps][4][64]; z [T][E] for tokens t0..t1-1.
 * force_libm != 0 takes the fmaf-call form (for the tests). */
void dsk_oracle_gate_fma(const float* xt, const float* wt, int32_t E, int32_t steps, int32_t t0, int32_t t1,
                         float* z, int32_t force_libm) {
  const chain_fn chain = force_libm ? chain_libm : pick();
  const int seg = (steps + SEGMENTS - 1) / SEGMENTS;
  const int64_t per = (int64_t)steps * VEC * LANES;
  float p[LANES], q[LANES];
  for (int t = t0; t < t1; ++t)
    for (int e = 0; e < E; ++e) {
      float zz = 0.0f;
      for (int sw = 0; sw < SEGMENTS; ++sw) {
        const int m0 = sw * seg, m1 = (sw + 1) * seg < steps ? (sw + 1) * seg : steps;
        for (int l = 0; l < LANES; ++l) p[l] = 0.0f;
        if (m0 < m1) chain(xt + t * per, wt + e * per, m0, m1, p);
        for (int s = 32; s >= 1; s >>= 1) {
          for (int l = 0; l < LANES; ++l) q[l] = p[l] + p[l ^ s];
          memcpy(p, q, sizeof p);
        }
        zz = sw == 0 ? p[0] : zz + p[0];
      }
      z[(int64_t)t * E + e] = zz;
    }
}
