/*
 * hi2 encode-path ORACLE — test infrastructure only.
 *
 * A plain-C CPU restatement of the reference's encode hot path (BlivionIaG/hi2,
 * torch reference code), used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker.  Nothing in the product
 * (hi2_amd/) links, loads or calls this file.
 *
 * Each function names the reference lines it restates.  Where the reference's
 * result depends on torch's CPU reduction or BLAS/LAPACK order, the oracle fixes
 * its own order (stated per function) and the tests hold it to the reference's
 * golden vectors (tests/golden/) at the tolerance that order difference allows.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fno-fast-math -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- IEEE half conversions (round to nearest even), torch's .to(float16) ---- */
uint16_t or_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or nan */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (ax >= 0x38800000u) { /* normal half range (>= 2^-14) */
    uint32_t mant = ax & 0x7fffffu;
    uint32_t exp = (ax >> 23) - 127 + 15;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry into exp is fine */
    return (uint16_t)(sign | h);
  }
  /* subnormal half or zero: value = ax as float; half ulp = 2^-24 */
  {
    float af;
    memcpy(&af, &ax, 4);
    /* scale to units of 2^-24 and round to nearest even (exact in double) */
    double v = (double)af * 16777216.0;
    double r = nearbyint(v); /* default rounding mode: nearest even */
    return (uint16_t)(sign | (uint32_t)r);
  }
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign;
    } else { /* subnormal: mant * 2^-24 */
      float v = (float)mant * (1.0f / 16777216.0f);
      memcpy(&x, &v, 4);
      x |= sign;
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (mant << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

static inline float f16r(float f) { return or_f16_to_f32(or_f32_to_f16(f)); }

static inline float bf16_to_f32(uint16_t b) {
  uint32_t x = (uint32_t)b << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* torch.round: half to even */
static inline float rne(float x) { return nearbyintf(x); }

/* clamp(0, n-1) with NaN propagating, as torch.clamp */
static inline float clampq(float q, float nm) {
  q = (q < 0.0f) ? 0.0f : q;
  q = (q > nm) ? nm : q;
  return q;
}

/* ---- hadamard / fwht_groups (hi2/format.py:22-41) ------------------------------
 * Order-16 transform of the flagged groups as the reference's fp32 matmul x @ H16
 * evaluates it: y_j = sequential FMA chain over i = 0..15 of x_i * H[i][j] from zero
 * (H entries +-1/4, Sylvester sign (-1)^popcount(i & j)). */
void or_fwht16(const float* x, float* y, int64_t rows, int64_t k, const uint8_t* flags) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < k / 16; ++g) {
      const float* xi = x + r * k + g * 16;
      float* yo = y + r * k + g * 16;
      if (!flags[g]) {
        for (int t = 0; t < 16; ++t) yo[t] = xi[t];
        continue;
      }
      float v[16];
      for (int t = 0; t < 16; ++t) v[t] = xi[t];
      for (int j = 0; j < 16; ++j) {
        float acc = 0.0f;
        for (int i = 0; i < 16; ++i)
          acc = fmaf(v[i], (__builtin_popcount(i & j) & 1) ? -0.25f : 0.25f, acc);
        yo[j] = acc;
      }
    }
  }
}

/* ---- torch's CPU float sum order (torch 2.10 aten/src/ATen/native/cpu/SumKernel.cpp,
 * cascade_sum -> vectorized_inner_sum -> row_sum -> multi_row_sum) ----------------
 * The reference's reductions (.sum(-1), .mean(-1)) over a contiguous inner dim run
 * in this order on the build machine: 8-float vector lanes, 4 independent vector
 * accumulators ("rows" of 4 vectors), a 4-level cascade with base 2^max(4,
 * ceil_log2(rows)/4) over the rows, then the 4 accumulators folded, the scalar tail,
 * then the 8 lanes added sequentially.  Verified equal to torch.sum bit for bit on
 * sizes 16..2^20 (tests/test_oracle.py). */
static int64_t ceil_log2_i64(int64_t x) {
  if (x <= 2) return 1;
  int64_t b = 0;
  uint64_t v = (uint64_t)(x - 1);
  while (v) {
    ++b;
    v >>= 1;
  }
  return b;
}

float or_torch_sum(const float* x, int64_t n) {
  enum { V = 8, ILP = 4, NL = 4 };
  const int64_t vec_size = n / V;
  const int64_t size_ilp = vec_size / ILP;
  float p[ILP][V];
  memset(p, 0, sizeof(p));
  if (size_ilp > 0) {
    int64_t lp = ceil_log2_i64(size_ilp) / NL;
    if (lp < 4) lp = 4;
    const int64_t step = (int64_t)1 << lp, lmask = step - 1;
    float acc[NL][ILP][V];
    memset(acc, 0, sizeof(acc));
    int64_t i = 0;
    while (i + step <= size_ilp) {
      for (int64_t j = 0; j < step; ++j)
        for (int k = 0; k < ILP; ++k)
          for (int v = 0; v < V; ++v) acc[0][k][v] += x[((i + j) * ILP + k) * V + v];
      i += step;
      for (int j = 1; j < NL; ++j) {
        for (int k = 0; k < ILP; ++k)
          for (int v = 0; v < V; ++v) {
            acc[j][k][v] += acc[j - 1][k][v];
            acc[j - 1][k][v] = 0.0f;
          }
        if (i & (lmask << (j * lp))) break;
      }
    }
    for (; i < size_ilp; ++i)
      for (int k = 0; k < ILP; ++k)
        for (int v = 0; v < V; ++v) acc[0][k][v] += x[(i * ILP + k) * V + v];
    for (int j = 1; j < NL; ++j)
      for (int k = 0; k < ILP; ++k)
        for (int v = 0; v < V; ++v) acc[0][k][v] += acc[j][k][v];
    memcpy(p, acc[0], sizeof(p));
  }
  for (int64_t i = size_ilp * ILP; i < vec_size; ++i)
    for (int v = 0; v < V; ++v) p[0][v] += x[i * V + v];
  for (int k = 1; k < ILP; ++k)
    for (int v = 0; v < V; ++v) p[0][v] += p[k][v];
  float out = 0.0f;
  for (int64_t i = vec_size * V; i < n; ++i) out += x[i];
  for (int v = 0; v < V; ++v) out += p[0][v];
  return out;
}

/* ---- fit_ladder (hi2/encode.py:30-92) ------------------------------------------
 * One (row, block) at a time; every elementwise op as the reference's torch ops
 * (separately rounded), every block sum in torch's order (or_torch_sum). */
static float recon_err(const float* w, const float* d, int B, float lo, float step, float nm,
                       float* tmp) {
  const float safe = (step == 0.0f) ? 1.0f : step;
  for (int t = 0; t < B; ++t) {
    float c = clampq(rne((w[t] - lo) / safe), nm);
    float rec = lo + c * step;
    float df = rec - w[t];
    tmp[t] = d[t] * (df * df);
  }
  return or_torch_sum(tmp, B);
}

void or_fit_ladder(const float* wb, const float* db, int64_t rows, int64_t nb, int B,
                   int n, const float* grid, int G, int ls, float* out_lo,
                   float* out_step) {
  const float nm = (float)(n - 1);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * nb; ++i) {
    float tmp[256], t2[256], t3[256], t4[256], t5[256];
    const float* w = wb + i * B;
    const float* d = db + (i % nb) * B;
    float mn = w[0], mx = w[0];
    for (int t = 1; t < B; ++t) {
      mn = (w[t] < mn) ? w[t] : mn;
      mx = (w[t] > mx) ? w[t] : mx;
    }
    const float span = mx - mn;
    float best_lo = 0, best_st = 0, best_err = 0;
    int first = 1;
    for (int a = 0; a < G; ++a) {
      const float lo = mn + grid[a] * span;
      for (int b = 0; b < G; ++b) {
        const float step = ((mx - grid[b] * span) - lo) / nm;
        const float err = recon_err(w, d, B, lo, step, nm, tmp);
        if (first || err < best_err) {
          best_lo = lo;
          best_st = step;
          best_err = err;
          first = 0;
        }
      }
    }
    for (int it = 0; it < ls; ++it) {
      /* codes of the current best ladder, then _lsq (hi2/encode.py:35-50) */
      const float safe = (best_st == 0.0f) ? 1.0f : best_st;
      float cs[256];
      for (int t = 0; t < B; ++t) cs[t] = clampq(rne((w[t] - best_lo) / safe), nm);
      const float sd = or_torch_sum(d, B);
      for (int t = 0; t < B; ++t) {
        const float dc = d[t] * cs[t];
        tmp[t] = dc;
        t2[t] = dc * cs[t];
        t3[t] = d[t] * w[t];
        t4[t] = dc * w[t];
      }
      const float sc = or_torch_sum(tmp, B), scc = or_torch_sum(t2, B);
      const float sw = or_torch_sum(t3, B), scw = or_torch_sum(t4, B);
      const float det = sd * scc - sc * sc;
      const int ok = fabsf(det) > 1e-20f;
      const float step = ok ? (sd * scw - sc * sw) / det : 0.0f;
      const float sdc = (sd < 1e-20f) ? 1e-20f : sd;
      for (int t = 0; t < B; ++t) t5[t] = w[t];
      const float lo = ok ? (sw - step * sc) / sdc : or_torch_sum(t5, B) / (float)B;
      const float err = recon_err(w, d, B, lo, step, nm, tmp);
      if (err < best_err && step > 0.0f) {
        best_lo = lo;
        best_st = step;
        best_err = err;
      }
    }
    out_lo[i] = best_lo;
    out_step[i] = best_st;
  }
}

/* ---- quantize_params + decode_params (hi2/encode.py:95-119, format.py:45-60) ---- */
void or_params(const float* lo, const float* step_in, int64_t rows, int64_t nb,
               uint8_t* lo_u8, uint8_t* step_u8, uint16_t* consts, float* lo_d,
               float* step_d) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* l = lo + r * nb;
    const float* s = step_in + r * nb;
    float smax = 0, lmin = l[0], lmax = l[0];
    for (int64_t b = 0; b < nb; ++b) {
      float st = s[b] < 0.0f ? 0.0f : s[b];
      if (b == 0 || st > smax) smax = st;
      lmin = (l[b] < lmin) ? l[b] : lmin;
      lmax = (l[b] > lmax) ? l[b] : lmax;
    }
    const uint16_t ss_h = or_f32_to_f16(smax / 255.0f);
    const float ss = or_f16_to_f32(ss_h);
    const uint16_t lm_h = or_f32_to_f16(lmin);
    const float lmf = or_f16_to_f32(lm_h);
    float span = lmax - lmf;
    span = span < 0.0f ? 0.0f : span;
    const uint16_t ls_h = or_f32_to_f16(span / 255.0f);
    const float lsf = or_f16_to_f32(ls_h);
    consts[r * 3 + 0] = lm_h;
    consts[r * 3 + 1] = ls_h;
    consts[r * 3 + 2] = ss_h;
    for (int64_t b = 0; b < nb; ++b) {
      float st = s[b] < 0.0f ? 0.0f : s[b];
      float su = 0.0f;
      if (ss > 0.0f) su = rne(st / (ss < 1e-30f ? 1e-30f : ss));
      su = su < 0.0f ? 0.0f : (su > 255.0f ? 255.0f : su);
      float lu = 0.0f;
      if (lsf > 0.0f) lu = rne((l[b] - lmf) / (lsf < 1e-30f ? 1e-30f : lsf));
      lu = lu < 0.0f ? 0.0f : (lu > 255.0f ? 255.0f : lu);
      const uint8_t lub = (uint8_t)lu, sub = (uint8_t)su;
      lo_u8[r * nb + b] = lub;
      step_u8[r * nb + b] = sub;
      /* decode: f64 multiply-add, one rounding to f32, then fp16 */
      const double v = (double)lub * (double)lsf + (double)lmf;
      lo_d[r * nb + b] = f16r((float)v);
      step_d[r * nb + b] = f16r((float)sub * ss);
    }
  }
}

/* ---- GPTQ column loop (hi2/hessian.py:235-264; op spec hi2/gptq_kernel.py:82-100)
 * wc [n, K] fp32 in rounding order (modified in place), u [K, K], lo_d/step_d
 * [n, nb], blk_of [K] block of each rounding-order column.  Outputs codes [n, K]
 * (rounding order), comp [n, K] (optional).  The intra-block loop follows the
 * reference op for op; the cross-block update wc[:, i2:] -= err1 @ u[i1:i2, i2:]
 * is accumulated in double per element and rounded once before the subtraction. */
int g_trail_mode = 1; /* 1: sequential fp32 FMA (the reference's BLAS order); 0: double */
void or_gptq_set_trailing_mode(int m) { g_trail_mode = m; }

void or_gptq_rows(float* wc, int64_t n, int64_t k, const float* u, const float* lo_d,
                  const float* step_d, int64_t nb, const int64_t* blk_of, int nlev,
                  uint8_t* codes, float* comp) {
  const float nm = (float)(nlev - 1);
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t r = 0; r < n; ++r) {
    float* w = wc + r * k;
    float err1[128];
    for (int64_t i1 = 0; i1 < k; i1 += 128) {
      const int64_t i2 = (i1 + 128 < k) ? i1 + 128 : k;
      const int L = (int)(i2 - i1);
      float w1[128];
      for (int c = 0; c < L; ++c) w1[c] = w[i1 + c];
      for (int i = 0; i < L; ++i) {
        const int64_t j = i1 + i;
        const int64_t b = blk_of[j];
        const float lo = lo_d[r * nb + b], st = step_d[r * nb + b];
        const float col = w1[i];
        const float safe = (st == 0.0f) ? 1.0f : st;
        float q = clampq(rne((col - lo) / safe), nm);
        if (st == 0.0f) q = 0.0f;
        const float wq = f16r(lo + q * st);
        codes[r * k + j] = (uint8_t)q;
        if (comp) comp[r * k + j] = col;
        const float* ui = u + j * k + i1;
        const float e = (col - wq) / ui[i];
        for (int c = i + 1; c < L; ++c) w1[c] = w1[c] - e * ui[c];
        err1[i] = e;
      }
      for (int64_t c = i2; c < k; ++c) {
        if (g_trail_mode == 1) {
          float acc = 0.0f;
          for (int i = 0; i < L; ++i) acc = fmaf(err1[i], u[(i1 + i) * k + c], acc);
          w[c] = w[c] - acc;
        } else {
          double acc = 0.0;
          for (int i = 0; i < L; ++i) acc += (double)err1[i] * (double)u[(i1 + i) * k + c];
          w[c] = w[c] - (float)acc;
        }
      }
    }
  }
}

/* One lazy block only (the fused kernel's contract, hi2/gptq_kernel.py:59-101):
 * wc read only, err1 [n, L] and codes/comp written at rounding-order positions.
 * row_grp/u_ptrs/blk/nmax select the factor, column map and code count per row. */
void or_gptq_block(const float* wc, int64_t n, int64_t k, int64_t i1, int L, float* err1,
                   uint8_t* codes, const float* lo, const float* st, int64_t ldp,
                   const int32_t* row_grp, const float* const* u_list, const int32_t* blk,
                   const float* nmax, float* comp) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) {
    const int g = row_grp[r];
    const float* u = u_list[g];
    const int32_t* bl = blk + (int64_t)g * k;
    const float nm = nmax[g];
    float w[128];
    for (int c = 0; c < L; ++c) w[c] = wc[r * k + i1 + c];
    for (int i = 0; i < L; ++i) {
      const int64_t j = i1 + i;
      const int b = bl[j];
      const float lo_j = lo[r * ldp + b], st_j = st[r * ldp + b];
      const float col = w[i];
      const float safe = (st_j == 0.0f) ? 1.0f : st_j;
      float q = clampq(rne((col - lo_j) / safe), nm);
      if (st_j == 0.0f) q = 0.0f;
      const float wq = f16r(lo_j + q * st_j);
      codes[r * k + j] = (uint8_t)q;
      if (comp) comp[r * k + j] = col;
      const float* ui = u + j * k + i1;
      const float e = (col - wq) / ui[i];
      for (int c = i + 1; c < L; ++c) w[c] = w[c] - e * ui[c];
      err1[r * L + i] = e;
    }
  }
}

/* ---- _finish (hi2/hessian.py:318-345) --------------------------------------------
 * Un-permute codes/comp (rounding order -> column order via perm), reconstruct
 * fp16(lo + code*step) in fp32, sse = sum_k d_k (rec - w)^2 in torch's sum order. */
void or_finish(const uint8_t* codes_ro, const float* comp_ro, const int64_t* perm,
               int64_t n, int64_t k, int64_t block, const float* lo_d, const float* step_d,
               const float* w, const float* d, uint8_t* codes, float* comp, float* sse) {
  const int64_t nb = k / block;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t j = 0; j < k; ++j) {
      const int64_t c = perm ? perm[j] : j;
      codes[r * k + c] = codes_ro[r * k + j];
      if (comp && comp_ro) comp[r * k + c] = comp_ro[r * k + j];
    }
    float* tmp = (float*)malloc((size_t)k * sizeof(float));
    for (int64_t c = 0; c < k; ++c) {
      const int64_t b = c / block;
      const float rec = f16r(lo_d[r * nb + b] + (float)codes[r * k + c] * step_d[r * nb + b]);
      const float df = rec - w[r * k + c];
      tmp[c] = d[c] * (df * df);
    }
    sse[r] = or_torch_sum(tmp, k);
    free(tmp);
  }
}

/* ---- HessianStats.update (hi2/hessian.py:35-40) ----------------------------------
 * S[K, K] += X^T X over T tokens, X given as bf16 bits (is_bf16) or fp32; every
 * element accumulated in double and rounded once when added to S. */
void or_hessian_update(const void* x, int is_bf16, int64_t t, int64_t k, float* s) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t a = 0; a < k; ++a) {
    double* acc = (double*)calloc((size_t)k, sizeof(double));
    for (int64_t i = 0; i < t; ++i) {
      double xa;
      if (is_bf16) xa = bf16_to_f32(((const uint16_t*)x)[i * k + a]);
      else xa = ((const float*)x)[i * k + a];
      if (xa == 0.0) continue;
      if (is_bf16) {
        const uint16_t* xr = (const uint16_t*)x + i * k;
        for (int64_t b = 0; b < k; ++b) acc[b] += xa * (double)bf16_to_f32(xr[b]);
      } else {
        const float* xr = (const float*)x + i * k;
        for (int64_t b = 0; b < k; ++b) acc[b] += xa * (double)xr[b];
      }
    }
    for (int64_t b = 0; b < k; ++b) s[a * k + b] = (float)((double)s[a * k + b] + acc[b]);
    free(acc);
  }
}

/* ---- transform_sigma (hi2/hessian.py:50-68) -------------------------------------
 * As the reference's fp32 ops: smoothing (s * inv_i) * inv_j with inv = 1 / col_scale,
 * then per 16x16 block the two einsums as sequential fp32 FMA chains from zero
 * (t1 = m_gi s, t2 = t1 m_gh^T; m = H16/4 on flagged groups, I otherwise), then
 * 0.5 * (s + s^T).  col_scale: fp16 bits or NULL; had [K/16]. */
void or_transform_sigma(const float* sigma, const uint16_t* col_scale, const uint8_t* had,
                        int64_t k, float* out) {
  float* s = (float*)malloc((size_t)(k * k) * sizeof(float));
  float* inv = NULL;
  if (col_scale) {
    inv = (float*)malloc((size_t)k * sizeof(float));
    for (int64_t i = 0; i < k; ++i) inv[i] = 1.0f / or_f16_to_f32(col_scale[i]);
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < k; ++i)
    for (int64_t j = 0; j < k; ++j)
      s[i * k + j] = inv ? (sigma[i * k + j] * inv[i]) * inv[j] : sigma[i * k + j];
  int any = 0;
  for (int64_t g = 0; g < k / 16; ++g) any |= had[g] != 0;
  if (any) {
    float m[2][16][16]; /* [0] = identity, [1] = H16 / 4 */
    for (int i = 0; i < 16; ++i)
      for (int j = 0; j < 16; ++j) {
        m[0][i][j] = (i == j) ? 1.0f : 0.0f;
        m[1][i][j] = (__builtin_popcount(i & j) & 1) ? -0.25f : 0.25f;
      }
    const int64_t g = k / 16;
#pragma omp parallel for schedule(static)
    for (int64_t gi = 0; gi < g; ++gi) {
      const float(*mi)[16] = m[had[gi] ? 1 : 0];
      for (int64_t gh = 0; gh < g; ++gh) {
        const float(*mh)[16] = m[had[gh] ? 1 : 0];
        float blkv[16][16], t1[16][16];
        for (int i = 0; i < 16; ++i)
          for (int j = 0; j < 16; ++j) blkv[i][j] = s[(gi * 16 + i) * k + gh * 16 + j];
        for (int i = 0; i < 16; ++i)
          for (int c = 0; c < 16; ++c) {
            float a = 0.0f;
            for (int j = 0; j < 16; ++j) a = fmaf(mi[i][j], blkv[j][c], a);
            t1[i][c] = a;
          }
        for (int i = 0; i < 16; ++i)
          for (int l = 0; l < 16; ++l) {
            float a = 0.0f;
            for (int c = 0; c < 16; ++c) a = fmaf(t1[i][c], mh[l][c], a);
            s[(gi * 16 + i) * k + gh * 16 + l] = a; /* block already read */
          }
      }
    }
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < k; ++i)
    for (int64_t j = 0; j < k; ++j) out[i * k + j] = 0.5f * (s[i * k + j] + s[j * k + i]);
  free(s);
  free(inv);
}

/* torch's CPU sum of a strided (non-contiguous) float vector, e.g. diagonal().sum():
 * SumKernel.cpp scalar_inner_sum -> row_sum -> multi_row_sum with 4 scalar
 * accumulators, the same 4-level cascade, the tail into accumulator 0, then folded. */
float or_torch_sum_strided(const float* x, int64_t n, int64_t stride) {
  enum { ILP = 4, NL = 4 };
  const int64_t size_ilp = n / ILP;
  float acc[NL][ILP];
  memset(acc, 0, sizeof(acc));
  if (size_ilp > 0) {
    int64_t lp = ceil_log2_i64(size_ilp) / NL;
    if (lp < 4) lp = 4;
    const int64_t step = (int64_t)1 << lp, lmask = step - 1;
    int64_t i = 0;
    while (i + step <= size_ilp) {
      for (int64_t j = 0; j < step; ++j)
        for (int q = 0; q < ILP; ++q) acc[0][q] += x[((i + j) * ILP + q) * stride];
      i += step;
      for (int l = 1; l < NL; ++l) {
        for (int q = 0; q < ILP; ++q) {
          acc[l][q] += acc[l - 1][q];
          acc[l - 1][q] = 0.0f;
        }
        if (i & (lmask << (l * lp))) break;
      }
    }
    for (; i < size_ilp; ++i)
      for (int q = 0; q < ILP; ++q) acc[0][q] += x[(i * ILP + q) * stride];
    for (int l = 1; l < NL; ++l)
      for (int q = 0; q < ILP; ++q) acc[0][q] += acc[l][q];
  }
  float p[ILP] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
  for (int64_t i = size_ilp * ILP; i < n; ++i) p[0] += x[i * stride];
  return ((p[0] + p[1]) + p[2]) + p[3];
}

/* ---- inverse_factor (hi2/hessian.py:71-86) ----------------------------------------
 * lam = damp * mean(diag) (clamped at 1e-12, fp32), attempts a = 0..5 with
 * lam * 10^a on the diagonal; per attempt the reference chain
 *   L = chol(h); Hinv = L^-T L^-1; U = chol_upper((Hinv + Hinv^T) / 2)
 * in double.  Returns the attempt that succeeded, or -1. */
static int chol_lower_d(double* a, int64_t k) {
  for (int64_t j = 0; j < k; ++j) {
    double dj = a[j * k + j];
    for (int64_t p = 0; p < j; ++p) dj -= a[j * k + p] * a[j * k + p];
    if (!(dj > 0.0)) return -1;
    dj = sqrt(dj);
    a[j * k + j] = dj;
#pragma omp parallel for schedule(static)
    for (int64_t i = j + 1; i < k; ++i) {
      double v = a[i * k + j];
      for (int64_t p = 0; p < j; ++p) v -= a[i * k + p] * a[j * k + p];
      a[i * k + j] = v / dj;
    }
  }
  for (int64_t i = 0; i < k; ++i)
    for (int64_t j = i + 1; j < k; ++j) a[i * k + j] = 0.0;
  return 0;
}

int or_inverse_factor(const float* hs, int64_t k, float damp, float* u_out) {
  float mean = or_torch_sum_strided(hs, k, k + 1) / (float)k;
  if (mean < 1e-12f) mean = 1e-12f;
  double* a = (double*)malloc((size_t)(k * k) * sizeof(double));
  double* linv = (double*)malloc((size_t)(k * k) * sizeof(double));
  int result = -1;
  for (int att = 0; att < 6 && result < 0; ++att) {
    float p10 = 1.0f;
    for (int q = 0; q < att; ++q) p10 *= 10.0f;
    const float lam = (damp * mean) * p10;
    for (int64_t i = 0; i < k; ++i)
      for (int64_t j = 0; j < k; ++j)
        a[i * k + j] = (double)(i == j ? hs[i * k + j] + lam : hs[i * k + j]);
    if (chol_lower_d(a, k)) continue;
    /* Linv = L^-1 (lower), column by column */
    memset(linv, 0, (size_t)(k * k) * sizeof(double));
#pragma omp parallel for schedule(dynamic, 8)
    for (int64_t c = 0; c < k; ++c) {
      linv[c * k + c] = 1.0 / a[c * k + c];
      for (int64_t i = c + 1; i < k; ++i) {
        double v = 0.0;
        for (int64_t p = c; p < i; ++p) v -= a[i * k + p] * linv[p * k + c];
        linv[i * k + c] = v / a[i * k + i];
      }
    }
    /* Hinv = Linv^T Linv, symmetric by construction */
#pragma omp parallel for schedule(dynamic, 8)
    for (int64_t i = 0; i < k; ++i)
      for (int64_t j = i; j < k; ++j) {
        double v = 0.0;
        const int64_t p0 = j; /* Linv[p][i], Linv[p][j] nonzero for p >= max(i, j) */
        for (int64_t p = p0; p < k; ++p) v += linv[p * k + i] * linv[p * k + j];
        a[i * k + j] = v;
        a[j * k + i] = v;
      }
    /* U = chol_upper(Hinv) = L2^T with L2 = chol_lower(Hinv) */
    if (chol_lower_d(a, k)) continue;
    for (int64_t i = 0; i < k; ++i)
      for (int64_t j = 0; j < k; ++j) u_out[i * k + j] = (j >= i) ? (float)a[j * k + i] : 0.0f;
    result = att;
  }
  free(a);
  free(linv);
  return result;
}

/* ---- pack_codes / assemble (hi2/format.py:73-85, 127-184) ------------------------
 * codes [rows, K] -> words [rows, K*nbits/32] int32, LSB first.  Returns the number
 * of codes outside [0, 2^nbits) (the reference raises ValueError when nonzero). */
int64_t or_pack_codes(const uint8_t* codes, int64_t rows, int64_t k, int nbits,
                      int32_t* words) {
  const int per = 32 / nbits;
  const int64_t nw = k / per;
  int64_t bad = 0;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t wi = 0; wi < nw; ++wi) {
      uint32_t v = 0;
      for (int i = 0; i < per; ++i) {
        uint32_t c = codes[r * k + wi * per + i];
        if (c >= (1u << nbits)) ++bad;
        v |= (c & ((1u << nbits) - 1u)) << (nbits * i);
      }
      words[r * nw + wi] = (int32_t)v;
    }
  return bad;
}

/* One piece of assemble: rows [r] (tensor row indices), codes [r, K], params
 * [r, nb, 2], consts [r, 3] fp16 bits scattered into the flat buffers at the
 * per-row offsets code_off / param_off (in words / blocks). */
int64_t or_assemble_piece(const int64_t* rows, int64_t r, const uint8_t* codes,
                          const uint8_t* params, const uint16_t* consts, int64_t k,
                          int nbits, int64_t block, const int64_t* code_off,
                          const int64_t* param_off, int32_t* out_codes, uint8_t* out_params,
                          uint16_t* out_consts) {
  const int per = 32 / nbits;
  const int64_t nw = k / per, nblk = k / block;
  int64_t bad = 0;
  for (int64_t i = 0; i < r; ++i) {
    const int64_t row = rows[i];
    bad += or_pack_codes(codes + i * k, 1, k, nbits, out_codes + code_off[row]);
    (void)nw;
    for (int64_t b = 0; b < nblk; ++b) {
      out_params[(param_off[row] + b) * 2 + 0] = params[(i * nblk + b) * 2 + 0];
      out_params[(param_off[row] + b) * 2 + 1] = params[(i * nblk + b) * 2 + 1];
    }
    for (int c = 0; c < 3; ++c) out_consts[row * 3 + c] = consts[i * 3 + c];
  }
  return bad;
}

/* ---- local code refinement (hi2/refine.py:43-106; column-loop op spec
 * hi2/refine_kernel.py:63-91) ------------------------------------------------------
 * Rows w [n, k] f32 (stored basis), codes [n, k] u8 (refined in place), decoded ladders
 * lo/st [n, ldp] f32 where row r's column j uses ladder block j / block[r], top[r] the
 * row's highest code, hs [k, k] f32.  Per row:
 *   e = fp16(lo + c*st) - w;  g = e @ hs, each element a sequential fp32 FMA chain over
 *   k in order (the oracle's fixed order for the reference's rank-k BLAS product);
 *   per sweep and 128-column block [b0, b1): the reference's column loop, every product
 *   and sum rounded separately, the candidates +1 then -1 compared as torch's max over
 *   the stacked pair (a NaN gain propagates and is never taken, ties keep +1); then
 *   g += (dw @ hs[b0:b1]) with the product a sequential FMA chain over the block's
 *   columns from zero and one addition (hi2/refine.py:99).
 * Rows are independent given hs, and a row whose sweep moves no code never moves again
 * (its g and codes are unchanged, so the next sweep repeats the same decisions): the
 * reference's stop after a sweep that moves nothing in any row is the same as stopping
 * each row after its own first such sweep.  moved[r] (optional) receives the number of
 * codes moved in row r over all sweeps.  Returns the number of sweeps the reference
 * runs: min(passes, 1 + the largest number of sweeps in which some row moved). */
int or_refine(const float* w, uint8_t* codes, int64_t n, int64_t k, const float* lo,
              const float* st, int64_t ldp, const int32_t* block, const float* top,
              const float* hs, int passes, int64_t* moved) {
  int most = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(max : most)
  for (int64_t r = 0; r < n; ++r) {
    float* g = (float*)malloc((size_t)k * sizeof(float));
    float* e = (float*)malloc((size_t)k * sizeof(float));
    uint8_t* c = codes + r * k;
    const float* lr = lo + r * ldp;
    const float* sr = st + r * ldp;
    const int64_t B = block[r];
    const float tp = top[r];
    for (int64_t j = 0; j < k; ++j)
      e[j] = f16r(lr[j / B] + (float)c[j] * sr[j / B]) - w[r * k + j];
    for (int64_t col = 0; col < k; ++col) {
      float acc = 0.0f;
      for (int64_t i = 0; i < k; ++i) acc = fmaf(e[i], hs[i * k + col], acc);
      g[col] = acc;
    }
    int64_t mv = 0;
    int sweeps_moved = 0;
    for (int p = 0; p < passes; ++p) {
      int64_t mp = 0;
      for (int64_t b0 = 0; b0 < k; b0 += 128) {
        const int L = (int)((k - b0 < 128) ? k - b0 : 128);
        float gb[128], dwb[128];
        for (int q = 0; q < L; ++q) gb[q] = g[b0 + q];
        for (int jj = 0; jj < L; ++jj) {
          const int64_t j = b0 + jj;
          const float lo_j = lr[j / B], st_j = sr[j / B];
          const float cj = (float)c[j];
          const float cur = f16r(lo_j + cj * st_j);
          const float hd = hs[j * k + j];
          const float gj = gb[jj];
          float gain[2], dw[2], cn[2];
          for (int t = 0; t < 2; ++t) {
            cn[t] = cj + (t == 0 ? 1.0f : -1.0f);
            dw[t] = f16r(lo_j + cn[t] * st_j) - cur;
            const int ok = (cn[t] >= 0.0f) && (cn[t] <= tp) && (st_j > 0.0f);
            const float t1 = 2.0f * dw[t];
            const float t2 = t1 * gj;
            const float t3 = dw[t] * dw[t];
            const float t4 = t3 * hd;
            gain[t] = ok ? -(t2 + t4) : -INFINITY;
          }
          /* torch max over [gain+, gain-]: NaN wins (never > 0), else the first largest */
          int which = 0;
          float best = gain[0];
          if (!isnan(gain[0]) && (isnan(gain[1]) || gain[1] > gain[0])) {
            which = 1;
            best = gain[1];
          }
          const int take = best > 0.0f;
          const float dwj = take ? dw[which] : 0.0f;
          if (take) {
            c[j] = (uint8_t)cn[which];
            ++mp;
          }
          dwb[jj] = dwj;
          const float* hr = hs + j * k + b0;
          for (int q = 0; q < L; ++q) gb[q] = gb[q] + dwj * hr[q];
        }
        for (int64_t col = 0; col < k; ++col) {
          float acc = 0.0f;
          for (int jj = 0; jj < L; ++jj) acc = fmaf(dwb[jj], hs[(b0 + jj) * k + col], acc);
          g[col] = g[col] + acc;
        }
      }
      mv += mp;
      if (mp == 0) break;
      ++sweeps_moved;
    }
    if (moved) moved[r] = mv;
    if (sweeps_moved > most) most = sweeps_moved;
    free(g);
    free(e);
  }
  return passes < most + 1 ? passes : most + 1;
}

/* ---- ColumnStats (hi2/stats.py:26-33) -----------------------------------------------
 * s [K/16, 16, 16] f64 += the 16 x 16 second moments of every column group of x [t, K]
 * (bf16 bits when is_bf16, else f32), chunk by chunk of 4096 tokens as the reference's
 * update: each chunk's moments in fp32, then added to s in f64.  The reference forms a
 * chunk's fp32 moments with torch's einsum; the oracle fixes its own order, the one the
 * GPU kernel uses: sub-chunks of 256 tokens, each a sequential fp32 FMA chain over its
 * tokens from zero, their results added in order (fp32) into the chunk's moment. */
void or_colstats_update(const void* x, int is_bf16, int64_t t, int64_t k, double* s) {
  const int64_t ng = k / 16;
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < ng; ++g) {
    for (int i = 0; i < 16; ++i)
      for (int j = 0; j < 16; ++j) {
        double acc = s[(g * 16 + i) * 16 + j];
        for (int64_t c0 = 0; c0 < t; c0 += 4096) {
          const int64_t c1 = (c0 + 4096 < t) ? c0 + 4096 : t;
          float chunk = 0.0f;
          for (int64_t s0 = c0; s0 < c1; s0 += 256) {
            const int64_t s1 = (s0 + 256 < c1) ? s0 + 256 : c1;
            float sub = 0.0f;
            for (int64_t r = s0; r < s1; ++r) {
              float a, b;
              if (is_bf16) {
                a = bf16_to_f32(((const uint16_t*)x)[r * k + g * 16 + i]);
                b = bf16_to_f32(((const uint16_t*)x)[r * k + g * 16 + j]);
              } else {
                a = ((const float*)x)[r * k + g * 16 + i];
                b = ((const float*)x)[r * k + g * 16 + j];
              }
              sub = fmaf(a, b, sub);
            }
            chunk = chunk + sub;
          }
          acc = acc + (double)chunk;
        }
        s[(g * 16 + i) * 16 + j] = acc;
      }
  }
}

/* ColumnStats.diag (hi2/stats.py:39-55): out [K] f32.  s = S / max(n, 1) in f64, times
 * inv_j inv_k when inv_scale (f32 [K]) is given ((s * inv_j) * inv_k); plain = s_ii; on a
 * flagged group rot_i = sum_j h_ij (sum_k s_jk h_ik) with h = H16 / 4, each sum
 * sequential in f64 without fused products (the reference's f64 einsum fixes its own
 * order; the difference is far below the f32 output's rounding). */
void or_colstats_diag(const double* S, int64_t k, int64_t n, const uint8_t* flags,
                      const float* inv_scale, float* out) {
  const int64_t ng = k / 16;
  const double nn = (double)(n > 1 ? n : 1);
  for (int64_t g = 0; g < ng; ++g) {
    double s[16][16];
    for (int j = 0; j < 16; ++j)
      for (int q = 0; q < 16; ++q) {
        double v = S[(g * 16 + j) * 16 + q] / nn;
        if (inv_scale) v = (v * (double)inv_scale[g * 16 + j]) * (double)inv_scale[g * 16 + q];
        s[j][q] = v;
      }
    for (int i = 0; i < 16; ++i) {
      double v = s[i][i];
      if (flags && flags[g]) {
        double rot = 0.0;
        for (int j = 0; j < 16; ++j) {
          double tj = 0.0;
          for (int q = 0; q < 16; ++q) {
            const double hq = (__builtin_popcount(i & q) & 1) ? -0.25 : 0.25;
            tj = tj + s[j][q] * hq;
          }
          const double hj = (__builtin_popcount(i & j) & 1) ? -0.25 : 0.25;
          rot = rot + hj * tj;
        }
        v = rot;
      }
      out[g * 16 + i] = (float)v;
    }
  }
}

/* ---- QAD decode (hi2/qad_kernel.py:57-189; hi2/qad.py:366-400) -------------------------- */

/* The block's fp16 lo and step from its continuous bytes (hi2/qad_kernel.py:60-69):
 * byte = clamp(rint(u), 0, 255) (fmin/fmax: a NaN byte reads as 0); lo = fp16(f32(f64(byte)
 * * f64(lo_scale) + f64(lo_min))), step = fp16(f32(byte) * step_scale). */
static void qad_ladder(float lo_u, float st_u, const uint16_t* c, float* lo, float* st) {
  const float lb = fminf(fmaxf(rne(lo_u), 0.0f), 255.0f);
  const float sb = fminf(fmaxf(rne(st_u), 0.0f), 255.0f);
  const double v = (double)lb * (double)or_f16_to_f32(c[1]) + (double)or_f16_to_f32(c[0]);
  *lo = f16r((float)v);
  *st = f16r(sb * or_f16_to_f32(c[2]));
}

/* q = clamp(rint(z), 0, nmax) with NaN kept (torch.clamp), 0 for a zero step
 * (hi2/qad.py:390-392). */
static float qad_code(float z, float nmax, int zero) {
  float q = rne(z);
  q = q < 0.0f ? 0.0f : q;
  q = q > nmax ? nmax : q;
  return zero ? 0.0f : q;
}

/* decode_fwd (hi2/qad_kernel.py:88-108; the value of hi2/qad.py:371-395): out[rows[r], j] =
 * fp16(f64(lo) + f64(q) * f64(step)), the f64 value converted as torch converts f64 to fp16
 * (through f32). */
void or_qad_decode_fwd(const float* latent, const float* unit, const float* lo_u,
                       const float* st_u, const uint16_t* consts, const int64_t* rows,
                       int64_t n_rows, int64_t k, int64_t block, float nmax, float* out) {
  const int64_t nblk = k / block;
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t b = 0; b < nblk; ++b) {
      float lo, st;
      qad_ladder(lo_u[r * nblk + b], st_u[r * nblk + b], consts + r * 3, &lo, &st);
      const int zero = st == 0.0f;
      const float safe = zero ? 1.0f : st;
      for (int64_t j = b * block; j < (b + 1) * block; ++j) {
        const int64_t off = rows[r] * k + j;
        float v = latent[off];
        if (unit) v = v * unit[off];
        const float q = qad_code((v - lo) / safe, nmax, zero);
        out[off] = f16r((float)((double)lo + (double)q * (double)st));
      }
    }
}

/* decode_bwd (hi2/qad_kernel.py:110-159): the straight-through gradients of
 * hi2/qad.py:380-399 in closed form; the per-block sums are the pairwise tree
 * s[i] += s[i + h] (i < h) for h = block/2, ..., 1, in fp32. */
void or_qad_decode_bwd(const float* grad, const float* latent, const float* unit,
                       const float* lo_u, const float* st_u, const uint16_t* consts,
                       const int64_t* rows, int64_t n_rows, int64_t k, int64_t block,
                       float nmax, float* g_latent, float* g_lo, float* g_st) {
  const int64_t nblk = k / block;
  float* s_lo = (float*)malloc(sizeof(float) * block);
  float* s_st = (float*)malloc(sizeof(float) * block);
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t b = 0; b < nblk; ++b) {
      float lo, st;
      const uint16_t* c = consts + r * 3;
      qad_ladder(lo_u[r * nblk + b], st_u[r * nblk + b], c, &lo, &st);
      const int zero = st == 0.0f;
      const float safe = zero ? 1.0f : st;
      for (int64_t t = 0; t < block; ++t) {
        const int64_t off = rows[r] * k + b * block + t;
        const float un = unit ? unit[off] : 1.0f;
        float v = latent[off];
        if (unit) v = v * un;
        const float z = (v - lo) / safe;
        const float q = qad_code(z, nmax, zero);
        const float G = grad[off];
        const int inside = z >= 0.0f && z <= nmax;
        const float gz = inside ? G * st : 0.0f;
        const float gv = gz / safe;
        g_latent[off] = unit ? gv * un : gv;
        s_lo[t] = G - gv;
        float a = G * q;
        if (!zero) a = a + (-gz) * (z / safe);
        s_st[t] = a;
      }
      for (int64_t h = block / 2; h > 0; h /= 2)
        for (int64_t i = 0; i < h; ++i) {
          s_lo[i] = s_lo[i] + s_lo[i + h];
          s_st[i] = s_st[i] + s_st[i + h];
        }
      g_lo[r * nblk + b] = s_lo[0] * or_f16_to_f32(c[1]);
      g_st[r * nblk + b] = s_st[0] * or_f16_to_f32(c[2]);
    }
  free(s_lo);
  free(s_st);
}

/* wht_scale (hi2/qad_kernel.py:165-189): per flagged 16-column group the butterfly
 * y[t] = (t & h) ? y[t ^ h] - y[t] : y[t] + y[t ^ h] for h = 1, 2, 4, 8, times 0.25; the
 * division by the fp16 scale after it, or before it with pre_div. */
void or_qad_wht_scale(const float* x, int64_t n_rows, int64_t k, const uint8_t* flags,
                      const uint16_t* scale, int pre_div, float* out) {
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t g = 0; g < k / 16; ++g) {
      float y[16], orig[16];
      for (int t = 0; t < 16; ++t) {
        float v = x[r * k + g * 16 + t];
        if (pre_div && scale) v = v / or_f16_to_f32(scale[g * 16 + t]);
        y[t] = orig[t] = v;
      }
      for (int h = 1; h < 16; h <<= 1) {
        float nxt[16];
        for (int t = 0; t < 16; ++t) nxt[t] = (t & h) ? y[t ^ h] - y[t] : y[t] + y[t ^ h];
        memcpy(y, nxt, sizeof(y));
      }
      for (int t = 0; t < 16; ++t) {
        float v = flags[g] ? y[t] * 0.25f : orig[t];
        if (!pre_div && scale) v = v / or_f16_to_f32(scale[g * 16 + t]);
        out[r * k + g * 16 + t] = v;
      }
    }
}
