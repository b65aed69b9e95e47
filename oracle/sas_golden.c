/*
 * sas_golden.c -- C restatement of the reference golden model for sparse
 * shared-KV attention.  TEST INFRASTRUCTURE ONLY: used by tests/ for parity
 * and by bench.py as the CPU baseline; never linked into the product.
 *
 * Algorithm (reference sparse_attn_sharedkv_tilelang/golden.py):
 *   - per (b, s): s_global = act_kv - act_q + s                      (golden.py:125)
 *   - window positions [max(s_global - win_left, 0), s_global]        (golden.py:129-131)
 *   - compressed ids: first min(K, thr) slots, -1 terminates, ids >= thr
 *     skipped, thr = floor((s_global + 1) / ratio)                     (golden.py:28-66)
 *     scenario 2: every id in [0, thr)                                 (golden.py:146-150)
 *   - paged row of position p: page = bt[b, p / BS], row p % BS; a
 *     negative page reads as zeros                                     (golden.py:247-268)
 *   - online softmax seeded with (row_max = sink, row_sum = 1), 512-row
 *     tiles, window tiles first then compressed tiles, P rounded to the
 *     query dtype before PV, output cast to the query dtype, lse =
 *     row_max + ln(row_sum)                                            (golden.py:156-200)
 * fp32 arithmetic throughout, as in the reference.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define SASG_TILE 512

enum { SASG_F32 = 0, SASG_BF16 = 1, SASG_F16 = 2, SASG_FP8E4M3 = 3 };

typedef struct {
  int32_t T, H, D, Dv, B;
  int32_t scenario, win_left, cmp_ratio, K;
  int32_t q_dtype, kv_dtype;
  int32_t ori_block_size, ori_table_len, ori_block_num;
  int32_t cmp_block_size, cmp_table_len, cmp_block_num;
  int64_t ori_block_stride, ori_row_stride; /* elements */
  int64_t cmp_block_stride, cmp_row_stride;
  float softmax_scale;
  int32_t nthreads;
} sasg_params;

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else { /* subnormal: renormalise */
      int sh = 0;
      while (!(m & 0x400)) { m <<= 1; sh++; }
      m &= 0x3ff;
      u = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
    }
  } else if (e == 0x1f) {
    u = s | 0x7f800000u | (m << 13);
  } else {
    u = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float fp8e4m3_to_f32(uint8_t v) {
  float sgn = (v & 0x80) ? -1.0f : 1.0f;
  int e = (v >> 3) & 0xf, m = v & 7;
  if (e == 0xf && m == 7) return NAN;
  if (e == 0) return sgn * ldexpf((float)m / 8.0f, -6);
  return sgn * ldexpf(1.0f + (float)m / 8.0f, e - 7);
}

static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x; /* NaN */
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float round_f16(float x) {
  /* round-to-nearest-even float -> half -> float, finite range only */
  if (isnan(x) || isinf(x)) return x;
  float ax = fabsf(x);
  if (ax >= 65520.0f) return copysignf(INFINITY, x);
  if (ax < ldexpf(1.0f, -14)) { /* subnormal half: quantum 2^-24 */
    float q = ldexpf(1.0f, -24);
    return copysignf(nearbyintf(ax / q) * q, x);
  }
  int ex;
  frexpf(ax, &ex); /* ax = f * 2^ex, f in [0.5,1) */
  float q = ldexpf(1.0f, ex - 11);
  return copysignf(nearbyintf(ax / q) * q, x);
}

static float round_to(float x, int dt) {
  if (dt == SASG_BF16) return round_bf16(x);
  if (dt == SASG_F16) return round_f16(x);
  return x;
}

static float load_elem(const void* base, int dt, int64_t i) {
  switch (dt) {
    case SASG_BF16: return bf16_to_f32(((const uint16_t*)base)[i]);
    case SASG_F16: return f16_to_f32(((const uint16_t*)base)[i]);
    case SASG_FP8E4M3: return fp8e4m3_to_f32(((const uint8_t*)base)[i]);
    default: return ((const float*)base)[i];
  }
}

static int64_t floor_div(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) q--;
  return q;
}

/* Pool row (page * BS + offset) of logical position pos, or -1 for an unused page. */
static int64_t paged_row(const int32_t* bt_row, int table_len, int block_size, int64_t pos) {
  int64_t blk = pos / block_size;
  if (blk >= table_len) return -1;
  int32_t page = bt_row[blk];
  if (page < 0) return -1;
  return (int64_t)page * block_size + pos % block_size;
}

/* Resolve the rows token (b, s) attends: window rows then compressed rows.
 * rows[] receives pool rows; n_ori/n_cmp the counts.  Returns 0, or -1 when
 * an index < -1 is met (outside the operator contract). */
static int resolve_token(const sasg_params* p, const int32_t* ori_bt, const int32_t* cmp_bt,
                         const int32_t* idx, int b, int t, int s, int act_q, int act_kv,
                         int64_t* rows, int* n_ori, int* n_cmp) {
  int64_t s_g = (int64_t)act_kv - act_q + s;
  int64_t left = s_g - p->win_left;
  if (left < 0) left = 0;
  int no = 0, nc = 0;
  for (int64_t pos = left; pos <= s_g; ++pos)
    rows[no++] = paged_row(ori_bt + (int64_t)b * p->ori_table_len, p->ori_table_len,
                           p->ori_block_size, pos);
  if (p->scenario >= 2) {
    int64_t thr = floor_div(s_g + 1, p->cmp_ratio);
    int64_t cmp_act = floor_div(act_kv, p->cmp_ratio);
    const int32_t* cbt = cmp_bt + (int64_t)b * p->cmp_table_len;
    if (p->scenario == 2) {
      for (int64_t id = 0; id < thr; ++id)
        rows[no + nc++] = paged_row(cbt, p->cmp_table_len, p->cmp_block_size, id);
    } else {
      int64_t vc = thr < p->K ? thr : p->K;
      const int32_t* ir = idx + (int64_t)t * p->K;
      for (int64_t i = 0; i < vc; ++i) {
        int32_t id = ir[i];
        if (id == -1) break;
        if (id < -1) return -1;
        int64_t end = (int64_t)id + 1;
        if (end > cmp_act) end = cmp_act;
        if (id >= thr) continue;
        if (end > thr) end = thr;
        for (int64_t j = id; j < end; ++j)
          rows[no + nc++] = paged_row(cbt, p->cmp_table_len, p->cmp_block_size, j);
      }
    }
  }
  *n_ori = no;
  *n_cmp = nc;
  return 0;
}

static int max_rows_per_token(const sasg_params* p, const int32_t* seqused_kv) {
  int64_t m = p->win_left + 1;
  if (p->scenario == 3) m += p->K;
  if (p->scenario == 2) {
    int64_t mx = 0;
    for (int b = 0; b < p->B; ++b) mx = seqused_kv[b] > mx ? seqused_kv[b] : mx;
    m += mx / p->cmp_ratio + 1;
  }
  return (int)m;
}

/* Map flat token -> (b, s) through q_prefix / act_q; -1 when no batch owns it. */
static void build_token_map(const sasg_params* p, const int32_t* q_prefix, const int32_t* act_q,
                            int32_t* tb, int32_t* ts) {
  for (int t = 0; t < p->T; ++t) tb[t] = -1;
  for (int b = 0; b < p->B; ++b)
    for (int s = 0; s < act_q[b]; ++s) {
      int64_t t = (int64_t)q_prefix[b] + s;
      if (t >= 0 && t < p->T) { tb[t] = b; ts[t] = s; }
    }
}

int sasg_resolve(const sasg_params* p, const int32_t* ori_bt, const int32_t* cmp_bt,
                 const int32_t* idx, const int32_t* q_prefix, const int32_t* act_q,
                 const int32_t* seqused_kv, int32_t max_rows, int64_t* rows_out,
                 int32_t* n_ori_out, int32_t* n_cmp_out) {
  int32_t* tb = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  int32_t* ts = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  int need = max_rows_per_token(p, seqused_kv);
  int64_t* tmp = (int64_t*)malloc(sizeof(int64_t) * need);
  int rc = 0;
  build_token_map(p, q_prefix, act_q, tb, ts);
  for (int t = 0; t < p->T && rc == 0; ++t) {
    n_ori_out[t] = n_cmp_out[t] = 0;
    if (tb[t] < 0) continue;
    int b = tb[t], no, nc;
    if (resolve_token(p, ori_bt, cmp_bt, idx, b, t, ts[t], act_q[b], seqused_kv[b], tmp, &no,
                      &nc)) { rc = -1; break; }
    if (no + nc > max_rows) { rc = -2; break; }
    memcpy(rows_out + (int64_t)t * max_rows, tmp, sizeof(int64_t) * (no + nc));
    n_ori_out[t] = no;
    n_cmp_out[t] = nc;
  }
  free(tmp); free(tb); free(ts);
  return rc;
}

int sasg_attention(const sasg_params* p, const void* q, const void* ori_kv,
                   const float* ori_scale, const int32_t* ori_bt, const void* cmp_kv,
                   const float* cmp_scale, const int32_t* cmp_bt, const int32_t* idx,
                   const int32_t* q_prefix, const int32_t* act_q, const int32_t* seqused_kv,
                   const float* sinks, const int32_t* tokens, int32_t n_tokens, float* out,
                   float* lse) {
  const int H = p->H, D = p->D, Dv = p->Dv;
  int32_t* tb = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  int32_t* ts = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  build_token_map(p, q_prefix, act_q, tb, ts);
  int nwork = tokens ? n_tokens : p->T;
  int need = max_rows_per_token(p, seqused_kv);
  int err = 0;
#ifdef _OPENMP
  if (p->nthreads > 0) omp_set_num_threads(p->nthreads);
#endif
#pragma omp parallel
  {
    int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * need);
    float* kt = (float*)malloc(sizeof(float) * (size_t)SASG_TILE * D);
    float* sc = (float*)malloc(sizeof(float) * (size_t)SASG_TILE);
    float* qf = (float*)malloc(sizeof(float) * (size_t)H * D);
    float* acc = (float*)malloc(sizeof(float) * (size_t)H * D);
    float* rmax = (float*)malloc(sizeof(float) * (size_t)H);
    float* rsum = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(dynamic, 1)
    for (int w = 0; w < nwork; ++w) {
      int t = tokens ? tokens[w] : w;
      if (t < 0 || t >= p->T) continue;
      float* ot = out + (int64_t)t * H * Dv;
      float* lt = lse + (int64_t)t * H;
      memset(ot, 0, sizeof(float) * (size_t)H * Dv);
      memset(lt, 0, sizeof(float) * (size_t)H);
      if (tb[t] < 0) continue;
      int b = tb[t], s = ts[t], no, nc;
      if (resolve_token(p, ori_bt, cmp_bt, idx, b, t, s, act_q[b], seqused_kv[b], rows, &no, &nc)) {
#pragma omp atomic write
        err = -1;
        continue;
      }
      for (int64_t i = 0; i < (int64_t)H * D; ++i)
        qf[i] = load_elem(q, p->q_dtype, (int64_t)t * H * D + i);
      for (int h = 0; h < H; ++h) { rmax[h] = sinks[h]; rsum[h] = 1.0f; }
      memset(acc, 0, sizeof(float) * (size_t)H * D);
      /* tile list: window tiles, then compressed tiles (never mixed). */
      int ntile_o = (no + SASG_TILE - 1) / SASG_TILE, ntile_c = (nc + SASG_TILE - 1) / SASG_TILE;
      for (int tile = 0; tile < ntile_o + ntile_c; ++tile) {
        int is_cmp = tile >= ntile_o;
        int r0 = is_cmp ? no + (tile - ntile_o) * SASG_TILE : tile * SASG_TILE;
        int rend = is_cmp ? no + nc : no;
        int n = rend - r0 < SASG_TILE ? rend - r0 : SASG_TILE;
        const void* pool = is_cmp ? cmp_kv : ori_kv;
        int bs = is_cmp ? p->cmp_block_size : p->ori_block_size;
        int64_t bstr = is_cmp ? p->cmp_block_stride : p->ori_block_stride;
        int64_t rstr = is_cmp ? p->cmp_row_stride : p->ori_row_stride;
        for (int j = 0; j < n; ++j) { /* gather the tile rows as fp32 (dequantised for fp8) */
          int64_t row = rows[r0 + j];
          float* kr = kt + (int64_t)j * D;
          if (row < 0) { memset(kr, 0, sizeof(float) * (size_t)D); continue; }
          int64_t base = (row / bs) * bstr + (row % bs) * rstr;
          float scl = 1.0f;
          if (p->kv_dtype == SASG_FP8E4M3) scl = (is_cmp ? cmp_scale : ori_scale)[row];
          for (int d = 0; d < D; ++d) {
            float v = load_elem(pool, p->kv_dtype, base + d);
            kr[d] = p->kv_dtype == SASG_FP8E4M3 ? v * scl : v;
          }
        }
        for (int h = 0; h < H; ++h) {
          const float* qh = qf + (int64_t)h * D;
          float* ah = acc + (int64_t)h * D;
          float tmax = -INFINITY;
          for (int j = 0; j < n; ++j) {
            const float* kr = kt + (int64_t)j * D;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qh[d] * kr[d];
            sc[j] = dot * p->softmax_scale;
            tmax = sc[j] > tmax ? sc[j] : tmax;
          }
          float m_old = rmax[h];
          float m_new = tmax > m_old ? tmax : m_old;
          float alpha = expf(m_old - m_new);
          float psum = 0.0f;
          for (int j = 0; j < n; ++j) {
            float pj = expf(sc[j] - m_new);
            psum += pj;
            sc[j] = round_to(pj, p->q_dtype);
          }
          rmax[h] = m_new;
          rsum[h] = alpha * rsum[h] + psum;
          for (int d = 0; d < D; ++d) ah[d] *= alpha;
          for (int j = 0; j < n; ++j) {
            const float* kr = kt + (int64_t)j * D;
            float pj = sc[j];
            for (int d = 0; d < D; ++d) ah[d] += pj * kr[d];
          }
        }
      }
      for (int h = 0; h < H; ++h) {
        for (int d = 0; d < Dv; ++d)
          ot[(int64_t)h * Dv + d] = round_to(acc[(int64_t)h * D + d] / rsum[h], p->q_dtype);
        lt[h] = rmax[h] + logf(rsum[h]);
      }
    }
    free(rows); free(kt); free(sc); free(qf); free(acc); free(rmax); free(rsum);
  }
  free(tb); free(ts);
  return err;
}

/* Mathematical reference for the accuracy check: the same resolved rows, the
 * one-shot sink softmax out = sum_j e^(x_j - m) V_j / (e^(sink - m) + sum_j
 * e^(x_j - m)) evaluated in double with no intermediate rounding (golden's
 * closed form golden.py:207-244 in float64).  Outputs are NOT rounded to the
 * query dtype.  Same argument list as sasg_attention. */
int sasg_attention_exact(const sasg_params* p, const void* q, const void* ori_kv,
                         const float* ori_scale, const int32_t* ori_bt, const void* cmp_kv,
                         const float* cmp_scale, const int32_t* cmp_bt, const int32_t* idx,
                         const int32_t* q_prefix, const int32_t* act_q, const int32_t* seqused_kv,
                         const float* sinks, const int32_t* tokens, int32_t n_tokens, float* out,
                         float* lse) {
  const int H = p->H, D = p->D, Dv = p->Dv;
  int32_t* tb = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  int32_t* ts = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  build_token_map(p, q_prefix, act_q, tb, ts);
  int nwork = tokens ? n_tokens : p->T;
  int need = max_rows_per_token(p, seqused_kv);
  int err = 0;
#ifdef _OPENMP
  if (p->nthreads > 0) omp_set_num_threads(p->nthreads);
#endif
#pragma omp parallel
  {
    int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * need);
    double* kv = (double*)malloc(sizeof(double) * (size_t)need * D);
    double* sc = (double*)malloc(sizeof(double) * (size_t)need);
    double* qh = (double*)malloc(sizeof(double) * (size_t)D);
    double* acc = (double*)malloc(sizeof(double) * (size_t)Dv);
#pragma omp for schedule(dynamic, 1)
    for (int w = 0; w < nwork; ++w) {
      int t = tokens ? tokens[w] : w;
      if (t < 0 || t >= p->T) continue;
      float* ot = out + (int64_t)t * H * Dv;
      float* lt = lse + (int64_t)t * H;
      memset(ot, 0, sizeof(float) * (size_t)H * Dv);
      memset(lt, 0, sizeof(float) * (size_t)H);
      if (tb[t] < 0) continue;
      int b = tb[t], no, nc;
      if (resolve_token(p, ori_bt, cmp_bt, idx, b, t, ts[t], act_q[b], seqused_kv[b], rows, &no,
                        &nc)) {
#pragma omp atomic write
        err = -1;
        continue;
      }
      int n = no + nc;
      for (int j = 0; j < n; ++j) {
        int is_cmp = j >= no;
        int64_t row = rows[j];
        double* kr = kv + (int64_t)j * D;
        if (row < 0) { for (int d = 0; d < D; ++d) kr[d] = 0.0; continue; }
        const void* pool = is_cmp ? cmp_kv : ori_kv;
        int bs = is_cmp ? p->cmp_block_size : p->ori_block_size;
        int64_t base = (row / bs) * (is_cmp ? p->cmp_block_stride : p->ori_block_stride) +
                       (row % bs) * (is_cmp ? p->cmp_row_stride : p->ori_row_stride);
        float scl = 1.0f;
        if (p->kv_dtype == SASG_FP8E4M3) scl = (is_cmp ? cmp_scale : ori_scale)[row];
        for (int d = 0; d < D; ++d) {
          float v = load_elem(pool, p->kv_dtype, base + d);
          kr[d] = p->kv_dtype == SASG_FP8E4M3 ? (double)(v * scl) : (double)v;
        }
      }
      for (int h = 0; h < H; ++h) {
        for (int d = 0; d < D; ++d) qh[d] = load_elem(q, p->q_dtype, ((int64_t)t * H + h) * D + d);
        double m = sinks[h];
        for (int j = 0; j < n; ++j) {
          const double* kr = kv + (int64_t)j * D;
          double dot = 0.0;
          for (int d = 0; d < D; ++d) dot += qh[d] * kr[d];
          sc[j] = dot * (double)p->softmax_scale;
          if (sc[j] > m) m = sc[j];
        }
        double l = isinf(sinks[h]) && sinks[h] < 0 ? 0.0 : exp((double)sinks[h] - m);
        for (int d = 0; d < Dv; ++d) acc[d] = 0.0;
        for (int j = 0; j < n; ++j) {
          double pj = exp(sc[j] - m);
          l += pj;
          const double* kr = kv + (int64_t)j * D;
          for (int d = 0; d < Dv; ++d) acc[d] += pj * kr[d];
        }
        for (int d = 0; d < Dv; ++d) ot[(int64_t)h * Dv + d] = (float)(acc[d] / l);
        lt[h] = (float)(m + log(l));
      }
    }
    free(rows); free(kv); free(sc); free(qh); free(acc);
  }
  free(tb); free(ts);
  return err;
}

/* Backward of the one-shot sink softmax over the same resolved rows, in double
 * (the reference has no backward; this is the gradient of sasg_attention_exact):
 * with P_j = e^(s_j - lse), out = sum_j P_j V_j, P_sink = e^(sink - lse),
 *   D = <dO, out>, dS_j = P_j (<dO, V_j> - D),
 *   dq = scale sum_j dS_j K_j, dsink = -sum_t P_sink D,
 *   dK_j += scale dS_j q, dV_j += P_j dO (both into the row's gradient).
 * dout [T, H, Dv] float; dq [T, H, D] float; dsinks [H] float; dori / dcmp
 * (float, the pools' shapes, zeroed by the caller) may be NULL.  Tokens listed
 * in `tokens` (all when NULL) are differentiated; the others' dq stays as given. */
int sasg_attention_bwd_exact(const sasg_params* p, const void* q, const void* ori_kv,
                             const float* ori_scale, const int32_t* ori_bt, const void* cmp_kv,
                             const float* cmp_scale, const int32_t* cmp_bt, const int32_t* idx,
                             const int32_t* q_prefix, const int32_t* act_q,
                             const int32_t* seqused_kv, const float* sinks, const float* dout,
                             const int32_t* tokens, int32_t n_tokens, float* dq, float* dsinks,
                             float* dori, float* dcmp) {
  const int H = p->H, D = p->D, Dv = p->Dv;
  int32_t* tb = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  int32_t* ts = (int32_t*)malloc(sizeof(int32_t) * (p->T > 0 ? p->T : 1));
  double* sterm = (double*)calloc((size_t)(p->T > 0 ? p->T : 1) * H, sizeof(double));
  build_token_map(p, q_prefix, act_q, tb, ts);
  int nwork = tokens ? n_tokens : p->T;
  int need = max_rows_per_token(p, seqused_kv);
  int err = 0;
#ifdef _OPENMP
  if (p->nthreads > 0) omp_set_num_threads(p->nthreads);
#endif
#pragma omp parallel
  {
    int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * need);
    int* is_cmp = (int*)malloc(sizeof(int) * need);
    double* kv = (double*)malloc(sizeof(double) * (size_t)need * D);
    double* sc = (double*)malloc(sizeof(double) * (size_t)need);
    double* qh = (double*)malloc(sizeof(double) * (size_t)D);
    double* oh = (double*)malloc(sizeof(double) * (size_t)Dv);
    double* gq = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int w = 0; w < nwork; ++w) {
      int t = tokens ? tokens[w] : w;
      if (t < 0 || t >= p->T) continue;
      float* dqt = dq + (int64_t)t * H * D;
      memset(dqt, 0, sizeof(float) * (size_t)H * D);
      if (tb[t] < 0) continue;
      int b = tb[t], no, nc;
      if (resolve_token(p, ori_bt, cmp_bt, idx, b, t, ts[t], act_q[b], seqused_kv[b], rows, &no,
                        &nc)) {
#pragma omp atomic write
        err = -1;
        continue;
      }
      int n = no + nc;
      for (int j = 0; j < n; ++j) {
        is_cmp[j] = j >= no;
        int64_t row = rows[j];
        double* kr = kv + (int64_t)j * D;
        if (row < 0) { for (int d = 0; d < D; ++d) kr[d] = 0.0; continue; }
        const void* pool = is_cmp[j] ? cmp_kv : ori_kv;
        int bs = is_cmp[j] ? p->cmp_block_size : p->ori_block_size;
        int64_t base = (row / bs) * (is_cmp[j] ? p->cmp_block_stride : p->ori_block_stride) +
                       (row % bs) * (is_cmp[j] ? p->cmp_row_stride : p->ori_row_stride);
        float scl = 1.0f;
        if (p->kv_dtype == SASG_FP8E4M3) scl = (is_cmp[j] ? cmp_scale : ori_scale)[row];
        for (int d = 0; d < D; ++d) {
          float v = load_elem(pool, p->kv_dtype, base + d);
          kr[d] = p->kv_dtype == SASG_FP8E4M3 ? (double)(v * scl) : (double)v;
        }
      }
      for (int h = 0; h < H; ++h) {
        for (int d = 0; d < D; ++d) qh[d] = load_elem(q, p->q_dtype, ((int64_t)t * H + h) * D + d);
        const float* doh = dout + ((int64_t)t * H + h) * Dv;
        double m = sinks[h];
        for (int j = 0; j < n; ++j) {
          const double* kr = kv + (int64_t)j * D;
          double dot = 0.0;
          for (int d = 0; d < D; ++d) dot += qh[d] * kr[d];
          sc[j] = dot * (double)p->softmax_scale;
          if (sc[j] > m) m = sc[j];
        }
        if (isinf(m) && m < 0) m = 0.0; /* a head with nothing to attend: all zero */
        double es = isinf(sinks[h]) && sinks[h] < 0 ? 0.0 : exp((double)sinks[h] - m);
        double l = es;
        for (int j = 0; j < n; ++j) { sc[j] = exp(sc[j] - m); l += sc[j]; }
        if (l <= 0.0) l = 1.0;
        for (int d = 0; d < Dv; ++d) oh[d] = 0.0;
        for (int j = 0; j < n; ++j) {
          sc[j] /= l; /* P_j */
          const double* kr = kv + (int64_t)j * D;
          for (int d = 0; d < Dv; ++d) oh[d] += sc[j] * kr[d];
        }
        double Dh = 0.0;
        for (int d = 0; d < Dv; ++d) Dh += (double)doh[d] * oh[d];
        sterm[(int64_t)t * H + h] = -(es / l) * Dh;
        for (int d = 0; d < D; ++d) gq[d] = 0.0;
        for (int j = 0; j < n; ++j) {
          const double* kr = kv + (int64_t)j * D;
          double dp = 0.0;
          for (int d = 0; d < Dv; ++d) dp += (double)doh[d] * kr[d];
          double ds = sc[j] * (dp - Dh);
          for (int d = 0; d < D; ++d) gq[d] += ds * kr[d];
          float* grad = is_cmp[j] ? dcmp : dori;
          if (grad && rows[j] >= 0) {
            int bs = is_cmp[j] ? p->cmp_block_size : p->ori_block_size;
            int64_t gb = (rows[j] / bs) * (int64_t)bs * D + (rows[j] % bs) * (int64_t)D;
            for (int d = 0; d < D; ++d) {
              double g = (double)p->softmax_scale * ds * qh[d] + (d < Dv ? sc[j] * doh[d] : 0.0);
#pragma omp atomic
              grad[gb + d] += (float)g;
            }
          }
        }
        for (int d = 0; d < D; ++d) dqt[(int64_t)h * D + d] = (float)((double)p->softmax_scale * gq[d]);
      }
    }
    free(rows); free(is_cmp); free(kv); free(sc); free(qh); free(oh); free(gq);
  }
  for (int h = 0; h < H; ++h) {
    double acc = 0.0;
    for (int t = 0; t < p->T; ++t) acc += sterm[(int64_t)t * H + h];
    dsinks[h] = (float)acc;
  }
  free(tb); free(ts); free(sterm);
  return err;
}

/* Test hook: the oracle's own rounding of n floats to the dtype dt (SASG_BF16 or
 * SASG_F16; other codes copy), so its rounding can be checked against a library. */
int sasg_round(int dt, const float* x, float* y, int64_t n) {
  if (!x || !y || n < 0) return -1;
  for (int64_t i = 0; i < n; ++i) y[i] = round_to(x[i], dt);
  return 0;
}

int sasg_version(void) { return 1; }
