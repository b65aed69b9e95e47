// sas_kernels.hip -- gfx950 kernels of the sparse shared-KV attention path.
//
//   plan_kernel     split-KV scheduler: per-token row spans (window + compressed)
//                   and work units balanced over the CUs; replaces the reference
//                   scheduler metadata.py:1018-1086 with a GPU pass that needs
//                   only the per-batch lengths.
//   resolve_kernel  compressed top-k index resolution (reference golden.py:28-66):
//                   examine the first min(K, thr) slots, -1 terminates, ids >= thr
//                   are skipped, survivors are compacted in slot order and mapped
//                   through the paged block table to pool rows.
//   fwd_kernel      per work unit: gather paged KV rows into LDS, S^T = K Q^T and
//                   O^T += V^T P^T on bf16/fp16 MFMA (32x32x16) with fp32
//                   accumulation, one sink-seeded online softmax across the window
//                   and compressed rows (golden.py:156-200); writes the final
//                   output or an un-normalised split partial (O, m, l).
//   combine_kernel  log-sum-exp merge of split partials.
//
// Work decomposition: one work unit = (token, contiguous range of its row list);
// the row list of a token is its window rows (raw KV pool) followed by its
// compressed rows (compressed KV pool).  All heads of the token are processed by
// one workgroup (heads x keys MFMA tiles, 32 heads per wave), so each KV row is
// read from HBM once per token.
#include <hip/hip_runtime.h>

#include "sas_common.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

namespace sas {

__device__ __forceinline__ int floor_div(int a, int b) {
  int q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

// ===========================================================================
// Planner
// ===========================================================================
struct TokInfo {
  int b, s, sg, nwin, winlo, ncmpmax;
};

// Token -> (batch, local position) through q_prefix / act_q: the owning batch is
// the last b with q_prefix[b] <= t (equal prefixes only occur for empty batches,
// which precede the batch that owns the tokens).
__device__ TokInfo token_info(const SasPlanArgs& a, const int* __restrict__ q_prefix,
                              const int* __restrict__ act_q, const int* __restrict__ seqused_kv,
                              int t) {
  TokInfo ti{-1, 0, 0, 0, 0, 0};
  int lo = 0, hi = a.B - 1, b = -1;
  while (lo <= hi) {
    int mid = (lo + hi) >> 1;
    if (q_prefix[mid] <= t) {
      b = mid;
      lo = mid + 1;
    } else {
      hi = mid - 1;
    }
  }
  if (b < 0) return ti;
  int s = t - q_prefix[b];
  int aq = act_q[b];
  if (s >= aq) return ti;
  int sg = seqused_kv[b] - aq + s;                    // golden.py:125
  int winlo = max(sg - a.win_left, 0);                // golden.py:130
  int nwin = max(sg + 1 - winlo, 0);                  // golden.py:129-131
  int ncmp = 0;
  if (a.scenario >= 2) {
    int thr = floor_div(sg + 1, a.cmp_ratio);         // golden.py:44, 147
    ncmp = a.K > 0 ? min(a.K, thr) : thr;             // golden.py:48 / 148 (list capacity)
    ncmp = max(ncmp, 0);
  }
  ti.b = b;
  ti.s = s;
  ti.sg = sg;
  ti.nwin = nwin;
  ti.winlo = winlo;
  ti.ncmpmax = ncmp;
  return ti;
}

constexpr int PLAN_NT = 1024;

__global__ __launch_bounds__(PLAN_NT) void plan_kernel(SasPlanArgs a,
                                                       const int* __restrict__ q_prefix,
                                                       const int* __restrict__ act_q,
                                                       const int* __restrict__ seqused_kv,
                                                       int* __restrict__ plan) {
  __shared__ long long red[PLAN_NT];
  __shared__ int scan_u[PLAN_NT], scan_s[PLAN_NT], scan_k[PLAN_NT];
  const int tid = threadIdx.x;
  const SasPlanLayout L = sas_plan_layout(a.T, a.target);
  int* tok = plan + L.off_tok;
  int* units = plan + L.off_units;
  int* stoks = plan + L.off_split_tokens;
  const int per = (a.T + PLAN_NT - 1) / PLAN_NT;
  const int t0 = min(a.T, tid * per), t1 = min(a.T, t0 + per);

  long long my_rows = 0;
  for (int t = t0; t < t1; ++t) {
    TokInfo ti = token_info(a, q_prefix, act_q, seqused_kv, t);
    int* r = tok + (size_t)t * SAS_TOK_W;
    r[TK_B] = ti.b;
    r[TK_S] = ti.s;
    r[TK_SG] = ti.sg;
    r[TK_NWIN] = ti.nwin;
    r[TK_WINLO] = ti.winlo;
    r[TK_NCMPMAX] = ti.ncmpmax;
    if (ti.b >= 0) my_rows += ti.nwin + ti.ncmpmax;
  }
  red[tid] = my_rows;
  __syncthreads();
  for (int off = PLAN_NT / 2; off > 0; off >>= 1) {
    if (tid < off) red[tid] += red[tid + off];
    __syncthreads();
  }
  const long long R = red[0];
  long long chunk = (R + a.target - 1) / a.target;
  if (chunk < SAS_MIN_CHUNK) chunk = SAS_MIN_CHUNK;
  chunk = (chunk + SAS_TILE - 1) / SAS_TILE * SAS_TILE;

  int my_u = 0, my_s = 0, my_k = 0;
  for (int t = t0; t < t1; ++t) {
    const int* r = tok + (size_t)t * SAS_TOK_W;
    long long rows = r[TK_B] >= 0 ? (long long)r[TK_NWIN] + r[TK_NCMPMAX] : 0;
    int splits = rows > chunk ? (int)((rows + chunk - 1) / chunk) : 1;
    my_u += splits;
    if (splits > 1) {
      my_s += splits;
      my_k += 1;
    }
  }
  scan_u[tid] = my_u;
  scan_s[tid] = my_s;
  scan_k[tid] = my_k;
  __syncthreads();
  for (int off = 1; off < PLAN_NT; off <<= 1) {  // inclusive Hillis-Steele scan
    int vu = 0, vs = 0, vk = 0;
    if (tid >= off) {
      vu = scan_u[tid - off];
      vs = scan_s[tid - off];
      vk = scan_k[tid - off];
    }
    __syncthreads();
    scan_u[tid] += vu;
    scan_s[tid] += vs;
    scan_k[tid] += vk;
    __syncthreads();
  }
  const int U = scan_u[PLAN_NT - 1];
  int ub = scan_u[tid] - my_u, sb = scan_s[tid] - my_s, kb = scan_k[tid] - my_k;
  for (int t = t0; t < t1; ++t) {
    int* r = tok + (size_t)t * SAS_TOK_W;
    const int b = r[TK_B];
    const long long rows = b >= 0 ? (long long)r[TK_NWIN] + r[TK_NCMPMAX] : 0;
    const int splits = rows > chunk ? (int)((rows + chunk - 1) / chunk) : 1;
    r[TK_SPLITS] = splits;
    r[TK_WSBASE] = splits > 1 ? sb : -1;
    long long ct = rows;
    if (splits > 1) ct = ((rows + splits - 1) / splits + SAS_TILE - 1) / SAS_TILE * SAS_TILE;
    for (int i = 0; i < splits; ++i) {
      // units are emitted in reverse order so the longest (latest prefill) tokens start first
      int* ur = units + (size_t)(U - 1 - (ub + i)) * SAS_UNIT_W;
      long long r0 = (long long)i * ct, r1 = r0 + ct < rows ? r0 + ct : rows;
      ur[0] = t;
      ur[1] = (int)r0;
      ur[2] = (int)r1;
      ur[3] = b >= 0 ? i : -1;
    }
    ub += splits;
    if (splits > 1) {
      stoks[kb++] = t;
      sb += splits;
    }
  }
  if (tid == 0) {
    plan[PH_MAGIC] = SAS_PLAN_MAGIC;
    plan[PH_VERSION] = SAS_PLAN_VERSION;
    plan[PH_T] = a.T;
    plan[PH_UNITS] = U;
    plan[PH_CHUNK] = (int)chunk;
    plan[PH_TARGET] = a.target;
    plan[PH_NSPLIT_TOKENS] = scan_k[PLAN_NT - 1];
    plan[PH_NSLOTS] = scan_s[PLAN_NT - 1];
    plan[PH_TOTAL_ROWS_LO] = (int)(R & 0xffffffff);
    plan[PH_TOTAL_ROWS_HI] = (int)(R >> 32);
    plan[PH_H] = a.H;
    plan[PH_UNIT_CAP] = (int)L.unit_cap;
    plan[PH_SCENARIO] = a.scenario;
    plan[PH_K] = a.K;
  }
}

// ===========================================================================
// Row resolution.  Writes each token's row-code list: the
// window rows (golden.py:129-131, paged as golden.py:247-268) and, in scenario 3,
// the resolved compressed rows (golden.py:28-66).  A code is a flat pool row
// (page * block_size + offset) or -1 for a row the reference reads as zeros
// (unused page).  Window codes index the raw pool, later codes the compressed pool.
// ===========================================================================
// The row every -1 code reads (zeros).
__device__ __attribute__((aligned(16))) uint8_t g_zero_row[1152] = {};

// Pool address of a row code (-1: the shared zero row).
__device__ __forceinline__ uint64_t code_addr(int code, const uint8_t* pool, int block_size,
                                              int64_t block_stride, int64_t row_stride, int esz) {
  if (code < 0) return (uint64_t)g_zero_row;
  const int page = code / block_size, off = code - page * block_size;
  return (uint64_t)(pool + ((size_t)page * block_stride + (size_t)off * row_stride) * esz);
}

__device__ __forceinline__ int paged_code(const int* __restrict__ bt_row, int table_len,
                                          int block_size, int block_num, int pos) {
  const int blk = pos / block_size;
  const int page = blk < table_len ? bt_row[blk] : -1;
  return (page < 0 || page >= block_num) ? -1 : page * block_size + (pos - blk * block_size);
}

// One workgroup (256 threads) per token.  Thread i owns index slots
// [RS_PER i, RS_PER (i + 1)) of the first min(K, thr) slots; the first -1 (a
// block-wide minimum) ends the list, ids outside [0, thr) are skipped, and the
// survivors keep their slot order through a block-wide exclusive scan.
constexpr int RS_NT = 256;
constexpr int RS_PER = 8;  // index slots per thread and chunk

constexpr int RS_CBT_LDS = 4096;  // compressed block-table entries staged in LDS

__global__ __launch_bounds__(RS_NT) void resolve_kernel(SasFwdArgs a, const int* __restrict__ plan,
                                                        const int* __restrict__ ori_bt,
                                                        const int* __restrict__ idx,
                                                        const int* __restrict__ cmp_bt,
                                                        int* __restrict__ rows_out,
                                                        int* __restrict__ ncmp_out,
                                                        uint64_t* __restrict__ addr_out,
                                                        const uint8_t* __restrict__ ori_kv,
                                                        const uint8_t* __restrict__ cmp_kv,
                                                        int esz) {
  __shared__ int s_wmin[RS_NT / 64];
  __shared__ int s_wsum[RS_NT / 64];
  __shared__ int s_cbt[RS_CBT_LDS];
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int* ir = idx + (size_t)t * a.K;
  const bool vec = (a.K & 3) == 0;  // index rows are 16-B aligned
  // Index slots [s0, s0 + RS_PER) below `bound`, all loaded before any is used
  // (-2: past the bound).
  auto load_slots = [&](int (&v)[RS_PER], int s0, int bound) {
    if (vec && s0 + RS_PER <= bound) {
#pragma unroll
      for (int k = 0; k < RS_PER; k += 4) {
        const int4 x = *reinterpret_cast<const int4*>(ir + s0 + k);
        v[k] = x.x;
        v[k + 1] = x.y;
        v[k + 2] = x.z;
        v[k + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < RS_PER; ++k) v[k] = s0 + k < bound ? ir[s0 + k] : -2;
    }
  };
  // First memory round trip: the token's plan record and, independent of it, the
  // first pass of its index slots.
  int v0[RS_PER];
  if (a.scenario == 3) load_slots(v0, tid * RS_PER, a.K);
  const int* tk = plan + SAS_PLAN_HDR + (size_t)t * SAS_TOK_W;
  const int b = tk[TK_B];
  if (b < 0) {
    if (tid == 0) ncmp_out[t] = 0;
    return;
  }
  int* out = rows_out + (size_t)t * a.list_stride;
  uint64_t* aout = addr_out + (size_t)t * a.list_stride;
  const int nwin = tk[TK_NWIN], winlo = tk[TK_WINLO];
  // Second: the window's block-table entries and the batch's compressed block-table
  // row, staged in LDS so the per-id page lookups below stay on chip.
  const int* cbt_g = cmp_bt + (size_t)b * a.cmp_table_len;
  const bool cbt_lds = a.scenario >= 2 && a.cmp_table_len <= RS_CBT_LDS;
  if (cbt_lds)
    for (int i = tid; i < a.cmp_table_len; i += RS_NT) s_cbt[i] = cbt_g[i];
  const int* obt = ori_bt + (size_t)b * a.ori_table_len;
  for (int r = tid; r < nwin; r += RS_NT) {
    const int code = paged_code(obt, a.ori_table_len, a.ori_block_size, a.ori_block_num, winlo + r);
    out[r] = code;
    aout[r] = code_addr(code, ori_kv, a.ori_block_size, a.ori_block_stride, a.ori_row_stride, esz);
  }
  aout += nwin;
  if (a.scenario == 1) {
    if (tid == 0) ncmp_out[t] = 0;
    return;
  }
  __syncthreads();  // s_cbt
  const int* cbt = cbt_lds ? s_cbt : cbt_g;
  out += nwin;  // compressed codes follow the window codes
  const int thr = floor_div(tk[TK_SG] + 1, a.cmp_ratio);
  if (a.scenario == 2) {  // golden.py:146-150: every compressed row below thr
    const int n = max(min(thr, a.K), 0);
    for (int j = tid; j < n; j += RS_NT) {
      const int code = paged_code(cbt, a.cmp_table_len, a.cmp_block_size, a.cmp_block_num, j);
      out[j] = code;
      aout[j] = code_addr(code, cmp_kv, a.cmp_block_size, a.cmp_block_stride, a.cmp_row_stride, esz);
    }
    if (tid == 0) ncmp_out[t] = n;
    return;
  }
  const int limit = max(min(a.K, thr), 0);  // golden.py:48
  // Passes of RS_NT * RS_PER slots; thread tid owns slots [RS_PER tid, RS_PER (tid + 1))
  // of a pass; the terminator, the survivors and their slot-order positions come
  // from block-wide reductions over registers.
  int emitted = 0;  // compressed rows written so far (block-uniform)
  for (int c0 = 0; c0 < limit; c0 += RS_NT * RS_PER) {
    const int s0 = c0 + tid * RS_PER;
    int v[RS_PER];
    if (c0 == 0) {
#pragma unroll
      for (int k = 0; k < RS_PER; ++k) v[k] = s0 + k < limit ? v0[k] : -2;
    } else {
      load_slots(v, s0, limit);
    }
    // golden.py:52-53: the first -1 terminates the list
    int first = limit;
#pragma unroll
    for (int k = RS_PER - 1; k >= 0; --k)
      if (v[k] == -1) first = s0 + k;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) first = min(first, __shfl_xor(first, off));
    if (lane == 0) s_wmin[w] = first;
    __syncthreads();
    int term = s_wmin[0];
#pragma unroll
    for (int j = 1; j < RS_NT / 64; ++j) term = min(term, s_wmin[j]);
    // golden.py:58-59: ids at or beyond thr are skipped (other negatives too)
    int cnt = 0;
    unsigned keep = 0;
#pragma unroll
    for (int k = 0; k < RS_PER; ++k)
      if (s0 + k < term && v[k] >= 0 && v[k] < thr) {
        keep |= 1u << k;
        ++cnt;
      }
    // block-wide exclusive scan of cnt: survivors keep their slot order
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int x = __shfl_up(incl, off);
      if (lane >= off) incl += x;
    }
    if (lane == 63) s_wsum[w] = incl;
    __syncthreads();
    int pos = emitted + incl - cnt, total = 0;
#pragma unroll
    for (int j = 0; j < RS_NT / 64; ++j) {
      if (j < w) pos += s_wsum[j];
      total += s_wsum[j];
    }
#pragma unroll
    for (int k = 0; k < RS_PER; ++k)
      if ((keep >> k) & 1u) {
        const int code = paged_code(cbt, a.cmp_table_len, a.cmp_block_size, a.cmp_block_num, v[k]);
        out[pos] = code;
        aout[pos++] = code_addr(code, cmp_kv, a.cmp_block_size, a.cmp_block_stride, a.cmp_row_stride, esz);
      }
    emitted += total;
    if (term < limit) break;  // the list ended in this pass
    __syncthreads();          // s_wmin / s_wsum are rewritten by the next pass
  }
  if (tid == 0) ncmp_out[t] = emitted;
}

// ===========================================================================
// Attention
// ===========================================================================
template <int QT>
__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (QT == 0)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// float -> 16-bit payload of the query dtype, round to nearest even.
template <int QT>
__device__ __forceinline__ uint32_t to_q16(float x) {
  if constexpr (QT == 0)
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
  else
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// Two floats -> two 16-bit values of the query dtype (round to nearest even),
// packed low = a, high = b: one v_cvt_pk_bf16_f32 for bf16.
template <int QT>
__device__ __forceinline__ uint32_t pack2_q16(float a, float b) {
  if constexpr (QT == 0) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, b2{(__bf16)a, (__bf16)b});
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, h2{(_Float16)a, (_Float16)b});
  }
}

// 16-bit payload of the query dtype -> float (exact).
template <int QT>
__device__ __forceinline__ float q16_to_f32(uint32_t v) {
  if constexpr (QT == 0)
    return __uint_as_float(v << 16);
  else
    return (float)__builtin_bit_cast(_Float16, (uint16_t)v);
}

// acc + the two 16-bit values packed in v (exact products with 1, fp32 sum).
template <int QT>
__device__ __forceinline__ float sum2_q16(uint32_t v, float acc) {
  if constexpr (QT == 0) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 one = {(__bf16)1.f, (__bf16)1.f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, v), one, acc, false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 one = {(_Float16)1.f, (_Float16)1.f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v), one, acc, false);
  }
}

// ===========================================================================
// Split-KV merge (log-sum-exp) of one (token, head): lane l merges columns
// [8 l, 8 l + 8) of the d_v = 512 partial outputs.  A partial holds O and its two
// normalisers (l_w: sum of the rounded P that entered O, for the output; l_e: sum
// of the exact P, for the LSE) in its own frame m; the merge rescales each by
// 2^(m_s - max_s m_s).  Only split 0 carries the sink, so it enters once.
// ===========================================================================
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// Log-sum-exp merge of the S split partials of head h of token t (partial slots
// base .., each an un-normalised O row with its (m, l_w, l_e)), by one wave: lane
// l owns d = 8 l .. 8 l + 7.  The partial records are read 64 at a time (lane j
// holds record j of a chunk), and partial rows are loaded 8 at a time before any
// is accumulated, so a merge costs a few memory round trips for any S.
constexpr int COMBINE_BATCH = 8;

template <int QT>
__device__ __forceinline__ void combine_head(int t, int h, int H, int S, int base,
                                             const float* __restrict__ ws_o,
                                             const float* __restrict__ ws_ml,
                                             uint16_t* __restrict__ out, float* __restrict__ lse) {
  constexpr int DV = 512;
  const int lane = threadIdx.x & 63;
  const float4* ml = reinterpret_cast<const float4*>(ws_ml);
  auto record = [&](int s0) {
    return s0 + lane < S ? ml[(size_t)(base + s0 + lane) * H + h] : make_float4(-INFINITY, 0.f, 0.f, 0.f);
  };
  const float4 rec0 = record(0);
  float mx = rec0.x;
  for (int s0 = 64; s0 < S; s0 += 64) mx = fmaxf(mx, record(s0).x);
  mx = wave_max(mx);  // the merged frame
  float l = 0.f, le = 0.f;
  float4 o0 = make_float4(0.f, 0.f, 0.f, 0.f), o1 = o0;
  for (int s0 = 0; s0 < S; s0 += 64) {
    const float4 rec = s0 == 0 ? rec0 : record(s0);
    const float wgt = rec.x == -INFINITY ? 0.f : exp2f(rec.x - mx);
    l += wgt * rec.y;
    le += wgt * rec.z;
    const int n = min(64, S - s0);
    for (int j0 = 0; j0 < n; j0 += COMBINE_BATCH) {
      float4 v[COMBINE_BATCH][2];
#pragma unroll
      for (int j = 0; j < COMBINE_BATCH; ++j) {
        const int jj = min(j0 + j, n - 1);
        const float4* src =
            reinterpret_cast<const float4*>(ws_o + ((size_t)(base + s0 + jj) * H + h) * DV) + 2 * lane;
        v[j][0] = src[0];
        v[j][1] = src[1];
      }
#pragma unroll
      for (int j = 0; j < COMBINE_BATCH; ++j) {
        if (j0 + j >= n) break;
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j0 + j));
        o0.x += w * v[j][0].x; o0.y += w * v[j][0].y; o0.z += w * v[j][0].z; o0.w += w * v[j][0].w;
        o1.x += w * v[j][1].x; o1.y += w * v[j][1].y; o1.z += w * v[j][1].z; o1.w += w * v[j][1].w;
      }
    }
  }
  l = wave_sum(l);
  le = wave_sum(le);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  u32x4_t o;
  o[0] = to_q16<QT>(o0.x * inv) | (to_q16<QT>(o0.y * inv) << 16);
  o[1] = to_q16<QT>(o0.z * inv) | (to_q16<QT>(o0.w * inv) << 16);
  o[2] = to_q16<QT>(o1.x * inv) | (to_q16<QT>(o1.y * inv) << 16);
  o[3] = to_q16<QT>(o1.z * inv) | (to_q16<QT>(o1.w * inv) << 16);
  reinterpret_cast<u32x4_t*>(out + ((size_t)t * H + h) * DV)[lane] = o;
  if (lse && lane == 0) lse[(size_t)t * H + h] = (mx + __log2f(le)) * 0.6931471805599453f;
}

// OCP FP8 E4M3FN code -> exact 16-bit value of the query dtype.
template <int QT>
__device__ __forceinline__ uint32_t fp8_to_q16(uint32_t v) {
  const uint32_t e = (v >> 3) & 15u, m = v & 7u;
  const uint32_t s = (v & 0x80u) << 8;
  if constexpr (QT == 0) {
    if (e == 15u && m == 7u) return s | 0x7FC0u;
    if (e == 0u) return m == 0u ? s : (s | (__float_as_uint((float)m * 0.001953125f) >> 16));
    return s | ((e + 120u) << 7) | (m << 4);
  } else {
    if (e == 15u && m == 7u) return s | 0x7E00u;
    if (e == 0u)
      return m == 0u ? s
                     : (s | (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((float)m * 0.001953125f)));
    return s | ((e + 8u) << 10) | (m << 7);
  }
}

// Source of rows that read as zeros (unused pages, tile padding).


// Online softmax (golden.py:184-196): m_run is the running maximum of the sink
// and every logit seen so far; a tile whose maximum exceeds it rescales O and l
// by 2^(m_old - m_new) before P = 2^(x - m_run) is formed, so P <= 1 and the
// row holding the maximum gets P = 1 exactly, as in the reference.  The rescale
// runs only when some head of the wave saw a larger maximum.
constexpr float LOG2E = 1.4426950408889634f;

template <int NW, int DQK, int QT, bool KV8>
__global__ __launch_bounds__(256, 1) void fwd_kernel(
    SasFwdArgs a, const uint16_t* __restrict__ q, const uint8_t* __restrict__ ori_kv,
    const uint8_t* __restrict__ cmp_kv, const float* __restrict__ ori_scale,
    const float* __restrict__ cmp_scale, const int* __restrict__ ori_bt,
    const int* __restrict__ cmp_bt, const int* __restrict__ rows_list,
    const int* __restrict__ ncmp, const float* __restrict__ sinks, const int* __restrict__ plan,
    uint16_t* __restrict__ out, float* __restrict__ lse, float* __restrict__ ws_o,
    float* __restrict__ ws_ml) {
  constexpr int DV = 512;
  constexpr int NT = 256;
  constexpr int ROWB = DQK * 2;          // LDS row bytes (16-bit elements)
  constexpr int CPR = ROWB / 16;         // 16-B chunks per LDS row: 72 / 64
  constexpr int KSTEPS = DQK / 16;       // MFMA k-steps of Q K^T
  constexpr int TILEB = SAS_TILE * ROWB;
  constexpr int NBUF = KV8 ? 1 : 2;      // DMA path double-buffers; fp8 stages through VGPRs
  constexpr int ESZ = KV8 ? 1 : 2;       // source element bytes
  constexpr int CPT = SAS_TILE * CPR / NT;  // DMA chunks per thread per tile (9 / 8)
  static_assert(SAS_TILE * CPR % NT == 0, "tile must split evenly over the workgroup");
  constexpr int SRC_CPR8 = DQK / 16;     // fp8: 16-B source chunks per row (36 / 32)
  constexpr int CPT8 = (SAS_TILE * SRC_CPR8 + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) uint8_t tiles[NBUF * TILEB];
  __shared__ const uint8_t* rowaddr[2][SAS_TILE];
  __shared__ float rowscale[SAS_TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 5;   // half-wave: selects the k-chunk / key quad
  const int li = lane & 31;  // MFMA row/column index within the 32-wide tile

  const int u = blockIdx.x;
  if (plan[PH_MAGIC] != SAS_PLAN_MAGIC || u >= plan[PH_UNITS]) return;
  const int* ur = plan + SAS_PLAN_HDR + (size_t)SAS_TOK_W * a.T + (size_t)u * SAS_UNIT_W;
  const int t = ur[0], split = ur[3];
  const int H = a.H;

  if (split < 0) {  // a q row no batch owns: zeros, as the reference's padded slots
    for (int i = tid; i < H * DV / 8; i += NT)
      reinterpret_cast<u32x4_t*>(out + (size_t)t * H * DV)[i] = u32x4_t{0, 0, 0, 0};
    if (lse)
      for (int i = tid; i < H; i += NT) lse[(size_t)t * H + i] = 0.f;
    return;
  }

  const int* tk = plan + SAS_PLAN_HDR + (size_t)t * SAS_TOK_W;
  const int nwin = tk[TK_NWIN];
  const int splits = tk[TK_SPLITS], wsbase = tk[TK_WSBASE];
  const int r0 = ur[1];
  const int r1 = min(ur[2], nwin + ncmp[t]);
  const int ntiles = r1 > r0 ? (r1 - r0 + SAS_TILE - 1) / SAS_TILE : 0;
  const int* codes = rows_list + (size_t)t * a.list_stride;

  // Row code of list row r (-1 = zero row); window rows first, then compressed rows.
  auto row_code = [&](int r) -> int { return r < r1 ? codes[r] : -1; };
  auto row_ptr = [&](int r, int code) -> const uint8_t* {
    if (code < 0) return g_zero_row;
    if (r < nwin) {
      const int page = code / a.ori_block_size, off = code - page * a.ori_block_size;
      return ori_kv + ((size_t)page * a.ori_block_stride + (size_t)off * a.ori_row_stride) * ESZ;
    }
    const int page = code / a.cmp_block_size, off = code - page * a.cmp_block_size;
    return cmp_kv + ((size_t)page * a.cmp_block_stride + (size_t)off * a.cmp_row_stride) * ESZ;
  };
  auto row_scale = [&](int r, int code) -> float {
    if (code < 0) return 0.f;
    return r < nwin ? ori_scale[code] : cmp_scale[code];
  };

  // ---- LDS addressing ----
  // Row-major tile; 16-B chunk c of row r lives at chunk (c ^ (r & 7)) of that row,
  // so each ds_read_b128 phase (8 lanes) and ds_read_b32 phase (32 lanes) hits
  // distinct banks.  Every operand read is a per-lane base plus a constant:
  //  * K, k-step ks: row li, chunk 2 ks + g            = kbase[ks & 3] + 128 (ks >> 2)
  //  * V^T, block pair mm, k-step kk, element e: row 16 kk + 8 (e >> 2) + 4 g + (e & 3),
  //    dword 32 mm + li                                 = vbase[e & 3] + (16 kk + 8 (e >> 2)) ROWB + 128 mm
  uint32_t kbase[4], vbase[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kbase[j] = li * ROWB + (((2 * j + g) ^ (li & 7)) * 16);
    vbase[j] = (4 * g + j) * ROWB + 16 * ((li >> 2) ^ (4 * g + j)) + 4 * (li & 3);
  }

  // ---- per-wave state: 32 heads per wave ----
  // Every wave computes (no divergence around the register tiles); head indices
  // past H (and waves past NW) are clamped onto valid heads and never stored.
  const int h = w * 32 + li;
  const bool hvalid = (w < NW) && (h < H);
  const int hc = min(h, H - 1);
  u32x4_t qf[KSTEPS];
  {
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(q + ((size_t)t * H + hc) * DQK);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[ks] = qrow[2 * ks + g];
  }
  const float sink2 = split == 0 ? sinks[hc] * LOG2E : -INFINITY;  // golden.py:162-163
  f32x16_t acc[16];
  float m_run = sink2, l_run = split == 0 ? 1.f : 0.f;  // golden.py:162-163

  // fp8: 16 source bytes -> two 16-bit chunks written to the (single) tile
  auto fp8_stage = [&](int it) {
    u32x4_t st[CPT8];
#pragma unroll
    for (int k = 0; k < CPT8; ++k) {
      const int c = tid + k * NT;
      const int cc = c < SAS_TILE * SRC_CPR8 ? c : 0;
      const int row = cc / SRC_CPR8, chk = cc - row * SRC_CPR8;
      st[k] = *reinterpret_cast<const u32x4_t*>(rowaddr[it & 1][row] + chk * 16);
    }
#pragma unroll
    for (int k = 0; k < CPT8; ++k) {
      const int c = tid + k * NT;
      if (c < SAS_TILE * SRC_CPR8) {
        const int row = c / SRC_CPR8, chk = c - row * SRC_CPR8;
#pragma unroll
        for (int hlf = 0; hlf < 2; ++hlf) {
          const uint32_t w0 = st[k][2 * hlf], w1 = st[k][2 * hlf + 1];
          u32x4_t o;
          o[0] = fp8_to_q16<QT>(w0 & 0xff) | (fp8_to_q16<QT>((w0 >> 8) & 0xff) << 16);
          o[1] = fp8_to_q16<QT>((w0 >> 16) & 0xff) | (fp8_to_q16<QT>(w0 >> 24) << 16);
          o[2] = fp8_to_q16<QT>(w1 & 0xff) | (fp8_to_q16<QT>((w1 >> 8) & 0xff) << 16);
          o[3] = fp8_to_q16<QT>((w1 >> 16) & 0xff) | (fp8_to_q16<QT>(w1 >> 24) << 16);
          const int ch = 2 * chk + hlf;
          *reinterpret_cast<u32x4_t*>(tiles + row * ROWB + ((ch ^ (row & 7)) * 16)) = o;
        }
      }
    }
  };
  // 16-bit KV: each lane DMAs 16 B of the tile straight into LDS.  Wave w's k-th
  // instruction fills LDS chunk slots [(4k + w) * 64, +64): slot s holds chunk
  // (s % CPR) ^ (row & 7) of row s / CPR.
  auto dma_tile = [&](int buf, int slot) {
    uint8_t* dst0 = tiles + buf * TILEB;
    // Recomputed per tile (an opaque copy of the lane id stops the compiler from
    // hoisting 2 x CPT loop-invariant VGPRs out of the tile loop).
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = (4 * k + w) * 64 + lane_v;
      const int row = s / CPR, pc = s - row * CPR;
      const uint8_t* src = rowaddr[slot][row] + ((pc ^ (row & 7)) * 16);
      __builtin_amdgcn_global_load_lds(
          (const void*)src,
          (__attribute__((address_space(3))) void*)(dst0 + (4 * k + w) * 64 * 16), 16, 0, 0);
    }
  };

  {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = f32x16_t{};

    // prologue: addresses of tiles 0 and 1; DMA of tile 0
    if (tid < SAS_TILE) {
      for (int j = 0; j < 2; ++j) {
        const int r = r0 + j * SAS_TILE + tid;
        const int code = row_code(r);
        rowaddr[j][tid] = row_ptr(r, code);
        if (KV8 && j == 0) rowscale[tid] = row_scale(r, code);
      }
    }
    __syncthreads();
    if (!KV8 && ntiles > 0) dma_tile(0, 0);

    for (int it = 0; it < ntiles; ++it) {
      const int buf = KV8 ? 0 : (it & 1);
      __syncthreads();  // all waves are done with tile it-1 (and its buffer)
      int code2 = -1;
      const int r2 = r0 + (it + 2) * SAS_TILE + tid;
      if (tid < SAS_TILE) code2 = row_code(r2);  // issued before the next DMA: ready at the wait
      if constexpr (!KV8) {
        if (it + 1 < ntiles) {
          dma_tile((it + 1) & 1, (it + 1) & 1);
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPT) : "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        if (tid < SAS_TILE) rowaddr[it & 1][tid] = row_ptr(r2, code2);
      } else {
        fp8_stage(it);
      }
      __syncthreads();  // tile it is in LDS for every wave
      const uint8_t* tile = tiles + buf * TILEB;
      const int nvalid = min(SAS_TILE, r1 - (r0 + it * SAS_TILE));

      // ---- S^T[key][head] = K Q^T : A = K rows (LDS), B = Q^T (registers) ----
      f32x16_t s = f32x16_t{};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const u32x4_t kf =
            *reinterpret_cast<const u32x4_t*>(tile + kbase[ks & 3] + (ks >> 2) * 128);
        s = mfma32<QT>(kf, qf[ks], s);
      }
      // C layout: register r holds key 8 (r / 4) + 4 g + r % 4 for head li.
      float x[16];
      float mt = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * g + (r & 3);
        float v = s[r] * a.scale_log2;
        if (KV8) v *= rowscale[key];
        x[r] = key < nvalid ? v : -INFINITY;
        mt = fmaxf(mt, x[r]);
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      if (__any(mt > m_run)) {  // golden.py:185-187,196: rescale O and l to the new maximum
        const float m_new = fmaxf(m_run, mt);
        const float alpha = m_new > m_run ? exp2f(m_run - m_new) : 1.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] *= alpha;
        l_run *= alpha;
        m_run = m_new;
      }
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[r] = exp2f(x[r] - m_run);
        ps += x[r];
      }
      ps += __shfl_xor(ps, 32);
      l_run += ps;
      // P^T as the B operand: k-step kk element e = register 8 kk + e.
      u32x4_t pk[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float p0 = x[8 * kk + 2 * e], p1 = x[8 * kk + 2 * e + 1];
          if (KV8) {  // V = fp8 * scale: fold the row scale into P
            p0 *= rowscale[16 * kk + 8 * ((2 * e) >> 2) + 4 * g + ((2 * e) & 3)];
            p1 *= rowscale[16 * kk + 8 * ((2 * e + 1) >> 2) + 4 * g + ((2 * e + 1) & 3)];
          }
          pk[kk][e] = to_q16<QT>(p0) | (to_q16<QT>(p1) << 16);
        }
      }
      // ---- O^T[d][head] += V^T P^T : A = V^T gathered from the row-major tile ----
      // Block pair mm covers d in [64 mm, 64 mm + 64): MFMA row li of block 2 mm + j
      // is d = 64 mm + 2 li + j, so one dword per key feeds both blocks of the pair.
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          uint32_t wv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            wv[e] = *reinterpret_cast<const uint32_t*>(
                tile + vbase[e & 3] + (16 * kk + 8 * (e >> 2)) * ROWB + 128 * mm);
          u32x4_t a0, a1;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a0[e] = __builtin_amdgcn_perm(wv[2 * e + 1], wv[2 * e], 0x05040100u);
            a1[e] = __builtin_amdgcn_perm(wv[2 * e + 1], wv[2 * e], 0x07060302u);
          }
          acc[2 * mm] = mfma32<QT>(a0, pk[kk], acc[2 * mm]);
          acc[2 * mm + 1] = mfma32<QT>(a1, pk[kk], acc[2 * mm + 1]);
        }
      }
      if constexpr (KV8) {
        __syncthreads();  // tile and scales consumed; next tile's scales may be written
        if (tid < SAS_TILE && it + 1 < ntiles) {
          const int r = r0 + (it + 1) * SAS_TILE + tid;
          const int code = row_code(r);
          rowaddr[(it + 1) & 1][tid] = row_ptr(r, code);
          rowscale[tid] = row_scale(r, code);
        }
      }
    }
  }

  // ---- epilogue ----
  if (!hvalid) return;
  if (splits == 1) {
    const float inv = 1.f / l_run;
    uint16_t* orow = out + ((size_t)t * H + h) * DV;
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        // registers 4 q4 .. 4 q4 + 3 of blocks 2 mm, 2 mm + 1 -> d = 64 mm + 16 q4 + 8 g + [0, 8)
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = to_q16<QT>(acc[2 * mm][4 * q4 + e] * inv) |
                 (to_q16<QT>(acc[2 * mm + 1][4 * q4 + e] * inv) << 16);
        *reinterpret_cast<u32x4_t*>(orow + 64 * mm + 16 * q4 + 8 * g) = o;
      }
    }
    if (lse && g == 0) lse[(size_t)t * H + h] = (m_run + __log2f(l_run)) * 0.6931471805599453f;
  } else {
    const int slot = wsbase + split;
    float* orow = ws_o + ((size_t)slot * H + h) * DV;
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        float4 v0, v1;
        v0.x = acc[2 * mm][4 * q4 + 0];
        v0.y = acc[2 * mm + 1][4 * q4 + 0];
        v0.z = acc[2 * mm][4 * q4 + 1];
        v0.w = acc[2 * mm + 1][4 * q4 + 1];
        v1.x = acc[2 * mm][4 * q4 + 2];
        v1.y = acc[2 * mm + 1][4 * q4 + 2];
        v1.z = acc[2 * mm][4 * q4 + 3];
        v1.w = acc[2 * mm + 1][4 * q4 + 3];
        float4* dst = reinterpret_cast<float4*>(orow + 64 * mm + 16 * q4 + 8 * g);
        dst[0] = v0;
        dst[1] = v1;
      }
    }
    if (g == 0)
      reinterpret_cast<float4*>(ws_ml)[(size_t)slot * H + h] = make_float4(m_run, l_run, l_run, 0.f);
  }
}

// ===========================================================================
// Split combine: one wave per (split token, head), grid-stride over the split
// tokens the plan recorded (a call without split tokens exits at once).
// ===========================================================================
constexpr int COMBINE_WAVES = 4;  // waves per workgroup

template <int QT>
__global__ __launch_bounds__(64 * COMBINE_WAVES) void combine_kernel(
    SasFwdArgs a, const int* __restrict__ plan, const float* __restrict__ ws_o,
    const float* __restrict__ ws_ml, uint16_t* __restrict__ out, float* __restrict__ lse) {
  const int H = a.H;
  const int items = plan[PH_NSPLIT_TOKENS] * H;  // (split token, head) pairs
  const SasPlanLayout L = sas_plan_layout(a.T, a.split_cap);
  const int wave = blockIdx.x * COMBINE_WAVES + (threadIdx.x >> 6);
  for (int item = wave; item < items; item += gridDim.x * COMBINE_WAVES) {
    const int i = item / H, h = item - i * H;
    const int t = plan[L.off_split_tokens + i];
    const int* tk = plan + SAS_PLAN_HDR + (size_t)t * SAS_TOK_W;
    combine_head<QT>(t, h, H, tk[TK_SPLITS], tk[TK_WSBASE], ws_o, ws_ml, out, lse);
  }
}

}  // namespace sas
