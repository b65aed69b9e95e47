// sas_backward.hip -- gfx950 kernels of the backward pass for the queries and sinks.
//
// The reference has no backward; it returns the LSE for one (api.py:32-35,
// 176-184).  With the forward's out and lse, P_j = e^(s_j - lse) is known exactly
// (no running maximum and no frame), and
//   D = <dO, out> - dlse,  dS_j = P_j (<dO, V_j> - D),  dq = scale sum_j dS_j K_j,
//   dsink = -sum_t e^(sink - lse) D
// over the same row lists the forward attends (the resolver's output).
//
//   bwd_prep_kernel   D and the sink term per (token, head); zeroes the dq rows
//                     that are accumulated by several units (split tokens) or
//                     that no batch owns.
//   bwd_dq_kernel     one workgroup per (work unit, 64 heads): each wave owns 16
//                     heads.  Per 32-row tile: S^T = K Q^T and dP^T = V dO^T as
//                     16x16x32 MFMAs (K rows from LDS, Q^T and dO^T fragments in
//                     registers), P and dS in registers, then dq^T += K^T dS^T
//                     (K^T from a transposed LDS copy of the tile, dS^T straight
//                     from the accumulator layout).
//   bwd_dsink_kernel  dsink[h] summed over tokens in a fixed order (one wave per
//                     head), so it is deterministic.
//
// MFMA 16x16x32 operand layouts (lane l, n = l & 15, g = l >> 4): A (16 x 32)
// lane holds row n, columns 8 g .. 8 g + 7; B (32 x 16) lane holds rows 8 g .. 8 g
// + 7 of column n; C (16 x 16) lane holds rows 4 g .. 4 g + 3 of column n.  For
// dq^T the contraction runs over the tile's 32 keys in the order k = 8 g + e ->
// key (e < 4 ? 4 g + e : 16 + 4 g + e - 4): exactly the keys the two S^T blocks
// leave in lane l, so dS^T needs no data movement.
#include <hip/hip_runtime.h>

#include "sas_common.h"

namespace sas {

typedef __bf16 bw_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 bw_f16x8 __attribute__((ext_vector_type(8)));
typedef float bw_f32x4 __attribute__((ext_vector_type(4)));

constexpr int BW_HEADS = 64;  // heads per workgroup: 4 waves x 16
constexpr int BW_TILE = 32;   // keys per tile

template <int QT>
__device__ __forceinline__ bw_f32x4 bw_mfma(const u32x4_t& a, const u32x4_t& b, const bw_f32x4& c) {
  if constexpr (QT == 0)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bw_bf16x8, a),
                                                   __builtin_bit_cast(bw_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(bw_f16x8, a),
                                                  __builtin_bit_cast(bw_f16x8, b), c, 0, 0, 0);
}

// D = <dO, out> (less dlse when the LSE has a gradient) and the sink term
// -e^(sink - lse) D of token t, one wave per head (lane l covers dimensions 8 l ..
// 8 l + 7 of d_v = 512).
template <int QT>
__global__ __launch_bounds__(256) void bwd_prep_kernel(SasFwdArgs a, int dqk,
                                                       const int* __restrict__ plan,
                                                       const uint16_t* __restrict__ dout,
                                                       const uint16_t* __restrict__ out,
                                                       const float* __restrict__ lse,
                                                       const float* __restrict__ dlse,
                                                       const float* __restrict__ sinks,
                                                       float* __restrict__ dterm,
                                                       float* __restrict__ sterm,
                                                       float* __restrict__ dq) {
  constexpr int DV = 512;
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool ok = plan_matches(plan, a);
  const int* tk = plan + SAS_PLAN_HDR + (size_t)t * SAS_TOK_W;
  const int b = ok ? tk[TK_B] : -1;
  const bool owned = b >= 0 && b < a.B;
  const bool zero_dq = !owned || tk[TK_SPLITS] > 1;
  for (int h = w; h < a.H; h += 4) {
    const size_t th = (size_t)t * a.H + h;
    float d = 0.f;
    if (owned) {
      const u32x4_t go = reinterpret_cast<const u32x4_t*>(dout + th * DV)[lane];
      const u32x4_t oo = reinterpret_cast<const u32x4_t*>(out + th * DV)[lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d = fmaf(q16_to_f32<QT>(go[e] & 0xffffu), q16_to_f32<QT>(oo[e] & 0xffffu), d);
        d = fmaf(q16_to_f32<QT>(go[e] >> 16), q16_to_f32<QT>(oo[e] >> 16), d);
      }
      d = wave_sum(d);
      // a gradient of the LSE: d lse / d s_j = P_j and d lse / d sink = P_sink, so it
      // enters as dS = P (dP - (D - dlse)) and dsink = -P_sink (D - dlse)
      if (dlse) d -= dlse[th];
    }
    if (lane == 0) {
      dterm[th] = d;
      const float s = sinks[h];
      // a sink of -inf has P_sink = 0 (lse may be -inf too when nothing is attended)
      sterm[th] = (!owned || s == -INFINITY || d == 0.f) ? 0.f : -__expf(s - lse[th]) * d;
    }
    if (zero_dq) {
      float4* row = reinterpret_cast<float4*>(dq + th * dqk);
      for (int i = lane; i < dqk / 4; i += 64) row[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

template <int DQK, int QT>
__global__ __launch_bounds__(256, 1) void bwd_dq_kernel(SasFwdArgs a, const uint16_t* __restrict__ q,
                                                        const uint16_t* __restrict__ dout,
                                                        const uint64_t* __restrict__ addr_list,
                                                        const int* __restrict__ ncmp,
                                                        const float* __restrict__ lse,
                                                        const float* __restrict__ dterm,
                                                        const int* __restrict__ plan,
                                                        float* __restrict__ dq) {
  constexpr int DV = 512;
  constexpr int KS = DQK / 32;         // k-steps of S^T = K Q^T (18 / 16)
  constexpr int VKS = DV / 32;         // k-steps of dP^T = V dO^T (16)
  constexpr int NDB = DQK / 16;        // 16-dimension blocks of dq^T (36 / 32)
  constexpr int CH = DQK / 8;          // 16-B chunks per row
  constexpr int KSTR = DQK * 2 + 16;   // row-major tile: row stride in bytes
  constexpr int TSTR = BW_TILE * 2 + 16;  // transposed tile: bytes per dimension row
  __shared__ __attribute__((aligned(16))) uint8_t kt[BW_TILE * KSTR];
  __shared__ __attribute__((aligned(16))) uint8_t ktt[DQK * TSTR];

  const int HG = (a.H + BW_HEADS - 1) / BW_HEADS;
  const int u = blockIdx.x / HG, hg = blockIdx.x - u * HG;
  if (!plan_matches(plan, a) || u >= plan[PH_UNITS]) return;  // refused plan: prep zeroed dq
  const int* ur = plan + SAS_PLAN_HDR + (size_t)SAS_TOK_W * a.T + (size_t)u * SAS_UNIT_W;
  const int t = ur[0], split = ur[3];
  if (split < 0) return;  // a q row no batch owns: zero (bwd_prep_kernel)
  const int* tk = plan + SAS_PLAN_HDR + (size_t)t * SAS_TOK_W;
  const int nwin = min(tk[TK_NWIN], a.win_left + 1);
  const int splits = tk[TK_SPLITS];
  const int r0 = ur[1];
  const int r1 = min(min(ur[2], nwin + ncmp[t]), a.list_stride);
  const int ntiles = r1 > r0 ? (r1 - r0 + BW_TILE - 1) / BW_TILE : 0;
  const uint64_t* alist = addr_list + (size_t)t * a.list_stride;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n16 = lane & 15, g = lane >> 4;
  const int h = hg * BW_HEADS + w * 16 + n16;
  const bool hvalid = h < a.H;
  const int hc = min(h, a.H - 1);
  const size_t th = (size_t)t * a.H + hc;

  u32x4_t qf[KS], of[VKS];
  {
    const u32x4_t* qr = reinterpret_cast<const u32x4_t*>(q + th * DQK);
    const u32x4_t* orow = reinterpret_cast<const u32x4_t*>(dout + th * DV);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = qr[4 * ks + g];
#pragma unroll
    for (int ks = 0; ks < VKS; ++ks) of[ks] = orow[4 * ks + g];
  }
  const float lse2 = lse[th] * LOG2E, dh = dterm[th];
  const float c = a.scale_log2;
  bw_f32x4 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = bw_f32x4{0.f, 0.f, 0.f, 0.f};

  for (int i = 0; i < ntiles; ++i) {
    const int rb = r0 + i * BW_TILE;
    __syncthreads();  // every wave is done with the previous tile
    for (int ch = tid; ch < BW_TILE * CH; ch += 256) {
      const int row = ch / CH, cc = ch - row * CH;
      u32x4_t v = u32x4_t{0, 0, 0, 0};
      if (rb + row < r1) v = reinterpret_cast<const u32x4_t*>(alist[rb + row])[cc];
      *reinterpret_cast<u32x4_t*>(kt + row * KSTR + cc * 16) = v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        *reinterpret_cast<uint16_t*>(ktt + (8 * cc + 2 * e) * TSTR + row * 2) = (uint16_t)(v[e] & 0xffffu);
        *reinterpret_cast<uint16_t*>(ktt + (8 * cc + 2 * e + 1) * TSTR + row * 2) = (uint16_t)(v[e] >> 16);
      }
    }
    __syncthreads();
    // S^T and dP^T: two blocks of 16 keys each
    bw_f32x4 s[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const uint8_t* kr = kt + (16 * kb + n16) * KSTR + 16 * g;
      s[kb] = bw_f32x4{0.f, 0.f, 0.f, 0.f};
      dp[kb] = bw_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(kr + 64 * ks);
        s[kb] = bw_mfma<QT>(av, qf[ks], s[kb]);
        if (ks < VKS) dp[kb] = bw_mfma<QT>(av, of[ks], dp[kb]);
      }
    }
    // P = e^(s - lse) and dS = P (dP - D) for keys 16 kb + 4 g + r of head n16
    float ds[8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool valid = rb + 16 * kb + 4 * g + r < r1;
        const float p = valid ? exp2f(fmaf(s[kb][r], c, -lse2)) : 0.f;
        ds[4 * kb + r] = p * (dp[kb][r] - dh);
      }
    u32x4_t bds;
#pragma unroll
    for (int e = 0; e < 4; ++e) bds[e] = pack2_q16<QT>(ds[2 * e], ds[2 * e + 1]);
    // dq^T += K^T dS^T: A = dimensions 16 db + n16 of keys 4 g .. 4 g + 3 and 16 + 4 g ..
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const uint8_t* tr = ktt + (16 * db + n16) * TSTR + 8 * g;
      const uint2 lo = *reinterpret_cast<const uint2*>(tr);
      const uint2 hi = *reinterpret_cast<const uint2*>(tr + 32);
      acc[db] = bw_mfma<QT>(u32x4_t{lo.x, lo.y, hi.x, hi.y}, bds, acc[db]);
    }
  }
  if (!hvalid) return;
  // lane holds dimensions 16 db + 4 g .. + 3 of head h
  const float scale = c * 0.6931471805599453f;
  float* dqr = dq + ((size_t)t * a.H + h) * DQK + 4 * g;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const float4 v = make_float4(acc[db][0] * scale, acc[db][1] * scale, acc[db][2] * scale,
                                 acc[db][3] * scale);
    if (splits > 1) {
      atomicAdd(dqr + 16 * db + 0, v.x);
      atomicAdd(dqr + 16 * db + 1, v.y);
      atomicAdd(dqr + 16 * db + 2, v.z);
      atomicAdd(dqr + 16 * db + 3, v.w);
    } else {
      *reinterpret_cast<float4*>(dqr + 16 * db) = v;
    }
  }
}

// dsink[h] = sum over tokens of the sink terms, lanes striding over tokens in a
// fixed order and a fixed reduction: deterministic.
__global__ __launch_bounds__(256) void bwd_dsink_kernel(int T, int H, const float* __restrict__ sterm,
                                                        float* __restrict__ dsinks) {
  const int h = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (h >= H) return;
  float acc = 0.f;
  for (int t = lane; t < T; t += 64) acc += sterm[(size_t)t * H + h];
  acc = wave_sum(acc);
  if (lane == 0) dsinks[h] = acc;
}

}  // namespace sas
