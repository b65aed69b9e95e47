// sas_attend.hip -- pipelined gfx950 attention kernel for 16-bit (bf16 / fp16) KV.
//
// One workgroup (4 waves, one per SIMD) processes one work unit of the split-KV
// plan: a contiguous range of one query token's row list (its window rows, then
// its compressed rows).  Wave w owns query heads [32 w, 32 w + 32); Q stays in
// VGPRs (36 x 16-B fragments at d_qk = 576) and the fp32 O^T accumulator of
// 512 x 32 fills the AGPRs.  KV rows are gathered 32 at a time (one tile) by
// direct global -> LDS DMA (16 B per lane) into a 4-slot ring, three tiles ahead
// of the one being consumed.
//
// Per tile, per wave (32 keys x 32 heads):
//   S^T = K Q^T      36 MFMA 32x32x16, A = K rows from LDS (ds_read_b128), B = Q
//   softmax          P = 2^(x - m) in a per-unit frame m, bf16(P)
//   O^T += V^T P^T   32 MFMA, A = V^T read transposed from LDS (ds_read_b64_tr_b16),
//                    B = P^T straight from the S^T accumulator registers
//
// Softmax (reference golden.py:156-200): the state of a head is (m, l, O) seeded
// with (sink, 1, 0) on the unit that holds the token's first rows.  O / l and
// m + ln l do not depend on the frame m, so the kernel fixes m after the first
// tile and never rescales the AGPR-resident O inside the loop (a VALU pass over
// 256 accumulators would cost as much as a tile of MFMA work and, worse, makes
// the compiler keep O in VGPRs).  Two normalisers are kept: l_w sums the
// bf16-rounded P that enter PV, so O / l_w is exactly a convex combination of
// the V rows (a one-hot softmax returns its row unchanged, as the reference's
// P = 1 does); l_e sums the unrounded P and gives the LSE.  A logit more than
// REDO_SLACK above the frame (where 2^SLACK times the row count nears the fp32
// range) makes the workgroup discard the pass and recompute the unit framed on
// the maximum each head observed (a second, separately inlined copy of the unit
// body, so the common path carries no extra live state).
//
// LDS tile = latent region (32 rows x 512 dims at a 1088-B row stride, i.e. 64 B
// of padding per row) + rope region (32 rows x 64 dims, 128-B rows; absent at
// d_qk = 512).  Latent 16-B chunk c of row r lives at chunk c ^ ((r >> 2) & 3);
// the padding puts rows r .. r+3 in different quarters of the 256-B bank line,
// the XOR separates rows 4 apart.  Rope chunk c of row r lives at c ^ ((r >> 1) & 7).
// With these, the b128 K reads (16 consecutive rows, one chunk) and the b64
// transposed V reads (4 rows x 4 chunks per 16 lanes) touch every bank once per
// 256 B, and the per-lane read offsets reduce to two registers plus immediates.
// A latent DMA instruction copies one whole row (64 lanes x 16 B), so its source
// is a wave-uniform row base plus a per-lane offset.
#include <hip/hip_runtime.h>

#include "sas_common.h"

namespace sas {

constexpr float REDO_SLACK = 64.f;

typedef __bf16 bf16x4_t __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef __fp16 f16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Workgroup barrier without the memory fences of __syncthreads(): those wait for
// every outstanding global load (vmcnt(0)), which would drain the DMA prefetch.
// LDS writes of this wave are completed first (lgkmcnt(0)); DMA landings are
// waited for explicitly with vmcnt before the barrier where needed.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Four 16-bit elements of one LDS column from four consecutive rows:
// ds_read_b64_tr_b16 hands lane i of a 16-lane group element r of the 8-byte
// chunk addressed by lane 4 r + (i >> 2) of that group, element (i & 3).
template <int QT>
__device__ __forceinline__ u32x2_t lds_read_tr16(const lds_u8* p) {
  typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4;
  typedef __attribute__((address_space(3))) f16x4_t lds_f16x4;
  if constexpr (QT == 0) {
    const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
    return __builtin_bit_cast(u32x2_t, v);
  } else {
    const f16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_f16x4*)p);
    return __builtin_bit_cast(u32x2_t, v);
  }
}

__device__ __forceinline__ u32x4_t lds_read_b128(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(p);
}

__device__ __forceinline__ void dma16(const uint8_t* src, lds_u8* dst) {
  __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)dst,
                                   16, 0, 0);
}

// Swizzle of the latent region: chunk c of row r sits at c ^ swz_a(r).
__device__ __forceinline__ int swz_a(int r) { return (r >> 2) & 3; }
// Swizzle of the rope region.
__device__ __forceinline__ int swz_b(int r) { return (r >> 1) & 7; }

template <int DQK>
struct AttendLds {
  static constexpr int TILEB = SAS_TILE * (1024 + 64) + SAS_TILE * (DQK - 512) * 2;
  uint8_t tiles[4 * TILEB];
  const uint8_t* rowaddr[4][SAS_TILE];
  int codes[4][SAS_TILE];  // row codes of the next tiles, fetched by DMA
  int far;                 // a logit of some head outgrew the frame
};

// One work unit u.  Returns true (workgroup-uniform) when the first pass must be
// redone; m_obs then holds each lane's observed maximum (log2 units), which the
// REDO instance takes as its frame.
template <int DQK, int QT, bool REDO>
__device__ __forceinline__ bool attend_unit(
    int u, AttendLds<DQK>& sm, const SasFwdArgs& a, const uint16_t* __restrict__ q,
    const uint8_t* __restrict__ ori_kv, const uint8_t* __restrict__ cmp_kv,
    const int* __restrict__ cmp_bt, const int* __restrict__ rows_list,
    const int* __restrict__ ncmp, const float* __restrict__ sinks, const int* __restrict__ plan,
    uint16_t* __restrict__ out, float* __restrict__ lse, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, float& m_obs) {
  constexpr int DV = 512;
  constexpr int NT = 256;
  constexpr int TILE = SAS_TILE;          // 32 keys
  constexpr int NSTAGE = 4;
  constexpr bool ROPE = DQK > DV;         // d_qk = 576: 64 rope dims after the latent 512
  static_assert(DQK == DV || DQK == DV + 64, "d_qk must be 512 or 576");
  constexpr int ROWA = DV * 2;            // latent bytes per row (1024)
  constexpr int STRA = ROWA + 64;         // latent LDS row stride
  constexpr int ROWR = (DQK - DV) * 2;    // rope bytes per row (128 or 0)
  constexpr int TILEA = TILE * STRA;
  constexpr int TILEB = TILEA + TILE * ROWR;
  constexpr int KSTEPS = DQK / 16;        // MFMA k-steps of Q K^T: 36 / 32
  constexpr int CPT = TILE / 4 + (ROPE ? 1 : 0);  // DMA instructions per wave per tile
  static_assert(TILE == 32, "the MFMA tiling assumes 32-key tiles");

  static_assert(AttendLds<DQK>::TILEB == TILEB, "LDS layout");
  lds_u8* const tiles = (lds_u8*)sm.tiles;
  auto& rowaddr = sm.rowaddr;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 5;   // half-wave
  const int li = lane & 31;  // MFMA column (head) / row index

  const int* ur = plan + SAS_PLAN_HDR + (size_t)SAS_TOK_W * a.T + (size_t)u * SAS_UNIT_W;
  const int t = ur[0], split = ur[3];
  const int H = a.H;

  if (split < 0) {  // a q row no batch owns: zeros, as the reference's padded slots
    for (int i = tid; i < H * DV / 8; i += NT)
      reinterpret_cast<u32x4_t*>(out + (size_t)t * H * DV)[i] = u32x4_t{0, 0, 0, 0};
    if (lse)
      for (int i = tid; i < H; i += NT) lse[(size_t)t * H + i] = 0.f;
    return false;
  }

  const int* tk = plan + SAS_PLAN_HDR + (size_t)t * SAS_TOK_W;
  const int b = tk[TK_B], nwin = tk[TK_NWIN];
  const int splits = tk[TK_SPLITS], wsbase = tk[TK_WSBASE];
  const int r0 = ur[1];
  const int r1 = min(ur[2], nwin + ncmp[t]);
  const int ntiles = r1 > r0 ? (r1 - r0 + TILE - 1) / TILE : 0;
  const int* codes = rows_list + (size_t)t * a.list_stride;

  // Row code of list row r (-1 = a row read as zeros): the token's list holds its
  // window rows, then its compressed rows, contiguously.
  auto row_code = [&](int r) -> int { return r < r1 ? codes[r] : -1; };
  auto row_ptr = [&](int r, int code) -> const uint8_t* {
    if (code < 0) return g_zero_row;
    if (r < nwin) {
      const int page = code / a.ori_block_size, off = code - page * a.ori_block_size;
      return ori_kv + ((size_t)page * a.ori_block_stride + (size_t)off * a.ori_row_stride) * 2;
    }
    const int page = code / a.cmp_block_size, off = code - page * a.cmp_block_size;
    return cmp_kv + ((size_t)page * a.cmp_block_stride + (size_t)off * a.cmp_row_stride) * 2;
  };

  // ---- per-lane LDS offsets (bytes within a tile) ----
  // K, latent k-step ks < 32: row li, chunk 2 ks + g -> kofs[ks & 1] + 64 (ks >> 1).
  // K, rope k-step 32 + j: row li, rope chunk 2 j + g -> kofs_r[j].
  uint32_t kofs[2], kofs_r[4];
  {
    const int f = swz_a(li);
#pragma unroll
    for (int j = 0; j < 2; ++j) kofs[j] = li * STRA + 16 * ((2 * j + g) ^ f);
    const int fr = swz_b(li);
#pragma unroll
    for (int j = 0; j < 4; ++j) kofs_r[j] = TILEA + li * ROWR + 16 * ((2 * j + g) ^ fr);
  }
  // V^T (A of O^T += V^T P^T).  MFMA row m of d-block mb is d = 32 mb + dmap(m) with
  // dmap(m) = 16 ((m >> 2) & 1) + 4 (m >> 3) + (m & 3), so accumulator register r of
  // lane (li, g) holds d = 32 mb + 16 g + r.  MFMA k index 8 g + e of k-step kk is key
  // 16 kk + 8 (e >> 2) + 4 g + (e & 3), matching where P^T sits in the S^T registers.
  // Lane l therefore supplies row 16 kk + 4 (l >> 5) + ((l >> 2) & 3) + 8 hf (hf = e >> 2)
  // at column 32 mb + 16 (l & 1) + 8 ((l >> 4) & 1) + 4 ((l >> 1) & 1): latent chunk
  // 4 mb + clo, clo = 2 (l & 1) + ((l >> 4) & 1), byte 8 ((l >> 1) & 1) within it.  The
  // row's swizzle only touches clo and depends on hf alone, so the offset is
  // vofs[hf] + 64 mb + 16 kk STRA.
  uint32_t vofs[2];
  {
    const int clo = 2 * (lane & 1) + ((lane >> 4) & 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = 4 * (lane >> 5) + ((lane >> 2) & 3) + 8 * hf;
      vofs[hf] = row * STRA + 16 * (clo ^ swz_a(row)) + 8 * ((lane >> 1) & 1);
    }
  }

  // ---- per-wave state: 32 heads per wave ----
  // Head indices past H are clamped onto a valid head and never stored.
  const int h = w * 32 + li;
  const bool hvalid = h < H;
  const int hc = min(h, H - 1);
  u32x4_t qf[KSTEPS];
  {
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(q + ((size_t)t * H + hc) * DQK);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[ks] = qrow[2 * ks + g];
  }
  f32x16_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x16_t{};
  // golden.py:162-163: the unit holding the token's first rows carries the sink
  const float sink2 = split == 0 ? sinks[hc] * LOG2E : -INFINITY;
  float m_run = REDO ? m_obs : sink2;  // redo: the frame is the maximum pass 1 observed

  // ---- gather: tile i goes to ring slot i & 3 ----
  // Latent: instruction k of wave w copies row 4 k + w; lane l fetches source chunk
  // l ^ swz_a(4 k + w) = l ^ (k & 3) into slot l.  Rope: wave w copies rows
  // 8 w .. 8 w + 7, lane l row 8 w + (l >> 3), slot l & 7 <- chunk (l & 7) ^ swz_b(row).
  const int wu = __builtin_amdgcn_readfirstlane(w);  // the wave index as a scalar
  const uint32_t ulane = (uint32_t)lane;
  auto dma_tile = [&](int i) {
    const int slot = i & (NSTAGE - 1);
    lds_u8* dstA = tiles + slot * TILEB;
    const uint64_t mine = (uint64_t)rowaddr[slot][4 * (lane & 7) + wu];
#pragma unroll
    for (int k = 0; k < TILE / 4; ++k) {
      const uint64_t rb = ((uint64_t)__builtin_amdgcn_readlane((uint32_t)(mine >> 32), k) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((uint32_t)mine, k);
      const uint32_t off = 16u * (ulane ^ (uint32_t)(k & 3));
      dma16((const uint8_t*)rb + off, dstA + (4 * k + wu) * STRA);
    }
    if constexpr (ROPE) {
      const int row = 8 * wu + (lane >> 3);
      const uint8_t* rr = rowaddr[slot][row];
      dma16(rr + (uint32_t)(ROWA + 16 * ((lane & 7) ^ swz_b(row))), dstA + TILEA + 8 * wu * ROWR);
    }
  };

  // Row codes of tile i reach LDS by a 4-byte DMA (wave 0, lanes < 32, slot i & 3)
  // so that no global load with a VGPR result sits inside the tile loop: the
  // compiler would have to drain every outstanding tile DMA to consume it.
  auto dma_codes = [&](int i) {
    const int r = r0 + i * TILE + lane;
    if (lane < TILE && r < r1)
      __builtin_amdgcn_global_load_lds((const void*)(codes + r),
                                       (__attribute__((address_space(3))) void*)&sm.codes[i & 3][0],
                                       4, 0, 0);
  };

  // Pipeline, per iteration it (one barrier):
  //   wait   until tile it has landed (tiles it+1, it+2 may still be in flight)
  //   wave 0 writes the row addresses of tile it+3 (codes DMA'd two iterations ago)
  //   barrier: tile it visible; every wave is done with tile it-1, whose slot
  //            (= slot of it+3) is free
  //   DMA    codes of tile it+5 (wave 0), then tile it+3 (all waves)
  //   compute S, softmax and PV of tile it
  // prologue: row addresses of tiles 0..2, codes of tiles 3 and 4, DMA of tiles 0..2
  if (!REDO && tid == 0) sm.far = 0;
  if (tid < 3 * TILE) {
    const int r = r0 + tid;  // tile tid / 32, row tid % 32
    rowaddr[tid / TILE][tid % TILE] = row_ptr(r, row_code(r));
  }
  lds_barrier();
  if (wu == 0) {
    if (ntiles > 3) dma_codes(3);
    if (ntiles > 4) dma_codes(4);
  }
  if (ntiles > 0) dma_tile(0);
  if (ntiles > 1) dma_tile(1);
  if (ntiles > 2) dma_tile(2);

  // O^T += V^T P^T for one tile
  auto pv = [&](const lds_u8* tl, const u32x4_t(&pk)[2]) {
#pragma unroll
    for (int mb = 0; mb < 16; ++mb) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const lds_u8* p = tl + 64 * mb + 16 * STRA * kk;
        const u32x2_t lo = lds_read_tr16<QT>(p + vofs[0]);
        const u32x2_t hi = lds_read_tr16<QT>(p + vofs[1]);
        const u32x4_t av = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        acc[mb] = mfma32<QT>(av, pk[kk], acc[mb]);
      }
    }
    // operand reads run one MFMA ahead of their MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int i = 0; i < 31; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  };

  // Per-lane partial sums over this lane's keys (the two half-waves of a head see
  // different keys); they are combined once, after the loop.
  float pe = 0.f;          // sum of P (LSE)
  float pw = 0.f;          // sum of bf16(P): what entered PV (output normaliser)
  float xobs = -INFINITY;  // max of x - m over the unit, for the overflow guard
  const float c = a.scale_log2;
  for (int it = 0; it < ntiles; ++it) {
    // tile it has landed (this wave's share): the tile DMAs issued after it (at most
    // two) may still be pending; wave 0's code DMAs were issued before those, so
    // the same count also completes the codes of tile it+3
    if (it + 2 < ntiles)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * CPT) : "memory");
    else if (it + 1 < ntiles)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CPT) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (wu == 0 && it + 3 < ntiles && lane < TILE) {
      const int r3 = r0 + (it + 3) * TILE + lane;
      rowaddr[(it + 3) & (NSTAGE - 1)][lane] =
          row_ptr(r3, r3 < r1 ? sm.codes[(it + 3) & 3][lane] : -1);
    }
    lds_barrier();
    if (wu == 0 && it + 5 < ntiles) dma_codes(it + 5);  // before the tile DMA (vmcnt order)
    if (it + 3 < ntiles) dma_tile(it + 3);

    const lds_u8* tl = tiles + (it & (NSTAGE - 1)) * TILEB;
    // ---- S^T = K Q^T (each K fragment is read one MFMA ahead) ----
    auto kread = [&](int ks) -> u32x4_t {
      return ks < 32 ? lds_read_b128(tl + kofs[ks & 1] + 64 * (ks >> 1))
                     : lds_read_b128(tl + kofs_r[(ks - 32) & 3]);
    };
    f32x16_t s = f32x16_t{};
    u32x4_t kcur = kread(0);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const u32x4_t knext = ks + 1 < KSTEPS ? kread(ks + 1) : kcur;
      s = mfma32<QT>(kcur, qf[ks], s);
      kcur = knext;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int i = 0; i < KSTEPS - 1; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read, one ahead
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);

    // ---- softmax ----
    // x = S c - m (log2 units); the first tile of the first pass fixes the frame m.
    const bool first = !REDO && it == 0;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = first ? s[r] * c : fmaf(s[r], c, -m_run);
    const int nvalid = r1 - (r0 + it * TILE);
    if (__builtin_expect(nvalid < TILE, 0)) {  // the unit's last tile: rows past r1
      const int lim = nvalid - 4 * g;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) >= lim) x[r] = -INFINITY;
    }
    if (first) {  // O is still zero: no rescale needed
      float mt = x[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mt = fmaxf(mt, x[r]);
      m_run = fmaxf(m_run, fmaxf(mt, __shfl_xor(mt, 32)));
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] -= m_run;
    }
    float xm = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) xm = fmaxf(xm, x[r]);
    xobs = fmaxf(xobs, xm);
    u32x4_t pk[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x[r] = __builtin_amdgcn_exp2f(x[r]);  // 2^x; below 2^-126 of the frame flushes to 0
      pe += x[r];
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pk[kk][e] = pack2_q16<QT>(x[8 * kk + 2 * e], x[8 * kk + 2 * e + 1]);
        pw = sum2_q16<QT>(pk[kk][e], pw);
      }
    // ---- O^T += V^T P^T ----
    pv(tl, pk);
  }
  pe += __shfl_xor(pe, 32);
  pw += __shfl_xor(pw, 32);
  xobs = fmaxf(xobs, __shfl_xor(xobs, 32));
  // golden.py:162-163: the sink seeds (m, l) = (sink, 1) on the token's first unit
  const float l_sink = split != 0 ? 0.f : (sink2 == m_run ? 1.f : exp2f(sink2 - m_run));
  const float l_e = l_sink + pe, l_w = l_sink + pw;

  // ---- overflow guard: a logit far above the frame redoes the whole unit ----
  if (!REDO) {
    if (__any(xobs > REDO_SLACK) && lane == 0) atomicOr(&sm.far, 1);
    lds_barrier();
    if (sm.far) {
      m_obs = m_run + xobs;
      return true;
    }
  }

  // ---- epilogue: lane (li, g) holds d = 32 mb + 16 g + r of head li ----
  if (!hvalid) return false;
  if (splits == 1) {
    const float inv = l_w > 0.f ? 1.f / l_w : 0.f;
    uint16_t* orow = out + ((size_t)t * H + h) * DV + 16 * g;
#pragma unroll
    for (int mb = 0; mb < 16; ++mb) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = to_q16<QT>(acc[mb][8 * hf + 2 * e] * inv) |
                 (to_q16<QT>(acc[mb][8 * hf + 2 * e + 1] * inv) << 16);
        *reinterpret_cast<u32x4_t*>(orow + 32 * mb + 8 * hf) = o;
      }
    }
    if (lse && g == 0) lse[(size_t)t * H + h] = (m_run + __log2f(l_e)) * 0.6931471805599453f;
  } else {
    const int slot = wsbase + split;
    float* orow = ws_o + ((size_t)slot * H + h) * DV + 16 * g;
#pragma unroll
    for (int mb = 0; mb < 16; ++mb) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        float4 v;
        v.x = acc[mb][4 * qd + 0];
        v.y = acc[mb][4 * qd + 1];
        v.z = acc[mb][4 * qd + 2];
        v.w = acc[mb][4 * qd + 3];
        *reinterpret_cast<float4*>(orow + 32 * mb + 4 * qd) = v;
      }
    }
    if (g == 0)
      reinterpret_cast<float4*>(ws_ml)[(size_t)slot * H + h] = make_float4(m_run, l_w, l_e, 0.f);
  }
  return false;
}

}  // namespace sas

namespace sas {

// One workgroup per work unit.
template <int DQK, int QT>
__global__ __launch_bounds__(256, 1) void attend_kernel(
    SasFwdArgs a, const uint16_t* __restrict__ q, const uint8_t* __restrict__ ori_kv,
    const uint8_t* __restrict__ cmp_kv, const int* __restrict__ cmp_bt,
    const int* __restrict__ rows_list, const int* __restrict__ ncmp,
    const float* __restrict__ sinks, const int* __restrict__ plan, uint16_t* __restrict__ out,
    float* __restrict__ lse, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  __shared__ __attribute__((aligned(16))) AttendLds<DQK> sm;
  const int u = blockIdx.x;
  if (plan[PH_MAGIC] != SAS_PLAN_MAGIC || u >= plan[PH_UNITS]) return;
  float m_obs = 0.f;
  if (attend_unit<DQK, QT, false>(u, sm, a, q, ori_kv, cmp_kv, cmp_bt, rows_list, ncmp, sinks,
                                  plan, out, lse, ws_o, ws_ml, m_obs)) {
    lds_barrier();  // every wave is done with the ring before the redo refills it
    attend_unit<DQK, QT, true>(u, sm, a, q, ori_kv, cmp_kv, cmp_bt, rows_list, ncmp, sinks, plan,
                               out, lse, ws_o, ws_ml, m_obs);
  }
}

}  // namespace sas
