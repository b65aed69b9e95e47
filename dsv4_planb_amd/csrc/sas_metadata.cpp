// sas_metadata.cpp -- host restatement of the reference scheduler that emits the
// int32[1024] SparseAttnSharedkvMetadata table (sparse_attn_sharedkv_tilelang/
// metadata.py:258-1086 of the reference).  The table layout, the cost model and
// the greedy cursor walk must match the reference exactly for callers that
// consume the table, so the steps below follow the reference's order; the code
// is organised as plain structs and free functions.
//
//   table        = FA rows [36][8] then FD rows [72][8]            (metadata.py:38-68)
//   block cost   = 6 * ceil(m / 16) + 10 * ceil(s2 / 64)             (metadata.py:428-438)
//   row spans    = window [s1 - preToken, s1 + nextToken] clipped, then
//                  min(#compressed, topk) compressed tokens, in 512-blocks
//                                                                    (metadata.py:479-547)
//   per core     = whole batches, then whole rows, within half a
//                  block's cost of max(avg remaining, max row cost)  (metadata.py:718-764, 872-923)
// Arithmetic that Python performs on unbounded integers (the INT64_MAX token
// limits) is done in 128 bits here.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/sas.h"

namespace {

typedef __int128 i128;
constexpr int64_t kInt64Max = INT64_MAX;
constexpr int kS2Base = 512;
constexpr int kTolRatio = 2;
constexpr int kFaW = 8, kFdW = 8;
enum { WIN_N = 0, WIN_T = 1, CMP_N = 2, CMP_T = 3 };
enum { MASK_DEFAULT = 0, MASK_ALL = 1, MASK_LEFT_UP = 2, MASK_RIGHT_DOWN = 3, MASK_BAND = 4 };

int64_t fdiv(int64_t a, int64_t b) {  // Python floor division
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}
int64_t fmod_py(int64_t a, int64_t b) { return a - fdiv(a, b) * b; }

struct BatchCache {
  int64_t b = 0, s1 = 0, s2 = 0;
  i128 pre_lu = 0, next_lu = 0;
};

struct RowCache {  // S1GCache of the reference
  int64_t b = 0, s1g = 0, s2_start = 0, s2_end = 0;
  int64_t win_s2_start = 0, win_s2_end = 0, cmp_s2_start = 0, cmp_s2_end = 0;
  int64_t cost = 0, last_block_cost = 0, block = 0, normal_block_cost = 0;
  int64_t win_block = 0, win_cost = 0, win_last = 0, win_normal = 0;
  int64_t cmp_block = 0, cmp_cost = 0, cmp_last = 0, cmp_normal = 0;
  int64_t cmp_tail = 0, win_tail = 0;
};

struct CoreCache {
  int64_t limit = 0, cost = 0, block = 0;
};

struct Cursor {  // AssignContext of the reference
  int64_t b = 0, bn2 = 0, s1g = 0, s2 = 0, core = 0, unassigned = 0, used = 0;
  int64_t kv_split_part = 1, fd_data_num = 1, bn2_cost = 0, bn2_block = 0;
  bool finished = false;
  BatchCache bc;
  RowCache rc;
  CoreCache cc;
};

struct Scheduler {
  // inputs
  int64_t nq = 0, nkv = 0, batch = 0, max_q = 0, max_kv = 0, topk = 0, ratio = -1;
  int ori_mask = 4, win_left = 127, win_right = 0, layout_q = 0, layout_kv = 0;
  bool has_cmp = true;
  int64_t aic = 24, aiv = 48;
  std::vector<int64_t> cu_q, cu_kv, used_q, used_kv;
  // derived
  i128 pre_token = 0, next_token = 0;
  int attn_mode = 1;
  bool s1g_layout = true, cfa = false, scfa = false;
  int64_t group = 0, m_base = 0;
  int64_t tc[4][4] = {{0}};
  // split info / cost info
  std::vector<int64_t> s1g_base, s1g_tail, s2_base, s2_tail;
  bool all_zero = true;
  std::vector<int64_t> bn2_cost, bn2_block, bn2_last;
  int64_t total_block = 0, total_cost = 0, max_row_cost = 0;
  // result
  int64_t used_core = 0, max_cost = 0, num_fd_head = 0, max_s2_split = 0, fd_used_vec = 0;
  std::vector<int64_t> bn2_end, g_s1_end, s2_end, first_fd_ws;
  std::vector<int64_t> fd_bn2, fd_m, fd_ws, fd_split, fd_msize, fd_idx, fd_mstart, fd_mnum;
  bool error = false;

  int64_t s1_size(int64_t b) const {
    if (!used_q.empty()) return used_q[b];
    if (layout_q == 1 && !cu_q.empty()) return cu_q[b + 1] - cu_q[b];
    return max_q;
  }
  int64_t s2_size(int64_t b) const {
    if (!used_kv.empty()) return used_kv[b];
    if (layout_kv == 1 && !cu_kv.empty()) return cu_kv[b + 1] - cu_kv[b];
    return max_kv;
  }

  void params_init() {
    if (!used_q.empty())
      batch = (int64_t)used_q.size();
    else if (layout_q == 1 && !cu_q.empty())
      batch = (int64_t)cu_q.size() - 1;
    if (ori_mask == MASK_DEFAULT) {
      pre_token = kInt64Max;
      next_token = kInt64Max;
      attn_mode = 0;
    } else if (ori_mask == MASK_RIGHT_DOWN) {
      pre_token = kInt64Max;
      next_token = 0;
      attn_mode = 1;
    } else {
      pre_token = win_left > -1 ? (i128)win_left : (i128)kInt64Max;
      next_token = 0;
      attn_mode = 1;
    }
    s1g_layout = layout_q == 0 || layout_q == 1 || layout_q == 2;
    group = nkv == 0 ? 0 : nq / nkv;
    if (has_cmp) {
      if (topk > 0)
        scfa = true;
      else
        cfa = true;
    }
    m_base = group;
  }

  i128 pre_left_up(int64_t s1, int64_t s2) const {
    return ori_mask == MASK_BAND ? (i128)s1 - s2 + pre_token : pre_token;
  }
  i128 next_left_up(int64_t s1, int64_t s2) const {
    if (ori_mask == MASK_DEFAULT || ori_mask == MASK_ALL || ori_mask == MASK_LEFT_UP) return next_token;
    if (ori_mask == MASK_RIGHT_DOWN) return (i128)s2 - s1;
    if (ori_mask == MASK_BAND) return (i128)s2 - s1 + next_token;
    return next_token;
  }

  static int64_t block_cost(int64_t m, int64_t s2) { return 6 * ((m + 15) >> 4) + 10 * ((s2 + 63) >> 6); }

  void cost_table(int64_t s1n, int64_t s2n, int64_t s1t, int64_t wt, int64_t ct) {
    tc[WIN_N][WIN_N] = block_cost(s1n, s2n);
    tc[WIN_T][WIN_N] = s1t == 0 ? 0 : block_cost(s1t, s2n);
    tc[WIN_N][WIN_T] = wt == 0 ? 0 : block_cost(s1n, wt);
    tc[WIN_T][WIN_T] = (s1t == 0 || wt == 0) ? 0 : block_cost(s1t, wt);
    if (has_cmp) {
      tc[CMP_N][CMP_N] = block_cost(s1n, s2n);
      tc[CMP_T][CMP_N] = s1t == 0 ? 0 : block_cost(s1t, s2n);
      tc[CMP_N][CMP_T] = ct == 0 ? 0 : block_cost(s1n, ct);
      tc[CMP_T][CMP_T] = (s1t == 0 || ct == 0) ? 0 : block_cost(s1t, ct);
    }
  }

  void s2_range(int64_t s1g_idx, const BatchCache& bc, i128* first, i128* last) const {
    if (bc.s1 == 0 || bc.s2 == 0) {
      *first = 0;
      *last = 0;
      return;
    }
    if (!attn_mode) {
      *first = 0;
      *last = bc.s2 - 1;
      return;
    }
    const int64_t g_first = s1g_idx * m_base;
    const int64_t g_last = std::min(g_first + m_base, bc.s1 * group) - 1;
    int64_t s1_first, s1_last;
    if (s1g_layout) {
      s1_first = fdiv(g_first, group);
      s1_last = fdiv(g_last, group);
    } else if (fdiv(g_first, bc.s1) == fdiv(g_last, bc.s1)) {
      s1_first = fmod_py(g_first, bc.s1);
      s1_last = fmod_py(g_last, bc.s1);
    } else {
      s1_first = 0;
      s1_last = bc.s1;
    }
    *first = (i128)s1_first - bc.pre_lu;
    *last = (i128)s1_last + bc.next_lu;
  }

  void batch_cache(int64_t b, BatchCache* bc) const {
    bc->b = b;
    bc->s1 = s1_size(b);
    bc->s2 = s2_size(b);
    bc->pre_lu = pre_left_up(bc->s1, bc->s2);
    bc->next_lu = next_left_up(bc->s1, bc->s2);
  }

  void block_range(i128 f, i128 l, const BatchCache& bc, RowCache* rc) const {
    int64_t last;
    if (f >= bc.s2 || l < 0 || l < f) {
      last = 0;
      rc->win_s2_start = rc->win_s2_end = rc->win_tail = 0;
    } else {
      const int64_t first = (int64_t)std::max<i128>(0, std::min<i128>(f, bc.s2 - 1));
      last = (int64_t)std::max<i128>(0, std::min<i128>(l, bc.s2 - 1));
      rc->win_s2_start = 0;
      rc->win_s2_end = fdiv(last - first, kS2Base) + 1;
      rc->win_tail = fmod_py(last - first + 1, kS2Base);
    }
    rc->cmp_s2_start = rc->win_s2_end;
    const int64_t cmp_last_tokens = (has_cmp && ratio > 0) ? fdiv(last + 1, ratio) : 0;
    int64_t act = 0;
    if (cfa)
      act = cmp_last_tokens;
    else if (scfa)
      act = std::min(cmp_last_tokens, topk);
    rc->cmp_s2_end = act == 0 ? rc->cmp_s2_start : rc->cmp_s2_start + fdiv(act - 1, kS2Base) + 1;
    rc->cmp_tail = fmod_py(act, kS2Base);
  }

  void side_cache(RowCache* rc, bool cmp) const {
    const int64_t start = cmp ? rc->cmp_s2_start : rc->win_s2_start;
    const int64_t end = cmp ? rc->cmp_s2_end : rc->win_s2_end;
    int64_t &blk = cmp ? rc->cmp_block : rc->win_block, &cost = cmp ? rc->cmp_cost : rc->win_cost,
            &lastc = cmp ? rc->cmp_last : rc->win_last, &norm = cmp ? rc->cmp_normal : rc->win_normal;
    if (start >= end) {
      blk = cost = lastc = norm = 0;
      return;
    }
    blk = end - start;
    const int64_t tail = (cmp ? rc->cmp_tail : rc->win_tail) != 0 ? 1 : 0;
    const int64_t normal = blk - tail;
    const int N = cmp ? CMP_N : WIN_N, TT = cmp ? CMP_T : WIN_T;
    const bool row_tail = rc->s1g == s1g_base[rc->b] - 1 && s1g_tail[rc->b] != 0;
    const int r = row_tail ? TT : N;
    cost = tc[r][N] * normal + tc[r][TT] * tail;
    lastc = tail > 0 ? tc[r][TT] : tc[r][N];
    norm = tc[r][N];
  }

  void row_cache(int64_t s1g_idx, const BatchCache& bc, RowCache* rc) {
    if (s1g_base[bc.b] == 0) {
      rc->cost = rc->last_block_cost = 0;
      rc->win_normal = rc->win_last = rc->cmp_normal = rc->cmp_last = 0;
      rc->block = 0;
      rc->s2_start = rc->cmp_s2_start = rc->s2_end = 0;
      return;
    }
    rc->b = bc.b;
    rc->s1g = s1g_idx;
    i128 f, l;
    s2_range(s1g_idx, bc, &f, &l);
    block_range(f, l, bc, rc);
    cost_table(m_base, kS2Base, s1g_tail[rc->b], rc->win_tail, rc->cmp_tail);
    side_cache(rc, false);
    side_cache(rc, true);
    rc->s2_start = rc->win_block > 0 ? rc->win_s2_start : rc->cmp_s2_start;
    if (rc->cmp_block > 0) {
      rc->last_block_cost = rc->cmp_last;
      rc->s2_end = rc->cmp_s2_end;
    } else {
      rc->last_block_cost = rc->win_last;
      rc->s2_end = rc->win_s2_end;
    }
    rc->block = rc->win_block + rc->cmp_block;
    rc->cost = rc->win_cost + rc->cmp_cost;
  }

  void split_info() {
    s1g_base.assign(batch, 0);
    s1g_tail.assign(batch, 0);
    s2_base.assign(batch, 0);
    s2_tail.assign(batch, 0);
    for (int64_t b = 0; b < batch; ++b) {
      const int64_t s1 = s1_size(b), s2 = s2_size(b);
      s1g_base[b] = fdiv(s1 * group + m_base - 1, m_base);
      s1g_tail[b] = fmod_py(s1 * group, m_base);
      s2_base[b] = fdiv(s2 + kS2Base - 1, kS2Base);
      s2_tail[b] = fmod_py(s2, kS2Base);
      if (s1g_base[b] != 0 && s2_base[b] != 0) all_zero = false;
    }
  }

  void cost_info() {
    bn2_cost.assign(batch, 0);
    bn2_block.assign(batch, 0);
    bn2_last.assign(batch, 0);
    if (all_zero) return;
    for (int64_t b = 0; b < batch; ++b) {
      if (s1_size(b) != 0 && s2_size(b) != 0) {
        BatchCache bc;
        RowCache rc;
        batch_cache(b, &bc);
        for (int64_t g = 0; g < s1g_base[b]; ++g) {
          row_cache(g, bc, &rc);
          bn2_cost[b] += rc.cost;
          bn2_block[b] += rc.block;
          max_row_cost = std::max(max_row_cost, rc.cost);
          if (rc.block > 0) bn2_last[b] = rc.last_block_cost;
        }
      }
      total_cost += bn2_cost[b] * nkv;
      total_block += bn2_block[b] * nkv;
    }
  }

  static bool within(int64_t limit, int64_t tol, int64_t value) { return limit + tol >= value; }

  void by_batch(Cursor* c) {
    if (c->finished) return;
    while (c->bn2_cost == 0 || within(c->cc.limit, fdiv(bn2_last[c->b], kTolRatio), c->cc.cost + c->bn2_cost)) {
      c->cc.cost += c->bn2_cost;
      c->cc.block += c->bn2_block;
      c->bn2 += 1;
      if (c->bn2 == batch * nkv) {
        c->s1g = 0;
        c->s2 = 0;
        c->finished = true;
        return;
      }
      if (fdiv(c->bn2, nkv) != c->b) {
        c->b = fdiv(c->bn2, nkv);
        batch_cache(c->b, &c->bc);
      }
      c->bn2_cost = bn2_cost[c->b];
      c->bn2_block = bn2_block[c->b];
      c->s1g = 0;
      row_cache(c->s1g, c->bc, &c->rc);
      c->s2 = c->rc.s2_start;
    }
  }

  void by_row(Cursor* c) {
    if (c->finished) return;
    while (within(c->cc.limit, fdiv(c->rc.last_block_cost, kTolRatio), c->cc.cost + c->rc.cost)) {
      c->cc.cost += c->rc.cost;
      c->cc.block += c->rc.block;
      c->bn2_cost = std::max<int64_t>(0, c->bn2_cost - c->rc.cost);
      c->bn2_block = std::max<int64_t>(0, c->bn2_block - c->rc.block);
      int64_t guard = 0;
      while (true) {
        c->s1g += 1;
        row_cache(c->s1g, c->bc, &c->rc);
        if (c->rc.block != 0) break;
        if (++guard > (int64_t)1 << 26) {  // the reference would not terminate here
          error = true;
          return;
        }
      }
      c->s2 = c->rc.s2_start;
    }
  }

  bool need_record_fd(const Cursor& c) const {
    if (c.core == 0 || c.kv_split_part <= 1) return false;
    if (c.bn2 == bn2_end[c.core - 1] && c.s1g == g_s1_end[c.core - 1]) return false;
    return true;
  }

  void record_fd(Cursor* c) {
    const int64_t sb = fdiv(bn2_end[c->core - 1], nkv);
    const int64_t sg = g_s1_end[c->core - 1];
    const int64_t s1 = s1_size(sb);
    const int64_t msize = sg == s1g_base[sb] - 1 ? s1 * group - sg * m_base : m_base;
    max_s2_split = std::max(max_s2_split, c->kv_split_part);
    fd_bn2[num_fd_head] = bn2_end[c->core - 1];
    fd_m[num_fd_head] = g_s1_end[c->core - 1];
    fd_ws[num_fd_head] = c->fd_data_num - c->kv_split_part;
    fd_split[num_fd_head] = c->kv_split_part;
    fd_msize[num_fd_head] = msize;
    num_fd_head += 1;
  }

  void assign_core(Cursor* c) {
    const int64_t avg = fdiv(c->unassigned, std::max<int64_t>(1, aic - c->core));
    c->cc = CoreCache();
    c->cc.limit = std::max(avg, max_row_cost);  // split-KV (FD) assignment is off, as in the reference
    by_batch(c);
    by_row(c);
    bn2_end[c->core] = c->bn2;
    g_s1_end[c->core] = c->s1g;
    s2_end[c->core] = c->s2;
    max_cost = std::max(max_cost, c->cc.cost);
    c->unassigned -= c->cc.cost;
    if (need_record_fd(*c)) {
      record_fd(c);
      c->kv_split_part = 1;
    }
    if (c->rc.s2_start < c->s2 && c->s2 <= c->rc.s2_end) c->kv_split_part += 1;
  }

  void split_plan() {
    if (aic == 0) return;
    max_cost = 0;
    used_core = 0;
    Cursor c;
    c.b = 0;
    c.s1g = 0;
    c.unassigned = total_cost;
    c.bn2_cost = bn2_cost[0];
    c.bn2_block = bn2_block[0];
    batch_cache(0, &c.bc);
    row_cache(0, c.bc, &c.rc);
    c.s2 = c.rc.s2_start;
    for (int64_t i = 0; i < aic; ++i) {
      if (c.finished || c.unassigned <= 0) break;
      c.core = i;
      assign_core(&c);
      if (error) return;
    }
    used_core = c.core + 1;
  }

  void split_fd() {
    int64_t total = 0;
    for (int64_t i = 0; i < num_fd_head; ++i) total += fd_split[i] * fd_msize[i];
    if (aiv == 0) return;
    const int64_t avg = fdiv(total, aiv);
    if (avg == 0) return;
    int64_t cur = 0;
    for (int64_t i = 0; i < num_fd_head; ++i) {
      const int64_t nvec = fdiv(fd_split[i] * fd_msize[i], avg);
      if (nvec == 0) continue;
      const int64_t am = fdiv(fd_msize[i], nvec);
      for (int64_t v = 0; v < nvec; ++v) {
        if (cur >= (int64_t)fd_idx.size()) break;
        fd_idx[cur] = i;
        fd_mstart[cur] = v * am;
        fd_mnum[cur] = v < nvec - 1 ? am : fd_msize[i] - v * am;
        cur += 1;
      }
    }
    fd_used_vec = cur;
  }

  void run(int32_t* out) {
    params_init();
    bn2_end.assign(aic, 0);
    g_s1_end.assign(aic, 0);
    s2_end.assign(aic, 0);
    first_fd_ws.assign(aic, 0);
    fd_bn2.assign(aic, 0);
    fd_m.assign(aic, 0);
    fd_ws.assign(aic, 0);
    fd_split.assign(aic, 0);
    fd_msize.assign(aic, 0);
    fd_idx.assign(aiv, 0);
    fd_mstart.assign(aiv, 0);
    fd_mnum.assign(aiv, 0);
    split_info();
    if (all_zero) {
      used_core = 1;
      bn2_end[0] = batch * nkv;
      g_s1_end[0] = 0;
      s2_end[0] = 0;
    } else {
      cost_info();
      used_core = 1;
      split_plan();
      if (error) return;
      if (num_fd_head > 0) split_fd();
      used_core = std::max<int64_t>(used_core, 1);
    }
    std::memset(out, 0, sizeof(int32_t) * SAS_META_SIZE);
    for (int64_t i = 0; i < SAS_AIC_CORE_NUM; ++i) {
      int32_t* row = out + i * kFaW;
      if (i >= used_core || i >= aic) continue;
      row[0] = 1;
      row[1] = (int32_t)(i == 0 ? 0 : bn2_end[i - 1]);
      row[2] = (int32_t)(i == 0 ? 0 : g_s1_end[i - 1]);
      row[3] = (int32_t)(i == 0 ? 0 : s2_end[i - 1]);
      row[4] = (int32_t)bn2_end[i];
      row[5] = (int32_t)g_s1_end[i];
      row[6] = (int32_t)s2_end[i];
      row[7] = (int32_t)first_fd_ws[i];
    }
    for (int64_t i = 0; i < SAS_AIV_CORE_NUM; ++i) {
      int32_t* row = out + SAS_AIC_CORE_NUM * kFaW + i * kFdW;
      if (i >= fd_used_vec || i >= aiv) continue;
      const int64_t k = fd_idx[i];
      row[0] = 1;
      row[1] = (int32_t)fd_bn2[k];
      row[2] = (int32_t)fd_m[k];
      row[3] = (int32_t)fd_ws[k];
      row[4] = (int32_t)fd_split[k];
      row[5] = (int32_t)fd_mstart[i];
      row[6] = (int32_t)fd_mnum[i];
    }
  }
};

}  // namespace

extern "C" int sas_metadata_legacy(const sas_meta_args_t* a, const int32_t* cu_seqlens_q,
                                   int32_t n_cu_q, const int32_t* cu_seqlens_ori_kv,
                                   int32_t n_cu_kv, const int32_t* seqused_q, int32_t n_seqused_q,
                                   const int32_t* seqused_kv, int32_t n_seqused_kv, int32_t* out) {
  if (!a || !out) return SAS_ERR_NULL;
  if (a->num_heads_kv <= 0 || a->num_heads_q <= 0 || a->num_heads_q < a->num_heads_kv)
    return SAS_ERR_METADATA;  // the reference divides by the group size
  if (a->aic_core_num < 0 || a->aiv_core_num < 0) return SAS_ERR_METADATA;
  Scheduler s;
  s.nq = a->num_heads_q;
  s.nkv = a->num_heads_kv;
  s.batch = a->batch_size;
  s.max_q = a->max_seqlen_q;
  s.max_kv = a->max_seqlen_kv;
  s.topk = a->cmp_topk;
  s.ratio = a->cmp_ratio;
  s.ori_mask = a->ori_mask_mode;
  s.win_left = a->ori_win_left;
  s.win_right = a->ori_win_right;
  s.layout_q = a->layout_q;
  s.layout_kv = a->layout_kv;
  s.has_cmp = a->has_cmp_kv != 0;
  s.aic = a->aic_core_num;
  s.aiv = a->aiv_core_num;
  auto take = [](const int32_t* p, int32_t n, std::vector<int64_t>* v) {
    if (p && n > 0) v->assign(p, p + n);
  };
  take(cu_seqlens_q, n_cu_q, &s.cu_q);
  take(cu_seqlens_ori_kv, n_cu_kv, &s.cu_kv);
  take(seqused_q, n_seqused_q, &s.used_q);
  take(seqused_kv, n_seqused_kv, &s.used_kv);
  // batch entries the schedule indexes must exist (the reference raises IndexError)
  int64_t B = s.batch;
  if (!s.used_q.empty()) B = (int64_t)s.used_q.size();
  else if (s.layout_q == 1 && !s.cu_q.empty()) B = (int64_t)s.cu_q.size() - 1;
  if (B < 1) return SAS_ERR_METADATA;
  if (!s.used_kv.empty() && (int64_t)s.used_kv.size() < B) return SAS_ERR_METADATA;
  if (s.used_kv.empty() && s.layout_kv == 1 && !s.cu_kv.empty() && (int64_t)s.cu_kv.size() < B + 1)
    return SAS_ERR_METADATA;
  s.run(out);
  return s.error ? SAS_ERR_METADATA : SAS_OK;
}
