// C-ABI of the collapsed GAT (kernels in gat_kernels.h, instantiated in the
// gat_inst_*.hip translation units so they compile in parallel).
#include "gat_fl.h"

namespace cign {
namespace gatk {
CIGN_GAT_DECLARE(float, 4)
CIGN_GAT_DECLARE(float, 8)
CIGN_GAT_DECLARE(float, 32)
CIGN_GAT_DECLARE(bf16, 4)
CIGN_GAT_DECLARE(bf16, 8)
CIGN_GAT_DECLARE(bf16, 32)
CIGN_GAT_FL_DECLARE(float)
CIGN_GAT_FL_DECLARE(bf16)
CIGN_GAT_FL_DECLARE_NARROW(bf16h)
CIGN_GAT_FL_DECLARE(bf16x)
}  // namespace gatk
}  // namespace cign

namespace cign {
namespace gatk {

// ---------------------------------------------------------------------------
// Host dispatch over (HP, CP).
// ---------------------------------------------------------------------------
inline int pow2ceil(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Heads are padded to HP lanes (4, 8 or 32; unused head lanes idle) and
// channels to CP-wide blocks (8, 16 or 32).
template <template <typename, int, int> class Launcher, typename T, typename... Args>
int dispatch_hc(int H, int C, Args&&... args) {
  const int HP = H <= 4 ? 4 : (H <= 8 ? 8 : 32);
  const int CP = C >= 32 ? 32 : (pow2ceil(C) < 8 ? 8 : pow2ceil(C));
#define CIGN_CASE(hp, cp) \
  if (HP == hp && CP == cp) return Launcher<T, hp, cp>::run(args...);
#define CIGN_CASES(hp) CIGN_CASE(hp, 8) CIGN_CASE(hp, 16) CIGN_CASE(hp, 32)
  CIGN_CASES(4) CIGN_CASES(8) CIGN_CASES(32)
#undef CIGN_CASES
#undef CIGN_CASE
  return set_error(kInvalid, "collapsed GAT: unsupported heads=%d channels=%d", H, C);
}

struct BwdLayout {
  int64_t grad_pre, gscore, wsum, bias_part, bias_l2, part_row, part_col, total;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// row_blocks = n_seg + ceil(n_light / 4) of the row schedule; one more bias
// partial is reserved because the feature-layout row grid (light rows split
// into one-per-wave and several-per-wave blocks) can be one block longer.
inline BwdLayout bwd_layout(int n, int nnz, int H, int C, int row_blocks, int n_seg_rows, int n_seg_cols) {
  BwdLayout L;
  row_blocks += 1;
  // Second-level grad_bias partials: (row_blocks + 63) / 64 for the pair
  // layout (partials of row blocks), kFlBiasBlocks for the feature layout
  // (partials of grad_pre rows).
  const int n_l2 = max((row_blocks + 63) / 64, kFlBiasBlocks);
  int64_t off = 0;
  // grad_pre rows of C + 4H floats: the feature layout keeps each row's
  // softmax record after its g_pre; the pair layout uses the first n*C.
  L.grad_pre = off; off = align256(off + 4LL * n * (C + 4LL * H));
  L.gscore = off; off = align256(off + 4LL * nnz * H);
  L.wsum = off; off = align256(off + 4LL * n * H);
  L.bias_part = off; off = align256(off + 4LL * row_blocks * C);
  L.bias_l2 = off; off = align256(off + 4LL * n_l2 * C);
  L.part_row = off; off = align256(off + 4LL * n_seg_rows * 3 * H);
  L.part_col = off; off = align256(off + 4LL * n_seg_cols * (static_cast<int64_t>(H) * C + H));
  L.total = off;
  return L;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int check_shape(const char* who, int n, int nnz, int H, int C) {
  if (n < 0 || nnz < 0) return set_error(kInvalid, "%s: negative sizes", who);
  if (H < 1 || H > kMaxH) return set_error(kInvalid, "%s: heads=%d outside [1, %d]", who, H, kMaxH);
  if (C < 1 || C > kMaxC) return set_error(kInvalid, "%s: channels=%d outside [1, %d]", who, C, kMaxC);
  return kOk;
}

__global__ void zero_floats(float* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// Feature-layout geometry of a shape: lanes per row L and chunks per lane V,
// or false. H <= 8 heads, C a multiple of the 16-byte chunk width W with cq =
// C/W a power of two (head sums and per-head dot products are butterflies
// over lane bits); narrow rows (H*cq <= 64 chunks) take L = pow2ceil(H*cq),
// V = 1; wide rows take L = 64 and V = H*cq/64 in {2, 3, 4, 6, 8} (cq <= 64
// divides 64, so a lane's chunks share one channel chunk).
inline bool fl_geom_w(int W, int H, int C, int& L, int& V) {
  const int cq = C / W;
  if (H < 1 || H > kFlHeads || C % W != 0 || cq < 1 || (cq & (cq - 1)) != 0) return false;
  const int nq = H * cq;
  if (nq <= kWave) {
    L = 1;
    while (L < nq) L <<= 1;
    V = 1;
    return true;
  }
  if (cq > kWave || nq % kWave != 0) return false;
  L = kWave;
  V = nq / kWave;
  return V == 2 || V == 3 || V == 4 || V == 6 || V == 8;
}

inline bool fl_geom(int dtype, int H, int C, int& L, int& V) {
  return fl_geom_w(dtype == kBF16 || dtype == kBF16F32 ? 8 : 4, H, C, L, V);
}

inline bool fl_ok(int dtype, int H, int C) {
  int L, V;
  return fl_geom(dtype, H, C, L, V);
}

// Whether bf16 features run the feature-layout kernels four values per lane
// (bf16h): graphs below the large-graph threshold, shapes whose rows stay
// narrow that way. At 211K edges (4 x 16 channels) a row then takes 16 lanes
// like fp32 instead of 8, each with half the work, which a launch of a few
// dependent memory rounds is bound by.
inline bool fl_half(int dtype, int H, int C, int64_t graph_nnz) {
  int L, V;
  return dtype == kBF16 && graph_nnz < big_graph_edges() && fl_ok(dtype, H, C) && fl_geom_w(4, H, C, L, V) &&
         V == 1;
}

// Calls go(integral_constant<L>, integral_constant<V>) for an instantiated
// (L, V) of the feature-layout kernels.
template <typename Go>
int fl_dispatch(int L, int V, Go&& go) {
  using std::integral_constant;
  if (V == 1) {
    switch (L) {
      case 1: return go(integral_constant<int, 1>(), integral_constant<int, 1>());
      case 2: return go(integral_constant<int, 2>(), integral_constant<int, 1>());
      case 4: return go(integral_constant<int, 4>(), integral_constant<int, 1>());
      case 8: return go(integral_constant<int, 8>(), integral_constant<int, 1>());
      case 16: return go(integral_constant<int, 16>(), integral_constant<int, 1>());
      case 32: return go(integral_constant<int, 32>(), integral_constant<int, 1>());
      default: return go(integral_constant<int, 64>(), integral_constant<int, 1>());
    }
  }
  switch (V) {
    case 2: return go(integral_constant<int, 64>(), integral_constant<int, 2>());
    case 3: return go(integral_constant<int, 64>(), integral_constant<int, 3>());
    case 4: return go(integral_constant<int, 64>(), integral_constant<int, 4>());
    case 6: return go(integral_constant<int, 64>(), integral_constant<int, 6>());
    default: return go(integral_constant<int, 64>(), integral_constant<int, 8>());
  }
}

// fl_dispatch for the narrow rows (V = 1) only.
template <typename Go>
int fl_dispatch_narrow(int L, Go&& go) {
  using std::integral_constant;
  switch (L) {
    case 1: return go(integral_constant<int, 1>(), integral_constant<int, 1>());
    case 2: return go(integral_constant<int, 2>(), integral_constant<int, 1>());
    case 4: return go(integral_constant<int, 4>(), integral_constant<int, 1>());
    case 8: return go(integral_constant<int, 8>(), integral_constant<int, 1>());
    case 16: return go(integral_constant<int, 16>(), integral_constant<int, 1>());
    case 32: return go(integral_constant<int, 32>(), integral_constant<int, 1>());
    default: return go(integral_constant<int, 64>(), integral_constant<int, 1>());
  }
}

inline int fl_lgcq_w(int W, int C) {
  int lg = 0;
  while ((1 << lg) < C / W) ++lg;
  return lg;
}

// Schedule geometry (light_max, seg_edges) each GAT pass runs on. The
// feature-layout kernels take any segment length that is a multiple of their
// 256-edge round (reported as seg_edges = 0, "any"); the pair-layout kernels
// need exactly kGatSeg.
inline void gat_geometry(int pass, int dtype, int H, int C, int& light, int& seg) {
  if (fl_ok(dtype, H, C)) {
    light = kFlLightMax;
    seg = 0;
  } else {
    light = kGatLight;
    seg = kGatSeg;
  }
}

// Host view of a schedule header (schedule.h).
struct Hdr {
  int n_light, n_seg, n_hrow;
};

inline int read_hdr(const char* who, const int32_t* info, int n, int light, int seg, Hdr& h) {
  if (!info) return set_error(kInvalid, "%s: null schedule header", who);
  h.n_light = info[0];
  h.n_seg = info[1];
  h.n_hrow = info[2];
  if (h.n_light + h.n_hrow != n) return set_error(kInvalid, "%s: schedule does not cover %d rows", who, n);
  const bool seg_ok = seg == 0 ? (info[3] > 0 && info[3] % kSegRound == 0) : info[3] == seg;
  if (info[4] != light || !seg_ok)
    return set_error(kInvalid, "%s: schedule built with light_max=%d seg_edges=%d; this pass needs light_max=%d and "
                     "seg_edges %s%d (cign_gat_schedule_params)", who, info[4], info[3], light,
                     seg == 0 ? "a multiple of " : "", seg == 0 ? kSegRound : seg);
  return kOk;
}

}  // namespace gatk
}  // namespace cign

using namespace cign;
using namespace cign::gatk;

extern "C" {

// Schedule geometry (light_max, seg_edges) the GAT pass (0 = forward on the
// CSR, 1 = backward on the CSR and the CSC) needs for this dtype / shape.
int cign_gat_schedule_params(int32_t pass, int32_t dtype, int32_t heads, int32_t channels, int32_t* light_max,
                             int32_t* seg_edges) {
  if (!light_max || !seg_edges) return set_error(kInvalid, "cign_gat_schedule_params: null output");
  int l, s;
  gat_geometry(pass, dtype, heads, channels, l, s);
  *light_max = l;
  *seg_edges = s;
  return kOk;
}

// fp32 workspace needed by cign_gat_fwd for a row schedule with n_seg
// segments: one partial {acc, accl, m, s, bl} per segment.
int64_t cign_gat_fwd_workspace_bytes(int32_t n_seg, int32_t heads, int32_t channels) {
  return 4LL * n_seg * (2LL * heads * channels + 3LL * heads);
}

// Floats of the per-row aggregate buffer of cign_gat_fwd / cign_gat_bwd for
// this shape, 0 when the shape's kernels do not use one.
int64_t cign_gat_row_agg_floats(int32_t dtype, int32_t n, int32_t heads, int32_t channels) {
  if (n < 0 || heads < 1 || channels < 1 || !fl_ok(dtype, heads, channels)) return 0;
  return static_cast<int64_t>(n) * heads * (2LL * channels + 1);
}

// Collapsed GAT forward. Replaces the ext `forward` of the reference
// (collapsed_gat_ext/collapsed_gat.cpp:45-72 -> collapsed_gat_cuda.cu:434-478).
}  // extern "C"

namespace {

// cign_gat_fwd over the whole graph (edge_base 0, graph_nnz = nnz) or one
// destination-row shard of it.
int gat_fwd_impl(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 const float* attn_row, const float* attn_col, const int32_t* col, const int32_t* row_sched,
                 const int32_t* row_sched_info, int32_t* row_counters, float negative_slope, const void* in_feat,
                 const float* bias, float attn_drop, uint64_t seed, void* out, float* pre, float* edge_max,
                 float* edge_sum, uint8_t* edge_mask, void* workspace, int64_t workspace_bytes, float* row_agg,
                 int64_t edge_base, int64_t graph_nnz) {
  int rc = check_shape("cign_gat_fwd", n, nnz, heads, channels);
  if (rc) return rc;
  if (!(attn_drop >= 0.0f && attn_drop < 1.0f)) return set_error(kInvalid, "cign_gat_fwd: attn_drop must be in [0,1)");
  Hdr hd;
  int light, seg;
  gat_geometry(0, dtype, heads, channels, light, seg);
  if ((rc = read_hdr("cign_gat_fwd", row_sched_info, n, light, seg, hd))) return rc;
  if (workspace_bytes < cign_gat_fwd_workspace_bytes(hd.n_seg, heads, channels))
    return set_error(kInvalid, "cign_gat_fwd: workspace too small");
  if (row_agg && (cign_gat_row_agg_floats(dtype, n, heads, channels) == 0 || !aligned16(row_agg)))
    return set_error(kInvalid, "cign_gat_fwd: row_agg must be null for this shape (cign_gat_row_agg_floats) or "
                     "16-byte aligned");
  if (n == 0) return kOk;
  const Sched s = make_sched(row_sched, hd.n_light, hd.n_seg, hd.n_hrow);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto fill = [&](auto* xt, auto* ot) {
    using T = std::remove_cv_t<std::remove_pointer_t<decltype(xt)>>;
    GatFwdArgs<T> a;
    a.n = n; a.H = heads; a.C = channels; a.graph_nnz = graph_nnz; a.mask_base = edge_base * heads;
    a.slope = negative_slope; a.p = attn_drop; a.seed = seed;
    a.vec = aligned16(xt) && (channels * static_cast<int>(sizeof(T))) % 16 == 0;
    a.attn_row = attn_row; a.attn_col = attn_col; a.col = col;
    a.x = xt; a.bias = bias; a.out = ot; a.pre = pre; a.emax = edge_max; a.esum = edge_sum;
    a.mask = edge_mask; a.partial = static_cast<float*>(workspace); a.counters = row_counters;
    a.agg = row_agg;
    int L, V;
    if (fl_geom_w(FlGeom<T>::W, heads, channels, L, V)) {
      if (!aligned16(xt) || !aligned16(ot) || !aligned16(pre))
        return set_error(kInvalid, "cign_gat_fwd: in_feat, out and pre must be 16-byte aligned");
      const int lgcq = fl_lgcq_w(FlGeom<T>::W, channels);
      auto go = [&](auto LC, auto VC) {
        return FwdFlLauncher<T, decltype(LC)::value, decltype(VC)::value>::run(st, a, s, row_sched_info, lgcq);
      };
      if constexpr (std::is_same_v<T, bf16h>) return fl_dispatch_narrow(L, go);  // fl_half: V = 1
      else return fl_dispatch(L, V, go);
    }
    if constexpr (std::is_same_v<T, bf16h>) return set_error(kInvalid, "cign_gat_fwd: bf16h needs a narrow shape");
    else if constexpr (std::is_same_v<T, bf16x>)
      return set_error(kInvalid, "cign_gat_fwd: dtype 2 (bf16 features, fp32 outputs) needs a feature-layout shape "
                       "(cign_gat_row_agg_floats > 0)");
    else return dispatch_hc<FwdLauncher, T>(heads, channels, st, a, s);
  };
  if (dtype == kF32) return fill(static_cast<const float*>(in_feat), static_cast<float*>(out));
  if (dtype == kBF16 && fl_half(dtype, heads, channels, graph_nnz))
    return fill(static_cast<const bf16h*>(in_feat), static_cast<bf16h*>(out));
  if (dtype == kBF16) return fill(static_cast<const bf16*>(in_feat), static_cast<bf16*>(out));
  if (dtype == kBF16F32) return fill(static_cast<const bf16x*>(in_feat), static_cast<float*>(out));
  return set_error(kInvalid, "cign_gat_fwd: unsupported dtype %d", dtype);
}

}  // namespace

extern "C" {

int cign_gat_fwd(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 const float* attn_row, const float* attn_col, const int32_t* col, const int32_t* row_sched,
                 const int32_t* row_sched_info, int32_t* row_counters, float negative_slope, const void* in_feat,
                 const float* bias, float attn_drop, uint64_t seed, void* out, float* pre, float* edge_max,
                 float* edge_sum, uint8_t* edge_mask, void* workspace, int64_t workspace_bytes, float* row_agg) {
  return gat_fwd_impl(stream, dtype, n, nnz, heads, channels, attn_row, attn_col, col, row_sched, row_sched_info,
                      row_counters, negative_slope, in_feat, bias, attn_drop, seed, out, pre, edge_max, edge_sum,
                      edge_mask, workspace, workspace_bytes, row_agg, 0, nnz);
}

int cign_gat_fwd_shard(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                       const float* attn_row, const float* attn_col, const int32_t* col, const int32_t* row_sched,
                       const int32_t* row_sched_info, int32_t* row_counters, float negative_slope,
                       const void* in_feat, const float* bias, float attn_drop, uint64_t seed, void* out, float* pre,
                       float* edge_max, float* edge_sum, uint8_t* edge_mask, void* workspace,
                       int64_t workspace_bytes, float* row_agg, int64_t edge_base, int64_t graph_nnz) {
  if (edge_base < 0 || graph_nnz < nnz || edge_base > graph_nnz - nnz)
    return set_error(kInvalid, "cign_gat_fwd_shard: edges [%lld, %lld) outside a graph of %lld edges",
                     static_cast<long long>(edge_base), static_cast<long long>(edge_base) + nnz,
                     static_cast<long long>(graph_nnz));
  return gat_fwd_impl(stream, dtype, n, nnz, heads, channels, attn_row, attn_col, col, row_sched, row_sched_info,
                      row_counters, negative_slope, in_feat, bias, attn_drop, seed, out, pre, edge_max, edge_sum,
                      edge_mask, workspace, workspace_bytes, row_agg, edge_base, graph_nnz);
}

int64_t cign_gat_bwd_workspace_bytes(int32_t n, int32_t nnz, int32_t heads, int32_t channels, int32_t row_blocks,
                                     int32_t n_seg_rows, int32_t n_seg_cols) {
  return bwd_layout(n, nnz, heads, channels, row_blocks, n_seg_rows, n_seg_cols).total;
}

}  // extern "C"

namespace {

// cign_gat_bwd over the whole graph (bias rows [0, n), graph_nnz = nnz) or
// one source-column shard of it.
int gat_bwd_impl(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 float negative_slope, float attn_drop, const int32_t* col, const int32_t* rowind,
                 const int32_t* perm, const float* edge_max, const float* edge_sum, const uint8_t* edge_mask,
                 const void* in_feat, const float* attn_row, const float* attn_col, const float* pre,
                 const void* grad_y, const int32_t* row_sched, const int32_t* row_sched_info,
                 int32_t* row_counters, const int32_t* col_sched, const int32_t* col_sched_info,
                 int32_t* col_counters, void* workspace, int64_t workspace_bytes, void* grad_feat,
                 float* grad_attn_row, float* grad_attn_col, float* grad_bias, const float* row_agg,
                 int32_t bias_lo, int32_t bias_n, int64_t graph_nnz) {
  int rc = check_shape("cign_gat_bwd", n, nnz, heads, channels);
  if (row_agg && (cign_gat_row_agg_floats(dtype, n, heads, channels) == 0 || !aligned16(row_agg)))
    return set_error(kInvalid, "cign_gat_bwd: row_agg must be null for this shape (cign_gat_row_agg_floats) or "
                     "16-byte aligned");
  if (rc) return rc;
  if (!(attn_drop >= 0.0f && attn_drop < 1.0f)) return set_error(kInvalid, "cign_gat_bwd: attn_drop must be in [0,1)");
  Hdr rh, ch;
  int light, seg;
  gat_geometry(1, dtype, heads, channels, light, seg);
  if ((rc = read_hdr("cign_gat_bwd (rows)", row_sched_info, n, light, seg, rh))) return rc;
  if ((rc = read_hdr("cign_gat_bwd (cols)", col_sched_info, n, light, seg, ch))) return rc;
  const Sched rs = make_sched(row_sched, rh.n_light, rh.n_seg, rh.n_hrow);
  const Sched cs = make_sched(col_sched, ch.n_light, ch.n_seg, ch.n_hrow);
  const int row_blocks = sched_blocks(rs);
  const BwdLayout L = bwd_layout(n, nnz, heads, channels, row_blocks, rh.n_seg, ch.n_seg);
  if (workspace_bytes < L.total) return set_error(kInvalid, "cign_gat_bwd: workspace too small (%lld < %lld)",
                                                  static_cast<long long>(workspace_bytes), static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n == 0) {
    hipLaunchKernelGGL(zero_floats, dim3((channels + kBlock - 1) / kBlock), dim3(kBlock), 0, st, grad_bias, channels);
    return check_launch("cign_gat_bwd");
  }
  char* ws = static_cast<char*>(workspace);
  auto fill = [&](auto* xt, auto* gyt, auto* gxt) {
    using T = std::remove_cv_t<std::remove_pointer_t<decltype(xt)>>;
    GatBwdArgs<T> a;
    a.n = n; a.nnz = nnz; a.H = heads; a.C = channels;
    a.graph_nnz = graph_nnz; a.bias_lo = bias_lo; a.bias_n = bias_n;
    a.slope = negative_slope; a.p = attn_drop; a.inv_h = 1.0f / static_cast<float>(heads);
    a.vec_x = aligned16(xt) && (channels * static_cast<int>(sizeof(T))) % 16 == 0;
    a.vec_gp = (channels % 4) == 0;
    a.col = col; a.rowind = rowind; a.perm = perm;
    a.emax = edge_max; a.esum = edge_sum; a.mask = edge_mask; a.x = xt;
    a.attn_row = attn_row; a.attn_col = attn_col; a.pre = pre; a.grad_y = gyt; a.agg = row_agg;
    a.grad_pre = reinterpret_cast<float*>(ws + L.grad_pre);
    a.gp_stride = channels;
    a.rowstat = nullptr;
    a.rs_stride = 0;
    a.gscore = reinterpret_cast<float*>(ws + L.gscore);
    a.wsum = reinterpret_cast<float*>(ws + L.wsum);
    a.bias_part = reinterpret_cast<float*>(ws + L.bias_part);
    a.bias_l2 = reinterpret_cast<float*>(ws + L.bias_l2);
    a.part_row = reinterpret_cast<float*>(ws + L.part_row);
    a.part_col = reinterpret_cast<float*>(ws + L.part_col);
    a.row_counters = row_counters; a.col_counters = col_counters;
    a.grad_feat = gxt; a.grad_attn_row = grad_attn_row; a.grad_attn_col = grad_attn_col; a.grad_bias = grad_bias;
    int FL, FV;
    if (fl_geom_w(FlGeom<T>::W, heads, channels, FL, FV)) {
      if (!aligned16(xt) || !aligned16(gyt) || !aligned16(gxt) || !aligned16(pre) || !aligned16(grad_bias))
        return set_error(kInvalid, "cign_gat_bwd: in_feat, pre, grad_y, grad_feat and grad_bias must be 16-byte "
                                   "aligned");
      // one contiguous record per destination row: g_pre, then H float4s
      a.gp_stride = channels + 4 * heads;
      a.rowstat = reinterpret_cast<float4*>(a.grad_pre + channels);
      a.rs_stride = a.gp_stride / 4;
      const int lgcq = fl_lgcq_w(FlGeom<T>::W, channels);
      auto go = [&](auto LC, auto VC) {
        constexpr int LL = decltype(LC)::value, VV = decltype(VC)::value;
        a.rows_blocks = BwdFlLauncher<T, LL, VV>::row_blocks(rs, row_sched_info);
        a.n_l2 = fl_bias_blocks(bias_n);
        return BwdFlLauncher<T, LL, VV>::run(st, a, rs, row_sched_info, cs, col_sched_info, lgcq);
      };
      if constexpr (std::is_same_v<T, bf16h>) return fl_dispatch_narrow(FL, go);  // fl_half: V = 1
      else return fl_dispatch(FL, FV, go);
    }
    a.rows_blocks = row_blocks;
    a.n_l2 = (row_blocks + 63) / 64;
    if constexpr (std::is_same_v<T, bf16h>) return set_error(kInvalid, "cign_gat_bwd: bf16h needs a narrow shape");
    else if constexpr (std::is_same_v<T, bf16x>)
      return set_error(kInvalid, "cign_gat_bwd: dtype 2 (bf16 features, fp32 outputs) needs a feature-layout shape "
                       "(cign_gat_row_agg_floats > 0)");
    else return dispatch_hc<BwdLauncher, T>(heads, channels, st, a, rs, cs);
  };
  if (dtype == kF32)
    return fill(static_cast<const float*>(in_feat), static_cast<const float*>(grad_y), static_cast<float*>(grad_feat));
  if (dtype == kBF16 && fl_half(dtype, heads, channels, graph_nnz))
    return fill(static_cast<const bf16h*>(in_feat), static_cast<const bf16h*>(grad_y), static_cast<bf16h*>(grad_feat));
  if (dtype == kBF16)
    return fill(static_cast<const bf16*>(in_feat), static_cast<const bf16*>(grad_y), static_cast<bf16*>(grad_feat));
  if (dtype == kBF16F32)
    return fill(static_cast<const bf16x*>(in_feat), static_cast<const float*>(grad_y), static_cast<float*>(grad_feat));
  return set_error(kInvalid, "cign_gat_bwd: unsupported dtype %d", dtype);
}

}  // namespace

extern "C" {

// Collapsed GAT backward. Replaces the ext `backward` of the reference
// (collapsed_gat_ext/collapsed_gat.cpp:74-102 -> collapsed_gat_cuda.cu:480-545).
int cign_gat_bwd(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 float negative_slope, float attn_drop, const int32_t* col, const int32_t* rowind,
                 const int32_t* perm, const float* edge_max, const float* edge_sum, const uint8_t* edge_mask,
                 const void* in_feat, const float* attn_row, const float* attn_col, const float* pre,
                 const void* grad_y, const int32_t* row_sched, const int32_t* row_sched_info,
                 int32_t* row_counters, const int32_t* col_sched, const int32_t* col_sched_info,
                 int32_t* col_counters, void* workspace, int64_t workspace_bytes, void* grad_feat,
                 float* grad_attn_row, float* grad_attn_col, float* grad_bias, const float* row_agg) {
  return gat_bwd_impl(stream, dtype, n, nnz, heads, channels, negative_slope, attn_drop, col, rowind, perm, edge_max,
                      edge_sum, edge_mask, in_feat, attn_row, attn_col, pre, grad_y, row_sched, row_sched_info,
                      row_counters, col_sched, col_sched_info, col_counters, workspace, workspace_bytes, grad_feat,
                      grad_attn_row, grad_attn_col, grad_bias, row_agg, 0, n, nnz);
}

int cign_gat_bwd_shard(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                       float negative_slope, float attn_drop, const int32_t* col, const int32_t* rowind,
                       const int32_t* perm, const float* edge_max, const float* edge_sum, const uint8_t* edge_mask,
                       const void* in_feat, const float* attn_row, const float* attn_col, const float* pre,
                       const void* grad_y, const int32_t* row_sched, const int32_t* row_sched_info,
                       int32_t* row_counters, const int32_t* col_sched, const int32_t* col_sched_info,
                       int32_t* col_counters, void* workspace, int64_t workspace_bytes, void* grad_feat,
                       float* grad_attn_row, float* grad_attn_col, float* grad_bias, const float* row_agg,
                       int32_t bias_row_lo, int32_t bias_rows, int64_t graph_nnz) {
  if (!row_agg || cign_gat_row_agg_floats(dtype, n, heads, channels) == 0)
    return set_error(kInvalid, "cign_gat_bwd_shard: needs the forward's row_agg (a feature-layout shape): the halo "
                     "destination rows have only part of their in-edges in a column shard");
  if (bias_row_lo < 0 || bias_rows < 0 || bias_row_lo > n - bias_rows)
    return set_error(kInvalid, "cign_gat_bwd_shard: bias rows [%d, %d) outside [0, %d)", bias_row_lo,
                     bias_row_lo + bias_rows, n);
  if (graph_nnz < nnz) return set_error(kInvalid, "cign_gat_bwd_shard: graph_nnz %lld < shard edges %d",
                                        static_cast<long long>(graph_nnz), nnz);
  return gat_bwd_impl(stream, dtype, n, nnz, heads, channels, negative_slope, attn_drop, col, rowind, perm, edge_max,
                      edge_sum, edge_mask, in_feat, attn_row, attn_col, pre, grad_y, row_sched, row_sched_info,
                      row_counters, col_sched, col_sched_info, col_counters, workspace, workspace_bytes, grad_feat,
                      grad_attn_row, grad_attn_col, grad_bias, row_agg, bias_row_lo, bias_rows, graph_nnz);
}

}  // extern "C"
