// Dense-rotation query preparation, split planning and the C-ABI entry of
// attention.  The attention work itself is the fused kernel of tq_attn_impl.h.
#include <algorithm>
#include <mutex>

#include "tq_attn_general.h"
#include "tq_attn_splitmerge.h"

namespace tq {

// ------------------------------------------------------------------ qprep ---
// Dense rotation only:
//   q_s = round_qdtype(q * scale_q)     (MLX weak-scalar multiply, :5802)
//   q_rot = q_s @ R_K^T                 (turboquant_cache.py:4144)
// Block (row block, coordinate block) computes q_rot[r][i] for QR query rows
// and 64 coordinates i.  Thread (i, quarter jq) holds the quarter jq of row
// i of R_K in registers and forms partial dot products with every query row
// of the block (the rows are LDS broadcasts: a wave shares jq); the four
// partials of (r, i) fold through LDS.  R_K crosses L2 once per QR query
// rows.  The launch is latency-bound (a few query rows per kv head), so QR is
// the largest of 16, 8, 4 that still gives one workgroup per CU.
constexpr int kQprepThreads = 256;

template <int QDT, int D, int QR>
__global__ __launch_bounds__(kQprepThreads) void qprep_kernel(AttnParams p, int64_t n_rows) {
  constexpr int JL = D / 4;  // coordinates j per thread
  __shared__ float4 s_q4[QR][D / 4];
  __shared__ float s_part[4][QR][64];
  const int tid = threadIdx.x;
  const int il = tid % 64;
  const int jq = tid / 64;
  const int i = blockIdx.y * 64 + il;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * QR;
  float4 rv[JL / 4];
  const float4* src = reinterpret_cast<const float4*>(p.krot + static_cast<int64_t>(i) * D + jq * JL);
#pragma unroll
  for (int m = 0; m < JL / 4; ++m) rv[m] = src[m];
  // query rows: thread (row r, segment) loads SEG consecutive elements with
  // independent loads (one index computation per thread)
  static_assert(kQprepThreads % QR == 0 && D * QR % kQprepThreads == 0, "one segment per thread");
  {
    constexpr int TPR = kQprepThreads / QR;  // threads per row
    constexpr int SEG = D / TPR;
    float* s_q = reinterpret_cast<float*>(s_q4);
    const int r = tid / TPR;
    const int j0 = (tid % TPR) * SEG;
    const int64_t row = row0 + r;  // (b*Hq + h)*L + l
    float v[SEG];
    if (row < n_rows) {
      // 32-bit index math (tq_attention rejects 2^31 rows or more)
      const int row32 = static_cast<int>(row);
      const int l = row32 % p.L;
      const int bh = row32 / p.L;
      const int h = bh % p.Hq;
      const int b = bh / p.Hq;
      const int64_t base = b * p.q_sb + h * p.q_sh + l * p.q_sl + j0;
#pragma unroll
      for (int e = 0; e < SEG; ++e) v[e] = load_elem<QDT>(p.q, base + e);
#pragma unroll
      for (int e = 0; e < SEG; ++e) v[e] = round_to<QDT>(v[e] * p.scale_q);
    } else {
#pragma unroll
      for (int e = 0; e < SEG; ++e) v[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < SEG; ++e) s_q[r * D + j0 + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int m = 0; m < JL / 4; ++m) {
      const float4 q = s_q4[r][jq * (JL / 4) + m];
      acc = fmaf(q.x, rv[m].x, acc);
      acc = fmaf(q.y, rv[m].y, acc);
      acc = fmaf(q.z, rv[m].z, acc);
      acc = fmaf(q.w, rv[m].w, acc);
    }
    s_part[jq][r][il] = acc;
  }
  __syncthreads();
  for (int o = tid; o < QR * 64; o += kQprepThreads) {
    const int r = o / 64;
    const int c = o % 64;
    if (row0 + r < n_rows)
      p.qrot[(row0 + r) * D + blockIdx.y * 64 + c] =
          (s_part[0][r][c] + s_part[1][r][c]) + (s_part[2][r][c] + s_part[3][r][c]);
  }
}

template <int D, int QR>
void launch_qprep_qr(const AttnParams& p, int q_dtype, int64_t rows, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((rows + QR - 1) / QR), D / 64);
  switch (q_dtype) {
    case TQ_DTYPE_F32: hipLaunchKernelGGL((qprep_kernel<TQ_DTYPE_F32, D, QR>), grid, dim3(kQprepThreads), 0, st, p, rows); break;
    case TQ_DTYPE_F16: hipLaunchKernelGGL((qprep_kernel<TQ_DTYPE_F16, D, QR>), grid, dim3(kQprepThreads), 0, st, p, rows); break;
    default: hipLaunchKernelGGL((qprep_kernel<TQ_DTYPE_BF16, D, QR>), grid, dim3(kQprepThreads), 0, st, p, rows); break;
  }
}

template <int D>
void launch_qprep(const AttnParams& p, int q_dtype, int64_t rows, hipStream_t st) {
  const int64_t blocks16 = (rows + 15) / 16 * (D / 64);
  const int64_t cus = device_cu_count();
  if (blocks16 >= cus)
    launch_qprep_qr<D, 16>(p, q_dtype, rows, st);
  else if (2 * blocks16 >= cus)
    launch_qprep_qr<D, 8>(p, q_dtype, rows, st);
  else
    launch_qprep_qr<D, 4>(p, q_dtype, rows, st);
}

// ------------------------------------------------------------- planning ---
bool small_rows_path(int kv_kind, int D, int rows) {
  return kv_kind == TQ_KV_PACKED && D <= 128 && rows <= 4;
}

bool rows16_path(int kv_kind, int D, int rows) {
  return kv_kind == TQ_KV_PACKED && D == 128 && rows > 4;
}

SplitPlan plan_splits(int B, int Hq, int Hkv, int L, int64_t T, int D, bool packed) {
  SplitPlan sp{};
  const int R = Hq / Hkv;
  const int rows = R * L;
  // matrix-core kernels (packed and plain): 16-row tiles; 4-row groups when
  // the GQA group is small (less LDS and fewer partial rows), and for d = 256
  // (registers).  A row group reads its kv head's cache once.
  (void)packed;
  sp.nq = (rows <= 4 || D >= 256) ? 4 : 16;
  sp.n_rg = (rows + sp.nq - 1) / sp.nq;
  const int64_t base = static_cast<int64_t>(B) * Hkv * sp.n_rg;
  // one workgroup in flight per CU (measured at the 32k-token decode: two or
  // three per CU, with twice or three times the splits, ran slower)
  const int64_t target = device_cu_count();
  int64_t ns = base > 0 ? (target + base - 1) / base : 1;
  const int64_t max_by_tokens = std::max<int64_t>(1, (T + 255) / 256);
  ns = std::max<int64_t>(1, std::min(ns, max_by_tokens));
  int64_t chunk = (T + ns - 1) / ns;
  chunk = std::max<int64_t>(256, (chunk + 255) / 256 * 256);  // whole sub-chunks for every wave
  chunk = std::min<int64_t>(chunk, kMaxChunk);
  sp.chunk = static_cast<int>(chunk);
  sp.n_splits = static_cast<int>(std::max<int64_t>(1, (T + chunk - 1) / chunk));
  return sp;
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Layout: [q_rot B*Hq*L*D][partial o groups*splits*nq*D]
// [partial (m, l) groups*splits*nq*2], groups = B * Hkv * n_rg.
int64_t workspace_bytes(const SplitPlan& sp, int B, int Hq, int Hkv, int L, int D) {
  const int64_t rows = static_cast<int64_t>(B) * Hq * L;
  const int64_t grows = static_cast<int64_t>(B) * Hkv * sp.n_rg * sp.nq;  // padded rows
  return align256(rows * D * 4) + align256(grows * sp.n_splits * D * 4) +
         align256(grows * sp.n_splits * 2 * 4);
}


}  // namespace tq

using namespace tq;

namespace {

// Workspace of one attention call: the larger of the tuned kernels' layout
// (either cache kind) and the general kernels' (the shapes outside the tuned
// ones); Prod keys add a projected-query region to the latter.
int64_t attention_workspace_bytes(int B, int Hq, int Hkv, int L, int dim, int64_t max_tokens, bool prod) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || dim <= 0 || max_tokens < 0 || Hq % Hkv)
    return 0;
  const int64_t T = std::max<int64_t>(max_tokens, 1);
  const int64_t tuned =
      std::max(workspace_bytes(plan_splits(B, Hq, Hkv, L, T, dim, true), B, Hq, Hkv, L, dim),
               workspace_bytes(plan_splits(B, Hq, Hkv, L, T, dim, false), B, Hq, Hkv, L, dim));
  return std::max(tuned, general_workspace_bytes(B, Hq, Hkv, L, dim, dim, T, prod));
}

}  // namespace

extern "C" int64_t tq_attention_workspace_size(int B, int Hq, int Hkv, int L, int dim,
                                               int64_t max_tokens) {
  return attention_workspace_bytes(B, Hq, Hkv, L, dim, max_tokens, false);
}

extern "C" int64_t tq_attention_prod_workspace_size(int B, int Hq, int Hkv, int L, int dim,
                                                    int64_t max_tokens) {
  return attention_workspace_bytes(B, Hq, Hkv, L, dim, max_tokens, true);
}

namespace {

// The key side of Prod-coded keys (tq_attention_prod); k / k_norms carry the
// MSE part at k_bits = bits - 1.
struct ProdKeys {
  const void* signs;
  const void* rnorms;
  const float* proj;
};

int attention_impl(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                   int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l, float scale,
                   int kv_kind, int kv_dtype, const void* k, const void* k_norms, const void* v,
                   const void* v_norms, int norm_dtype, int k_bits, int v_bits,
                   const float* k_codebook, const float* v_codebook, int rot_kind,
                   const float* k_rot, const float* v_rot, int64_t capacity, int64_t max_tokens,
                   const int32_t* seq_starts, const int32_t* seq_lens, int causal, void* out,
                   void* workspace, int64_t workspace_bytes_given, void* stream,
                   const ProdKeys* prod) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || L < 1 || Hq % Hkv)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: bad heads/L (Hq %d, Hkv %d, L %d)", Hq, Hkv, L);
  // Shapes outside the tuned kernels (other head dims; Prod keys beyond
  // d <= 128 and 4 rows per kv head, or 1-bit Prod) run the general kernels.
  const bool tuned_dim = dim == 64 || dim == 128 || dim == 256;
  const bool prod_small = prod && dim <= 128 && static_cast<int64_t>(Hq / Hkv) * L <= 4 && k_bits >= 1;
  const bool tile = !prod && tile_rows_path(kv_kind, dim, dim, (Hq / Hkv) * L);
  if (!tuned_dim || (prod && !prod_small) || tile) {
    GenCall c{};
    c.q = q;
    c.q_dtype = q_dtype;
    c.B = B;
    c.Hq = Hq;
    c.Hkv = Hkv;
    c.L = L;
    c.Dk = dim;
    c.Dv = dim;
    c.q_sb = q_stride_b;
    c.q_sh = q_stride_h;
    c.q_sl = q_stride_l;
    c.scale = scale;
    c.kv_kind = kv_kind;
    c.kv_dtype = kv_dtype;
    c.k = k;
    c.k_norms = k_norms;
    c.k_signs = prod ? prod->signs : nullptr;
    c.k_rnorms = prod ? prod->rnorms : nullptr;
    c.k_bits = prod ? k_bits + 1 : k_bits;  // the Prod width
    c.k_codebook = k_codebook;
    c.k_rot_kind = rot_kind;
    c.k_rot = k_rot;
    c.projection = prod ? prod->proj : nullptr;
    c.v = v;
    c.v_norms = v_norms;
    c.v_bits = v_bits;
    c.v_codebook = v_codebook;
    c.v_rot_kind = rot_kind;
    c.v_rot = v_rot;
    c.norm_dtype = norm_dtype;
    c.capacity = capacity;
    c.max_tokens = max_tokens;
    c.seq_starts = seq_starts;
    c.seq_lens = seq_lens;
    c.causal = causal;
    c.mask_kind = TQ_MASK_NONE;
    c.out = out;
    c.workspace = workspace;
    c.workspace_bytes = workspace_bytes_given;
    c.stream = stream;
    return general_attention(c);
  }
  if (q_dtype != TQ_DTYPE_F32 && q_dtype != TQ_DTYPE_F16 && q_dtype != TQ_DTYPE_BF16)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: q_dtype %d", q_dtype);
  if (capacity > INT32_MAX)
    return fail(TQ_ERR_UNSUPPORTED, "attention: capacity %lld above 2^31 - 1 tokens", (long long)capacity);
  if (max_tokens < 0 || max_tokens > capacity)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: max_tokens %lld > capacity %lld",
                (long long)max_tokens, (long long)capacity);
  if (prod) {
    // Prod keys here: the small row-group kernel (<= 4 query rows per kv head, d <= 128)
    if (k_bits > 3)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: Prod keys of %d bits (1..4)", k_bits + 1);
    if (rot_kind != TQ_ROT_HADAMARD)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: Prod keys use the Hadamard rotation");
    if (max_tokens > 0 && (!prod->signs || !prod->rnorms))
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null Prod key pointer");
    if (!prod->proj) return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null projection matrix");
  }
  if (kv_kind == TQ_KV_PACKED || kv_kind == TQ_KV_PROD) {
    if (k_bits < 1 || k_bits > 4 || v_bits < 1 || v_bits > 4)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: bits k=%d v=%d not in 1..4", k_bits, v_bits);
    if (norm_dtype != TQ_DTYPE_F32 && norm_dtype != TQ_DTYPE_F16)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: norm_dtype %d", norm_dtype);
    if (rot_kind != TQ_ROT_HADAMARD && rot_kind != TQ_ROT_DENSE)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: rot_kind %d", rot_kind);
    if (!k_codebook || !v_codebook || !k_rot || !v_rot)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null codec pointer");
    if (max_tokens > 0 && (!k_norms || !v_norms))
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null norms pointer");
    // the kernel addresses one (sequence, kv head) row with 32-bit byte offsets
    if (capacity * (static_cast<int64_t>(dim) * std::max(k_bits, v_bits) / 8) > UINT32_MAX)
      return fail(TQ_ERR_UNSUPPORTED, "attention: a packed row of %lld tokens exceeds 4 GiB",
                  (long long)capacity);
  } else if (kv_kind == TQ_KV_PLAIN) {
    if (kv_dtype != TQ_DTYPE_F16 && kv_dtype != TQ_DTYPE_BF16)
      return fail(TQ_ERR_INVALID_ARGUMENT, "attention: plain kv_dtype %d", kv_dtype);
    if (capacity * static_cast<int64_t>(dim) * 2 > UINT32_MAX)
      return fail(TQ_ERR_UNSUPPORTED, "attention: a plain row of %lld tokens exceeds 4 GiB",
                  (long long)capacity);
  } else {
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: kv_kind %d", kv_kind);
  }
  if (B == 0) return TQ_OK;
  if (!q || !out || !workspace) return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null pointer");
  if (max_tokens > 0 && (!k || !v)) return fail(TQ_ERR_INVALID_ARGUMENT, "attention: null cache pointer");
  const int64_t T = std::max<int64_t>(max_tokens, 1);
  // the small row-group kernels carry the kv head count in a 12-bit field
  if (small_rows_path(kv_kind, dim, (Hq / Hkv) * L) && Hkv >= (1 << kSmallRowsHkvBits))
    return fail(TQ_ERR_UNSUPPORTED, "attention: %d kv heads (at most %d with <= 4 query rows per kv head)",
                Hkv, (1 << kSmallRowsHkvBits) - 1);
  const SplitPlan sp = plan_splits(B, Hq, Hkv, L, T, dim, kv_kind == TQ_KV_PACKED);
  if (static_cast<int64_t>(B) * Hkv * sp.n_rg > kMaxGroups)
    return fail(TQ_ERR_UNSUPPORTED, "attention: %lld (batch, kv head, row group) groups > %d",
                (long long)B * Hkv * sp.n_rg, kMaxGroups);
  if (sp.n_splits > kMaxSplits)
    return fail(TQ_ERR_UNSUPPORTED, "attention: %lld tokens exceed %d splits of %d",
                (long long)T, kMaxSplits, sp.chunk);
  const int64_t need = workspace_bytes(sp, B, Hq, Hkv, L, dim);
  if (workspace_bytes_given < need)
    return fail(TQ_ERR_WORKSPACE, "attention: workspace %lld < %lld bytes",
                (long long)workspace_bytes_given, (long long)need);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: workspace must be 256-byte aligned");

  AttnParams p{};
  p.q = q;
  p.q_sb = q_stride_b;
  p.q_sh = q_stride_h;
  p.q_sl = q_stride_l;
  p.q_dtype = q_dtype;
  p.scale_q = host_round_to(q_dtype, scale);
  p.k = k;
  p.kn = k_norms;
  p.v = v;
  p.vn = v_norms;
  p.norm_dtype = norm_dtype;
  p.kcb = k_codebook;
  p.vcb = v_codebook;
  p.rot_kind = kv_kind == TQ_KV_PLAIN ? TQ_ROT_HADAMARD : rot_kind;  // plain: no rotation is read
  p.krot = k_rot;
  p.vrot = v_rot;
  p.seq_lens = seq_lens;
  p.seq_starts = seq_starts;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.L = L;
  p.R = Hq / Hkv;
  p.D = dim;
  for (int r = 0; r < 4; ++r) {
    p.row_head[r] = r / L;
    p.row_lpos[r] = r % L;
  }
  p.cap = capacity;
  p.T = max_tokens;
  p.causal = causal ? 1 : 0;
  p.n_splits = sp.n_splits;
  p.chunk = sp.chunk;
  p.n_rg = sp.n_rg;
  p.nq = sp.nq;
  const int64_t rows = static_cast<int64_t>(B) * Hq * L;
  if (rows >= (int64_t(1) << 31))
    return fail(TQ_ERR_UNSUPPORTED, "attention: %lld query rows", static_cast<long long>(rows));
  char* ws = static_cast<char*>(workspace);
  p.qrot = reinterpret_cast<float*>(ws);
  ws += (rows * dim * 4 + 255) / 256 * 256;
  p.po = reinterpret_cast<float*>(ws);
  ws += (static_cast<int64_t>(B) * Hkv * sp.n_rg * sp.nq * sp.n_splits * dim * 4 + 255) / 256 * 256;
  p.pml = reinterpret_cast<float*>(ws);
  p.out = out;

  hipStream_t st = static_cast<hipStream_t>(stream);
  p.rscale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(dim)));
  // the staged row-group kernel and the 16-row kernel leave Hadamard
  // partials in the rotated basis
  p.merge_rot = (kv_kind == TQ_KV_PACKED && !prod && rot_kind == TQ_ROT_HADAMARD &&
                 (small_rows_path(kv_kind, dim, (Hq / Hkv) * L) || rows16_path(kv_kind, dim, (Hq / Hkv) * L)))
                    ? 1
                    : 0;
  int rc = TQ_OK;
  if (prod) {
    // q_proj = q_s @ P^T into the rotated-query region (unused by the Hadamard rotation)
    p.ksg = prod->signs;
    p.krn = prod->rnorms;
    p.qproj = p.qrot;
    p.qjl_scale = static_cast<float>(__builtin_sqrt(3.14159265358979323846 / 2.0) / dim);
    AttnParams pq = p;
    pq.krot = prod->proj;
    switch (dim) {
      case 64: launch_qprep<64>(pq, q_dtype, rows, st); break;
      default: launch_qprep<128>(pq, q_dtype, rows, st); break;
    }
    rc = check_launch("qprep_kernel (q @ P^T)");
    if (rc) return rc;
  }
  if (kv_kind == TQ_KV_PACKED && rot_kind == TQ_ROT_DENSE) {
    switch (dim) {
      case 64: launch_qprep<64>(p, q_dtype, rows, st); break;
      case 128: launch_qprep<128>(p, q_dtype, rows, st); break;
      default: launch_qprep<256>(p, q_dtype, rows, st); break;
    }
    rc = check_launch("qprep_kernel");
    if (rc) return rc;
  }
  p.T = max_tokens;
  switch (dim) {
    case 64: rc = launch_partial_d64(p, kv_kind, kv_dtype, k_bits, v_bits, st); break;
    case 128: rc = launch_partial_d128(p, kv_kind, kv_dtype, k_bits, v_bits, st); break;
    default: rc = launch_partial_d256(p, kv_kind, kv_dtype, k_bits, v_bits, st); break;
  }
  if (rc || sp.n_splits == 1) return rc;
  // the splits' partials are merged by a second kernel
  // one workgroup per query row; for the dense rotation one per 64 output
  // columns of a row group (R_V^-1 is read once per row group)
  if (p.merge_rot) {
    // partials in the rotated basis: 4-row groups (staged kernel) or 16-row
    // groups (d = 128)
    const int valid = (seq_starts || seq_lens) ? -1 : static_cast<int>((T + sp.chunk - 1) / sp.chunk);
    const dim3 rgrid(static_cast<unsigned>(sp.nq), static_cast<unsigned>(Hkv * sp.n_rg), static_cast<unsigned>(B));
    if (sp.nq == 16 && dim == 128)
      hipLaunchKernelGGL((attn_merge_rot_kernel<128, 16>), rgrid, dim3(kWave), 0, st, p.po, p.pml, p.vrot,
                         sp.n_splits, valid, Hkv, sp.n_rg, p);
    else if (sp.nq == 4 && dim == 64)
      hipLaunchKernelGGL((attn_merge_rot_kernel<64, 4>), rgrid, dim3(kWave), 0, st, p.po, p.pml, p.vrot,
                         sp.n_splits, valid, Hkv, sp.n_rg, p);
    else if (sp.nq == 4 && dim == 128)
      hipLaunchKernelGGL((attn_merge_rot_kernel<128, 4>), rgrid, dim3(kWave), 0, st, p.po, p.pml, p.vrot,
                         sp.n_splits, valid, Hkv, sp.n_rg, p);
    else
      return fail(TQ_ERR_UNSUPPORTED, "attention: no rotated-basis merge for %d-row groups at dim %d", sp.nq, dim);
    return check_launch("attn_merge_rot_kernel");
  }
  const unsigned mx = rot_kind == TQ_ROT_DENSE ? static_cast<unsigned>(dim / 64) : static_cast<unsigned>(sp.nq);
  const dim3 mgrid(mx, static_cast<unsigned>(Hkv * sp.n_rg), static_cast<unsigned>(B));
  switch (dim) {
    case 64: hipLaunchKernelGGL(attn_merge_kernel<64>, mgrid, dim3(kMergeThreads), 0, st, p); break;
    case 128: hipLaunchKernelGGL(attn_merge_kernel<128>, mgrid, dim3(kMergeThreads), 0, st, p); break;
    default: hipLaunchKernelGGL(attn_merge_kernel<256>, mgrid, dim3(kMergeThreads), 0, st, p); break;
  }
  return check_launch("attn_merge_kernel");
}

}  // namespace

extern "C" int tq_attention_ranged(const void* q, int q_dtype, int B, int Hq, int Hkv, int L,
                                   int dim, int64_t q_stride_b, int64_t q_stride_h,
                                   int64_t q_stride_l, float scale, int kv_kind, int kv_dtype,
                                   const void* k, const void* k_norms, const void* v,
                                   const void* v_norms, int norm_dtype, int k_bits, int v_bits,
                                   const float* k_codebook, const float* v_codebook, int rot_kind,
                                   const float* k_rot, const float* v_rot, int64_t capacity,
                                   int64_t max_tokens, const int32_t* seq_starts,
                                   const int32_t* seq_lens, int causal, void* out, void* workspace,
                                   int64_t workspace_bytes_given, void* stream) {
  if (kv_kind != TQ_KV_PACKED && kv_kind != TQ_KV_PLAIN)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention: kv_kind %d", kv_kind);
  return attention_impl(q, q_dtype, B, Hq, Hkv, L, dim, q_stride_b, q_stride_h, q_stride_l, scale,
                        kv_kind, kv_dtype, k, k_norms, v, v_norms, norm_dtype, k_bits, v_bits,
                        k_codebook, v_codebook, rot_kind, k_rot, v_rot, capacity, max_tokens,
                        seq_starts, seq_lens, causal, out, workspace, workspace_bytes_given, stream,
                        nullptr);
}

extern "C" int tq_attention(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                            int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l,
                            float scale, int kv_kind, int kv_dtype, const void* k,
                            const void* k_norms, const void* v, const void* v_norms,
                            int norm_dtype, int k_bits, int v_bits, const float* k_codebook,
                            const float* v_codebook, int rot_kind, const float* k_rot,
                            const float* v_rot, int64_t capacity, int64_t max_tokens,
                            const int32_t* seq_lens, int causal, void* out, void* workspace,
                            int64_t workspace_bytes_given, void* stream) {
  return tq_attention_ranged(q, q_dtype, B, Hq, Hkv, L, dim, q_stride_b, q_stride_h, q_stride_l,
                             scale, kv_kind, kv_dtype, k, k_norms, v, v_norms, norm_dtype, k_bits,
                             v_bits, k_codebook, v_codebook, rot_kind, k_rot, v_rot, capacity,
                             max_tokens, nullptr, seq_lens, causal, out, workspace,
                             workspace_bytes_given, stream);
}

// ------------------------------------------------------------ no-alloc ----
// Attention scratch for callers that cannot allocate (graph capture, serving
// loops).  Each device holds its own copy of this array for the life of the
// process.  In host code `scratch` names a host-side stand-in, not device
// memory: kernels and copies take the per-device address from
// hipGetSymbolAddress instead.
namespace {

constexpr int64_t kScratchBytes = TQ_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's scratch address, looked up once per device (with that
// device current) and kept.
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TQ_ERR_HIP, "attention (no-alloc): hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(TQ_ERR_UNSUPPORTED, "attention (no-alloc): device %d beyond %d", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(TQ_ERR_HIP, "attention (no-alloc): hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TQ_OK;
}

}  // namespace

extern "C" int tq_attention_noalloc(const void* q, int q_dtype, int B, int Hq, int Hkv, int L,
                                    int dim, int64_t q_stride_b, int64_t q_stride_h,
                                    int64_t q_stride_l, float scale, int kv_kind, int kv_dtype,
                                    const void* k, const void* k_norms, const void* v,
                                    const void* v_norms, int norm_dtype, int k_bits, int v_bits,
                                    const float* k_codebook, const float* v_codebook, int rot_kind,
                                    const float* k_rot, const float* v_rot, int64_t capacity,
                                    int64_t max_tokens, const int32_t* seq_starts,
                                    const int32_t* seq_lens, int causal, void* out, void* stream) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || L < 1 || dim <= 0 || max_tokens < 0 || Hq % Hkv)
    return fail(TQ_ERR_INVALID_ARGUMENT, "attention (no-alloc): bad shape (B %d, Hq %d, Hkv %d, L %d, dim %d)",
                B, Hq, Hkv, L, dim);
  if (B == 0) return TQ_OK;
  const int64_t need = tq_attention_workspace_size(B, Hq, Hkv, L, dim, max_tokens);
  if (need > kScratchBytes)
    return fail(TQ_ERR_WORKSPACE, "attention (no-alloc): the problem needs %lld bytes of scratch, "
                "above the static %lld; use tq_attention with a caller workspace",
                (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return tq_attention_ranged(q, q_dtype, B, Hq, Hkv, L, dim, q_stride_b, q_stride_h, q_stride_l,
                             scale, kv_kind, kv_dtype, k, k_norms, v, v_norms, norm_dtype, k_bits,
                             v_bits, k_codebook, v_codebook, rot_kind, k_rot, v_rot, capacity,
                             max_tokens, seq_starts, seq_lens, causal, out, ws, kScratchBytes, stream);
}

extern "C" int tq_attention_prod(const void* q, int q_dtype, int B, int Hq, int Hkv, int L, int dim,
                                 int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_l,
                                 float scale, const void* k_mse, const void* k_norms,
                                 const void* k_signs, const void* k_residual_norms, int k_bits,
                                 const float* k_mse_codebook, const float* k_rot_signs,
                                 const float* projection, const void* v, const void* v_norms,
                                 int v_bits, const float* v_codebook, const float* v_rot_signs,
                                 int norm_dtype, int64_t capacity, int64_t max_tokens,
                                 const int32_t* seq_starts, const int32_t* seq_lens, int causal,
                                 void* out, void* workspace, int64_t workspace_bytes_given,
                                 void* stream) {
  const ProdKeys pk{k_signs, k_residual_norms, projection};
  return attention_impl(q, q_dtype, B, Hq, Hkv, L, dim, q_stride_b, q_stride_h, q_stride_l, scale,
                        TQ_KV_PROD, 0, k_mse, k_norms, v, v_norms, norm_dtype, k_bits - 1, v_bits,
                        k_mse_codebook, v_codebook, TQ_ROT_HADAMARD, k_rot_signs, v_rot_signs,
                        capacity, max_tokens, seq_starts, seq_lens, causal, out, workspace,
                        workspace_bytes_given, stream, &pk);
}

#ifdef TQ_PHASE_STAMPS
// Phase stamps of the last attn_merge_rot_kernel launch (stamps build only).
extern "C" int tq_dbg_merge_stamps(void* dst, long long bytes) {
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(tq::g_merge_stamps), bytes) == hipSuccess ? 0 : 1;
}
#endif
