// INT8 W8A8 entry points: raw int32, per-tensor and per-channel fused
// epilogues, and the fused gate/up FFN pair.
#include <mutex>
#include "launch.hpp"

using namespace c4q;

namespace {

int check_i8_args(const void* a, int64_t lda, const void* b, int64_t ldb, const void* d,
                  int64_t ldd, int64_t M, int64_t N, int64_t K, const char* what) {
  C4Q_REQUIRE(M >= 0 && N >= 0 && K >= 0, C4Q_ERR_SHAPE, "%s: negative size M=%lld N=%lld K=%lld",
              what, (long long)M, (long long)N, (long long)K);
  C4Q_REQUIRE(lda >= K && ldb >= K && ldd >= N, C4Q_ERR_SHAPE,
              "%s: row stride smaller than the row (lda=%lld ldb=%lld ldd=%lld)", what,
              (long long)lda, (long long)ldb, (long long)ldd);
  if (M > 0 && N > 0) {
    C4Q_REQUIRE(d != nullptr, C4Q_ERR_ARG, "%s: null output", what);
    C4Q_REQUIRE(K == 0 || (a != nullptr && b != nullptr), C4Q_ERR_ARG, "%s: null operand", what);
  }
  return C4Q_OK;
}

}  // namespace

extern "C" int c4q_i8_gemm_nt_i32(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                  int32_t* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                  void* stream) {
  const char* what = "c4q_i8_gemm_nt_i32";
  int st = check_i8_args(a, lda, b, ldb, c, ldc, M, N, K, what);
  if (st) return st;
  EpiI32 epi{{c, ldc, rows_vec16(c, ldc, 4)}};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                    uint16_t* d, int64_t ldd, const float* row_scale,
                                    const uint16_t* bias, int64_t M, int64_t N, int64_t K,
                                    void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused";
  int st = check_i8_args(a, lda, b, ldb, d, ldd, M, N, K, what);
  if (st) return st;
  C4Q_REQUIRE(M == 0 || N == 0 || row_scale != nullptr, C4Q_ERR_ARG, "%s: null row_scale", what);
  EpiRowScale epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, bias};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                       uint16_t* d, int64_t ldd, const float* row_scale,
                                       const float* col_scale, const uint16_t* bias, int64_t M,
                                       int64_t N, int64_t K, void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs";
  int st = check_i8_args(a, lda, b, ldb, d, ldd, M, N, K, what);
  if (st) return st;
  C4Q_REQUIRE(M == 0 || N == 0 || (row_scale != nullptr && col_scale != nullptr), C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  EpiRowColScale epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, col_scale, bias};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs_f16(const int8_t* a, int64_t lda, const int8_t* b,
                                           int64_t ldb, uint16_t* d, int64_t ldd,
                                           const float* row_scale, const float* col_scale,
                                           const uint16_t* bias, int64_t M, int64_t N, int64_t K,
                                           void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs_f16";
  int st = check_i8_args(a, lda, b, ldb, d, ldd, M, N, K, what);
  if (st) return st;
  C4Q_REQUIRE(M == 0 || N == 0 || (row_scale != nullptr && col_scale != nullptr), C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  EpiRowColScaleF16 epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, col_scale, bias};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs_qkv(const int8_t* a, int64_t lda, const int8_t* b,
                                           int64_t ldb, uint16_t* q, uint16_t* k, uint16_t* v,
                                           const float* row_scale, const float* col_scale,
                                           const uint16_t* bias, int64_t M, int64_t K, int64_t H,
                                           int64_t D, void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs_qkv";
  C4Q_REQUIRE(H > 0 && D > 0 && D % 8 == 0, C4Q_ERR_SHAPE,
              "%s: need H > 0 and D > 0 a multiple of 8 (H=%lld D=%lld)", what, (long long)H,
              (long long)D);
  const int64_t N = 3 * H * D;
  C4Q_REQUIRE(N < (1ll << 31) && M < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
  int st = check_i8_args(a, lda, b, ldb, q, N, M, N, K, what);
  if (st) return st;
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(k != nullptr && v != nullptr, C4Q_ERR_ARG, "%s: null K/V output", what);
  C4Q_REQUIRE(row_scale != nullptr && col_scale != nullptr, C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  const int vec = aligned16(q) && aligned16(k) && aligned16(v);
  const int64_t koff = (int64_t)(reinterpret_cast<intptr_t>(k) - reinterpret_cast<intptr_t>(q));
  const int64_t voff = (int64_t)(reinterpret_cast<intptr_t>(v) - reinterpret_cast<intptr_t>(q));
  EpiRowColScaleQKV epi{{{q, N, vec}, row_scale, col_scale, bias}, koff, voff, M,
                        (uint32_t)(H * D), (uint32_t)D};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

namespace {

// In-place Q/K RMSNorm + partial RoPE over the attention layout [1, H, M,
// 128] of Q and K: the second pass of the two-pass route (after the QKV
// scatter), with the lane map and arithmetic of epilogue_head_norm (8
// rows per wave: lane l holds row l/8, columns 64 h + 8 (l%8) + k). Rows
// are taken 8 consecutive tokens of one (kind, head) per wave, chunk by
// chunk of 8 tokens, so the 2H waves of a chunk read its freqs rows from
// the cache. A row is read whole before any lane writes it.
// `kinds` = 2: Q and K (K at epi.koff, normalized with the K weight);
// 1: one tensor at epi.d with the weight at epi.qw.
template <bool UNITS>
__global__ void __launch_bounds__(256) head_norm_rope_kernel(EpiQKVNormRope epi, int64_t H,
                                                             int kinds) {
  using St = Strip<128>;
  using Map = StoreMap<128, uint16_t>;
  __shared__ __attribute__((aligned(16))) float rows[4][St::kBytes / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, prow = lane >> 3;
  // wave w covers 8 consecutive tokens of one (kind, head) row set: chunk
  // c of 8 tokens, then (kind, head) t -- a wave reads 2 KB contiguous, and
  // the 2H waves of a chunk share its 8 freqs rows through the cache
  const uint32_t wv = blockIdx.x * 4u + (uint32_t)wave;   // < 2^31 (checked by the host)
  const uint32_t h2 = (uint32_t)(kinds * H);
  const uint32_t c8 = wv / h2, t = wv - c8 * h2;
  const int64_t m = (int64_t)c8 * 8 + prow;
  const bool live = m < epi.rows;
  const uint32_t kind = t >= (uint32_t)H ? 1u : 0u;
  const int64_t hd = (int64_t)(t - kind * (uint32_t)H);
  uint8_t* row = static_cast<uint8_t*>(epi.d) + epi.koff * (int64_t)kind + (hd * epi.rows + m) * 256;
  const float* wp = epi.weight(kind);
  float x[16], w[16], y[16];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = Map::col(lane, 2 * h);
    uint4 u{0, 0, 0, 0};
    if (live) u = *reinterpret_cast<const uint4*>(row + c * 2);
    const uint32_t p[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[8 * h + 2 * e] = bf16lo(p[e]);
      x[8 * h + 2 * e + 1] = bf16hi(p[e]);
    }
#pragma unroll
    for (int k = 0; k < 8; k += 4) {
      const float4 f = *reinterpret_cast<const float4*>(wp + c + k);
      w[8 * h + k] = f.x; w[8 * h + k + 1] = f.y; w[8 * h + k + 2] = f.z; w[8 * h + k + 3] = f.w;
    }
  }
  const int R = epi.pairs;
  const uint8_t* frow = reinterpret_cast<const uint8_t*>(epi.freqs) + (live ? m : 0) * R * 8;
  uint32_t fw[16];
  int pc[2];
  uint32_t swap[2];
  bool pass[2];
  if constexpr (UNITS) {
    // R % 8 == 0: each 8-column unit lies in one rotation half or past 2R;
    // its freqs words load with constant offsets (see epilogue_head_norm)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c0 = Map::col(lane, 2 * h);
      const bool first = c0 < R, second = !first && c0 < 2 * R;
      pass[h] = !first && !second;
      pc[h] = first ? c0 + R : (second ? c0 - R : c0);
      swap[h] = second ? 16u : 0u;
      if (live && !pass[h]) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(
            frow + (first ? 8 * c0 : 8 * (c0 - R) + 4));
#pragma unroll
        for (int k = 0; k < 8; ++k) fw[8 * h + k] = p[2 * k];
      }
    }
  }
  head_rms_norm(x, w, epi.eps, y);
  float* sf = rows[wave];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int k = 0; k < 8; k += 4)
      *reinterpret_cast<float4*>(sf + St::word(prow, Map::col(lane, 2 * h) + k)) =
          float4{y[8 * h + k], y[8 * h + k + 1], y[8 * h + k + 2], y[8 * h + k + 3]};
  lds_fence_wave();
  if (!live) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c0 = Map::col(lane, 2 * h);
    float o[8];
    if constexpr (UNITS) {
      float yp[8];
#pragma unroll
      for (int k = 0; k < 8; k += 4) {
        const float4 t4 = *reinterpret_cast<const float4*>(sf + St::word(prow, pc[h] + k));
        yp[k] = t4.x; yp[k + 1] = t4.y; yp[k + 2] = t4.z; yp[k + 3] = t4.w;
      }
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        // rope_split_half for two columns, their diagonal products rounded
        // by one paired conversion (the final rounding is the store's)
        const uint32_t f0 = __builtin_amdgcn_alignbit(fw[8 * h + k], fw[8 * h + k], swap[h]);
        const uint32_t f1 = __builtin_amdgcn_alignbit(fw[8 * h + k + 1], fw[8 * h + k + 1], swap[h]);
        const uint32_t dp = bf16x2_rne(bf16lo(f0) * y[8 * h + k], bf16lo(f1) * y[8 * h + k + 1]);
        const float r0 = bf16lo(dp) + bf16hi(f0) * yp[k];
        const float r1 = bf16hi(dp) + bf16hi(f1) * yp[k + 1];
        o[k] = pass[h] ? y[8 * h + k] : r0;
        o[k + 1] = pass[h] ? y[8 * h + k + 1] : r1;
      }
    } else {
      const uint32_t* fr = reinterpret_cast<const uint32_t*>(frow);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int d = c0 + k;
        o[k] = y[8 * h + k];
        if (d < 2 * R) {
          const bool second = d >= R;
          const int ii = second ? d - R : d;
          const float yp = sf[St::word(prow, second ? ii : d + R)];
          o[k] = rope_split_half(o[k], yp, fr[2 * ii + (second ? 1 : 0)], second);
        }
      }
    }
    *reinterpret_cast<uint4*>(row + c0 * 2) =
        uint4{bf16x2_rne(o[0], o[1]), bf16x2_rne(o[2], o[3]), bf16x2_rne(o[4], o[5]),
              bf16x2_rne(o[6], o[7])};
  }
}

}  // namespace

extern "C" int c4q_i8_gemm_nt_fused_cs_qkv_rms_rope(
    const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, uint16_t* q, uint16_t* k,
    uint16_t* v, const float* row_scale, const float* col_scale, const uint16_t* bias,
    const uint16_t* freqs, const float* q_weight, const float* k_weight, int64_t M, int64_t K,
    int64_t H, int64_t R, float eps, void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs_qkv_rms_rope";
  constexpr int64_t D = 128;
  C4Q_REQUIRE(H > 0 && R >= 0 && 2 * R <= D, C4Q_ERR_SHAPE,
              "%s: need H > 0 and 0 <= 2R <= 128 (H=%lld R=%lld)", what, (long long)H,
              (long long)R);
  const int64_t N = 3 * H * D;
  C4Q_REQUIRE(N < (1ll << 31) && M < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
  int st = check_i8_args(a, lda, b, ldb, q, N, M, N, K, what);
  if (st) return st;
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(k != nullptr && v != nullptr, C4Q_ERR_ARG, "%s: null K/V output", what);
  C4Q_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v), C4Q_ERR_ARG,
              "%s: Q, K and V must be 16-byte aligned", what);
  C4Q_REQUIRE(row_scale != nullptr && col_scale != nullptr, C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  C4Q_REQUIRE(q_weight != nullptr && k_weight != nullptr && aligned16(q_weight) &&
                  aligned16(k_weight),
              C4Q_ERR_ARG, "%s: q_weight/k_weight must be non-null and 16-byte aligned", what);
  C4Q_REQUIRE(R == 0 || (freqs != nullptr && (reinterpret_cast<uintptr_t>(freqs) & 3u) == 0),
              C4Q_ERR_ARG, "%s: freqs must be non-null and 4-byte aligned", what);
  const int64_t koff = (int64_t)(reinterpret_cast<intptr_t>(k) - reinterpret_cast<intptr_t>(q));
  const int64_t voff = (int64_t)(reinterpret_cast<intptr_t>(v) - reinterpret_cast<intptr_t>(q));
  const int64_t kwoff =
      (int64_t)(reinterpret_cast<intptr_t>(k_weight) - reinterpret_cast<intptr_t>(q_weight));
  EpiQKVNormRope epi{{{{q, N, 1}, row_scale, col_scale, bias}, koff, voff, M, (uint32_t)(H * D),
                      (uint32_t)D},
                     reinterpret_cast<const uint32_t*>(freqs), q_weight, kwoff, (int32_t)R, eps};
  hipStream_t s = as_stream(stream);
  const uint8_t* a8 = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* b8 = reinterpret_cast<const uint8_t*>(b);
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(b) && lda % 16 == 0 &&
                     ldb % 16 == 0 && tile_offsets_fit(lda, ldb);
  const Src2 sa{a8, a8, lda, M}, sb{b8, b8, ldb, N};
  auto op_for = [](auto t) { return OpI8T<decltype(t)::KS8>{}; };
  // Two routes, identical bytes. Fused: the projection with the norm/RoPE
  // epilogue (whole 8-column units per rotation half, so R % 8 == 0). Two
  // passes: the QKV scatter (the general 8-wave tiles), then the in-place
  // norm/RoPE pass over Q and K, which mostly re-reads them from the
  // Infinity Cache. On MI355X the second is the faster at H3's shapes
  // (56 heads, K 5376: 1020 vs 1113 us at 8192 tokens, 726 vs 775 at 5378,
  // 2121 vs 2085 at 17000), the norm epilogue's VALU work being exposed in
  // the fused kernel; C4Q_QKV_NORM_FUSE=1 selects the fused route.
  const char* fuse_env = getenv("C4Q_QKV_NORM_FUSE");
  const bool fuse = fuse_env && fuse_env[0] == '1' && fuse_env[1] == 0;
  if (tiled && R % 8 == 0 && fuse)
    return run_tiles<false>(M, N, N, K, sa, sb, nullptr, epi, s, what, op_for, HeadTiles{});
  // the QKV scatter, then the norm/RoPE pass over Q and K in place
  const EpiRowColScaleQKV& scatter = epi;
  st = tiled ? run_tiles<false>(M, N, N, K, sa, sb, nullptr, scatter, s, what, op_for)
             : launch_generic(M, N, K, GenI8::make(a8, lda, b8, ldb), scatter, s, what);
  if (st) return st;
  const int64_t blocks = cdiv(cdiv(M, 8) * 2 * H, 4);     // one wave per 8 tokens x (kind, head)
  C4Q_REQUIRE(blocks < (1ll << 29), C4Q_ERR_SHAPE, "%s: problem too large", what);
  if (R % 8 == 0)
    hipLaunchKernelGGL(head_norm_rope_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, epi, H, 2);
  else
    hipLaunchKernelGGL(head_norm_rope_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, epi, H, 2);
  return check_launch(what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs_qkv_lora_part(
    const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, uint16_t* out,
    const float* row_scale, const float* col_scale, const uint16_t* bias, const uint16_t* delta,
    const uint16_t* freqs, const float* norm_weight, int64_t M, int64_t K, int64_t H, int64_t R,
    int kind, float delta_scale, float eps, void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs_qkv_lora_part";
  constexpr int64_t D = 128;
  C4Q_REQUIRE(kind >= 0 && kind <= 2, C4Q_ERR_ARG, "%s: kind must be Q=0, K=1 or V=2 (got %d)",
              what, kind);
  C4Q_REQUIRE(H > 0, C4Q_ERR_SHAPE, "%s: need H > 0 (H=%lld)", what, (long long)H);
  C4Q_REQUIRE(kind == 2 || (R >= 0 && 2 * R <= D), C4Q_ERR_SHAPE,
              "%s: need 0 <= 2R <= 128 (R=%lld)", what, (long long)R);
  const int64_t N = H * D;
  C4Q_REQUIRE(N < (1ll << 31) && M < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
  int st = check_i8_args(a, lda, b, ldb, out, N, M, N, K, what);
  if (st) return st;
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(aligned16(out), C4Q_ERR_ARG, "%s: out must be 16-byte aligned", what);
  C4Q_REQUIRE(row_scale != nullptr && col_scale != nullptr, C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  C4Q_REQUIRE(delta != nullptr && (reinterpret_cast<uintptr_t>(delta) & 7u) == 0, C4Q_ERR_ARG,
              "%s: delta must be non-null and 8-byte aligned", what);
  if (kind != 2) {
    C4Q_REQUIRE(norm_weight != nullptr && aligned16(norm_weight), C4Q_ERR_ARG,
                "%s: norm_weight must be non-null and 16-byte aligned", what);
    C4Q_REQUIRE(R == 0 || (freqs != nullptr && (reinterpret_cast<uintptr_t>(freqs) & 3u) == 0),
                C4Q_ERR_ARG, "%s: freqs must be non-null and 4-byte aligned", what);
  }
  // the partition's scatter with the delta term, then (Q, K) the in-place
  // norm/RoPE pass of the two-pass QKV route over the one tensor
  const float ls = bf16_f32(bf16_rte(delta_scale));
  EpiQKVLora epi{{{{out, N, 1}, row_scale, col_scale, bias}, 0, 0, M, (uint32_t)N, (uint32_t)D},
                 delta, ls};
  hipStream_t s = as_stream(stream);
  const uint8_t* a8 = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* b8 = reinterpret_cast<const uint8_t*>(b);
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(b) && lda % 16 == 0 &&
                     ldb % 16 == 0 && tile_offsets_fit(lda, ldb);
  const Src2 sa{a8, a8, lda, M}, sb{b8, b8, ldb, N};
  auto op_for = [](auto t) { return OpI8T<decltype(t)::KS8>{}; };
  st = tiled ? run_tiles<false>(M, N, N, K, sa, sb, nullptr, epi, s, what, op_for)
             : launch_generic(M, N, K, GenI8::make(a8, lda, b8, ldb), epi, s, what);
  if (st || kind == 2) return st;
  EpiQKVNormRope norm{{{{out, N, 1}, row_scale, col_scale, bias}, 0, 0, M, (uint32_t)N,
                       (uint32_t)D},
                      reinterpret_cast<const uint32_t*>(freqs), norm_weight, 0, (int32_t)R, eps};
  const int64_t blocks = cdiv(cdiv(M, 8) * H, 4);     // one wave per 8 tokens x head
  C4Q_REQUIRE(blocks < (1ll << 29), C4Q_ERR_SHAPE, "%s: problem too large", what);
  if (R % 8 == 0)
    hipLaunchKernelGGL(head_norm_rope_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, norm, H, 1);
  else
    hipLaunchKernelGGL(head_norm_rope_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, norm, H, 1);
  return check_launch(what);
}

extern "C" int c4q_i8_mlp_bridge_prequant(const int8_t* a, int64_t lda, const int8_t* w1,
                                          int64_t ldw, const float* row_scale,
                                          const float* col_scale, const uint16_t* bias,
                                          const uint16_t* silu_table, int64_t M, int64_t K,
                                          int64_t W, int64_t tile_rows, uint16_t* wide,
                                          uint16_t* rot, int8_t* q, float* scales, void* stream) {
  const char* what = "c4q_i8_mlp_bridge_prequant";
  C4Q_REQUIRE(M >= 0 && K >= 0 && W > 0 && W % 512 == 0, C4Q_ERR_SHAPE,
              "%s: need W = 2F > 0 with F a multiple of 256 (W=%lld)", what, (long long)W);
  C4Q_REQUIRE(tile_rows > 0, C4Q_ERR_SHAPE, "%s: tile_rows must be positive", what);
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(wide && q && scales && silu_table, C4Q_ERR_ARG, "%s: null buffer", what);
  const int64_t F = W / 2;
  // rows of F <= 15360 fit the one-pass SwiGLU + ConvRot + quant (the
  // rotated row stays in LDS); wider rows go through `rot`
  const bool one_pass = F * 2 <= 30 * 1024;
  C4Q_REQUIRE(one_pass || rot != nullptr, C4Q_ERR_ARG, "%s: null rot scratch", what);
  // per chunk of rows: FC1 with the per-channel epilogue into `wide`, then
  // SwiGLU + ConvRot + rowwise quant into the chunk's q rows
  for (int64_t r0 = 0; r0 < M; r0 += tile_rows) {
    const int64_t rows = M - r0 < tile_rows ? M - r0 : tile_rows;
    int st = c4q_i8_gemm_nt_fused_cs(a + r0 * lda, lda, w1, ldw, wide, W, row_scale + r0, col_scale,
                                     bias, rows, W, K, stream);
    if (st == C4Q_OK && one_pass)
      st = c4q_i8_swiglu_rot_quant(wide, rows, F, silu_table, q + r0 * F, scales + r0, stream);
    if (st == C4Q_OK && !one_pass) {
      st = c4q_i8_swiglu_rot(wide, rows, F, silu_table, rot, stream);
      if (st == C4Q_OK)
        st = c4q_i8_quant_rowwise(rot, C4Q_BF16, F, q + r0 * F, F, scales + r0, rows, F, stream);
    }
    if (st != C4Q_OK) return st;
  }
  return C4Q_OK;
}

// ---- MLP bridge without allocations ---------------------------------------
// The bridge's FC1 staging (`wide`, and `rot` for F > 15360) lives in one
// file-scope device array per GPU instead of caller scratch. Host code never
// passes the array's name to a kernel or a copy: it passes the address that
// hipGetSymbolAddress returns for the current device, looked up once per
// device on the entry point's first call there.
static __device__ __align__(256) uint16_t scratch[C4Q_BRIDGE_SCRATCH_BYTES / 2];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {nullptr};

int bridge_scratch(uint16_t** out, const char* what) {
  int dev = -1;
  C4Q_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64, C4Q_ERR_HIP,
              "%s: no current HIP device (or device index >= 64)", what);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    C4Q_REQUIRE(e == hipSuccess && p != nullptr, C4Q_ERR_HIP,
                "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<uint16_t*>(g_scratch_ptr[dev]);
  return C4Q_OK;
}
}  // namespace

extern "C" int c4q_i8_mlp_bridge_prequant_noalloc(const int8_t* a, int64_t lda, const int8_t* w1,
                                                  int64_t ldw, const float* row_scale,
                                                  const float* col_scale, const uint16_t* bias,
                                                  const uint16_t* silu_table, int64_t M,
                                                  int64_t K, int64_t W, int8_t* q, float* scales,
                                                  void* stream) {
  const char* what = "c4q_i8_mlp_bridge_prequant_noalloc";
  C4Q_REQUIRE(M >= 0 && K >= 0 && W > 0 && W % 512 == 0, C4Q_ERR_SHAPE,
              "%s: need W = 2F > 0 with F a multiple of 256 (W=%lld)", what, (long long)W);
  if (M == 0) return C4Q_OK;
  const int64_t F = W / 2;
  const bool one_pass = F * 2 <= 30 * 1024;
  // staging bytes per FC1 row: the bf16 row [2F], plus its rotated half [F]
  // on the two-pass route
  const int64_t row_bytes = one_pass ? 4 * F : 6 * F;
  const int64_t fit = C4Q_BRIDGE_SCRATCH_BYTES / row_bytes;
  int64_t rows = M <= fit ? M : fit / 128 * 128;
  C4Q_REQUIRE(rows >= 1 && (rows == M || rows >= 128), C4Q_ERR_SHAPE,
              "%s: a chunk of 128 FC1 rows of F=%lld needs %lld bytes of staging, more than the "
              "%lld-byte scratch; use c4q_i8_mlp_bridge_prequant with caller scratch",
              what, (long long)F, (long long)(128 * row_bytes),
              (long long)C4Q_BRIDGE_SCRATCH_BYTES);
  uint16_t* base = nullptr;
  const int st = bridge_scratch(&base, what);
  if (st != C4Q_OK) return st;
  uint16_t* wide = base;
  uint16_t* rot = one_pass ? nullptr : base + rows * W;
  return c4q_i8_mlp_bridge_prequant(a, lda, w1, ldw, row_scale, col_scale, bias, silu_table, M, K,
                                    W, rows, wide, rot, q, scales, stream);
}

extern "C" int c4q_i8_ffn_pair(const int8_t* a, int64_t lda, const int8_t* w_gate,
                               const int8_t* w_up, int64_t ldw, uint16_t* d, int64_t ldd,
                               const float* row_scale, const float* gate_scale,
                               const float* up_scale, const uint16_t* table_gate,
                               const uint16_t* table_up, int64_t M, int64_t N_out, int64_t K,
                               void* stream) {
  const char* what = "c4q_i8_ffn_pair";
  int st = check_i8_args(a, lda, w_gate, ldw, d, ldd, M, N_out, K, what);
  if (st) return st;
  if (M == 0 || N_out == 0) return C4Q_OK;
  C4Q_REQUIRE(K == 0 || w_up != nullptr, C4Q_ERR_ARG, "%s: null w_up", what);
  C4Q_REQUIRE(row_scale && gate_scale && up_scale, C4Q_ERR_ARG, "%s: null scale", what);
  hipStream_t s = as_stream(stream);
  EpiPair epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, gate_scale, up_scale, table_gate, table_up};
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(w_gate) &&
                     aligned16(w_up) && lda % 16 == 0 && ldw % 16 == 0 && tile_offsets_fit(lda, ldw);
  if (!tiled) {
    const int64_t nbx = cdiv(N_out, 64);
    const int64_t blocks = nbx * cdiv(M, 4);
    C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
    hipLaunchKernelGGL((pair_generic_kernel<EpiPair>), dim3((unsigned)blocks), dim3(256), 0, s, M,
                       N_out, K, nbx, a, lda, w_gate, w_up, ldw, epi);
    return check_launch(what);
  }
  const Src2 sa{reinterpret_cast<const uint8_t*>(a), reinterpret_cast<const uint8_t*>(a), lda, M};
  const Src2 sb{reinterpret_cast<const uint8_t*>(w_gate), reinterpret_cast<const uint8_t*>(w_up),
                ldw, N_out};
  return run_tiles<true>(M, 2 * N_out, 2 * N_out, K, sa, sb, nullptr, epi, s, what,
                         [](auto t) { return OpI8T<decltype(t)::KS8>{}; });
}
