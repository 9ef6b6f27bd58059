// Swin-T camera backbone context (drop-in for reference src/cuda_swin.cu).
//
// Data layout in HBM:
//   x    fp32 [tokens, C]   residual stream, NHWC token order, in place
//   xn   fp16 [tokens, C]   stage 0: LayerNorm output -> fused W-MSA input,
//                           reused for the attention output
//   big  fp16 [tokens, 4C]  QKV [tokens, 3C], later the GELU hidden [tokens, 4C]
// Window partitioning never materialises: the attention kernel gathers its 49
// (padded, cyclically shifted) tokens straight from the token-major QKV rows
// and scatters its output back the same way, so QKV and proj run as plain
// token GEMMs over B*H*W rows instead of windows*49 rows.
//
// 16-bit words are fp16 (stored in the bf16 container type): every GEMM and
// the attention run on the fp16 MFMA with fp32 accumulation.
//
//   xh   fp16 [tokens, C]   stages 1-3: fp16 copy of x, the A operand of the
//                           LN-folded QKV / fc1 linears and patch merges
//                           (ln_fold.h); two buffers, alternating per stage,
//                           because a merge reads one stage's copy while
//                           writing the next (stage 0's copy, for its merge
//                           only, is written over xn)
//   stats float2 [tokens, C/64] (mean, M2) of x per 64-channel group, written
//                           with xh, read by the LN-folded linears (two, like
//                           xh; stage 0's, one group of all 96 channels, at the
//                           front of big)
//
// Per block at stages 1-3: QKV GEMM(LN1 folded, fp16) -> window attention ->
// proj GEMM(+bias, += into x; writes xh and stats) -> fc1 GEMM(LN2 folded,
// GELU, fp16) -> fc2 GEMM(+bias, += into x; writes xh and stats): no
// LayerNorm pass.  Stage 0 (C = 96) runs LN2 -> fc1 -> GELU -> fc2 ->
// residual as one fused kernel whose hidden layer stays on chip (swin_mlp.h),
// with the proj GEMM and its residual fused in front; it also writes the next
// block's LN1 output (the last block: xh and the row statistics), and the
// patch embedding's epilogue writes block 0's, so stage 0 launches no
// LayerNorm either.  The three patch merges fold their LayerNorm over 4C the
// same way, reading the 2x2 tokens straight from xh.
#include "bf_cuda_swin.h"
#include "bfhip_debug.h"
#include "bfhip_profile.h"
#include "conv_core.h"
#include "host_util.h"
#include "linear.h"
#include "ln_fold.h"
#include "swin_kernels.h"
#include "swin_mlp.h"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <mutex>
#include <vector>

using namespace bfhip;

namespace {

constexpr int kC[4] = {96, 192, 384, 768};
constexpr int kHeads[4] = {3, 6, 12, 24};
constexpr int kDepth[4] = {2, 2, 6, 2};

// Fused proj + MLP configuration of stage 0: one 16-token fragment per wave,
// four waves, three weight chunks in flight (measured best on MI355X at
// 6x256x704).
using MlpS0 = MlpCfg<96, 1, 4, 3, true>;
constexpr bool kFusedMlp[4] = {true, false, false, false};
// Stages whose QKV projection runs inside the attention kernel (one workgroup
// per window, window_msa_kernel).  Measured at 6x256x704: stage 0 26.5 us
// fused vs 32.8 us for QKV GEMM + attention (the 39 MB of q, k, v stay on
// chip); stage 1 25.5 us vs 23.1 us (six waves of ~226 VGPRs per window and
// 390 windows), so it keeps the separate kernels.  At stage 2 a variant with
// LayerNorm-1 applied on load (six of a window's twelve heads per workgroup,
// weight fragments streamed from L2 four k-steps ahead) took 21.9 us vs 19.0
// us for QKV GEMM + attention: one workgroup per CU at 234 VGPRs, each wave
// waiting on its weight chunks.
constexpr bool kFusedWmsa[4] = {true, false, false, false};

struct BlockW {
    const float *n1s, *n1b, *n2s, *n2b, *qkv_b, *proj_b, *fc1_b, *fc2_b, *bias_mat;
    // Stages 1-3: qkv_w and fc1_w hold the LN-folded weights W' (ln_fold.h),
    // with their centring-correction tables (per-group column sums) and
    // shifts d.
    const bf16 *qkv_corr, *fc1_corr;
    const float *qkv_d, *fc1_d;
    const bf16 *qkv_w, *proj_w, *fc1_w, *fc2_w;
    const bf16 *mlp_w;      // fc1/fc2 packed for the fused MLP (fused stages only)
    const bf16 *mlp_proj;   // proj packed for the fused MLP (fused stages only)
    const bf16 *attn_term;  // relative bias + shift mask per window type (attn_term_kernel)
};

struct BlockOff {
    size_t n1s, n1b, n2s, n2b, qkv_b, proj_b, fc1_b, fc2_b, bias_mat, qkv_w, proj_w, fc1_w, fc2_w;
    size_t qkv_corr, qkv_d, fc1_corr, fc1_d;
    size_t mlp_w, mlp_proj, attn_term;
};

}  // namespace

struct bf_cuda_swin {
    size_t batches, input_h, input_w, resident_bytes;
    int h[4], w[4];
    unsigned char *params, *acts;
    const bf16 *patch_w;
    const float *patch_b, *patch_ns, *patch_nb;
    BlockW blocks[4][6];
    const float *out_s[3], *out_b[3];
    const bf16 *merge_w[3];           // LN-folded, columns in tap-major order
    const bf16 *merge_corr[3];        // centring-correction tables (ln_fold.h)
    const float *merge_d[3];
    float *x;      // the fp32 residual stream (stage 2's at x + x2_off, the others at x)
    size_t x2_off;
    bf16 *xn, *big;
    bf16 *xh[2];
    float2 *stats[2];
};

namespace {

// Stage st's fp32 residual stream.  Stage 2's lies after stage 1's, so the
// merges after stages 1 and 2 never write over the rows that the same
// launch's output LayerNorm reads (merge_out_ln_kernel).
float *stage_x(bf_cuda_swin *s, int st) { return st == 2 ? s->x + s->x2_off : s->x; }

// A linear fed by a LayerNorm, folded (ln_fold.h): W'[j][kk] =
// fp16(g[k] W[j][k]) with k = perm(kk) (identity when perm is null),
// c[q][j] = sum of the fp16 W' row over the folded columns of statistics
// group q (group_cols columns each), d_j = b_j + sum_k beta_k W[j][k] (b may
// be null); sums in double.
struct FoldedLinear {
    std::vector<uint16_t> w;
    std::vector<float> c, d;  // c: [K / group_cols][N]
    // c as the GEMM epilogue's centring-correction table (ln_fold.h,
    // LnCorr): per column, fp16(c[q][j]) at k-slots 2q and 2q + 1, zero up to
    // the next multiple of 32 slots.
    std::vector<uint16_t> corr() const {
        const size_t N = d.size(), groups = c.size() / N;
        const size_t slots = (2 * groups + 31) / 32 * 32;
        std::vector<uint16_t> t(N * slots, 0);
        for (size_t j = 0; j < N; ++j)
            for (size_t q = 0; q < groups; ++q)
                t[j * slots + 2 * q] = t[j * slots + 2 * q + 1] = f16_bits(c[q * N + j]);
        return t;
    }
};

// Column order of the patch-merge reduction weights: folded column q*C + ch
// reads the reference's unfold column ch*4 + q (nn.Unfold order, channel then
// tap q = 2 ky + kx; swin_backbone.c:287-296), the tap-major order in which
// DmaMergeRows gathers the 2x2 tokens.
std::vector<int> merge_tap_order(int C) {
    std::vector<int> perm(4 * (size_t)C);
    for (int q = 0; q < 4; ++q)
        for (int ch = 0; ch < C; ++ch) perm[(size_t)q * C + ch] = ch * 4 + q;
    return perm;
}

FoldedLinear fold_ln(const float *W, const float *b, const float *g, const float *beta, int N,
                     int K, const std::vector<int> *perm, int group_cols) {
    FoldedLinear f;
    const int groups = K / group_cols;
    f.w.resize((size_t)N * K);
    f.c.resize((size_t)groups * N);
    f.d.resize(N);
    for (int j = 0; j < N; ++j) {
        const float *row = W + (size_t)j * K;
        double ds = b ? (double)b[j] : 0.0;
        for (int q = 0; q < groups; ++q) {
            double cs = 0.0;
            for (int kk = q * group_cols; kk < (q + 1) * group_cols; ++kk) {
                const int k = perm ? (*perm)[kk] : kk;
                const uint16_t h = f16_bits(g[k] * row[k]);
                f.w[(size_t)j * K + kk] = h;
                cs += (double)f16_value(h);
                ds += (double)beta[k] * (double)row[k];
            }
            f.c[(size_t)q * N + j] = (float)cs;
        }
        f.d[j] = (float)ds;
    }
    return f;
}

// Tiles of 64 tokens x 64 channels (792 / 396 blocks for C = 192 / 384 at
// 6 x 256 x 704), 32 tokens at C = 768 (396 blocks).  Measured on MI355X at
// 6 x 256 x 704: 6.5 / 5.6 / 5.0 us vs 9.3 / 7.4 / 6.6 us for one block per
// 16 / 8 / 4 whole rows that computed its own statistics (frame -5 us).
void launch_out_ln(int C, const float *x, const float2 *stats, float *out, const float *g,
                   const float *b, int rows, int hw, hipStream_t s) {
    const bool vec = hw % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const OutLnArgs a{x, stats, out, g, b, rows, hw, vec};
    switch (C) {
        case 192:
            hipLaunchKernelGGL((out_ln_kernel<3, 64>), dim3((rows + 63) / 64, 3), dim3(256), 0, s, a);
            break;
        case 384:
            hipLaunchKernelGGL((out_ln_kernel<6, 64>), dim3((rows + 63) / 64, 6), dim3(256), 0, s, a);
            break;
        case 768:
            hipLaunchKernelGGL((out_ln_kernel<12, 32>), dim3((rows + 31) / 32, 12), dim3(256), 0, s, a);
            break;
        default: break;
    }
}

}  // namespace

extern "C" void bf_cuda_swin_destroy(bf_cuda_swin *s) {
    if (!s) return;
    if (s->params) (void)hipFree(s->params);
    if (s->acts) (void)hipFree(s->acts);
    std::free(s);
}

extern "C" size_t bf_cuda_swin_resident_bytes(const bf_cuda_swin *s) {
    return s ? s->resident_bytes : 0;
}

static int swin_build(bf_cuda_swin *s, const bf_model *model, size_t batches, size_t input_h,
                      size_t input_w, char *error, size_t cap) {
    s->batches = batches;
    s->input_h = input_h;
    s->input_w = input_w;
    s->h[0] = (int)(input_h / 4);
    s->w[0] = (int)(input_w / 4);
    for (int i = 1; i < 4; ++i) {
        s->h[i] = (s->h[i - 1] + 1) / 2;
        s->w[i] = (s->w[i - 1] + 1) / 2;
    }

    ParamArena arena;
    char name[224];
    size_t o_patch_w, o_patch_b, o_patch_ns, o_patch_nb;
    BlockOff off[4][6];
    size_t o_mw[3], o_os[3], o_ob[3], o_mc[3] = {}, o_md[3] = {};
    {
        const float *pw = bind_f32(model, "image_backbone.patch_embed.projection.weight",
                                   {96, 3, 4, 4}, error, cap);
        const float *pb = bind_f32(model, "image_backbone.patch_embed.projection.bias", {96},
                                   error, cap);
        const float *ns = bind_f32(model, "image_backbone.patch_embed.norm.weight", {96}, error,
                                   cap);
        const float *nb = bind_f32(model, "image_backbone.patch_embed.norm.bias", {96}, error,
                                   cap);
        if (!pw || !pb || !ns || !nb) return 0;
        o_patch_w = arena.add_f16(pw, 96 * 48);
        o_patch_b = arena.add_f32(pb, 96);
        o_patch_ns = arena.add_f32(ns, 96);
        o_patch_nb = arena.add_f32(nb, 96);
    }
    for (int st = 0; st < 4; ++st) {
        const uint32_t c = (uint32_t)kC[st], hd = (uint32_t)kHeads[st];
        for (int b = 0; b < kDepth[st]; ++b) {
            BlockOff &o = off[st][b];
#define BF_F32(SUFFIX, ...)                                                                  \
    (std::snprintf(name, sizeof(name), "image_backbone.stages.%d.blocks.%d.%s", st, b, SUFFIX), \
     bind_f32(model, name, {__VA_ARGS__}, error, cap))
            const float *n1s = BF_F32("norm1.weight", c), *n1b = BF_F32("norm1.bias", c);
            const float *table = BF_F32("attn.w_msa.relative_position_bias_table", 169, hd);
            std::snprintf(name, sizeof(name),
                          "image_backbone.stages.%d.blocks.%d.attn.w_msa.relative_position_index",
                          st, b);
            const uint32_t idims[2] = {49, 49};
            const int64_t *index =
                (const int64_t *)bind_tensor(model, name, BF_DTYPE_I64, 2, idims, error, cap);
            const float *qkv_w = BF_F32("attn.w_msa.qkv.weight", 3 * c, c);
            const float *qkv_b = BF_F32("attn.w_msa.qkv.bias", 3 * c);
            const float *proj_w = BF_F32("attn.w_msa.proj.weight", c, c);
            const float *proj_b = BF_F32("attn.w_msa.proj.bias", c);
            const float *n2s = BF_F32("norm2.weight", c), *n2b = BF_F32("norm2.bias", c);
            const float *fc1_w = BF_F32("ffn.layers.0.0.weight", 4 * c, c);
            const float *fc1_b = BF_F32("ffn.layers.0.0.bias", 4 * c);
            const float *fc2_w = BF_F32("ffn.layers.1.weight", c, 4 * c);
            const float *fc2_b = BF_F32("ffn.layers.1.bias", c);
#undef BF_F32
            if (!n1s || !n1b || !table || !index || !qkv_w || !qkv_b || !proj_w || !proj_b ||
                !n2s || !n2b || !fc1_w || !fc1_b || !fc2_w || !fc2_b)
                return 0;
            // Dense per-head bias matrix [heads][49][49] gathered through the
            // checkpoint's index table (bounds as reference swin.c:34-37).
            std::vector<float> bias((size_t)hd * 49 * 49);
            for (int q = 0; q < 49 * 49; ++q) {
                const int64_t r = index[q];
                if (r < 0 || r >= 169) {
                    fail(error, cap, "stage %d block %d: relative_position_index out of range",
                         st, b);
                    return 0;
                }
                for (uint32_t hh = 0; hh < hd; ++hh) bias[(size_t)hh * 2401 + q] = table[r * hd + hh];
            }
            o.n1s = arena.add_f32(n1s, c); o.n1b = arena.add_f32(n1b, c);
            o.n2s = arena.add_f32(n2s, c); o.n2b = arena.add_f32(n2b, c);
            o.qkv_b = arena.add_f32(qkv_b, 3 * c); o.proj_b = arena.add_f32(proj_b, c);
            o.fc1_b = arena.add_f32(fc1_b, 4 * c); o.fc2_b = arena.add_f32(fc2_b, c);
            o.bias_mat = arena.add_f32(bias);
            o.attn_term = arena.add(nullptr, attn_term_elems((int)hd, (b & 1) ? 3 : 0) * 2);
            o.proj_w = arena.add_f16(proj_w, (size_t)c * c);
            o.fc2_w = arena.add_f16(fc2_w, (size_t)4 * c * c);
            o.qkv_corr = o.qkv_d = o.fc1_corr = o.fc1_d = 0;
            if (st == 0) {  // fused window MSA and MLP: LayerNorm kept explicit
                o.qkv_w = arena.add_f16(qkv_w, (size_t)3 * c * c);
                o.fc1_w = arena.add_f16(fc1_w, (size_t)4 * c * c);
            } else {
                const FoldedLinear fq = fold_ln(qkv_w, qkv_b, n1s, n1b, 3 * c, c, nullptr, kStatCols);
                const FoldedLinear f1 = fold_ln(fc1_w, fc1_b, n2s, n2b, 4 * c, c, nullptr, kStatCols);
                o.qkv_w = arena.add(fq.w.data(), fq.w.size() * 2);
                const std::vector<uint16_t> qc = fq.corr(), fc = f1.corr();
                o.qkv_corr = arena.add(qc.data(), qc.size() * 2);
                o.qkv_d = arena.add_f32(fq.d);
                o.fc1_w = arena.add(f1.w.data(), f1.w.size() * 2);
                o.fc1_corr = arena.add(fc.data(), fc.size() * 2);
                o.fc1_d = arena.add_f32(f1.d);
            }
            o.mlp_w = o.mlp_proj = 0;
            if (kFusedMlp[st]) {
                std::vector<uint16_t> packed((size_t)MlpS0::kChunks * MlpS0::kChunkBytes / 2);
                pack_mlp_weights<MlpS0>(fc1_w, fc2_w, fc1_b, packed.data(), f16_bits);
                o.mlp_w = arena.add(packed.data(), packed.size() * 2);
                std::vector<uint16_t> proj((size_t)c * c);
                pack_proj_weights<MlpS0>(proj_w, proj.data(), f16_bits);
                o.mlp_proj = arena.add(proj.data(), proj.size() * 2);
            }
        }
    }
    for (int st = 0; st < 3; ++st) {
        const uint32_t c = (uint32_t)kC[st];
        std::snprintf(name, sizeof(name), "image_backbone.stages.%d.downsample.norm.weight", st);
        const float *ms = bind_f32(model, name, {4 * c}, error, cap);
        std::snprintf(name, sizeof(name), "image_backbone.stages.%d.downsample.norm.bias", st);
        const float *mb = bind_f32(model, name, {4 * c}, error, cap);
        std::snprintf(name, sizeof(name), "image_backbone.stages.%d.downsample.reduction.weight", st);
        const float *mw = bind_f32(model, name, {2 * c, 4 * c}, error, cap);
        std::snprintf(name, sizeof(name), "image_backbone.norm%d.weight", st + 1);
        const float *os = bind_f32(model, name, {(uint32_t)kC[st + 1]}, error, cap);
        std::snprintf(name, sizeof(name), "image_backbone.norm%d.bias", st + 1);
        const float *ob = bind_f32(model, name, {(uint32_t)kC[st + 1]}, error, cap);
        if (!ms || !mb || !mw || !os || !ob) return 0;
        const std::vector<int> perm = merge_tap_order((int)c);
        // Statistics groups of the merge input: 64 channels of each of the
        // four tokens, or each whole 96-channel token at stage 0.
        const int gcols = c % kStatCols ? (int)c : kStatCols;
        const FoldedLinear fm = fold_ln(mw, nullptr, ms, mb, 2 * c, 4 * c, &perm, gcols);
        o_mw[st] = arena.add(fm.w.data(), fm.w.size() * 2);
        const std::vector<uint16_t> mc = fm.corr();
        o_mc[st] = arena.add(mc.data(), mc.size() * 2);
        o_md[st] = arena.add_f32(fm.d);
        o_os[st] = arena.add_f32(os, kC[st + 1]);
        o_ob[st] = arena.add_f32(ob, kC[st + 1]);
    }
    {
        if (!hip_ok(hipMalloc(&s->params, arena.host.size()), error, cap, "allocate Swin parameters") ||
            !hip_ok(hipMemcpy(s->params, arena.host.data(), arena.host.size(), hipMemcpyHostToDevice),
                    error, cap, "upload Swin parameters"))
            return 0;
        s->resident_bytes += arena.host.size();
        unsigned char *p = s->params;
        auto F = [p](size_t o) { return (const float *)(p + o); };
        auto H = [p](size_t o) { return (const bf16 *)(p + o); };
        s->patch_w = H(o_patch_w); s->patch_b = F(o_patch_b);
        s->patch_ns = F(o_patch_ns); s->patch_nb = F(o_patch_nb);
        for (int st = 0; st < 4; ++st)
            for (int b = 0; b < kDepth[st]; ++b) {
                const BlockOff &o = off[st][b];
                BlockW &w = s->blocks[st][b];
                w.n1s = F(o.n1s); w.n1b = F(o.n1b); w.n2s = F(o.n2s); w.n2b = F(o.n2b);
                w.qkv_b = F(o.qkv_b); w.proj_b = F(o.proj_b); w.fc1_b = F(o.fc1_b);
                w.fc2_b = F(o.fc2_b); w.bias_mat = F(o.bias_mat);
                w.qkv_w = H(o.qkv_w); w.proj_w = H(o.proj_w); w.fc1_w = H(o.fc1_w);
                w.fc2_w = H(o.fc2_w);
                w.qkv_corr = st ? H(o.qkv_corr) : nullptr; w.qkv_d = st ? F(o.qkv_d) : nullptr;
                w.fc1_corr = st ? H(o.fc1_corr) : nullptr; w.fc1_d = st ? F(o.fc1_d) : nullptr;
                w.mlp_w = kFusedMlp[st] ? H(o.mlp_w) : nullptr;
                w.mlp_proj = kFusedMlp[st] ? H(o.mlp_proj) : nullptr;
                w.attn_term = H(o.attn_term);
            }
        for (int st = 0; st < 3; ++st) {
            s->merge_w[st] = H(o_mw[st]); s->out_s[st] = F(o_os[st]); s->out_b[st] = F(o_ob[st]);
            s->merge_corr[st] = H(o_mc[st]);
            s->merge_d[st] = F(o_md[st]);
        }
        // Attention score terms (relative bias + shift mask, in the kernel's
        // accumulator order) from the uploaded bias matrices.
        for (int st = 0; st < 4; ++st)
            for (int b = 0; b < kDepth[st]; ++b) {
                const int shift = (b & 1) ? 3 : 0, heads = kHeads[st];
                const int wy_n = (s->h[st] + 6) / 7, wx_n = (s->w[st] + 6) / 7;
                hipLaunchKernelGGL(attn_term_kernel, dim3(window_types(shift) * heads * 8), dim3(64), 0,
                                   nullptr, s->blocks[st][b].bias_mat,
                                   const_cast<bf16 *>(s->blocks[st][b].attn_term), heads, wy_n, wx_n,
                                   shift);
            }
        if (!launch_ok(error, cap, "build attention terms") ||
            !hip_ok(hipDeviceSynchronize(), error, cap, "build attention terms"))
            return 0;
    }
    {
        size_t x_elems = 0, xn_elems = 0, big_elems = 0, xh_elems = 0, stat_elems = 0;
        const size_t tok1 = batches * (size_t)s->h[1] * s->w[1];
        const size_t tok2 = batches * (size_t)s->h[2] * s->w[2];
        s->x2_off = (tok1 * kC[1] + 63) & ~size_t(63);  // 256-byte aligned
        x_elems = s->x2_off + tok2 * kC[2];
        for (int st = 0; st < 4; ++st) {
            const size_t t = batches * (size_t)s->h[st] * s->w[st];
            x_elems = std::max(x_elems, t * kC[st]);
            // Stage 0's copy and statistics (one group of all 96 channels per
            // token) live in xn and big, which are free when it ends; the
            // activation layout is that of stages 1-3 alone (changing it
            // measured up to 9 us per frame slower).
            if (st > 0) {
                xh_elems = std::max(xh_elems, t * kC[st]);
                stat_elems = std::max(stat_elems, t * (kC[st] / kStatCols));
            }
            xn_elems = std::max(xn_elems, t * kC[st]);
            big_elems = std::max(big_elems, t * 4 * kC[st]);
            if (st < 3) {
                const size_t t2 = batches * (size_t)s->h[st + 1] * s->w[st + 1];
                xn_elems = std::max(xn_elems, t2 * 4 * kC[st]);
            }
        }
        // The linears address their 16-bit operands through 32-bit buffer offsets.
        if (std::max(std::max(xn_elems, big_elems), xh_elems) * 2 >= (size_t(1) << 31)) {
            fail(error, cap, "Swin batch too large: %zu images exceed the 2 GiB activation limit",
                 batches);
            return 0;
        }
        const size_t x_bytes = (x_elems * 4 + 255) & ~size_t(255);
        const size_t xn_bytes = (xn_elems * 2 + 255) & ~size_t(255);
        const size_t big_bytes = (big_elems * 2 + 255) & ~size_t(255);
        const size_t xh_bytes = (xh_elems * 2 + 255) & ~size_t(255);
        const size_t stat_bytes = (stat_elems * sizeof(float2) + 255) & ~size_t(255);
        const size_t total = x_bytes + xn_bytes + big_bytes + 2 * (xh_bytes + stat_bytes);
        if (!hip_ok(hipMalloc(&s->acts, total), error, cap, "allocate Swin activations"))
            return 0;
        unsigned char *p = s->acts;
        s->x = (float *)p;
        s->xn = (bf16 *)(p += x_bytes);
        s->big = (bf16 *)(p += xn_bytes);
        p += big_bytes;
        for (int i = 0; i < 2; ++i) {
            s->xh[i] = (bf16 *)p;
            s->stats[i] = (float2 *)(p + xh_bytes);
            p += xh_bytes + stat_bytes;
        }
        s->resident_bytes += total;
    }
    return 1;
}

extern "C" int bf_cuda_swin_create(const bf_model *model, size_t batches, size_t input_h,
                                   size_t input_w, bf_cuda_swin **out, char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!model || !out || !batches || !input_h || !input_w || (input_h % 4) || (input_w % 4) ||
        batches > INT_MAX || input_h > INT_MAX || input_w > INT_MAX)
        return fail(error, cap, "invalid HIP Swin contract");
    // Stage-0 hidden activations ([tokens, 384]) must index within int range.
    if ((unsigned long long)batches * (input_h / 4) * (input_w / 4) * 384ull > (unsigned long long)INT_MAX)
        return fail(error, cap, "HIP Swin input is too large");
    bf_cuda_swin *s = (bf_cuda_swin *)std::calloc(1, sizeof(*s));
    if (!s) return fail(error, cap, "Swin host allocation failed");
    if (!swin_build(s, model, batches, input_h, input_w, error, cap)) {
        bf_cuda_swin_destroy(s);
        return 0;
    }
    *out = s;
    return 1;
}

namespace {

// The launches of one frame, factored per op so that the forward and the
// profiling hook (bfhip_swin_profile_op) run exactly the same kernels.
void patch_embed(bf_cuda_swin *s, const float *images, hipStream_t stream) {
    // 4x4/s4 conv 3->96 straight from NCHW images into NHWC tokens; the
    // epilogue holds whole rows and applies the patch norm (-> x) and block
    // 0's LN1 (-> xn).
    using T = Tile<64, 96, 32, 1, 2, true>;
    const int B = (int)s->batches;
    ConvGeom g{};
    g.N = B; g.Ci = 3; g.IH = (int)s->input_h; g.IW = (int)s->input_w;
    g.OH = s->h[0]; g.OW = s->w[0]; g.KH = 4; g.KW = 4; g.SH = 4; g.SW = 4;
    g.PH = 0; g.PW = 0; g.transpose = 0;
    g.M = B * s->h[0] * s->w[0]; g.K = 48;
    LoadRowsBf16<T::BN, T::BK, T::kThreads> bl{s->patch_w, 48, 96, 48};
    const BlockW &b0 = s->blocks[0][0];
    EpiPatchNorms epi{stage_x(s, 0), s->xn, s->patch_b, s->patch_ns, s->patch_nb, b0.n1s, b0.n1b, g.M};
    if (((uintptr_t)images & 15) == 0) {  // IW % 4 == 0 by contract: float4 patch rows
        LoadPatch4x4<T::BM, T::BK, T::kThreads, true> al{images, g};
        launch_gemm<T>(al, bl, epi, g.M, 96, 48, stream);
    } else {
        LoadConvA<T::BM, T::BK, T::kThreads, 4, 4, SrcNCHW, true> al{};
        al.src = SrcNCHW{images, 3, g.IH, g.IW};
        al.g = g;
        launch_gemm<T>(al, bl, epi, g.M, 96, 48, stream);
    }
}

// The fp16 copy of x and its row statistics that stage st's folded consumers
// read: xh / stats of its parity at stages 1-3; at stage 0, whose last block
// writes them for the merge only, xn (the attention rows it overwrites in
// place) and the front of big (free then).
bf16 *stage_xh(bf_cuda_swin *s, int st) { return st ? s->xh[st & 1] : s->xn; }
float2 *stage_stats(bf_cuda_swin *s, int st) {
    return st ? s->stats[st & 1] : reinterpret_cast<float2 *>(s->big);
}

// Calls f(std::integral_constant<int, C / 64>) for the channel counts of
// stages 1-3 (the statistics groups per token).
template <class F>
void with_groups(int C, F &&f) {
    switch (C) {
        case 192: f(std::integral_constant<int, 3>{}); break;
        case 384: f(std::integral_constant<int, 6>{}); break;
        case 768: f(std::integral_constant<int, 12>{}); break;
        default: break;
    }
}

void block_op(bf_cuda_swin *s, int st, int b, int op, hipStream_t stream) {
    const int B = (int)s->batches, C = kC[st], heads = kHeads[st], H = s->h[st], W = s->w[st];
    const int T = B * H * W, wy_n = (H + 6) / 7, wx_n = (W + 6) / 7;
    const int items = B * wy_n * wx_n * heads;
    const BlockW &w = s->blocks[st][b];
    bf16 *xh = s->xh[st & 1];
    float2 *stats = s->stats[st & 1];
    switch (op) {
        case BFHIP_SWIN_QKV:  // LN1 folded
            with_groups(C, [&](auto g) {
                using Src = LnRows<decltype(g)::value>;
                linear_f16(xh, w.qkv_w, T, 3 * C, C,
                           EpiLnF16<false, Src>{s->big, w.qkv_d, w.qkv_corr, Src{stats}, 3 * C, T, 3 * C},
                           stream);
            });
            break;
        case BFHIP_SWIN_ATTENTION:
            hipLaunchKernelGGL(window_attention_kernel, dim3((items + kAttnWaves - 1) / kAttnWaves),
                               dim3(64 * kAttnWaves), 0, stream, s->big, w.qkv_b, w.attn_term,
                               s->xn, H, W, C, heads, wy_n, wx_n, (b & 1) ? 3 : 0, items);
            break;
        case BFHIP_SWIN_WMSA:
            // xn -> attention output, in place: a window's rows are gathered
            // into LDS before any wave of that window writes, and windows
            // own disjoint token rows.
            if (C == 96)
                hipLaunchKernelGGL(window_msa_kernel<96>, dim3(B * wy_n * wx_n), dim3(64 * 3), 0,
                                   stream, s->xn, w.qkv_w, w.qkv_b, w.attn_term, s->xn, H, W, wy_n,
                                   wx_n, (b & 1) ? 3 : 0);
            else
                hipLaunchKernelGGL(window_msa_kernel<192>, dim3(B * wy_n * wx_n), dim3(64 * 6), 0,
                                   stream, s->xn, w.qkv_w, w.qkv_b, w.attn_term, s->xn, H, W, wy_n,
                                   wx_n, (b & 1) ? 3 : 0);
            break;
        case BFHIP_SWIN_PROJ:
            linear_f16(s->xn, w.proj_w, T, C, C,
                       EpiStatsRows<false, true>{stage_x(s, st), xh, stats, w.proj_b, nullptr, {}, T, C},
                       stream);
            break;
        case BFHIP_SWIN_FC1:  // LN2 folded
            with_groups(C, [&](auto g) {
                using Src = LnRows<decltype(g)::value>;
                linear_f16(xh, w.fc1_w, T, 4 * C, C,
                           EpiLnF16<true, Src>{s->big, w.fc1_d, w.fc1_corr, Src{stats}, 4 * C, T, 4 * C},
                           stream);
            });
            break;
        case BFHIP_SWIN_FC2:
            // The last block of a stage leaves x and its row statistics for
            // the stage-output norm (and, before stage 3, the patch merge).
            linear_f16(s->big, w.fc2_w, T, C, 4 * C,
                       EpiStatsRows<false, true>{stage_x(s, st), xh, stats, w.fc2_b, nullptr, {}, T, C},
                       stream);
            break;
        case BFHIP_SWIN_MLP: {
            // The next block's LN1 is fused into the epilogue; the last block
            // of the stage writes xh and the row statistics for the patch
            // merge, which folds its LayerNorm (x itself is not read again).
            const bool next = b + 1 < kDepth[st];
            const BlockW *nw = next ? &s->blocks[st][b + 1] : nullptr;
            // proj reads the attention output in xn; LN1' overwrites it row by row.
            launch_swin_mlp<MlpS0>(stage_x(s, st), s->xn, w.mlp_proj, w.proj_b, w.n2s, w.n2b, w.mlp_w,
                                   w.fc1_b, w.fc2_b, nw ? nw->n1s : nullptr,
                                   nw ? nw->n1b : nullptr, next ? s->xn : nullptr, T, stream,
                                   next ? nullptr : stage_xh(s, st),
                                   next ? nullptr : stage_stats(s, st));
            break;
        }
        default:
            break;
    }
}

// The ops one block launches, in order (no LayerNorm launch: the patch
// embedding writes stage 0's first LN1, the fused MLP the next ones, and the
// other stages fold theirs into the linears).
int block_ops(int st, int b, int *ops) {
    (void)b;
    int n = 0;
    if (kFusedWmsa[st]) {
        ops[n++] = BFHIP_SWIN_WMSA;  // QKV + attention
    } else {
        ops[n++] = BFHIP_SWIN_QKV;
        ops[n++] = BFHIP_SWIN_ATTENTION;
    }
    if (kFusedMlp[st]) {
        ops[n++] = BFHIP_SWIN_MLP;  // proj + residual + LN2 + fc1 + fc2 + residual (+ LN1')
    } else {
        ops[n++] = BFHIP_SWIN_PROJ;
        ops[n++] = BFHIP_SWIN_FC1;
        ops[n++] = BFHIP_SWIN_FC2;
    }
    return n;
}

// A patch merge and the stage-output LayerNorm of the same stage in one
// launch: workgroups [0, tiles) are the merge's tiles (the first ids, so
// their XCD mapping is the standalone launch's), the rest the LayerNorm's
// 64-token x 64-channel tiles (OutLn).  Both read stage st's activations;
// the merge writes stage st + 1's residual into the other parity buffer, so
// the two are independent, and the LayerNorm's HBM-bound tiles fill the CU
// slots the merge leaves free instead of running after it.  The branch is
// uniform per workgroup.
template <bool SPEC, class T, class ALoad, class BLoad, class Epi, int G, int THREADS>
__global__ __launch_bounds__(THREADS) void merge_out_ln_kernel(ALoad al, BLoad bl, Epi epi, int M,
                                                               int N, int K, int tiles_n,
                                                               int tiles, OutLnArgs o) {
    using LN = OutLn<G, 64, THREADS>;
    constexpr size_t kM = dma_smem_bytes<T, Epi>();
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kM > LN::kSmem ? kM : LN::kSmem];
    const int bid = (int)blockIdx.x;
    if (bid < tiles) {
        const int pid = xcd_swizzle(bid, tiles);
        if constexpr (SPEC)
            gemm_spec_block<T>(al, bl, epi, M, N, K, tiles_n, pid, smem);
        else
            gemm_dma_block<T>(al, bl, epi, M, N, K, tiles_n, pid, smem);
        return;
    }
    const int r = bid - tiles;
    LN::block(o, r / G, r % G, smem);
}

// Patch merge after stage st with its LayerNorm over 4C folded: the A operand
// gathers the 2x2 tokens from xh, the statistics combine the tokens' group
// partials (groups of 64 channels, or the whole 96-channel token at stage 0),
// and the epilogue writes the next stage's x, xh and stats.  Tiles as
// linear_f16 picks for these (N, K); LW > 0 runs the tile on the
// wave-specialised pipeline with LW loader waves (measured on MI355X for the
// second merge, 1056 x 768 x 1536: 7.3 vs 8.9 us).  The gather and its tile
// are merge_gemm's, which bfhip_debug_swin_merge_gather also runs.  With
// `ln` (stages 1 and 2), stage st's output LayerNorm runs in the same launch
// (merge_out_ln_kernel, G = C / 64 statistics groups).
template <int C, class T, int LW, class Epi>
void merge_gemm(const bf16 *xh, int B, int H, int W, const bf16 *w, int N, const Epi &epi,
                hipStream_t stream, const OutLnArgs *ln = nullptr) {
    const int T2 = B * ((H + 1) / 2) * ((W + 1) / 2);
    constexpr int kLoadThreads = LW > 0 ? LW * kWave : T::kThreads;
    DmaMergeRows<T::BM, T::BK, kLoadThreads, C> al{};
    al.base = xh;
    al.batches = B;
    al.H = H;
    al.W = W;
    DmaRowsBf16<T::BN, T::BK, kLoadThreads> bl{w, 4 * C, N, 4 * C};
    if constexpr (C % kStatCols == 0) {
        if (ln) {
            constexpr int G = C / kStatCols, kThreads = T::kThreads + (LW > 0 ? LW * kWave : 0);
            const int tiles_n = (N + T::BN - 1) / T::BN;
            const int tiles = (T2 + T::BM - 1) / T::BM * tiles_n;
            const int ln_blocks = (ln->rows + 63) / 64 * G;
            hipLaunchKernelGGL((merge_out_ln_kernel<(LW > 0), T, decltype(al), decltype(bl), Epi, G, kThreads>),
                               dim3(tiles + ln_blocks), dim3(kThreads), 0, stream, al, bl, epi, T2, N,
                               4 * C, tiles_n, tiles, *ln);
            return;
        }
    }
    if constexpr (LW > 0)
        launch_gemm_spec<T>(al, bl, epi, T2, N, 4 * C, stream);
    else
        launch_gemm_dma<T>(al, bl, epi, T2, N, 4 * C, stream);
}

template <int C, class T, int LW = 0>
void merge_folded(bf_cuda_swin *s, int st, hipStream_t stream, const OutLnArgs *ln = nullptr) {
    const int B = (int)s->batches, H = s->h[st], W = s->w[st];
    const int T2 = B * s->h[st + 1] * s->w[st + 1];
    const int nx = (st + 1) & 1;
    constexpr bool kWhole = C % kStatCols != 0;  // one group per token
    using Src = LnMerge<kWhole ? 1 : C / kStatCols, kWhole ? C : kStatCols>;
    EpiStatsRows<true, false, Src> epi{stage_x(s, st + 1), s->xh[nx],     s->stats[nx],
                                       s->merge_d[st], s->merge_corr[st], Src{stage_stats(s, st), H, W},
                                       T2,            2 * C};
    merge_gemm<C, T, LW>(stage_xh(s, st), B, H, W, s->merge_w[st], 2 * C, epi, stream, ln);
}

// The merge tiles per stage.
using MergeT0 = DmaTile<128, 64, 64, 2, 2, 2, true>;
using MergeT1 = DmaTile<64, 64, 64, 2, 2, 2, true>;
using MergeT2 = DmaTile<64, 64, 128, 2, 2, 3, true>;
constexpr int kMergeLoaders2 = 4;

// The merge after stage st; with `ln`, stage st's output LayerNorm in the
// same launch (stages 1 and 2).
void merge_op(bf_cuda_swin *s, int st, hipStream_t stream, const OutLnArgs *ln = nullptr) {
    if (st == 0)
        merge_folded<96, MergeT0>(s, st, stream);
    else if (st == 1)
        merge_folded<192, MergeT1>(s, st, stream, ln);
    else
        merge_folded<384, MergeT2, kMergeLoaders2>(s, st, stream, ln);
}

// Stage st's output LayerNorm into `out` (NCHW fp32).
OutLnArgs out_ln_args(bf_cuda_swin *s, int st, float *out) {
    const int T = (int)s->batches * s->h[st] * s->w[st], hw = s->h[st] * s->w[st];
    return OutLnArgs{stage_x(s, st), stage_stats(s, st), out, s->out_s[st - 1], s->out_b[st - 1], T,
                     hw, hw % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0};
}

}  // namespace

extern "C" int bf_cuda_swin_forward(bf_cuda_swin *s, const float *images, float *out1,
                                    float *out2, float *out3, void *stream_value, char *error,
                                    size_t cap) {
    if (!s || !images || !out1 || !out2 || !out3)
        return fail(error, cap, "invalid HIP Swin buffers");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_value);
    float *outputs[3] = {out1, out2, out3};
    patch_embed(s, images, stream);
    for (int st = 0; st < 4; ++st) {
        for (int b = 0; b < kDepth[st]; ++b) {
            int ops[8];
            const int n = block_ops(st, b, ops);
            for (int i = 0; i < n; ++i) block_op(s, st, b, ops[i], stream);
        }
        // Stage outputs: stage 3's alone, stages 1 and 2 in the merge's launch.
        if (st == 3) {
            const int T = (int)s->batches * s->h[st] * s->w[st];
            launch_out_ln(kC[st], stage_x(s, st), stage_stats(s, st), outputs[st - 1], s->out_s[st - 1],
                          s->out_b[st - 1], T, s->h[st] * s->w[st], stream);
        } else if (st > 0) {
            const OutLnArgs ln = out_ln_args(s, st, outputs[st - 1]);
            merge_op(s, st, stream, &ln);
        } else {
            merge_op(s, st, stream);
        }
    }
    return launch_ok(error, cap, "launch HIP Swin graph");
}

extern "C" int bfhip_swin_profile_op(bf_cuda_swin *s, int stage, int block, int op, void *stream,
                                     char *error, size_t cap) {
    if (!s || stage < 0 || stage > 3 || block < 0 || block >= kDepth[stage] ||
        op < BFHIP_SWIN_LN1 || op > BFHIP_SWIN_WMSA || (op == BFHIP_SWIN_MERGE && stage > 2))
        return fail(error, cap, "invalid HIP Swin profiling op");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (op == BFHIP_SWIN_MERGE) {
        merge_op(s, stage, st);
    } else {
        int ops[8];
        const int n = block_ops(stage, block, ops);
        if (std::find(ops, ops + n, op) == ops + n)
            return fail(error, cap, "stage %d block %d does not launch op %d", stage, block, op);
        block_op(s, stage, block, op, st);
    }
    return launch_ok(error, cap, "launch HIP Swin profiling op");
}

extern "C" int bfhip_swin_profile_io(bf_cuda_swin *s, int stage, int op, const float *images,
                                     float *out, void *stream, char *error, size_t cap) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (s && op == BFHIP_SWIN_PATCH_EMBED && stage == 0 && images) {
        patch_embed(s, images, st);
    } else if (s && op == BFHIP_SWIN_OUT_NORM && stage >= 1 && stage <= 3 && out) {
        const int T = (int)s->batches * s->h[stage] * s->w[stage];
        launch_out_ln(kC[stage], stage_x(s, stage), stage_stats(s, stage), out, s->out_s[stage - 1],
                      s->out_b[stage - 1], T, s->h[stage] * s->w[stage], st);
    } else if (s && op == BFHIP_SWIN_MERGE_OUT_NORM && stage >= 1 && stage <= 2 && out) {
        const OutLnArgs ln = out_ln_args(s, stage, out);
        merge_op(s, stage, st, &ln);
    } else {
        return fail(error, cap, "invalid HIP Swin profiling io call");
    }
    return launch_ok(error, cap, "launch HIP Swin profiling io op");
}

extern "C" int bfhip_debug_window_map(int batches, int height, int width, int shift, int *token,
                                      int *label, void *stream, char *error, size_t cap) {
    if (!token || !label || batches <= 0 || height <= 0 || width <= 0 || shift < 0 || shift >= 7)
        return fail(error, cap, "invalid window-map probe");
    const long long wy_n = (height + 6) / 7, wx_n = (width + 6) / 7;
    const long long total = (long long)batches * wy_n * wx_n * 49;
    if (total > INT_MAX || (long long)batches * height * width > INT_MAX)
        return fail(error, cap, "window-map probe is too large");
    hipLaunchKernelGGL(window_map_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), token, label, batches, height, width,
                       (int)wy_n, (int)wx_n, shift);
    return launch_ok(error, cap, "launch window-map probe");
}

namespace {

// Contract of the window-attention probes: returns the (window, head) item
// count, or 0 with a message in error.
int window_attention_items(const void *qkv, const float *qkv_bias, const float *bias_mat,
                           const void *out, int batches, int height, int width, int channels,
                           int heads, int shift, char *error, size_t cap) {
    if (!qkv || !qkv_bias || !bias_mat || !out || batches <= 0 || height <= 0 || width <= 0 ||
        heads <= 0 || channels != 32 * heads || shift < 0 || shift >= 7)
        return fail(error, cap, "invalid window-attention probe");
    const long long wy_n = (height + 6) / 7, wx_n = (width + 6) / 7;
    const long long items = (long long)batches * wy_n * wx_n * heads;
    if (items > INT_MAX || (long long)batches * height * width * 3 * channels > INT_MAX)
        return fail(error, cap, "window-attention probe is too large");
    if ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(qkv_bias) |
         reinterpret_cast<uintptr_t>(out)) & 15)
        return fail(error, cap, "window-attention probe buffers must be 16-byte aligned");
    return (int)items;
}

// Builds the score terms with the context's builder into `term` (at least
// attn_term_elems(heads, shift) words), then runs the attention kernel.
void window_attention_launch(const void *qkv, const float *qkv_bias, const float *bias_mat,
                             void *out, bf16 *term, int height, int width, int channels,
                             int heads, int shift, int items, hipStream_t s) {
    const int wy_n = (height + 6) / 7, wx_n = (width + 6) / 7;
    hipLaunchKernelGGL(attn_term_kernel, dim3(window_types(shift) * heads * 8), dim3(64), 0, s,
                       bias_mat, term, heads, wy_n, wx_n, shift);
    hipLaunchKernelGGL(window_attention_kernel, dim3((unsigned)((items + kAttnWaves - 1) / kAttnWaves)),
                       dim3(64 * kAttnWaves), 0, s, static_cast<const bf16 *>(qkv), qkv_bias, term,
                       static_cast<bf16 *>(out), height, width, channels, heads, wy_n, wx_n, shift,
                       items);
}

}  // namespace

extern "C" int bfhip_debug_window_attention(const void *qkv, const float *qkv_bias,
                                            const float *bias_mat, void *out, int batches,
                                            int height, int width, int channels, int heads,
                                            int shift, void *stream, char *error, size_t cap) {
    const int items = window_attention_items(qkv, qkv_bias, bias_mat, out, batches, height, width,
                                             channels, heads, shift, error, cap);
    if (!items) return 0;
    // The probe builds the score terms into its own buffer (test path only:
    // it allocates and synchronises).
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    bf16 *term = nullptr;
    if (!hip_ok(hipMalloc(&term, attn_term_elems(heads, shift) * 2), error, cap,
                "allocate probe attention terms"))
        return 0;
    window_attention_launch(qkv, qkv_bias, bias_mat, out, term, height, width, channels, heads,
                            shift, items, s);
    const int ok = launch_ok(error, cap, "launch window-attention probe") &&
                   hip_ok(hipStreamSynchronize(s), error, cap, "window-attention probe");
    (void)hipFree(term);
    return ok;
}

// ---- Window attention without allocation ---------------------------------
// The score terms of one call (window types x heads x 8 KiB of fp16) go to a
// file-scope device array instead of a per-call allocation: at most
// kScratchHeads heads, 4 x 32 x 8 KiB = 1 MiB on every device the library
// runs this entry point on, held until the process ends.  Every call on a
// device rebuilds the terms it reads before reading them (no state carries
// over between calls and nothing needs clearing), and all calls on a device
// share the array: calls that overlap in time on one device (different
// streams, or host threads) race on it.
namespace {
constexpr int kScratchHeads = 32;
constexpr size_t kScratchElems = (size_t)4 * kScratchHeads * 8 * 64 * 8;
static_assert(kScratchElems >= attn_term_elems(kScratchHeads, 1), "scratch covers the largest term");
}  // namespace

// The score terms are fp16 words; the attention kernel takes them through the
// library's 16-bit word pointer type (bf16 *), which carries either format.
static __device__ __align__(256) uint16_t scratch[kScratchElems];

namespace {
// This device's copy of `scratch`: the host-side name of the array is not a
// device address, so it is resolved with the device current, on every call (a
// host-side lookup that allocates nothing; nothing cached can go stale after a
// device reset or a reload of the code object), and only the resolved pointer
// is ever passed to a kernel.
bf16 *scratch_on(int device, char *error, size_t cap) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        fail(error, cap, "resolve the window-attention scratch array on HIP device %d: %s", device,
             e != hipSuccess ? hipGetErrorString(e) : "null address");
        return nullptr;
    }
    return static_cast<bf16 *>(p);  // fp16 words (see `scratch`)
}
}  // namespace

extern "C" int bfhip_debug_window_attention_noalloc(const void *qkv, const float *qkv_bias,
                                                    const float *bias_mat, void *out, int batches,
                                                    int height, int width, int channels, int heads,
                                                    int shift, void *stream, char *error,
                                                    size_t cap) {
    const int items = window_attention_items(qkv, qkv_bias, bias_mat, out, batches, height, width,
                                             channels, heads, shift, error, cap);
    if (!items) return 0;
    if (heads > kScratchHeads)
        return fail(error, cap,
                    "window attention without allocation supports at most %d heads (got %d)",
                    kScratchHeads, heads);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int device = -1, stream_device = -1;
    if (!hip_ok(hipGetDevice(&device), error, cap, "query the current HIP device") ||
        !hip_ok(hipStreamGetDevice(s, &stream_device), error, cap, "query the stream's device"))
        return 0;
    if (stream_device != device)
        return fail(error, cap, "stream belongs to HIP device %d, but device %d is current",
                    stream_device, device);
    bf16 *term = scratch_on(device, error, cap);
    if (!term) return 0;
    window_attention_launch(qkv, qkv_bias, bias_mat, out, term, height, width, channels, heads,
                            shift, items, s);
    return launch_ok(error, cap, "launch window attention without allocation");
}

// ---- Patch-merge gather probe (include/bfhip_debug.h) ----------------------
// The merge of stage `stage` on the caller's fp16 tokens xh [B, H, W, C] with
// identity reduction weights whose columns go through merge_tap_order (as the
// folded weights do at create) and a plain fp32 store: the output row m is
// then the reference's unfold row, out[m][c*4 + q] = xh[token q of m][c].
extern "C" int bfhip_debug_swin_merge_gather(bf_cuda_swin *s, int stage, const void *xh, float *out,
                                             void *stream, char *error, size_t cap) {
    if (!s || stage < 0 || stage > 2 || !xh || !out) return fail(error, cap, "invalid merge gather probe");
    if (((uintptr_t)xh & 15) || ((uintptr_t)out & 15))
        return fail(error, cap, "merge gather probe buffers must be 16-byte aligned");
    const int C = kC[stage], B = (int)s->batches, H = s->h[stage], W = s->w[stage];
    const int T2 = B * s->h[stage + 1] * s->w[stage + 1];
    const std::vector<int> perm = merge_tap_order(C);
    std::vector<uint16_t> wt((size_t)4 * C * 4 * C, 0);  // [4C outputs][4C columns]
    for (int kk = 0; kk < 4 * C; ++kk) wt[(size_t)perm[kk] * 4 * C + kk] = 0x3C00;  // fp16 1.0
    bf16 *w = nullptr;
    if (!hip_ok(hipMalloc(&w, wt.size() * 2), error, cap, "allocate merge probe weights")) return 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int ok = hip_ok(hipMemcpy(w, wt.data(), wt.size() * 2, hipMemcpyHostToDevice), error, cap,
                    "upload merge probe weights");
    if (ok) {
        const EpiRowsF32 epi{out, nullptr, 4 * C, T2, 4 * C, 0};
        const bf16 *x = static_cast<const bf16 *>(xh);
        // Same (C, tile, loader waves) per stage as merge_op; the reduction
        // runs over 4C outputs here instead of 2C.
        if (stage == 0)
            merge_gemm<96, MergeT0, 0>(x, B, H, W, w, 4 * C, epi, st);
        else if (stage == 1)
            merge_gemm<192, MergeT1, 0>(x, B, H, W, w, 4 * C, epi, st);
        else
            merge_gemm<384, MergeT2, kMergeLoaders2>(x, B, H, W, w, 4 * C, epi, st);
        ok = launch_ok(error, cap, "launch merge gather probe") &&
             hip_ok(hipStreamSynchronize(st), error, cap, "merge gather probe");
    }
    (void)hipFree(w);
    return ok;
}
