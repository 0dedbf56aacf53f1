// K7: the encoder layer's feed-forward block in one kernel
// (feedForward, arctic.zig:760-811):
//
//   Y = LayerNorm( X + ( GELU(X W1^T s1 + b1) W2^T s2 + b2 ) )
//
// for X [T, 384] f32, W1 int8 codes [1536, 384] with f16 scales s1, W2
// int8 codes [384, 1536] with scales s2 (matmul_w8a32.zig:40-55: sum of x q,
// times the row's scale, plus bias), the tanh-form GELU (arctic.zig:750-756)
// and a two-pass LayerNorm over each 384-wide row (layernorm.zig:26-117).
// The 1536-wide intermediate H never leaves the chip: the unfused pair writes
// and re-reads it as f32 (830 MB per layer at 67 590 tokens).
//
// Arithmetic is the reference's f32: activations are split into an exact
// f16 pair x = hi + lo + r (|r| <= 2^-22 |x| for 2^-3 <= |x| < 65504,
// split_f32x8), weight codes are exact in f16, and each product runs as
// hi q + lo q through v_mfma_f32_16x16x32_f16 into an f32 accumulator.
// The caller guarantees that X and H lie inside the split's range (the
// model checks it from the weights at upload; rows that need scaling run
// on the unfused GEMMs).
//
// Design (gfx950):
//   - One workgroup of four waves per CU, one wave per SIMD, so every wave
//     has the SIMD's whole register file (VGPRs and AGPRs).  Each wave owns
//     16 tokens from the first product to the stored LayerNorm row: their X
//     as f16 hi/lo halves in VGPRs (the MFMA B operand of the first GEMM),
//     the raw f32 X in AGPRs (the residual), the 16 x 384 output sums in
//     VGPRs, and the current chunk of H.  Nothing but the weights goes
//     through LDS, and no wave waits for another except at the stage
//     barrier of the weight ring.
//   - The weights are widened once, at upload, to f16 in the order the
//     MFMA reads them (mlp_pack_kernel): 1 KiB fragments in which lane l's
//     16 bytes are its eight A-operand values, so every fragment read is one
//     conflict-free ds_read_b128.  Widening int8 codes in registers costs
//     eight VALU ops per fragment; measured with two MFMAs per fragment, that
//     halved the matrix-core rate (1.0 against 1.7 PFLOP/s).
//   - The intermediate runs in 24 chunks of 64 features; each chunk is four
//     24 KiB stages of the ring (W1 rows of the chunk over k 0..191 and
//     192..383, then W2 columns of the chunk for outputs 0..191 and
//     192..383), streamed HBM/L2 -> LDS by the direct-to-LDS loads, three
//     stages ahead.  The stage stream is the same for every 64-token panel.
//   - The H chunk needs no transpose: the first GEMM's result tile (token
//     lane % 16, features 4 (lane / 16) + e) is the second GEMM's B operand
//     for a k order in which MFMA slot 8 g + i holds feature 4 g + i (i < 4)
//     or 16 + 4 g + i - 4 (i >= 4) of a 32-feature step; the packed W2
//     fragments follow that k order.  W2's rows are packed so that the
//     output tile pair (2 j, 2 j + 1) leaves lane (t, g) with outputs 32 j +
//     8 g .. 32 j + 8 g + 7 of token t: the same columns as the lane's X
//     registers, so the residual add is lane-local and each LayerNorm row's
//     statistics reduce over the four lanes of its token with two row swaps.
//   - Two more modes share the ring and the first GEMM: the O-projection
//     mode runs the attention output's projection, residual and LayerNorm
//     (arctic.zig:716-746) at the head of each panel, so the layer's h1 is
//     formed in registers; the QKV mode runs the attention's input
//     projection (the first GEMM alone over W_qkv, each 64-column chunk
//     stored from its accumulators).
//   - Blocks deal the panels round robin; the last, partial round is split
//     by chunks over the CUs it would leave idle (TailSplit): a part sums
//     its chunks only, and mlp_tail_kernel adds the parts (in the QKV mode
//     the parts write disjoint columns, with nothing to add).
#include <algorithm>

#include "pipe.h"

namespace {

constexpr int kD = 384;                      // hidden size
constexpr int kF = 1536;                     // intermediate size
constexpr int kFC = 64;                      // intermediate features per chunk
constexpr int kChunks = kF / kFC;            // 24
constexpr int kWaves = 4;                    // one per SIMD
constexpr int kTokW = 16;                    // tokens per wave
constexpr int kBM = kWaves * kTokW;          // tokens per panel
constexpr int kFrag = 1024;                  // bytes of one A fragment (64 lanes x 8 f16)
constexpr int kStageFrags = 24;
constexpr int kStage = kStageFrags * kFrag;  // 24 KiB
constexpr int kSPC = 4;                      // stages per chunk
constexpr int kSPP = kChunks * kSPC;         // stages per panel
constexpr int kLW = kStageFrags / kWaves;    // direct-to-LDS loads per wave per stage
constexpr int kXJ = kD / 32;                 // 32-wide k steps of the first GEMM
constexpr int kYT = kD / 16;                 // 16-row output tiles of the second GEMM
constexpr int kXL = 2 * kXJ;                 // 16-byte X loads per lane per panel
constexpr size_t kPackHalves = (size_t)kChunks * kSPC * kStageFrags * (kFrag / 2);
static_assert(kStageFrags % kWaves == 0, "a stage splits evenly over the waves");
static_assert(kPackHalves * 2 == (size_t)2 * kD * kF * 2, "the pack holds both weight matrices as f16");

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// The packed f16 layout (halves): stage (c, q) at ((c * 4 + q) * 24 + f) *
// 512 + lane * 8 + i for fragment f, lane l = 16 g + rho:
//   q = 0, 1 (first GEMM, k steps j = 6 q + f / 4, feature tile ft = f % 4):
//       W1[64 c + 16 ft + rho][32 j + 8 g + i]
//   q = 2, 3 (second GEMM, output tile ot = 12 (q - 2) + f / 2, k step
//       jj = f % 2): W2[w2_row(ot, rho)][64 c + 32 jj + w2_k(g, i)]
__host__ __device__ constexpr int w2_row(int ot, int rho) {
    return 32 * (ot / 2) + 8 * (rho / 4) + 4 * (ot % 2) + rho % 4;
}
__host__ __device__ constexpr int w2_k(int g, int i) { return i < 4 ? 4 * g + i : 16 + 4 * g + i - 4; }

// W8T codes (biased u = q + 128, stage-tiled in 384-row blocks; see
// tile_codes_w8_kernel) -> q as f16, exactly.
__device__ __forceinline__ _Float16 w8t_code(const uint8_t *w, int k_pad, int n, int k) {
    const size_t o = (((size_t)(n / 384) * (k_pad / 64) + k / 64) * 384 + n % 384) * 64 + k % 64;
    return (_Float16)((int)w[o] - 128);
}

// One thread per (stage, fragment, lane): eight f16 values.
__global__ void mlp_pack_kernel(const uint8_t *__restrict__ w1, const uint8_t *__restrict__ w2,
                                _Float16 *__restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= kChunks * kSPC * kStageFrags * 64) return;
    const int lane = idx % 64, f = idx / 64 % kStageFrags, q = idx / (64 * kStageFrags) % kSPC;
    const int c = idx / (64 * kStageFrags * kSPC);
    const int rho = lane % 16, g = lane / 16;
    half8_t v;
    if (q < 2) {
        const int j = 6 * q + f / 4, ft = f % 4;
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = w8t_code(w1, kD, kFC * c + 16 * ft + rho, 32 * j + 8 * g + i);
    } else {
        const int ot = 12 * (q - 2) + f / 2, jj = f % 2;
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = w8t_code(w2, kF, w2_row(ot, rho), kFC * c + 32 * jj + w2_k(g, i));
    }
    *(half8_t *)(out + (size_t)idx * 8) = v;
}

// The O-projection's codes (W_o [384, 384] in W8T) -> its 12 stages, one per
// 32-wide k step s, fragment f = output tile ot (rows ordered as W2's, so
// that its sums land in the lanes of X's columns): lane l = 16 g + rho,
// value i = W_o[w2_row(ot, rho)][32 s + 8 g + i].
constexpr int kOStages = kD / 32;
__global__ void mlp_opack_kernel(const uint8_t *__restrict__ wo, _Float16 *__restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= kOStages * kStageFrags * 64) return;
    const int lane = idx % 64, ot = idx / 64 % kStageFrags, st = idx / (64 * kStageFrags);
    const int rho = lane % 16, g = lane / 16;
    half8_t v;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = w8t_code(wo, kD, w2_row(ot, rho), 32 * st + 8 * g + i);
    *(half8_t *)(out + (size_t)idx * 8) = v;
}

// The attention's input projection (QKV mode): W_qkv [1152, 384] in 18
// chunks of 64 rows, two stages each (k 0..191, 192..383), in the first
// GEMM's fragment layout: stage 2 c + q, fragment f (k step jp = f / 4,
// row tile ft = f % 4), lane l = 16 g + rho, value i =
// W_qkv[64 c + 16 ft + rho][32 (6 q + jp) + 8 g + i].
constexpr int kFQ = 3 * kD;          // 1152 outputs
constexpr int kQChunks = kFQ / kFC;  // 18
__global__ void qkv_pack_kernel(const uint8_t *__restrict__ w, _Float16 *__restrict__ out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 2 * kQChunks * kStageFrags * 64) return;
    const int lane = idx % 64, f = idx / 64 % kStageFrags, sq = idx / (64 * kStageFrags);
    const int c = sq / 2, q = sq % 2, rho = lane % 16, g = lane / 16;
    const int j = 6 * q + f / 4, ft = f % 4;
    half8_t v;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = w8t_code(w, kD, kFC * c + 16 * ft + rho, 32 * j + 8 * g + i);
    *(half8_t *)(out + (size_t)idx * 8) = v;
}

// A value parked in an accumulation register (AGPR) until it is read back:
// the raw X of a wave's tokens (its residual) stays there through the panel,
// outside the VGPRs the products use.
#ifdef TZH_EMULATION
__device__ __forceinline__ float park(float v) { return v; }
__device__ __forceinline__ float unpark(float a) { return a; }
#else
__device__ __forceinline__ float park(float v) {
    float a;
    asm("v_accvgpr_write_b32 %0, %1" : "=a"(a) : "v"(v));
    return a;
}
__device__ __forceinline__ float unpark(float a) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
}
#endif

// s_waitcnt vmcnt(n) lgkmcnt(0) for the counts the feed-forward modes' ring
// can need (n = 6 a + 24 b, a <= 2, b <= 2); any other n waits for
// everything.
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
    case 60: wait_vm_lgkm0<60>(); break;
    case 54: wait_vm_lgkm0<54>(); break;
    case 48: wait_vm_lgkm0<48>(); break;
    case 36: wait_vm_lgkm0<36>(); break;
    case 30: wait_vm_lgkm0<30>(); break;
    case 24: wait_vm_lgkm0<24>(); break;
    case 12: wait_vm_lgkm0<12>(); break;
    case 6: wait_vm_lgkm0<6>(); break;
    default: wait_vm_lgkm0<0>(); break;
    }
}

// The QKV mode's counts (two stages' loads, stores in fours, X loads in
// 24s): s_waitcnt vmcnt(n') lgkmcnt(0) for n' = n rounded down to a
// multiple of 4 (at most 60), which waits for at most three more ops than
// needed; a four-level tree of uniform branches.
__device__ __forceinline__ void wait_vm_n4(int n) {
    const int k = (n > 63 ? 63 : n) >> 2;  // 0 .. 15
    if (k & 8) {
        if (k & 4) {
            if (k & 2) {
                if (k & 1) wait_vm_lgkm0<60>(); else wait_vm_lgkm0<56>();
            } else {
                if (k & 1) wait_vm_lgkm0<52>(); else wait_vm_lgkm0<48>();
            }
        } else {
            if (k & 2) {
                if (k & 1) wait_vm_lgkm0<44>(); else wait_vm_lgkm0<40>();
            } else {
                if (k & 1) wait_vm_lgkm0<36>(); else wait_vm_lgkm0<32>();
            }
        }
    } else {
        if (k & 4) {
            if (k & 2) {
                if (k & 1) wait_vm_lgkm0<28>(); else wait_vm_lgkm0<24>();
            } else {
                if (k & 1) wait_vm_lgkm0<20>(); else wait_vm_lgkm0<16>();
            }
        } else {
            if (k & 2) {
                if (k & 1) wait_vm_lgkm0<12>(); else wait_vm_lgkm0<8>();
            } else {
                if (k & 1) wait_vm_lgkm0<4>(); else wait_vm_lgkm0<0>();
            }
        }
    }
}

// Where one wave's loads of a ring stage go (its kLW fragments of the
// stage).  ALWAYS: the stage exists; otherwise src null means no stage.
template <bool ALWAYS>
struct StageDma {
    static constexpr bool kAlways = ALWAYS;
    const char *src;
    char *dst;
};

// The attention output's side of an encoder layer, for the O-projection
// mode of mlp_fused_kernel: the attention context, the layer's input (the
// first LayerNorm's residual), W_o's stages (mlp_opack_kernel), its scales
// and bias, and the first LayerNorm's gamma and beta.
struct OProj {
    const float *ctx, *res;
    const _Float16 *wp;
    const uint16_t *s;
    const float *b, *gamma, *beta;
};

// The last, partial round of panels split by intermediate chunks over the
// CUs the round would leave idle.  Panels 0 .. full - 1 run whole, dealt
// round robin over the blocks; with parts > 1, each later panel runs as
// `parts` parts of kChunks / parts chunks each (block b: panel full + b /
// parts, part b % parts).  A part stores its raw output sums (codes times
// H, before scale and bias) to sums[(tp parts + part) 64 + token][384]
// (tp = panel - full); in the O-projection mode part 0 also stores X (the
// feed-forward's residual, formed on chip) to xs[tp 64 + token][384].
// mlp_tail_kernel adds the parts and finishes the rows.
struct TailSplit {
    int full, parts;
    float *sums, *xs;
};

// MODE 0: the feed-forward block.  MODE 1 (OP), the O-projection mode:
// each panel first forms X = LayerNorm(res + (ctx W_o^T s_o + b_o))
// (arctic.zig:716-746) in registers, from 12 more weight stages (W_o's,
// streamed ahead of the feed-forward's) and the first LayerNorm in the
// lanes, then runs the feed-forward block on it.  MODE 2 (QKV): the first
// GEMM alone over W_qkv (qkv_pack_kernel), Y [T, 1152] = X W_qkv^T s1 + b1
// (arctic.zig:639-650, matmul_w8a32.zig:40-55), each 64-column chunk
// stored from the accumulators.
template <int MODE>
__global__ void __launch_bounds__((MODE == 2 ? 2 : 1) * kWaves * 64) mlp_fused_kernel(
    const float *__restrict__ X, const _Float16 *__restrict__ Wp, const uint16_t *__restrict__ s1,
    const float *__restrict__ b1, const uint16_t *__restrict__ s2, const float *__restrict__ b2,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps, float *__restrict__ Y, int T,
    OProj op, TailSplit ts) {
    constexpr bool OP = MODE == 1, QKV = MODE == 2;
    // waves of a block: the QKV mode, at about 290 registers a wave, runs
    // two waves per SIMD on 128-token panels (the same weight stream feeds
    // twice the tokens, and each SIMD has a second wave to issue MFMAs
    // while one waits); its loads per wave per stage halve
    constexpr int kWv = QKV ? 2 * kWaves : kWaves;
    constexpr int kLWv = kStageFrags / kWv;
    constexpr int kBMv = kWv * kTokW;
    constexpr int kO = OP ? kOStages : 0;           // O-projection stages at the head of each panel
    constexpr int kSP = QKV ? 2 * kQChunks : kO + kSPP;  // stages per panel
    constexpr int kNC = QKV ? kQChunks : kChunks;   // chunks per panel
    static_assert(kSP % 4 == 0, "a panel's stages fill whole turns of the ring");
    __shared__ __attribute__((aligned(16))) char st[4][kStage];  // the weight ring
    __shared__ __attribute__((aligned(16))) float p1[2][kF];  // s1, b1
    __shared__ __attribute__((aligned(16))) float p2[4][kD];  // s2, b2, gamma, beta
    __shared__ __attribute__((aligned(16))) float p0[OP ? 4 : 1][OP ? kD : 4];  // s_o, b_o, LayerNorm 1

    // (lane quantities are formed where they are used, from lane_now())
    const int tid = threadIdx.x;
    const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int panels = (T + kBMv - 1) / kBMv;
    const int count = (int)blockIdx.x < ts.full ? (ts.full - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    // this block's part of a split panel, if any: chunks c0 .. c0 + nc - 1
    const bool tail = ts.parts > 1 && (int)blockIdx.x < (panels - ts.full) * ts.parts;
    const int tpanel = ts.full + (int)blockIdx.x / ts.parts, tpart = (int)blockIdx.x % ts.parts;
    const int nc = kNC / ts.parts, c0 = tpart * nc;
    const int SF = count * kSP;  // stages of the whole panels
    const int S = SF + (tail ? (QKV ? 2 * nc : kO + kSPC * nc) : 0);  // stages this block streams
    if (S == 0) return;

    // per-feature parameters -> LDS (visible after the first stage barrier)
    for (int i = tid; i < (QKV ? kFQ : kF); i += kWv * 64) {
        p1[0][i] = f16_bits_to_f32(s1[i]);
        p1[1][i] = b1[i];
    }
    for (int i = tid; i < (QKV ? 0 : kD); i += kWv * 64) {
        p2[0][i] = f16_bits_to_f32(s2[i]);
        p2[1][i] = b2[i];
        p2[2][i] = gamma[i];
        p2[3][i] = beta[i];
        if constexpr (OP) {
            p0[0][i] = f16_bits_to_f32(op.s[i]);
            p0[1][i] = op.b[i];
            p0[2][i] = op.gamma[i];
            p0[3][i] = op.beta[i];
        }
    }

    // The stage stream of a panel, skewed by one chunk so that the GELU of
    // chunk p runs between the products of the second GEMM of chunk p - 1
    // (the matrix cores would otherwise idle through it, with one wave per
    // SIMD):
    //   s = 0, 1:            W1 of chunk 0 (k 0..191, 192..383)
    //   s = 4p - 2, 4p - 1:  W1 of chunk p          (p = 1 .. 23)
    //   s = 4p, 4p + 1:      W2 of chunk p - 1      (outputs 0..191, 192..383)
    //   s = 94, 95:          W2 of chunk 23
    // (after the O-projection's kO stages in the O-projection mode; a part
    // of a split panel streams the same for its chunks c0 .. c0 + n - 1).
    // Stage u of the block sits in ring slot u % 4; pack_stage gives the
    // pack's stage (4 c + q) at feed-forward stream position s.
    auto pack_stage = [](int s, int cb, int n) __attribute__((always_inline)) {
        // (selects, not branches: one wave per SIMD has nothing to hide a
        // branch behind)
        const int p = cb + ((s + 2) >> 2), r = (s + 2) & 3, last = kSPC * n - 2;
        int v = r < 2 ? 4 * p + r : 4 * (p - 1) + r;
        v = s < 2 ? 4 * cb + s : v;
        return s >= last ? 4 * (cb + n - 1) + 2 + (s - last) : v;
    };
    char *const ring = &st[0][0];
    const char *const wsrc = (const char *)Wp + (size_t)wu * kLWv * kFrag;
    const char *const osrc = OP ? (const char *)op.wp + (size_t)wu * kLWv * kFrag : nullptr;
    // stage u's loads; WHOLE: u is a feed-forward stage of a whole panel
    auto dma_of = [&](int u, auto wholec) __attribute__((always_inline)) {
        const char *src;
        if constexpr (QKV) {
            // (QKV mode: the pack's stages in order, a part's from 2 c0)
            src = wsrc + (size_t)(decltype(wholec)::value ? u % kSP : (u >= SF ? 2 * c0 + u - SF : u % kSP)) * kStage;
        } else if constexpr (decltype(wholec)::value) {
            src = wsrc + (size_t)pack_stage(u % kSP - kO, 0, kChunks) * kStage;
        } else {
            const bool tl = u >= SF;
            const int sp = tl ? u - SF : u % kSP;
            src = OP && sp < kO ? osrc + (size_t)sp * kStage
                                : wsrc + (size_t)pack_stage(sp - kO, tl ? c0 : 0, tl ? nc : kChunks) * kStage;
        }
        return StageDma<true>{src, ring + (u & 3) * kStage + wu * kLWv * kFrag};
    };
    auto dma_one = [&](const auto &d, int i) __attribute__((always_inline)) {
        if (i < kLWv && (std::decay_t<decltype(d)>::kAlways || d.src))
            dma16(d.src + i * kFrag, (uint32_t)lane_now() * 16, d.dst + i * kFrag);
    };

    // Rows of the wave's tokens in the B-operand layout: lane (tl, g), k
    // step j: src[t][32 j + 8 g .. 32 j + 8 g + 7] (rows past T clamped to
    // T - 1).  load_x: the activation a panel starts from (X, or the
    // attention context in the O-projection mode).
    f32x4_t xn[kXL];
    auto load_rows = [&](const float *src, int panel) __attribute__((always_inline)) {
        const int ln = lane_now();
        int t = panel * kBMv + wu * kTokW + (ln & 15);
        t = t < T ? t : T - 1;
        const float *row = src + (size_t)t * kD + 8 * (ln >> 4);
#pragma unroll
        for (int j = 0; j < kXJ; j++) {
            xn[2 * j] = *(const f32x4_t *)(row + 32 * j);
            vmem_load_issued();
            xn[2 * j + 1] = *(const f32x4_t *)(row + 32 * j + 4);
            vmem_load_issued();
        }
    };
    auto load_x = [&](int panel) __attribute__((always_inline)) { load_rows(OP ? op.ctx : X, panel); };
    half8_t xh[kXJ], xl[kXJ];
    float xr[kXJ * 8];  // parked raw X: xr[8 j + i] = X[t][32 j + 8 g + i]
    // xn -> the f16 halves xh, xl; PARK: xn is the feed-forward's X, kept as
    // its residual (the attention context of the O-projection mode is not)
    auto split_x = [&](auto parkc) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kXJ; j++) {
            split_f32x8(xn[2 * j], xn[2 * j + 1], xh[j], xl[j]);
            if constexpr (decltype(parkc)::value)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    xr[8 * j + i] = park(xn[2 * j][i]);
                    xr[8 * j + 4 + i] = park(xn[2 * j + 1][i]);
                }
        }
    };

    f32x4_t yacc[kYT];  // lane (tl, g), tile ot: outputs w2_row(ot, 4 g + e)
    f32x4_t hacc[4];    // lane (tl, g), tile ft: features 64 c + 16 ft + 4 g + e
    // H of chunks p (being formed) and p - 1 (being multiplied) as the
    // second GEMM's B operand: hbh/hbl[p % 2][jj], k step jj = tiles 2 jj,
    // 2 jj + 1
    half8_t hbh[2][2], hbl[2][2];

    // Ops this wave issued after stage u's loads when step u waits for them:
    // the loads of stages u + 1 and u + 2 and the extra X loads and stores
    // issued after stage u's loads, by the step that issued them (ext0: the
    // step before this one, ext1, ext2: the two before it).  Step kinds:
    // MID (the steps away from a panel's ends): two stages' loads, and stage
    // u + 3 exists; GEN: the count computed at run time, stage u + 3 exists
    // (a panel's first steps); END: both at run time (its last steps).
    int ext0 = 0, ext1 = 0, ext2 = 0;
    // QKV mode: of those, the ops each step issued after its last stage load
    // (its stores go out between its loads; those before the last load of
    // stage u do not count for u's wait)
    int pst0 = 0, pst1 = 0, pst2 = 0;
    auto step_begin = [&](auto kindc, int u) __attribute__((always_inline)) {
        constexpr int K = decltype(kindc)::value;
        if constexpr (K == 0) {
            wait_vm_lgkm0<2 * kLWv>();
            lds_barrier_only();  // every wave's stage u landed; stage u - 1 fully read
            return dma_of(u + 3, std::true_type{});  // (the middle steps load their own panel's stages)
        } else {
            const int ahead = K == 1 || S - 1 - u >= 2 ? 2 : S - 1 - u;
            if constexpr (QKV)
                wait_vm_n4(kLWv * ahead + ext0 + ext1 + pst2);
            else
                wait_vm_n(kLWv * ahead + ext0 + ext1 + ext2);
            lds_barrier_only();
            ext2 = ext1;
            ext1 = ext0;
            ext0 = 0;
            pst2 = pst1;
            pst1 = pst0;
            pst0 = 0;
            if constexpr (K == 1) {
                return dma_of(u + 3, std::false_type{});
            } else {
                if (u + 3 >= S) return StageDma<false>{nullptr, nullptr};
                const StageDma<true> d = dma_of(u + 3, std::false_type{});
                return StageDma<false>{d.src, d.dst};
            }
        }
    };

    // QKV mode, a middle step: every step stores two of the last chunk's
    // four vectors, after its third and sixth groups' loads, so its wait
    // counts two stages' loads, the stores after stage u's last load (one
    // with six loads a step, both with three) and the two stores of each
    // of the two steps since: 17 with four waves, 12 with eight.  The records
    // of extra ops move on as in the counted steps, for the panel's last
    // steps.
    auto step_mid_q = [&](int u) __attribute__((always_inline)) {
        wait_vm_lgkm0<2 * kLWv + (kLWv == 3 ? 2 : 1) + 4>();
        lds_barrier_only();
        ext2 = ext1;
        ext1 = ext0;
        ext0 = 0;
        pst2 = pst1;
        pst1 = pst0;
        pst0 = 0;
        return dma_of(u + 3, std::true_type{});
    };

    // The lane's byte offset in a fragment, recomputed in each stage (an
    // opaque copy): the compiler otherwise keeps every fragment address of
    // every stage in its own VGPR for the whole kernel.
    auto lane_off = [&]() __attribute__((always_inline)) { return lane_now() * 16; };
    // first GEMM, half q of the chunk's k: H^T tiles += W1 fragments x X.
    // The fragments of k step jp + 1 are read before the products of step
    // jp are issued (two register sets), so the LDS latency hides behind
    // eight MFMAs; one of the six loads of stage u + 3 goes out per k step,
    // then hook(jp) (the QKV mode's stores).
    auto gemm1 = [&](auto qc, const char *sb, const auto &d, auto hook) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value;
        constexpr int j0 = 6 * q;
        sb += lane_off();
        if constexpr (q == 0)
#pragma unroll
            for (int ft = 0; ft < 4; ft++) hacc[ft] = f32x4_t{};
        half8_t a[2][4];
#pragma unroll
        for (int ft = 0; ft < 4; ft++) a[0][ft] = *(const half8_t *)(sb + ft * kFrag);
#pragma unroll
        for (int jp = 0; jp < 6; jp++) {
            if (jp + 1 < 6)
#pragma unroll
                for (int ft = 0; ft < 4; ft++)
                    a[(jp + 1) & 1][ft] = *(const half8_t *)(sb + ((jp + 1) * 4 + ft) * kFrag);
            dma_one(d, jp);
            hook(jp);
            sched_fence();
#pragma unroll
            for (int ft = 0; ft < 4; ft++)
                hacc[ft] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[jp & 1][ft], xh[j0 + jp], hacc[ft], 0, 0, 0);
#pragma unroll
            for (int ft = 0; ft < 4; ft++)
                hacc[ft] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[jp & 1][ft], xl[j0 + jp], hacc[ft], 0, 0, 0);
        }
    };
    // H = GELU(sum * s1 + b1) (matmul_w8a32.zig:55, arctic.zig:774-776) of
    // tile ft of chunk c
    auto gelu_tile = [&](int c, int ft) __attribute__((always_inline)) {
        const int f = kFC * c + 16 * ft + 4 * (lane_now() >> 4);
        const f32x4_t s = *(const f32x4_t *)&p1[0][f];
        const f32x4_t b = *(const f32x4_t *)&p1[1][f];
        f32x4_t v;
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = gelu_fast(hacc[ft][e] * s[e] + b[e]);
        return v;
    };
    // second GEMM, output tiles 12 (q - 2) .. + 11 of the chunk whose H is in
    // buffer HB: Y^T tiles += W2 fragments x H, in six half-groups hg (tiles
    // 4 (hg / 2) .. + 3 at k step hg % 2): each tile's two dependent products
    // of a half-group have three other tiles' between them, the next
    // half-group's fragments are read before this one's products are issued,
    // and one load of stage u + 3 goes out per half-group.  gc >= 0:
    // meanwhile k step q - 2 of chunk gc's GELU, into buffer HB ^ 1.
    auto gemm2 = [&](auto qc, auto hbc, const char *sb, const auto &d, int gc) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value, o0 = 12 * (q - 2), jg = q - 2;
        constexpr int HB = decltype(hbc)::value;
        sb += lane_off();
        half8_t a[2][4];
        f32x4_t gv[2];
        auto read = [&](int buf, int hg) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < 4; t++)
                a[buf][t] = *(const half8_t *)(sb + ((4 * (hg >> 1) + t) * 2 + (hg & 1)) * kFrag);
        };
        read(0, 0);
#pragma unroll
        for (int hg = 0; hg < 6; hg++) {
            if (hg + 1 < 6) read((hg + 1) & 1, hg + 1);
            dma_one(d, hg);
            sched_fence();
            const int jj = hg & 1, o = o0 + 4 * (hg >> 1);
#pragma unroll
            for (int t = 0; t < 4; t++)
                yacc[o + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[hg & 1][t], hbh[HB][jj], yacc[o + t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; t++)
                yacc[o + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[hg & 1][t], hbl[HB][jj], yacc[o + t], 0, 0, 0);
            if (gc >= 0) {
                if (hg == 1) gv[0] = gelu_tile(gc, 2 * jg);
                if (hg == 3) gv[1] = gelu_tile(gc, 2 * jg + 1);
                if (hg == 5) split_f32x8(gv[0], gv[1], hbh[HB ^ 1][jg], hbl[HB ^ 1][jg]);
            }
        }
    };

    // O-projection mode, k step j of W_o (the panel's stage j): Y^T tiles of
    // the 384 outputs += W_o fragments x ctx, in six groups of four tiles
    // (hi then lo products, so each tile's two have three others between
    // them), the next group's fragments read before this group's products,
    // one load of stage u + 3 per group
    auto gemm_o = [&](int j, const char *sb, const auto &d) __attribute__((always_inline)) {
        sb += lane_off();
        half8_t a[2][4];
        auto read = [&](int buf, int og) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < 4; t++) a[buf][t] = *(const half8_t *)(sb + (4 * og + t) * kFrag);
        };
        read(0, 0);
#pragma unroll
        for (int og = 0; og < 6; og++) {
            if (og + 1 < 6) read((og + 1) & 1, og + 1);
            dma_one(d, og);
            sched_fence();
#pragma unroll
            for (int t = 0; t < 4; t++)
                yacc[4 * og + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[og & 1][t], xh[j], yacc[4 * og + t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; t++)
                yacc[4 * og + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[og & 1][t], xl[j], yacc[4 * og + t], 0, 0, 0);
        }
    };
    // O-projection mode: X = LayerNorm(res + (sum * s_o + b_o)) (arctic.zig:
    // 716-746, the two-pass LayerNorm of layernorm.zig:26-117) into xn, from
    // the sums in yacc and res in xn; the pre-norm row replaces the sums
    auto layernorm1 = [&]() __attribute__((always_inline)) {
        const int g = lane_now() >> 4;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < kXJ; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int n = 32 * j + 8 * g + 4 * h;
                const f32x4_t s = *(const f32x4_t *)&p0[0][n];
                const f32x4_t b = *(const f32x4_t *)&p0[1][n];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // input + (sum * s + bias)  (arctic.zig:720)
                    const float v = xn[2 * j + h][e] + (yacc[2 * j + h][e] * s[e] + b[e]);
                    yacc[2 * j + h][e] = v;
                    sum += v;
                }
            }
        const float mean = sum_over_rows(sum) / (float)kD;
        float sq = 0.0f;
#pragma unroll
        for (int o = 0; o < kYT; o++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float d = yacc[o][e] - mean;
                sq += d * d;
            }
        const float inv_std = 1.0f / sqrtf(sum_over_rows(sq) / (float)kD + eps);
#pragma unroll
        for (int j = 0; j < kXJ; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int n = 32 * j + 8 * g + 4 * h;
                const f32x4_t gg = *(const f32x4_t *)&p0[2][n];
                const f32x4_t bt = *(const f32x4_t *)&p0[3][n];
#pragma unroll
                for (int e = 0; e < 4; e++) xn[2 * j + h][e] = ((yacc[2 * j + h][e] - mean) * inv_std) * gg[e] + bt[e];
            }
    };

    // residual + bias, LayerNorm (arctic.zig:780-783, layernorm.zig:26-117),
    // store; returns whether every token of the wave was stored (then all 24
    // store instructions were issued with every lane on).  The pre-norm row
    // replaces the sums in place.
    auto epilogue = [&](int panel) __attribute__((always_inline)) {
        const int ln = lane_now(), g = ln >> 4;
        const int t = panel * kBMv + wu * kTokW + (ln & 15);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < kXJ; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int n = 32 * j + 8 * g + 4 * h;
                const f32x4_t s = *(const f32x4_t *)&p2[0][n];
                const f32x4_t b = *(const f32x4_t *)&p2[1][n];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // input + (sum * s + bias)  (arctic.zig:780-781)
                    const float v = unpark(xr[8 * j + 4 * h + e]) + (yacc[2 * j + h][e] * s[e] + b[e]);
                    yacc[2 * j + h][e] = v;
                    sum += v;
                }
            }
        const float mean = sum_over_rows(sum) / (float)kD;
        float sq = 0.0f;
#pragma unroll
        for (int o = 0; o < kYT; o++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float d = yacc[o][e] - mean;
                sq += d * d;
            }
        const float inv_std = 1.0f / sqrtf(sum_over_rows(sq) / (float)kD + eps);
        const bool full = panel * kBMv + wu * kTokW + kTokW <= T;  // uniform
#pragma unroll
        for (int j = 0; j < kXJ; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int n = 32 * j + 8 * g + 4 * h;
                const f32x4_t gg = *(const f32x4_t *)&p2[2][n];
                const f32x4_t bt = *(const f32x4_t *)&p2[3][n];
                f32x4_t y;
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = ((yacc[2 * j + h][e] - mean) * inv_std) * gg[e] + bt[e];
                if (t < T) {
                    *(f32x4_t *)(Y + (size_t)t * kD + n) = y;
                    vmem_store_issued();
                }
            }
        return full;
    };

    // QKV mode: a chunk's outputs, sum * s + b (matmul_w8a32.zig:55), wait
    // in registers (vq: lane (tl, g), vector k = columns 16 k + 4 g .. + 3
    // of token tl of chunk pend_c of panel pend_panel) and go out one at a
    // time during the next chunk's steps, so that the stores trickle
    // between the matrix products instead of stalling the wave in a burst.
    // Rows past T are clamped to T - 1: those lanes hold row T - 1's own
    // values (the same X row, the same products), so every store goes out.
    f32x4_t vq[4];
    bool pend = false;
    int pend_panel = 0, pend_c = 0;
    auto qkv_finish = [&](int c, int panel) __attribute__((always_inline)) {
        const int g = lane_now() >> 4;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int f = kFC * c + 16 * k + 4 * g;
            const f32x4_t sc = *(const f32x4_t *)&p1[0][f];
            const f32x4_t bs = *(const f32x4_t *)&p1[1][f];
#pragma unroll
            for (int e = 0; e < 4; e++) vq[k][e] = hacc[k][e] * sc[e] + bs[e];
        }
        pend = true;
        pend_panel = panel;
        pend_c = c;
    };
    // store vector k of the pending chunk; POST: after the step's last load
    auto qkv_put = [&](int k, bool post) __attribute__((always_inline)) {
        if (!pend) return;
        const int ln = lane_now();
        int t = pend_panel * kBMv + wu * kTokW + (ln & 15);
        t = t < T ? t : T - 1;
        *(f32x4_t *)(Y + (size_t)t * kFQ + kFC * pend_c + 16 * k + 4 * (ln >> 4)) = vq[k];
        vmem_store_issued();
        ext0 += 1;
        if (post) pst0 += 1;
    };
    // QKV mode, chunk c of a panel (stages u, u + 1): the first GEMM's two
    // halves, storing the last chunk's vectors 0, 1 during the first and 2,
    // 3 during the second (after loads 3 and 6 of each), then this chunk's
    // outputs.  KIND as for the periods; with nextp >= 0 the next panel's X
    // loads go out in the second step (counted with the first).
    auto qkv_chunk = [&](auto kindc, int u, int c, int panel, int nextp) __attribute__((always_inline)) {
        auto hook_a = [&](int jp) __attribute__((always_inline)) {
            if (jp == 2) qkv_put(0, 2 >= kLWv - 1);
            if (jp == 5) qkv_put(1, true);
        };
        auto hook_b = [&](int jp) __attribute__((always_inline)) {
            if (jp == 2) qkv_put(2, 2 >= kLWv - 1);
            if (jp == 5) qkv_put(3, true);
        };
        if constexpr (decltype(kindc)::value == 0) {
            auto d = step_mid_q(u);
            gemm1(std::integral_constant<int, 0>{}, ring + (u & 3) * kStage, d, hook_a);
            d = step_mid_q(u + 1);
            gemm1(std::integral_constant<int, 1>{}, ring + ((u + 1) & 3) * kStage, d, hook_b);
        } else {
            auto d = step_begin(kindc, u);
            gemm1(std::integral_constant<int, 0>{}, ring + (u & 3) * kStage, d, hook_a);
            d = step_begin(kindc, u + 1);
            if (nextp >= 0) {
                load_x(nextp);
                ext1 += kXL;
                pst1 += kXL;
            }
            gemm1(std::integral_constant<int, 1>{}, ring + ((u + 1) & 3) * kStage, d, hook_b);
        }
        qkv_finish(c, panel);
    };

    // Period p of panel i (p = 0 .. 24; block stages from u0): the first
    // GEMM of chunk p (p <= 23; two stages), then the second GEMM of chunk
    // p - 1 (p >= 1; two stages) with chunk p's GELU between its products.
    // PK 0: p = 0 (its GELU alone), 1: 1 <= p <= 23, 2: p = 24.  KIND: the
    // step kind of its stages (GEN, END next to a panel's ends, else MID).
    // PAR: chunk p's H goes to buffer PAR, chunk p - 1's is in PAR ^ 1 (p &
    // 1, or p - c0 for a part).  At p = 23 the loads of panel nextp's X
    // (if nextp >= 0) go out once this panel's first GEMM is done, before
    // the loads of the stage after next (counted with the step before, after
    // whose stage loads they are issued).
    auto period = [&](auto pkc, auto kindc, auto parc, int u0, int p, int nextp) __attribute__((always_inline)) {
        constexpr int PK = decltype(pkc)::value, PAR = decltype(parc)::value;
        constexpr int S1 = PK == 0 ? 0 : 2;  // ring slots of this period's first two stages
        if constexpr (PK <= 1) {
            auto d = step_begin(kindc, u0);
            gemm1(std::integral_constant<int, 0>{}, st[S1], d, [](int) {});
            d = step_begin(kindc, u0 + 1);
            gemm1(std::integral_constant<int, 1>{}, st[S1 + 1], d, [](int) {});
        }
        if constexpr (PK == 0) {
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
                split_f32x8(gelu_tile(p, 2 * jj), gelu_tile(p, 2 * jj + 1), hbh[0][jj], hbl[0][jj]);
        } else {
            constexpr int S2 = PK == 1 ? 0 : 2;  // ring slots of the second GEMM's stages
            const int u2 = PK == 1 ? u0 + 2 : u0;
            const int gc = PK == 1 ? p : -1;
            auto d = step_begin(kindc, u2);
            if (PK == 1 && p == kChunks - 1 && nextp >= 0) {
                load_x(nextp);
                ext1 += kXL;
            }
            gemm2(std::integral_constant<int, 2>{}, std::integral_constant<int, PAR ^ 1>{}, st[S2], d, gc);
            d = step_begin(kindc, u2 + 1);
            gemm2(std::integral_constant<int, 3>{}, std::integral_constant<int, PAR ^ 1>{}, st[S2 + 1], d, gc);
        }
    };
    using std::integral_constant;
    using Mid = integral_constant<int, 0>;
    using Gen = integral_constant<int, 1>;
    using End = integral_constant<int, 2>;
    using P0 = integral_constant<int, 0>;
    using P1 = integral_constant<int, 1>;

    // the O-projection's stages (waits counted at run time: the first three
    // follow the last panel's stores, the last issues the residual's loads),
    // then the first LayerNorm
    auto o_phase = [&](int panel, int ub) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kO; j++) {
            const auto d = step_begin(Gen{}, ub + j);
            if (j == kO - 1) {
                // the residual, once the context's first halves are done
                // with (counted with the step before, after whose stage
                // loads it is issued)
                load_rows(op.res, panel);
                ext1 += kXL;
            }
            gemm_o(j, st[j & 3], d);
        }
        layernorm1();
        split_x(std::true_type{});
#pragma unroll
        for (int o = 0; o < kYT; o++) yacc[o] = f32x4_t{};
    };

    load_x(count > 0 ? (int)blockIdx.x : tpanel);
#pragma unroll
    for (int u = 0; u < 3; u++)
        if (u < S) {
            const auto d = dma_of(u, std::false_type{});
#pragma unroll
            for (int k = 0; k < kLWv; k++) dma_one(d, k);
        }
    split_x(std::integral_constant<bool, MODE == 0>{});
    if constexpr (QKV) {
        // whole panels: the first three chunks count their waits at run time
        // (the last panel's stores), the last two as the block's stream may
        // end.  The next panel's X is loaded after the panel (two waves a
        // SIMD leave no registers to hold it through the panel); the wait
        // for it before its split retires every op before it, so it needs no
        // count of its own.
        for (int i = 0; i < count; i++) {
            const int panel = blockIdx.x + i * gridDim.x;
            const int nextp = i + 1 < count ? panel + (int)gridDim.x : (tail ? tpanel : -1);
            const int ub = i * kSP;
            qkv_chunk(Gen{}, ub, 0, panel, -1);
            qkv_chunk(Gen{}, ub + 2, 1, panel, -1);
            qkv_chunk(Gen{}, ub + 4, 2, panel, -1);
            for (int c = 3; c < kQChunks - 2; c++) qkv_chunk(Mid{}, ub + 2 * c, c, panel, -1);
            qkv_chunk(End{}, ub + 2 * (kQChunks - 2), kQChunks - 2, panel, -1);
            qkv_chunk(End{}, ub + 2 * (kQChunks - 1), kQChunks - 1, panel, -1);
            if (nextp >= 0) {
                load_x(nextp);
                split_x(std::false_type{});
            }
        }
        // this block's part of a split panel: its chunks' columns
        if (tail)
            for (int cr = 0; cr < nc; cr++) qkv_chunk(End{}, SF + 2 * cr, c0 + cr, tpanel, -1);
        // the last chunk's vectors (no wait follows them)
#pragma unroll
        for (int k = 0; k < 4; k++) qkv_put(k, true);
        return;
    }
    for (int i = 0; i < count; i++) {
        const int panel = blockIdx.x + i * gridDim.x;
        const int nextp = i + 1 < count ? panel + (int)gridDim.x : (tail ? tpanel : -1);
#pragma unroll
        for (int o = 0; o < kYT; o++) yacc[o] = f32x4_t{};
        int ub = i * kSP;
        if constexpr (OP) {
            o_phase(panel, ub);
            ub += kO;
        }
        period(P0{}, Gen{}, P0{}, ub, 0, nextp);
        period(P1{}, Gen{}, P1{}, ub + 2, 1, nextp);
        for (int p = 2; p < kChunks - 2; p += 2) {
            period(P1{}, Mid{}, P0{}, ub + 4 * p - 2, p, nextp);
            period(P1{}, Mid{}, P1{}, ub + 4 * p + 2, p + 1, nextp);
        }
        period(P1{}, Mid{}, P0{}, ub + 4 * (kChunks - 2) - 2, kChunks - 2, nextp);
        period(P1{}, End{}, P1{}, ub + 4 * (kChunks - 1) - 2, kChunks - 1, nextp);
        period(integral_constant<int, 2>{}, End{}, P0{}, ub + kSPP - 2, kChunks, nextp);
        const bool full = epilogue(panel);
        ext0 = full ? kXL : 0;  // the stores, after the loads of the panel's last step
        if (nextp >= 0) split_x(std::integral_constant<bool, MODE == 0>{});
    }
    if (tail) {
        // this block's part of a split panel: its chunks' periods (every
        // step's wait counted at run time; the stream ends with the part),
        // then its raw sums (and, part 0, X) to the scratch
#pragma unroll
        for (int o = 0; o < kYT; o++) yacc[o] = f32x4_t{};
        int ub = SF;
        if constexpr (OP) {
            o_phase(tpanel, ub);
            ub += kO;
            if (tpart == 0) {
                // X, the residual, now (not parked through the part); issued
                // after the last O step's stage loads, counted with that step
                const int ln = lane_now(), g = ln >> 4;
                float *const px = ts.xs + ((size_t)(tpanel - ts.full) * kBMv + wu * kTokW + (ln & 15)) * kD;
#pragma unroll
                for (int j = 0; j < kXJ; j++)
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        f32x4_t x;
#pragma unroll
                        for (int e = 0; e < 4; e++) x[e] = unpark(xr[8 * j + 4 * h + e]);
                        *(f32x4_t *)(px + 32 * j + 8 * g + 4 * h) = x;
                        vmem_store_issued();
                    }
                ext0 += kXL;
            }
        }
        period(P0{}, End{}, P0{}, ub, c0, -1);
        for (int pr = 1; pr < nc; pr += 2) {
            period(P1{}, End{}, P1{}, ub + 4 * pr - 2, c0 + pr, -1);
            if (pr + 1 < nc) period(P1{}, End{}, P0{}, ub + 4 * pr + 2, c0 + pr + 1, -1);
        }
        if (nc & 1)
            period(integral_constant<int, 2>{}, End{}, P1{}, ub + kSPC * nc - 2, c0 + nc, -1);
        else
            period(integral_constant<int, 2>{}, End{}, P0{}, ub + kSPC * nc - 2, c0 + nc, -1);
        const int ln = lane_now(), g = ln >> 4;
        float *const ps =
            ts.sums + (((size_t)(tpanel - ts.full) * ts.parts + tpart) * kBMv + wu * kTokW + (ln & 15)) * kD;
#pragma unroll
        for (int j = 0; j < kXJ; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                *(f32x4_t *)(ps + 32 * j + 8 * g + 4 * h) = yacc[2 * j + h];
                vmem_store_issued();
            }
    }
}

// Rows t0 .. T - 1 of the split panels (the tail parts of mlp_fused_kernel):
// Y = LayerNorm(X + ((sum over parts) * s2 + b2)) with the parts' sums added
// in part order (arctic.zig:780-783; the LayerNorm of layernorm.zig:26-117,
// two-pass as in the fused kernel's epilogue); xs: X's row t0 + r at r.
// One wave per row, lane l holding columns 6 l .. 6 l + 5.
__global__ void __launch_bounds__(256) mlp_tail_kernel(const float *__restrict__ sums, const float *__restrict__ xs,
                                                       int parts, const uint16_t *__restrict__ s2,
                                                       const float *__restrict__ b2, const float *__restrict__ gamma,
                                                       const float *__restrict__ beta, float eps,
                                                       float *__restrict__ Y, int t0, int T) {
    const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (t0 + row >= T) return;
    const int lane = threadIdx.x & 63, tp = row / kBM, tok = row % kBM;
    const int n0 = 6 * lane;
    float acc[6];
    for (int p = 0; p < parts; p++) {
        const float *sr = sums + (((size_t)tp * parts + p) * kBM + tok) * kD + n0;
#pragma unroll
        for (int e = 0; e < 6; e++) acc[e] = p == 0 ? sr[e] : acc[e] + sr[e];
    }
    const float *xr = xs + (size_t)row * kD + n0;
    float v[6], sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 6; e++) {
        v[e] = xr[e] + (acc[e] * f16_bits_to_f32(s2[n0 + e]) + b2[n0 + e]);
        sum += v[e];
    }
    const float mean = wave_sum(sum) / (float)kD;
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < 6; e++) sq += (v[e] - mean) * (v[e] - mean);
    const float inv_std = 1.0f / sqrtf(wave_sum(sq) / (float)kD + eps);
    float *yr = Y + (size_t)(t0 + row) * kD + n0;
#pragma unroll
    for (int e = 0; e < 6; e++) yr[e] = ((v[e] - mean) * inv_std) * gamma[n0 + e] + beta[n0 + e];
}

}  // namespace

// W8T codes of the two feed-forward linears (w1: 1536 rows of 384, w2: 384
// rows of 1536) -> the f16 fragment pack of mlp_fused_kernel
// (tzh_mlp_pack_bytes bytes, 16-byte aligned).
size_t tzh_mlp_pack_bytes() { return kPackHalves * 2; }

int tzh_mlp_pack_launch(hipStream_t st, const void *w1, const void *w2, void *out) {
    if (!w1 || !w2 || !out || ((uintptr_t)out & 15)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad MLP pack operands");
    const int threads = kChunks * kSPC * kStageFrags * 64;
    hipLaunchKernelGGL(mlp_pack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       (const uint8_t *)w1, (const uint8_t *)w2, (_Float16 *)out);
    TZH_LAUNCHED("mlp_pack_kernel");
    return TZH_OK;
}

// W_o's codes (W8T, [384, 384]) -> the O-projection's stages for
// mlp_fused_kernel (tzh_mlp_opack_bytes bytes, 16-byte aligned).
size_t tzh_mlp_opack_bytes() { return (size_t)kOStages * kStage; }

int tzh_mlp_opack_launch(hipStream_t st, const void *wo, void *out) {
    if (!wo || !out || ((uintptr_t)out & 15)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad O-projection pack operands");
    const int threads = kOStages * kStageFrags * 64;
    hipLaunchKernelGGL(mlp_opack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, (const uint8_t *)wo,
                       (_Float16 *)out);
    TZH_LAUNCHED("mlp_opack_kernel");
    return TZH_OK;
}

namespace {

// The split of the last round for t tokens on num_cus CUs: the most parts
// (a divisor of the 24 chunks) whose blocks fit the CUs the round leaves
// idle, when the scratch holds their sums; otherwise none (parts = 1).
TailSplit choose_tail(int64_t t, int num_cus, size_t scratch_bytes) {
    const int panels = (int)((t + kBM - 1) / kBM);
    const int rest = panels % num_cus;
    TailSplit ts{panels, 1, nullptr, nullptr};
    if (rest == 0) return ts;
    for (int parts : {24, 12, 8, 6, 4, 3, 2}) {
        const size_t need = (size_t)rest * (parts + 1) * kBM * kD * 4;
        if (rest * parts <= num_cus && need <= scratch_bytes) {
            ts.full = panels - rest;
            ts.parts = parts;
            return ts;
        }
    }
    return ts;
}

}  // namespace

// Scratch bytes the split of the last round can use on num_cus CUs, at most
// (any token count).
size_t tzh_mlp_tail_bytes(int num_cus) {
    size_t most = 0;
    for (int rest = 1; rest <= num_cus / 2; rest++) {
        const TailSplit ts = choose_tail((int64_t)rest * kBM, num_cus, (size_t)-1);
        most = std::max(most, (size_t)rest * (ts.parts + 1) * kBM * kD * 4);
    }
    return most;
}

// Y = LayerNorm(X + GELU(X W1^T s1 + b1) W2^T s2 + b2) for X, Y [t, 384]
// f32 (16-byte aligned, not overlapping) with the pack of W1 and W2.  With
// the O-projection (opack non-null): X = LayerNorm(res + (ctx W_o^T s_o +
// b_o)) with gamma1, beta1 is formed on chip first, from ctx and res [t,
// 384] f32 (x unused).  Y may be res itself (each token's residual row is
// read, and its output row written, by the same wave, in that order) but
// may not overlap ctx or overlap res partly.  scratch (16-byte aligned,
// overlapping none of them; may be null): room for the split of the last
// round (tzh_mlp_tail_bytes); without enough, that round runs whole panels.
int tzh_mlp_fused_launch(hipStream_t st, int num_cus, const float *x, const void *pack, const uint16_t *s1,
                         const float *b1, const uint16_t *s2, const float *b2, const float *gamma, const float *beta,
                         float eps, float *y, int64_t t, const float *ctx, const float *res, const void *opack,
                         const uint16_t *so, const float *bo, const float *gamma1, const float *beta1, void *scratch,
                         size_t scratch_bytes) {
    if (t < 0 || t > ((int64_t)1 << 30)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad token count %lld", (long long)t);
    if (t == 0) return TZH_OK;
    const bool op = opack != nullptr;
    if (op) x = ctx;  // the activations the kernel loads
    if (!x || !pack || !s1 || !b1 || !s2 || !b2 || !gamma || !beta || !y ||
        (op && (!res || !so || !bo || !gamma1 || !beta1)))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "null MLP operand");
    if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)pack | (op ? (uintptr_t)res | (uintptr_t)opack : 0)) & 15)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "MLP operands must be 16-byte aligned");
    const size_t bytes = (size_t)t * kD * 4;
    auto overlap = [&](const void *a, const void *b) {
        return (const char *)a < (const char *)b + bytes && (const char *)b < (const char *)a + bytes;
    };
    if (overlap(x, y) || (op && res != y && overlap(res, y)))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "MLP input and output overlap");
    if (num_cus < 1) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad CU count %d", num_cus);
    if ((uintptr_t)scratch & 15) return tzh_fail(TZH_ERR_INVALID_ARGS, "MLP scratch must be 16-byte aligned");
    const int panels = (int)((t + kBM - 1) / kBM);
    TailSplit ts = choose_tail(t, num_cus, scratch ? scratch_bytes : 0);
    const int rest = panels - ts.full;
    int grid = panels < num_cus ? panels : num_cus;
    if (ts.parts > 1) {
        ts.sums = (float *)scratch;
        ts.xs = op ? ts.sums + (size_t)rest * ts.parts * kBM * kD : nullptr;
        grid = ts.full > 0 ? num_cus : rest * ts.parts;
    }
    const OProj o{ctx, res, (const _Float16 *)opack, so, bo, gamma1, beta1};
    if (op)
        hipLaunchKernelGGL(mlp_fused_kernel<1>, dim3((unsigned)grid), dim3(kWaves * 64), 0, st, x,
                           (const _Float16 *)pack, s1, b1, s2, b2, gamma, beta, eps, y, (int)t, o, ts);
    else
        hipLaunchKernelGGL(mlp_fused_kernel<0>, dim3((unsigned)grid), dim3(kWaves * 64), 0, st, x,
                           (const _Float16 *)pack, s1, b1, s2, b2, gamma, beta, eps, y, (int)t, o, ts);
    TZH_LAUNCHED("mlp_fused_kernel");
    if (ts.parts > 1) {
        const int t0 = ts.full * kBM, rows = (int)t - t0;
        hipLaunchKernelGGL(mlp_tail_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, ts.sums,
                           op ? (const float *)ts.xs : x + (size_t)t0 * kD, ts.parts, s2, b2, gamma, beta, eps, y, t0,
                           (int)t);
        TZH_LAUNCHED("mlp_tail_kernel");
    }
    return TZH_OK;
}

// W_qkv's codes (W8T, [1152, 384]) -> the QKV mode's stages
// (tzh_qkv_pack_bytes bytes, 16-byte aligned).
size_t tzh_qkv_pack_bytes() { return (size_t)2 * kQChunks * kStage; }

int tzh_qkv_pack_launch(hipStream_t st, const void *w, void *out) {
    if (!w || !out || ((uintptr_t)out & 15)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad QKV pack operands");
    const int threads = 2 * kQChunks * kStageFrags * 64;
    hipLaunchKernelGGL(qkv_pack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, (const uint8_t *)w,
                       (_Float16 *)out);
    TZH_LAUNCHED("qkv_pack_kernel");
    return TZH_OK;
}

// Y [t, 1152] = X W_qkv^T s + b for X [t, 384] f32 (16-byte aligned, not
// overlapping Y) with the QKV pack, on the fused kernel's QKV mode: the
// last, partial round of panels split by chunks over the idle CUs (the
// parts write disjoint columns; nothing to add up).
int tzh_qkv_fused_launch(hipStream_t st, int num_cus, const float *x, const void *pack, const uint16_t *s,
                         const float *b, float *y, int64_t t) {
    if (t < 0 || t > ((int64_t)1 << 30)) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad token count %lld", (long long)t);
    if (t == 0) return TZH_OK;
    if (!x || !pack || !s || !b || !y) return tzh_fail(TZH_ERR_INVALID_ARGS, "null QKV operand");
    if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)pack) & 15)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "QKV operands must be 16-byte aligned");
    if ((const char *)x < (const char *)(y + (size_t)t * kFQ) && (const char *)y < (const char *)(x + (size_t)t * kD))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "QKV input and output overlap");
    if (num_cus < 1) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad CU count %d", num_cus);
    constexpr int kBMq = 2 * kBM;  // the QKV mode's panels (eight waves)
    const int panels = (int)((t + kBMq - 1) / kBMq), rest = panels % num_cus;
    TailSplit ts{panels, 1, nullptr, nullptr};
    if (rest > 0)
        for (int parts : {18, 9, 6, 3, 2})
            if (rest * parts <= num_cus) {
                ts.full = panels - rest;
                ts.parts = parts;
                break;
            }
    const int grid = ts.parts > 1 ? (ts.full > 0 ? num_cus : rest * ts.parts) : std::min(panels, num_cus);
    hipLaunchKernelGGL(mlp_fused_kernel<2>, dim3((unsigned)grid), dim3(2 * kWaves * 64), 0, st, x, (const _Float16 *)pack,
                       s, b, nullptr, nullptr, nullptr, nullptr, 0.0f, y, (int)t, OProj{}, ts);
    TZH_LAUNCHED("mlp_fused_kernel");
    return TZH_OK;
}
