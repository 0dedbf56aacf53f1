// K4: variable-length multi-head self-attention on MFMA (head_dim 32).
//
// Restates the attention core of selfAttention (arctic.zig:660-713): per
// head, S = Q_h K_h^T, S *= 1/sqrt(head_dim), row softmax (max, exp(x-max),
// sum, divide), O_h = P V_h.  Sequences are packed back to back
// (cu_seqlens), each attends only to its own keys, so the result equals the
// reference's per-sequence unpadded forward.
//
// Design (gfx950): one workgroup per (sequence, head); its K and V^T
// (L <= 512 keys) are staged in LDS once and every wave walks 16-query
// tiles over them.  S^T = K Q^T and O^T = V^T P^T use
// v_mfma_f32_16x16x32_f16 so that each lane owns one query.  The loop is
// VALU-bound (one exp per score against 128 MFMA flops), so per score it
// spends one FMA (scale and running max folded into the exp2 argument), one
// exp2, half a max3 and half a packed convert: the row max crosses the four
// lane rows with permlane swaps, keys past the end are masked only in the
// last 64-key block, and the row sum is a third MFMA against a ones operand
// (it sums the same f16 probabilities the P V product uses).  Softmax is the
// online (running max / rescale) form; the division by the row sum happens
// once at the end.
#include "common.h"

#include <algorithm>
#include <climits>
#include <vector>

namespace {

constexpr int kHeadDim = 32;
constexpr int kMaxKeys = 512;
constexpr int K_LD = kHeadDim + 8;     // halves per K row in LDS (80 B: conflict-free 16-byte reads)
constexpr int V_LD = kMaxKeys + 8;     // halves per V^T row in LDS (1040 B: likewise)
constexpr int kWaves = 8;              // waves per workgroup (2 workgroups per CU by LDS)
constexpr int kQueryTiles = 1;         // 16-query tiles a wave carries at once
constexpr float kLazyLog2 = 8.0f;      // softmax reference-point slack (exp2 units)
constexpr float kLazySum = 32768.0f;   // f32 kernel: bound on a lane's block sum of probabilities

// V^T row layout: within each 32-key group, the keys the PV operand of lane
// row g takes ({4g..4g+3} and {16+4g..16+4g+3}, the order the S^T
// accumulators hold them in) are stored at 8g..8g+7, so one 16-byte read
// fetches them: key j of a group sits at 8 * ((j % 16) / 4) + 4 * (j / 16) + j % 4.

template <int NW, int QT>
__global__ void __launch_bounds__(NW * 64) attn_varlen_kernel(const _Float16 *__restrict__ qkv, int ld,
                                                          _Float16 *__restrict__ out, int ld_out,
                                                          const int *__restrict__ cu_seqlens,
                                                          const int *__restrict__ order, int batch, int n_heads,
                                                          int hidden, float scale_log2) {
    __shared__ __attribute__((aligned(16))) _Float16 Ks[kMaxKeys * K_LD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[kHeadDim * V_LD];

    // Workgroups go to the XCDs round-robin (block b on XCD b % 8), each XCD
    // with its own L2.  Heads 2k and 2k+1 of a sequence share every 128-byte
    // line of its Q/K/V rows (64 bytes each), so they get blocks b and b + 8:
    // same XCD, dispatched together, each line read from HBM once.  With an
    // odd head count blocks map to (sequence, head) in order.
    int item, h;
    if (n_heads % 2 == 0) {
        const int pairs = n_heads / 2;
        const int hp = (int)(blockIdx.x / 16) * 8 + (int)(blockIdx.x % 8);  // (sequence, head pair)
        item = hp / pairs;
        h = 2 * (hp % pairs) + (int)(blockIdx.x / 8) % 2;
    } else {
        item = blockIdx.x / n_heads;
        h = blockIdx.x % n_heads;
    }
    if (item >= batch) return;  // padding blocks of the pair layout (whole workgroup)
    const int b = order ? order[item] : item;
    const int start = cu_seqlens[b];
    // the host validates lengths; the clamp keeps every LDS index in bounds regardless
    const int L = min(max(cu_seqlens[b + 1] - start, 0), kMaxKeys);
    const int Lp = (L + 63) & ~63;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    const _Float16 *qbase = qkv + (size_t)start * ld + h * kHeadDim;
    const _Float16 *kbase = qbase + hidden;
    const _Float16 *vbase = qbase + 2 * hidden;

    // keys L..Lp-1 are zero-filled: their probabilities are 0 and 0 * V must stay 0
    for (int idx = tid; idx < Lp * 4; idx += NW * 64) {
        const int key = idx >> 2, c = (idx & 3) * 8;
        half8_t kv = {};
        if (key < L) kv = *(const half8_t *)(kbase + (size_t)key * ld + c);
        *(half8_t *)(Ks + key * K_LD + c) = kv;
    }
    // V^T: each lane loads an 8-key x 8-dim block (the keys one PV operand
    // read takes), transposes it in registers and writes eight 16-byte rows
    // (lanes 0..15 of a write cover sixteen distinct bank slots).
    {
        const int gq = lane & 3, kg = (lane >> 2) & 3, c = lane >> 4;
        for (int kb = 128 * w; kb < Lp; kb += 128 * NW) {
            const int k0 = kb + 32 * kg + 4 * gq;  // keys k0 + {0..3} and k0 + 16 + {0..3}
            half8_t v[8];
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const int key = k0 + (r & 3) + 16 * (r >> 2);
                v[r] = half8_t{};
                if (key < L) v[r] = *(const half8_t *)(vbase + (size_t)key * ld + 8 * c);
            }
#pragma unroll
            for (int d = 0; d < 8; d++) {
                half8_t col;
#pragma unroll
                for (int r = 0; r < 8; r++) col[r] = v[r][d];
                *(half8_t *)(Vt + (8 * c + d) * V_LD + kb + 32 * kg + 8 * gq) = col;
            }
        }
    }
    __syncthreads();

    const int g = lane >> 4;   // lane row: k-slots 8g..8g+7, C rows 4g..4g+3
    const int ql = lane & 15;  // query (C column) owned by this lane in each tile
    const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
    // A wave can carry QT 16-query tiles at once (they share every K and V
    // fragment read).  One tile per wave measured fastest on MI355X at the
    // Arctic lengths: twice the tasks balance the waves of a block better.
    for (int q0 = w * 16 * QT; q0 < L; q0 += NW * 16 * QT) {
        half8_t qf[QT];
        float m[QT];  // running max of the raw scores
        f32x4_t o0[QT], o1[QT], lsum[QT];
#pragma unroll
        for (int j = 0; j < QT; j++) {
            const int qrow = q0 + 16 * j + ql;
            qf[j] = half8_t{};
            if (qrow < L) qf[j] = *(const half8_t *)(qbase + (size_t)qrow * ld + g * 8);
            m[j] = -INFINITY;
            o0[j] = o1[j] = lsum[j] = f32x4_t{0, 0, 0, 0};
        }
        for (int kb0 = 0; kb0 < Lp; kb0 += 64) {
            f32x4_t s[QT][4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const half8_t kf = *(const half8_t *)(Ks + (kb0 + 16 * t + ql) * K_LD + g * 8);
#pragma unroll
                for (int j = 0; j < QT; j++)
                    s[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[j], f32x4_t{0, 0, 0, 0}, 0, 0, 0);
            }
            if (kb0 + 64 > L) {  // the block holding the sequence end (wave-uniform)
                const int rem = L - kb0 - 4 * g;  // element (t, i) is key kb0 + 4g + 16t + i
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const bool past = 16 * t + i >= rem;
#pragma unroll
                        for (int j = 0; j < QT; j++) s[j][t][i] = past ? -INFINITY : s[j][t][i];
                    }
            }
#pragma unroll
            for (int j = 0; j < QT; j++) {
                float mx = s[j][0][0];
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[j][t][i]);
                // finite: every 64-key block below Lp holds a key < L
                mx = max_over_rows(mx);
                // Lazy rescaling: the reference point m only moves (and the
                // accumulators are rescaled) when some lane's block max
                // exceeds it by more than kLazyLog2 in the exp2 domain, so the
                // probabilities stay <= 2^kLazyLog2 (f16 and f32 hold them
                // exactly as well as values <= 1) and most blocks skip the
                // rescale.  The first block always moves m off -inf.
                if (wave_any((mx - m[j]) * scale_log2 > kLazyLog2)) {
                    const float m_new = fmaxf(m[j], mx);
                    const float alpha = __builtin_amdgcn_exp2f((m[j] - m_new) * scale_log2);  // 0 on the first block
                    o0[j] *= alpha;
                    o1[j] *= alpha;
                    lsum[j] *= alpha;
                    m[j] = m_new;
                }
                const float mc = m[j] * scale_log2;
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        s[j][t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][t][i], scale_log2, -mc));
            }
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const int kv = kb0 + 32 * st + 8 * g;
                const half8_t va = *(const half8_t *)(Vt + ql * V_LD + kv);
                const half8_t vb = *(const half8_t *)(Vt + (16 + ql) * V_LD + kv);
#pragma unroll
                for (int j = 0; j < QT; j++) {
                    half8_t pf;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        pf[i] = (_Float16)s[j][2 * st][i];
                        pf[4 + i] = (_Float16)s[j][2 * st + 1][i];
                    }
                    o0[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf, o0[j], 0, 0, 0);
                    o1[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb, pf, o1[j], 0, 0, 0);
                    lsum[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf, lsum[j], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < QT; j++) {
            const int qrow = q0 + 16 * j + ql;
            if (qrow < L) {
                const float inv = 1.0f / lsum[j][0];  // every row of the ones product holds the row sum
                _Float16 *dst = out + (size_t)(start + qrow) * ld_out + h * kHeadDim + 4 * g;
                half4_t r0, r1;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    r0[i] = (_Float16)(o0[j][i] * inv);
                    r1[i] = (_Float16)(o1[j][i] * inv);
                }
                *(half4_t *)dst = r0;
                *(half4_t *)(dst + 16) = r1;
            }
        }
    }
}

// f32 attention (the reference's arithmetic).  Q, K and V are split into
// f16 pairs x = hi + lo (hi = f16(x), lo = f16(x - hi), exact to about 2^-22
// relative) and every product a.b of two split operands is formed as
// hi.hi + hi.lo + lo.hi on the MFMA with f32 accumulation (lo.lo is below
// 2^-22 relative); the probabilities are split the same way for P V.  K and
// V^T are staged in LDS as hi and lo planes (145 KiB: one workgroup per CU).
//
// Q is scaled by log2(e)/sqrt(head_dim) before it is split, and the S^T
// accumulators start at minus the query's reference point, so the MFMAs
// deliver exp2 arguments directly: no VALU work per score before the exp.
// The row sum adds the f32 probabilities on the VALU: the values P V
// weights with, to f32 rounding.  (As a fourth and fifth MFMA against a ones
// operand it measured 2 % slower.)  Only the first key block of a query
// tile takes a row max; later blocks test the lane's sum of their 16
// probabilities against kLazySum, which bounds every probability as the
// max would, and a block past it (rare) recomputes its scores to rescale.
// That removes about 12 of 78 VALU ops per block (1 % faster).
constexpr int kWavesF32 = 16;

template <int NW>
__global__ void __launch_bounds__(NW * 64) attn_varlen_f32_kernel(const float *__restrict__ qkv, int ld,
                                                              float *__restrict__ out, int ld_out,
                                                              const int *__restrict__ cu_seqlens,
                                                              const int *__restrict__ order, int batch, int n_heads,
                                                              int hidden, float scale_log2, unsigned *queue) {
    // V^T hi, V^T lo, K hi, K lo in one array, V^T first: the four V^T reads
    // of a 32-key step then lie within 64 KiB of one address register (the
    // DS offset field), as do the K reads of a block.
    constexpr int kVPlane = kHeadDim * V_LD, kKPlane = kMaxKeys * K_LD;
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * kVPlane + 2 * kKPlane];
    _Float16 *const Vt0 = lds, *const Vt1 = lds + kVPlane;
    _Float16 *const Ks0 = lds + 2 * kVPlane, *const Ks1 = Ks0 + kKPlane;

    static_assert(NW * 32 == kMaxKeys, "one 32-key V^T group per wave");
    static_assert(kMaxKeys == 2 * NW * 16, "two 16-query tiles per wave");
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, ql = lane & 15;
    const int gq = lane & 3, dp = lane >> 2;  // V staging: slot group, dim pair
    const int n_items = batch * n_heads;

    // Persistent blocks over items (item j: the j / n_heads-th sequence of
    // `order`, longest first, head j % n_heads).  Block b starts with item b
    // and then takes the next untaken item from queue[0] (a work queue:
    // statically dealt, the slowest block ran 10 % past the mean).  The next
    // item's K and V rows are loaded into registers while this item's
    // queries run, so a block's loads overlap its MFMA work: with one 145 KiB
    // workgroup per CU nothing else would hide them.
    struct Item {
        int start, L, h;
    };
    auto item_of = [&](int j) {
        const int s = j / n_heads;
        const int b = order ? order[s] : s;
        const int start = cu_seqlens[b];
        // the host validates lengths; the clamp keeps every LDS index in bounds regardless
        return Item{start, min(max(cu_seqlens[b + 1] - start, 0), kMaxKeys), j % n_heads};
    };
    // prefetch registers: K units u = tid + 1024 i (key u / 4, dims 8 (u % 4)
    // + [0, 8)) and V keys 32 w + 4 gq + (r % 4) + 16 (r / 4), dims 2 dp and
    // 2 dp + 1; rows past the sequence load its last row (same line, same
    // instruction count for every length)
    f32x4_t pk[4];
    f32x2_t pv[8];
    auto prefetch = [&](const Item &it) {
        if (it.L == 0) return;
        const float *kb = qkv + (size_t)it.start * ld + hidden + it.h * kHeadDim;
        const float *vb = kb + hidden;
        const int last = it.L - 1;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int u = tid + NW * 64 * i;
            const float *src = kb + (size_t)min(u >> 2, last) * ld + (u & 3) * 8;
            pk[2 * i] = *(const f32x4_t *)src;
            pk[2 * i + 1] = *(const f32x4_t *)(src + 4);
        }
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int key = 32 * w + 4 * gq + (r & 3) + 16 * (r >> 2);
            pv[r] = *(const f32x2_t *)(vb + (size_t)min(key, last) * ld + 2 * dp);
        }
    };
    // prefetched K / V -> hi and lo planes.  Keys L .. Lp-1 hold copies of
    // the last row: finite, and their scores are masked, so they weigh 0.
    auto stage = [&](const Item &it) {
        const int Lp = (it.L + 63) & ~63;
        // the LDS addresses below are recomputed per item from a laundered
        // thread id: hoisted, they would hold registers through the compute
        int stid = threadIdx.x;
        asm volatile("" : "+v"(stid));
        const int sgq = stid & 3, sdp = (stid & 63) >> 2;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int u = stid + NW * 64 * i, key = u >> 2, c = (u & 3) * 8;
            if (key < Lp) {
                half8_t hi, lo;
                split_f32x8(pk[2 * i], pk[2 * i + 1], hi, lo);
                *(half8_t *)(Ks0 + key * K_LD + c) = hi;
                *(half8_t *)(Ks1 + key * K_LD + c) = lo;
            }
        }
        // V^T in the PV operand order (see the V^T layout note): a wave per
        // 32-key group; 16 lanes read a whole 128-byte row; one 16-byte piece
        // per dim and plane
        const int kb = 32 * w;
        if (kb < Lp) {
            uint32_t hi[8], lo[8];  // key r: dims 2 sdp, 2 sdp + 1 as f16 pairs
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const f32x2_t v = pv[r];
                hi[r] = __builtin_bit_cast(uint32_t, half2_t{(_Float16)v[0], (_Float16)v[1]});
                lo[r] = split_lo_pair(hi[r], v[0], v[1]);
            }
#pragma unroll
            for (int part = 0; part < 2; part++) {
                const uint32_t *x = part ? lo : hi;
                _Float16 *const plane = part ? Vt1 : Vt0;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    // keys (2i, 2i + 1) of dim 2 sdp + e as one f16 pair
                    u32x4v col;
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        col[i] = e ? (x[2 * i] >> 16) | (x[2 * i + 1] & 0xffff0000u)
                                   : (x[2 * i] & 0xffffu) | (x[2 * i + 1] << 16);
                    *(u32x4v *)(plane + (2 * sdp + e) * V_LD + kb + 8 * sgq) = col;
                }
            }
        }
    };

    const f32x4_t scale4 = {scale_log2, scale_log2, scale_log2, scale_log2};
    __shared__ int next_item;
    int j = blockIdx.x;
    if (j >= n_items) return;
    Item cur = item_of(j);
    prefetch(cur);
    while (j < n_items) {
        // the queue's counter starts at 0 in every launch (reset below)
        if (tid == 0) next_item = (int)gridDim.x + (int)atomicAdd(queue, 1u);
        const int L = cur.L, Lp = (L + 63) & ~63;
        const float *qbase = qkv + (size_t)cur.start * ld + cur.h * kHeadDim;
        // Q rows of this wave's first query tile (16 w), clamped to the
        // sequence; loaded before staging so that their latency overlaps it
        auto load_q = [&](int q0, f32x4_t &qa, f32x4_t &qb) {
            if (L > 0) {
                const float *src = qbase + (size_t)min(q0 + ql, L - 1) * ld + g * 8;
                qa = *(const f32x4_t *)src;
                qb = *(const f32x4_t *)(src + 4);
            }
        };
        f32x4_t qa = {0, 0, 0, 0}, qb = {0, 0, 0, 0};
        load_q(16 * w, qa, qb);
        stage(cur);
        __syncthreads();
        // Q is split before the next item's loads are issued, so that its
        // wait does not include them; the second tile's Q (16 (w + NW), only
        // where L > 256) is loaded when the first tile is done
        half8_t qh, qlo;
        split_f32x8(qa * scale4, qb * scale4, qh, qlo);
        const int jn = next_item;  // written before the barrier above, rewritten after the one below
        const Item nxt = jn < n_items ? item_of(jn) : Item{0, 0, 0};
        prefetch(nxt);

        for (int t2 = 0; t2 < 2; t2++) {
            const int q0 = 16 * (w + NW * t2);
            if (q0 >= L) break;
            const int qrow = q0 + ql;
            if (t2) {
                load_q(q0, qa, qb);
                split_f32x8(qa * scale4, qb * scale4, qh, qlo);
            }
            // m: the query's reference point in exp2 units, set to the first
            // block's max.  Later blocks take no max: a block moves m only
            // when some lane's sum of its 16 probabilities exceeds kLazySum,
            // which keeps every probability below f16's range limit (its
            // hi/lo split keeps 22 bits at any magnitude); such a block
            // recomputes its scores and rescales before its P V products.
            float m = 0.0f, lsum = 0.0f;
            f32x4_t o0 = {0, 0, 0, 0}, o1 = {0, 0, 0, 0};
            const _Float16 *kp0 = Ks0 + ql * K_LD + g * 8;
            const _Float16 *vp0 = Vt0 + ql * V_LD + 8 * g;
            // the block's exp2 arguments s - m (keys past L: -inf)
            auto scores = [&](int kb0, f32x4_t(&s)[4]) {
                // one address register for the block's eight K reads (DS
                // offsets of up to 44 800 bytes); left to itself the compiler
                // forms each address with an add, as the K planes start past 64 KiB
                int koff = kb0 * K_LD;
                asm volatile("" : "+v"(koff));
                const _Float16 *kblk = kp0 + koff;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const _Float16 *kp = kblk + 16 * t * K_LD;
                    const half8_t kh = *(const half8_t *)kp;
                    const half8_t kl = *(const half8_t *)(kp + kKPlane);
                    f32x4_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh, f32x4_t{-m, -m, -m, -m}, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qlo, acc, 0, 0, 0);
                    s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh, acc, 0, 0, 0);
                }
                if (kb0 + 64 > L) {
                    // (4 g laundered: folded into the 16 compares' constants
                    // it would take 16 registers for the whole kernel)
                    int g4 = 4 * g;
                    asm volatile("" : "+v"(g4));
                    const int rem = L - kb0 - g4;
#pragma unroll
                    for (int t = 0; t < 4; t++)
#pragma unroll
                        for (int i = 0; i < 4; i++) s[t][i] = 16 * t + i >= rem ? -INFINITY : s[t][i];
                }
            };
            // the row's max over the block, in every lane row (finite: every
            // 64-key block below Lp holds a key < L)
            auto row_max = [&](const f32x4_t(&s)[4]) {
                float mx = s[0][0];
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[t][i]);
                return max_over_rows(mx);
            };
            // s -> 2^s in place; returns the lane's sum of the 16
            auto exps = [&](f32x4_t(&s)[4]) {
                float bs = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        s[t][i] = __builtin_amdgcn_exp2f(s[t][i]);
                        bs = t + i == 0 ? s[t][i] : bs + s[t][i];
                    }
                return bs;
            };
            for (int kb0 = 0; kb0 < Lp; kb0 += 64) {
                f32x4_t s[4];
                scores(kb0, s);
                // (a laundered test: peeled, the first block's copy of the
                // loop body took the registers of long-lived values)
                int first = kb0 == 0;
                asm volatile("" : "+v"(first));
                if (wave_any(first)) {
                    const float d = row_max(s);
                    m = d;
#pragma unroll
                    for (int t = 0; t < 4; t++) s[t] -= f32x4_t{d, d, d, d};
                }
                float bs = exps(s);
                if (wave_any(bs > kLazySum)) {
                    scores(kb0, s);
                    const float d = fmaxf(row_max(s), 0.0f);
                    const float alpha = __builtin_amdgcn_exp2f(-d);
                    o0 *= alpha;
                    o1 *= alpha;
                    lsum *= alpha;
                    m += d;
#pragma unroll
                    for (int t = 0; t < 4; t++) s[t] -= f32x4_t{d, d, d, d};
                    bs = exps(s);
                }
                lsum += bs;
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    const _Float16 *vp = vp0 + kb0 + 32 * st;
                    const half8_t vah = *(const half8_t *)vp;
                    const half8_t val = *(const half8_t *)(vp + kVPlane);
                    const half8_t vbh = *(const half8_t *)(vp + 16 * V_LD);
                    const half8_t vbl = *(const half8_t *)(vp + kVPlane + 16 * V_LD);
                    half8_t ph, pl;
                    split_f32x8(f32x4_t{s[2 * st][0], s[2 * st][1], s[2 * st][2], s[2 * st][3]},
                                f32x4_t{s[2 * st + 1][0], s[2 * st + 1][1], s[2 * st + 1][2], s[2 * st + 1][3]},
                                ph, pl);
                    o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(val, ph, o0, 0, 0, 0);
                    o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vah, pl, o0, 0, 0, 0);
                    o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vah, ph, o0, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vbl, ph, o1, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vbh, pl, o1, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(vbh, ph, o1, 0, 0, 0);
                }
            }
            // the query's whole row sum, in every lane row
            const float total = sum_over_rows(lsum);
            if (qrow < L) {
                const float inv = 1.0f / total;
                float *dst = out + (size_t)(cur.start + qrow) * ld_out + cur.h * kHeadDim + 4 * g;
                *(f32x4_t *)dst = o0 * inv;
                *(f32x4_t *)(dst + 16) = o1 * inv;
            }
        }
        __syncthreads();  // every read of this item's planes precedes the next item's staging
        cur = nxt;
        j = jn;
    }
    // Each block takes exactly one index past the end, after its last item;
    // the last block to get here returns both counters to 0 for the next
    // launch (every take of this launch has happened by then).
    if (tid == 0 && atomicAdd(queue + 1, 1u) == gridDim.x - 1) {
        atomicExch(queue, 0u);
        atomicExch(queue + 1, 0u);
    }
}

}  // namespace

// qkv: [T, 3*hidden] (Q | K | V per token), out: [T, hidden], both f16 or
// both f32 (f32: the split-product kernel above).
// order: sequence ids (longest first) so the long blocks start early.
// num_cus: the f32 kernel's persistent grid (one workgroup per CU); queue:
// its work-queue counters (two, zero between launches: tzh_ctx_work_queue).
int tzh_attention_launch(hipStream_t st, int num_cus, unsigned *queue, const void *qkv, void *out, int32_t dtype,
                         const int *cu_seqlens, const int *order, int batch, int n_heads, int hidden) {
    if (hidden != n_heads * kHeadDim)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "attention kernel needs head_dim 32 (hidden %d, heads %d)", hidden,
                        n_heads);
    if (dtype != TZH_F16 && dtype != TZH_F32) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "attention needs F16 or F32");
    if (batch <= 0) return TZH_OK;
    const float scale = 1.0f / sqrtf((float)kHeadDim);  // arctic.zig:649
    const float scale_log2 = scale * 1.4426950408889634f;
    if (dtype == TZH_F32) {
        if (!queue) return tzh_fail(TZH_ERR_INVALID_ARGS, "internal: attention without its work queue");
        if ((int64_t)batch * n_heads > INT32_MAX) return tzh_fail(TZH_ERR_TOO_LARGE, "attention: too many (sequence, head) items");
        const int64_t blocks = std::min<int64_t>((int64_t)batch * n_heads, std::max(num_cus, 1));
        hipLaunchKernelGGL((attn_varlen_f32_kernel<kWavesF32>), dim3((unsigned)blocks), dim3(kWavesF32 * 64), 0, st,
                           (const float *)qkv, 3 * hidden, (float *)out, hidden, cu_seqlens, order, batch, n_heads,
                           hidden, scale_log2, queue);
        TZH_LAUNCHED("attn_varlen_f32_kernel");
        return TZH_OK;
    }
    // head-pair layout: 16 blocks per 8 (sequence, head pair)s
    const int64_t blocks = n_heads % 2 == 0 ? ((int64_t)batch * (n_heads / 2) + 7) / 8 * 16 : (int64_t)batch * n_heads;
    hipLaunchKernelGGL((attn_varlen_kernel<kWaves, kQueryTiles>), dim3((unsigned)blocks), dim3(kWaves * 64), 0, st,
                       (const _Float16 *)qkv, 3 * hidden, (_Float16 *)out, hidden, cu_seqlens, order, batch, n_heads,
                       hidden, scale_log2);
    TZH_LAUNCHED("attn_varlen_kernel");
    return TZH_OK;
}

extern "C" int tzh_attention_varlen(tzh_ctx *ctx, const void *qkv, void *out, int32_t dtype,
                                    const int32_t *cu_seqlens, int32_t batch, int32_t n_heads, int32_t hidden) {
    tzh_clear_error();
    TZH_TRY(tzh_ctx_enter(ctx));
    if (dtype != TZH_F16 && dtype != TZH_F32) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "attention needs F16 or F32");
    if (batch < 0 || n_heads <= 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad batch/heads");
    if (batch > 0 && (!qkv || !out || !cu_seqlens)) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    if (batch == 0) return TZH_OK;
    std::vector<int32_t> cu((size_t)batch + 1);
    TZH_HIP(hipMemcpyAsync(cu.data(), cu_seqlens, cu.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    TZH_HIP(hipStreamSynchronize(ctx->stream));
    if (cu[0] < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "cu_seqlens[0] is negative");
    for (int32_t b = 0; b < batch; b++) {
        const int32_t L = cu[(size_t)b + 1] - cu[(size_t)b];
        if (L < 1 || L > kMaxKeys)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "sequence %d has length %d (must be 1..%d)", b, L, kMaxKeys);
    }
    unsigned *queue = nullptr;
    TZH_TRY(tzh_ctx_work_queue(ctx, &queue));
    return tzh_attention_launch(ctx->stream, ctx->num_cus, queue, qkv, out, dtype, cu_seqlens, nullptr, batch, n_heads,
                                hidden);
}
