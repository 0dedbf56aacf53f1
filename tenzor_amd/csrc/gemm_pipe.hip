// K3: activations x int8-valued weight codes on MFMA, with the operand tiles
// streamed HBM/L2 -> LDS by the gfx950 direct-to-LDS loads
// (global_load_lds_dwordx4) through an NS-deep ring of stage buffers.
//
//   C[t, n] = epi( (sum_k X[t,k] * Wc[n,k]) * f32(scale[n]) + bias[n] )
//
// the sums of matmulTransposeB_f32_i8_rowScale_bias (matmul_w8a32.zig:14-57).
// Weight codes are exact in f16 (|q| <= 127).  f32 activations (the
// reference's arithmetic) are split into an f16 pair x = hi + lo + r: hi =
// f16(x), lo = f16(x - hi) (x - hi is exact in f32), |r| <= 2^-22 |x| for
// |x| >= 2^-3 and <= 2^-25 otherwise (split_f32x8), once per stage, in
// place in the LDS tile; both halves go through the MFMA against the same
// codes into one f32 accumulator, so every product is that of an f32
// operand to about 22 bits, summed in f32.  The split is valid for |x| <
// 65504 (the f16 range); f16 activations (the opt-in fast model path) take
// one MFMA.  Epilogues: bias, bias + GELU (arctic.zig:771-776),
// bias + residual + LayerNorm over the full 384-wide row (arctic.zig:716-746,
// layernorm.zig:26-117, two-pass mean / biased variance).
//
// Design:
//   - The MFMA computes C^T tiles (weights as the A operand, tokens as B):
//     each lane then owns four consecutive output columns of one token, so
//     a token's LayerNorm statistics reduce in registers, across the two
//     half-waves, then across the waves of the row in LDS.  f16 results
//     are turned into whole 64-byte row pieces through a wave-private LDS
//     tile before they are stored; f32 ones are stored as 16-byte vectors
//     straight from the accumulators.
//   - Persistent blocks (one per CU): the (row panel, column tile) work units
//     are dealt out XCD by XCD so that the column tiles of a row panel run
//     together on one XCD and share its L2, and the stage ring runs across
//     unit boundaries, so the next unit's tiles are already in flight while
//     a unit's epilogue runs.
//   - Each stage buffer is its own __shared__ array: the compiler can then
//     tell a read of stage s from the in-flight loads of stages s+1.. and
//     does not drain the ring before every LDS read.  Stage completion is
//     tracked with explicit vmcnt waits (in-order counter; every vector
//     memory op issued after a stage's loads is counted as still pending).
//   - Rows of each tile are 16-byte-chunk XOR-swizzled so that the sixteen
//     rows one ds_read_b128 cycle serves (16 lanes x 16 B = the 256 bytes of
//     the 64 LDS banks) land on sixteen different bank slots.
#include <type_traits>

#include "pipe.h"

namespace {

constexpr int kXcds = 8;  // MI355X: 8 XCDs of 32 CUs


typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Stores one 32-token x 32-column f16 fragment given in the MFMA D layout
// (this lane: token lane%32; element 4g+q is column 8g + 4*(lane/32) + q)
// as whole 64-byte row pieces.  Output rows are 16-byte chunks spread over
// 32 rows per store instruction otherwise, which costs the L2 one request
// per 16 bytes; here a swap between the half-waves gives each lane two
// complete 16-byte column chunks of its token, a wave-private 2 KiB LDS tile
// (chunks XOR-swizzled by row/4: conflict-free both ways) transposes them,
// and each store instruction writes sixteen full 64-byte rows.
//   ws: the wave's staging tile; dst: &C[t0][c0]; ld: row pitch (elements);
//   rows: how many of the 32 tokens lie inside the matrix.
// Issues two store instructions per lane (fewer where rows < 32).
__device__ __forceinline__ void store_frag_f16(char *ws, const float (&v)[16], _Float16 *dst, int ld, int rows) {
    const int lane = threadIdx.x & 63, l31 = lane & 31, half = lane >> 5;
    uint32_t pk[4][2];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const half2_t h0 = {(_Float16)v[4 * g], (_Float16)v[4 * g + 1]};
        const half2_t h1 = {(_Float16)v[4 * g + 2], (_Float16)v[4 * g + 3]};
        pk[g][0] = __builtin_bit_cast(uint32_t, h0);
        pk[g][1] = __builtin_bit_cast(uint32_t, h1);
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        // lower half-wave keeps group 2k and receives the upper one's;
        // upper half-wave keeps group 2k+1 and receives the lower one's
        uint32_t x0 = pk[2 * k][0], x1 = pk[2 * k][1], y0 = pk[2 * k + 1][0], y1 = pk[2 * k + 1][1];
        lane_swap32(x0, y0);
        lane_swap32(x1, y1);
        const int c = 2 * k + half;  // columns 8c .. 8c+7
        *(u32x4_t *)(ws + l31 * 64 + ((c ^ ((l31 >> 2) & 3)) << 4)) = u32x4_t{x0, x1, y0, y1};
    }
    wave_lds_order();
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int q = i * 64 + lane, row = q >> 2, c = q & 3;
        const u32x4_t d = *(const u32x4_t *)(ws + row * 64 + ((c ^ ((row >> 2) & 3)) << 4));
        if (row < rows) {
            *(u32x4_t *)(dst + (size_t)row * ld + c * 8) = d;
            vmem_store_issued();
        }
    }
    wave_lds_order();
}

// Stores one 32-token x 32-column f32 fragment given in the MFMA D layout
// (as store_frag_f16) as whole 128-byte row pieces: each lane writes its
// four 16-byte column chunks to a wave-private 4 KiB LDS tile (chunks
// XOR-swizzled by row/2: conflict-free both ways), and each of the four
// store instructions then writes eight complete rows.
//   ws: the wave's staging tile; dst: &C[t0][c0]; ld: row pitch (elements,
//   a multiple of 4 with dst 16-byte aligned); rows: how many of the 32
//   tokens lie inside the matrix.  Issues four store instructions per lane
//   (fewer where rows < 32).
__device__ __forceinline__ void store_frag_f32(char *ws, const f32x16_t &v, float *dst, int ld, int rows) {
    const int lane = threadIdx.x & 63, l31 = lane & 31, half = lane >> 5;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int c = 2 * g + half;  // columns 4c .. 4c+3
        *(f32x4_t *)(ws + l31 * 128 + ((c ^ ((l31 >> 1) & 7)) << 4)) =
            f32x4_t{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
    }
    wave_lds_order();
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int row = 8 * j + (lane >> 3), c = lane & 7;
        const f32x4_t d = *(const f32x4_t *)(ws + row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
        if (row < rows) {
            *(f32x4_t *)(dst + (size_t)row * ld + c * 4) = d;
            vmem_store_issued();
        }
    }
    wave_lds_order();
}

// Eight biased int8 weight codes (u = q + 128, little-endian in d0, d1) ->
// f16 q, exactly: v_perm_b32 makes each code the low mantissa byte of an f16
// with exponent 10 (bits 0x64uu = 1024 + u), and a packed f16 subtraction of
// 1152 = 1024 + 128 leaves q; every value is an integer below 2048, so
// nothing rounds.
__device__ __forceinline__ half8_t codes_to_f16(uint32_t d0, uint32_t d1) {
    const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    half8_t r;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t d = i ? d1 : d0;
        const half2_t lo = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, d, 0x04010400u)) - off;
        const half2_t hi = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, d, 0x04030402u)) - off;
        r[4 * i + 0] = lo[0];
        r[4 * i + 1] = lo[1];
        r[4 * i + 2] = hi[0];
        r[4 * i + 3] = hi[1];
    }
    return r;
}

// Tile of rows x ROW_BYTES (k contiguous) as laid out in LDS.
template <int ROW_BYTES_>
struct TileFmt {
    static constexpr int ROW_BYTES = ROW_BYTES_;
    static constexpr int CPR = ROW_BYTES / 16;    // 16-byte chunks per row
    static constexpr int RPI = 64 / CPR;          // rows per DMA instruction (64 lanes x 16 B)
    static constexpr int RPW = 256 / ROW_BYTES;   // rows sharing one 256-byte bank window
    __device__ static __forceinline__ int swz(int r) { return (r / RPW) & (CPR - 1); }
    // the swizzle of a DMA group's rows depends on the group index only
    // through its parity (128-byte rows: 8-row groups, 2 rows per window)
    static constexpr bool PARITY = (RPI / RPW) % CPR != 0;
};

// W8: the weight codes stay one byte each (biased, u = q + 128) in HBM and
// in LDS, which halves the weight stream, and are widened to f16 in
// registers after each fragment read.
// WTB > 0: the weight codes are stored stage-tiled: for each block of WTB
// rows (a multiple of BN) and each k stage, the WTB x BK codes are one
// contiguous span, rows BK codes apart (tile_codes_w8_kernel writes it), so
// a stage's weight tile is read from consecutive memory.
// The tiled layout's k stages are 64 codes wide (TK); a configuration with
// BK = 32 reads each tiled stage as two halves (rows TK codes apart in
// memory, BK codes per row in LDS).
template <int BM_, int BN_, int BK_, int WM_, int WN_, int NS_, bool W8_ = false, int WTB_ = 0, int XE_ = 2>
struct PipeCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, NS = NS_;
    static constexpr int XE = XE_;  // bytes per activation element: 2 (f16) or 4 (f32, split hi/lo)
    static constexpr bool W8 = W8_, WT = WTB_ > 0;
    static constexpr int WTB = WTB_ > 0 ? WTB_ : BN_;
    static_assert(WTB % BN_ == 0, "weight tile blocks hold whole column tiles");
    static constexpr int TK = 64;                          // k codes per tiled stage in memory
    static_assert(!WT || TK % BK_ == 0, "a k stage covers a whole part of a tiled stage");
    static constexpr int SPT = WT ? TK / BK_ : 1;           // k stages per tiled stage
    static constexpr int NW = WM * WN, THREADS = NW * 64;
    static constexpr int TMF = BM / WM / 32;  // token fragments per wave
    static constexpr int TNF = BN / WN / 32;  // weight fragments per wave
    static constexpr int WEB = W8 ? 1 : 2;    // bytes per weight code
    using FX = TileFmt<BK * XE>;
    using FW = TileFmt<BK * WEB>;
    static_assert(!W8 || BK % 32 == 0, "int8 weights: whole 16-byte chunks per half-wave");
    static constexpr int X_BYTES = BM * BK * XE, W_BYTES = BN * BK * WEB, STAGE = X_BYTES + W_BYTES;
    static constexpr int XG = BM / FX::RPI, WG = BN / FW::RPI;  // DMA instructions per tile
    static constexpr int LX = XG / NW, LW = WG / NW, L = LX + LW;
    static_assert(XG % NW == 0 && WG % NW == 0, "DMA groups must split evenly over the waves");
    static_assert(TMF >= 1 && TNF >= 1, "wave tile too small");
    static_assert(NS >= 2 && NS <= 4, "2..4 stages");
    // LDS of one block (stage ring + parameter table + LayerNorm statistics
    // + per-wave output staging tiles) and how many such blocks a CU's
    // 160 KiB holds
    // (staged: output through per-wave LDS tiles, 2 KiB for f16 output and
    // 4 KiB for f32 output of f32-activation configurations)
    static constexpr int stage_tile(bool staged, bool f32_out) {
        return !staged ? 16 : f32_out ? (XE == 4 ? NW * 4096 : 16) : NW * 2048;
    }
    static constexpr int lds_bytes(bool ln, bool staged = true, bool f32_out = false) {
        return NS * STAGE + (ln ? 4 * BN * 4 + 2 * BM * WN * 4 : 2 * 1536 * 4) + stage_tile(staged, f32_out);
    }
    static constexpr int blocks_per_cu(bool ln, bool staged = true, bool f32_out = false) {
        return 163840 / lds_bytes(ln, staged, f32_out) > 2 ? 2 : 163840 / lds_bytes(ln, staged, f32_out);
    }
};


// Wait until at most L*A + E vector memory ops are outstanding, A chosen at
// run time from {0..AMAX} (the largest A <= ahead) and E from {0, E1, E2}
// (extra = 0, 1, 2).  On gfx9 every vector memory op (loads, stores,
// direct-to-LDS loads) retires from vmcnt in issue order, so when at least
// L*A + E ops were issued after a stage's loads, this guarantees that stage
// has landed.  E counts the epilogue's own loads and stores issued after
// them: without it the ring would wait for those too.
template <int AMAX, int L, int E1, int E2>
__device__ __forceinline__ void wait_stage(int ahead, int extra) {
    if constexpr (AMAX == 0) {
        if (extra == 2)
            wait_vm_lgkm0<E2>();
        else if (extra == 1)
            wait_vm_lgkm0<E1>();
        else
            wait_vm_lgkm0<0>();
    } else {
        if (ahead >= AMAX) {
            if (extra == 2)
                wait_vm_lgkm0<L * AMAX + E2>();
            else if (extra == 1)
                wait_vm_lgkm0<L * AMAX + E1>();
            else
                wait_vm_lgkm0<L * AMAX>();
        } else {
            wait_stage<AMAX - 1, L, E1, E2>(ahead, extra);
        }
    }
}

template <typename TC>
__device__ __forceinline__ void store4(TC *p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<_Float16>(_Float16 *p, float a, float b, float c, float d) {
    half4_t h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
    *(half4_t *)p = h;
}
template <>
__device__ __forceinline__ void store4<float>(float *p, float a, float b, float c, float d) {
    *(f32x4_t *)p = f32x4_t{a, b, c, d};
}

// EPI_RES: bias + residual without the LayerNorm, stored as f32: the
// pre-normalisation rows of a split LayerNorm tile (see launch_ln).
enum { EPI_BIAS = 0, EPI_GELU = 1, EPI_LN = 2, EPI_RES = 3 };

// Row scaling (RS; f32 activations only).  Each activation row enters the
// split as X[t,:] * 2^e with e an exact power-of-two exponent per row and
// unit, chosen online: the split of a stage takes the row's largest
// magnitude M over that stage (the eight lanes that hold the row's 64
// values reduce it), and the row's first stage with M > 0 sets e so that
// M 2^e lies in [2^14, 2^15); a later stage whose maximum would reach 2^15
// at the current e lowers e to that stage's choice.  Every stage's e goes
// to LDS (a ring of three), and each wave that accumulates the row
// multiplies its sums by 2^(e_new - e_old) when e drops, before that
// stage's MFMAs (exact: a power of two); the epilogue multiplies the sums by
// 2^-e.  So the hi/lo split keeps its 2^-22 relative residual for every
// value within 2^17 of the row's largest so far, whatever the row's scale,
// no finite row overflows the f16 halves, and the sums are f32 sums of the
// products.  A row's inf or NaN reaches the sums as NaN.
template <int EPI, typename TC, typename P, typename TR = TC, typename TX = _Float16, bool RS = false>
__global__ void __launch_bounds__(P::THREADS) linear_pipe_kernel(
    const TX *__restrict__ X, const void *__restrict__ Wc, const uint16_t *__restrict__ scale,
    const float *__restrict__ bias, TC *__restrict__ C, int M, int K, int N, const TR *__restrict__ R,
    const float *__restrict__ gamma, const float *__restrict__ beta, float eps, int ldc, int n_valid) {
    using FX = typename P::FX;
    using FW = typename P::FW;
    constexpr int BM = P::BM, BN = P::BN, BK = P::BK, NS = P::NS, TMF = P::TMF, TNF = P::TNF;
    constexpr int XROWB = FX::ROW_BYTES, WROWB = FW::ROW_BYTES, WEB = P::WEB;
    constexpr bool W8 = P::W8;
    constexpr int XE = (int)sizeof(TX);
    constexpr bool XF32 = XE == 4;
    static_assert(XE == P::XE, "configuration built for another activation type");
    static_assert(!RS || XF32, "row scaling is for f32 activations");
    constexpr bool LN = EPI == EPI_LN;
    static_assert(!LN || P::WN * TNF * 32 == BN, "LayerNorm tiles cover whole rows");
    constexpr int NPAR = LN ? 4 : 2;                        // per-column parameters kept in LDS
    constexpr int MAXN = LN ? BN : 1536;

    __shared__ __attribute__((aligned(16))) char st0[P::STAGE];
    __shared__ __attribute__((aligned(16))) char st1[P::STAGE];
    __shared__ __attribute__((aligned(16))) char st2[NS > 2 ? P::STAGE : 16];
    __shared__ __attribute__((aligned(16))) char st3[NS > 3 ? P::STAGE : 16];
    __shared__ __attribute__((aligned(16))) float par[NPAR][MAXN];
    __shared__ float stat0[LN ? BM * P::WN : 1], stat1[LN ? BM * P::WN : 1];
    // RS: the row exponents stage t was split with, in slot t % 3 (written by
    // the split of stage t in step t - 1; read in step t by the waves that
    // multiply the stage, by the split of stage t + 1 (which writes slot
    // (t + 1) % 3) and, at a unit's last stage, by its epilogue)
    constexpr int kUnset = -100000;  // no nonzero value in the row yet (its sums are exact zeros)
    __shared__ int e_st[RS ? 3 : 1][RS ? BM : 1];
    // f16 output goes through LDS, except from the f32-activation LayerNorm
    // kernel, which has no registers to spare for the staging
    constexpr bool STAGED = std::is_same<TC, _Float16>::value && !(XF32 && LN);
    // f32 output of the bias epilogues of the f32-activation configurations
    // too (whole 128-byte row pieces per store instruction), for units whose
    // columns all exist.  Not the LayerNorm epilogue: its 384 output columns
    // are a small share of its traffic, and the staging would spill registers.
    constexpr bool STAGED32 = std::is_same<TC, float>::value && P::XE == 4 && EPI != EPI_RES && EPI != EPI_LN;
    __shared__ __attribute__((aligned(16))) char epi_ws[P::stage_tile(STAGED || STAGED32, STAGED32)];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w / P::WN, wn = w % P::WN;
    const int KT = K / BK;
    const bool cvec = (ldc & 3) == 0 && ((uintptr_t)C & 15) == 0;
    const int nbn = N / BN;  // column tiles per row panel (1 with the LayerNorm epilogue)
    // Work units are (row panel, column tile) pairs.  Workgroups go to the
    // XCDs round-robin (block b on XCD b % 8) and each XCD has its own L2.
    // Panel p belongs to XCD p % 8, and an XCD's units, column tile fastest,
    // are dealt to its blocks one per block per round: the column tiles of a
    // panel run at the same time on one XCD, so its activations come from
    // HBM once and from L2 for the other tiles.  Unit i of this block is
    // j = slot + i * spx of its XCD.
    const int nxcd = gridDim.x % kXcds == 0 ? kXcds : 1;
    const int xcd = blockIdx.x % nxcd, spx = gridDim.x / nxcd, slot = blockIdx.x / nxcd;
    const int panels = (M + BM - 1) / BM;
    const int xunits = (panels - xcd + nxcd - 1) / nxcd * nbn;  // units of this XCD
    const int count = slot < xunits ? (xunits - slot + spx - 1) / spx : 0;
    const int S = count * KT;
    auto unit_m0 = [&](int i) __attribute__((always_inline)) {
        return ((slot + i * spx) / nbn * nxcd + xcd) * BM;
    };
    auto unit_n0 = [&](int i) __attribute__((always_inline)) { return (slot + i * spx) % nbn * BN; };

    // per-column parameters -> LDS (visible after the first stage barrier)
    // Columns n_valid .. N-1 are padding (zero codes): their parameters are
    // never read from memory and their outputs never stored.
    for (int i = tid; i < N; i += P::THREADS) {
        par[0][i] = i < n_valid ? f16_bits_to_f32(scale[i]) : 0.0f;
        par[1][i] = bias && i < n_valid ? bias[i] : 0.0f;
        if constexpr (LN) {
            par[2][i] = gamma[i];
            par[3][i] = beta[i];
        }
    }

    // --- DMA issue state -------------------------------------------------
    // Each lane fetches one 16-byte chunk per DMA instruction: source address
    // = wave-uniform row base (scalar) + a small per-lane byte offset.
    const int wu = __builtin_amdgcn_readfirstlane(w);                // wave index, uniform
    const int r_in = lane / FX::CPR;                                 // row inside an X DMA group
    const int rw_in = lane / FW::CPR;                                // row inside a W DMA group
    const int wchunk_e = (lane % FW::CPR) ^ FW::swz(rw_in);
    const int wchunk_o = (lane % FW::CPR) ^ FW::swz(FW::RPI + rw_in);
    constexpr int WTROWB = P::TK * WEB;           // bytes per row of a tiled stage in memory
    const int w_pitch = P::WT ? WTROWB : K * WEB;  // bytes between weight rows in memory
    const uint32_t w_loff_e = (uint32_t)(rw_in * w_pitch + wchunk_e * 16);  // bytes, same for every unit
    const uint32_t w_loff_o = (uint32_t)(rw_in * w_pitch + wchunk_o * 16);
    const char *const Xb = (const char *)X;
    const char *const Wb = (const char *)Wc;
    int iu = 0, ikt = 0;                                             // next stage to issue
    int x_row0[P::LX];                                               // uniform first row of each X group
    uint32_t x_loff[P::LX];                                          // per-lane byte offset (row clamp)
    const char *w_unit = nullptr;                                    // uniform: first W row of the wave
    auto set_unit = [&](int i) __attribute__((always_inline)) {
        const int m0 = unit_m0(i), n0 = unit_n0(i);
#pragma unroll
        for (int i = 0; i < P::LX; i++) {
            int r0 = m0 + (wu * P::LX + i) * FX::RPI;
            r0 = r0 < M ? r0 : M - 1;
            const int r = r0 + r_in < M ? r0 + r_in : M - 1;
            x_row0[i] = r0;
            // logical 16-byte chunk that lands at this lane's slot of its tile row
            const int chunk = (lane % FX::CPR) ^ FX::swz((wu * P::LX + i) * FX::RPI + r_in);
            x_loff[i] = (uint32_t)((r - r0) * K * XE + chunk * 16);
        }
        w_unit = P::WT ? Wb + (size_t)(n0 / P::WTB) * K * P::WTB * WEB +
                             (size_t)(n0 % P::WTB + wu * P::LW * FW::RPI) * WTROWB
                       : Wb + (size_t)(n0 + wu * P::LW * FW::RPI) * K * WEB;
    };
    // A stage's loads: this wave's X pieces (i < LX) and weight pieces
    // (i < LW), then the advance to the next stage's position.
    auto issue_x = [&](char *buf, int i) __attribute__((always_inline)) {
        dma16(Xb + ((size_t)x_row0[i] * K * XE + (size_t)ikt * BK * XE), x_loff[i],
              buf + (wu * P::LX + i) * FX::RPI * XROWB);
    };
    auto issue_w = [&](char *buf, int i) __attribute__((always_inline)) {
        dma16(w_unit + (P::WT ? (size_t)(ikt / P::SPT) * P::WTB * WTROWB + (size_t)(ikt % P::SPT) * WROWB +
                                    (size_t)i * FW::RPI * WTROWB
                              : (size_t)i * FW::RPI * K * WEB + (size_t)ikt * BK * WEB),
              (FW::PARITY && ((wu * P::LW + i) & 1)) ? w_loff_o : w_loff_e,
              buf + P::X_BYTES + (wu * P::LW + i) * FW::RPI * WROWB);
    };
    auto advance = [&]() __attribute__((always_inline)) {
        if (++ikt == KT) {
            ikt = 0;
            if (++iu < count) set_unit(iu);
        }
    };
    auto issue = [&](char *buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < P::LX; i++) issue_x(buf, i);
#pragma unroll
        for (int i = 0; i < P::LW; i++) issue_w(buf, i);
        advance();
    };

    // --- fragment read offsets -------------------------------------------
    const int l31 = lane & 31, half = lane >> 5;
    // The MFMA takes 8 k-values per lane (lanes 32..63 the upper 8 of its 16).
    // f16 weights: MFMA ks of a stage covers k = 16 ks .. 16 ks + 15.  int8
    // weights: a 16-byte read holds 16 codes, so half-wave h takes k = 32 h +
    // 8 ks .. 32 h + 8 ks + 7 in MFMA ks (BK = 64; BK = 32: 16 h + 8 ks), the
    // X operand following the same k.
    // f32 activations: the 8 k-values are two 16-byte chunks, 2 cx and 2 cx + 1.
    const int fx = FX::swz(l31), fw = FW::swz(l31);
    int xoff[BK / 16], xoff1[BK / 16], woff[BK / 16];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) {
        const int cx = W8 ? (BK / 16) * half + ks : 2 * ks + half;
        const int row = (wm * TMF * 32 + l31) * XROWB;
        xoff[ks] = row + (((XF32 ? 2 * cx : cx) ^ fx) << 4);
        xoff1[ks] = row + (((2 * cx + 1) ^ fx) << 4);
        const int cw = W8 ? (BK / 32) * half + ks / 2 : 2 * ks + half;  // W8: ks and ks+1 share a read
        woff[ks] = P::X_BYTES + (wn * TNF * 32 + l31) * WROWB + ((cw ^ fw) << 4);
    }

    f32x16_t acc[TNF][TMF];
#pragma unroll
    for (int a = 0; a < TNF; a++)
#pragma unroll
        for (int b = 0; b < TMF; b++) acc[a][b] = f32x16_t{};

    // f32 activations: each wave splits, in place, the X rows its own DMA
    // groups loaded (rows wu*LX*RPI .. +LX*RPI), once its own loads of the
    // stage have landed, in the step before the one that reads them; that
    // step's barrier then makes them visible to every wave.
    // Each 32-byte group of 8 consecutive k of a row, logical chunks 2p and
    // 2p+1, becomes hi in chunk 2p and lo in chunk 2p+1; eight lanes take
    // the eight groups of one row.
    auto split_own = [&](char *buf, int t) __attribute__((always_inline)) {
        if constexpr (XF32) {
            constexpr int GPR = BK / 8, ROWS_W = P::LX * FX::RPI;
            static_assert((ROWS_W * GPR) % 64 == 0, "whole groups per lane");
            // the offsets are recomputed here (a few VALU ops) rather than
            // kept in registers across the whole kernel
            int ln = lane;
            asm volatile("" : "+v"(ln));
#pragma unroll
            for (int c = 0; c < ROWS_W * GPR / 64; c++) {
                const int g = c * 64 + ln, r = wu * ROWS_W + g / GPR, p = g % GPR;
                char *row = buf + r * XROWB;
                f32x4_t *c0 = (f32x4_t *)(row + (((2 * p) ^ FX::swz(r)) << 4));
                f32x4_t *c1 = (f32x4_t *)(row + (((2 * p + 1) ^ FX::swz(r)) << 4));
                f32x4_t x0 = *c0, x1 = *c1;
                if constexpr (RS) {
                    // the row's largest magnitude over this stage: the GPR
                    // consecutive lanes that hold its groups of eight
                    float mx = fmaxf(fmaxf(fmaxf(fabsf(x0[0]), fabsf(x0[1])), fmaxf(fabsf(x0[2]), fabsf(x0[3]))),
                                     fmaxf(fmaxf(fabsf(x1[0]), fabsf(x1[1])), fmaxf(fabsf(x1[2]), fabsf(x1[3]))));
                    static_assert(GPR == 4 || GPR == 8, "a row's lanes: a quad or an aligned group of eight");
                    mx = fmaxf(mx, dpp_f32<0xB1>(mx));  // lane ^ 1
                    mx = fmaxf(mx, dpp_f32<0x4E>(mx));  // lane ^ 2
                    if constexpr (GPR == 8) mx = fmaxf(mx, dpp_f32<0x141>(mx));  // the other quad of the eight
                    const int prev = t % KT == 0 ? kUnset : e_st[(t + 2) % 3][r];
                    int e = prev;
                    if (mx > 0.0f && mx < INFINITY) {  // zero, inf and NaN rows keep theirs
                        const int want = 15 - __builtin_amdgcn_frexp_expf(mx);  // mx 2^want in [2^14, 2^15)
                        e = prev == kUnset || want < prev ? want : prev;
                    }
                    if (p == 0) e_st[t % 3][r] = e;
                    const int es = e == kUnset ? 0 : e;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        x0[q] = __builtin_amdgcn_ldexpf(x0[q], es);
                        x1[q] = __builtin_amdgcn_ldexpf(x1[q], es);
                    }
                }
                half8_t hi, lo;
                split_f32x8(x0, x1, hi, lo);
                *(half8_t *)c0 = hi;
                *(half8_t *)c1 = lo;
            }
        }
    };
    // nb: the stage buffer whose loads are issued during this compute, spread
    // over its first KS k steps (f32 activations: issued back to back after
    // the barrier, every wave's loads at once, the issue took 14 % of the
    // GEMM; spread over two steps FFN1 went from 231 to 224 us, over three
    // 221 -> 224 and over four the two-stage ring waited for them; f16
    // activations: all at the first step, spreading measured 2 % slower);
    // null: none
    constexpr int KS = XF32 ? 2 : 1;
    constexpr int XPER = (P::LX + KS - 1) / KS, WPER = (P::LW + KS - 1) / KS;
    auto compute = [&](const char *buf, char *nb, int t) __attribute__((always_inline)) {
        if constexpr (RS)
            if (t % KT != 0) {
                // a row whose exponent dropped at stage t: its sums so far
                // times 2^(e_t - e_{t-1}), before this stage's products
#pragma unroll
                for (int b = 0; b < TMF; b++) {
                    const int row = wm * TMF * 32 + b * 32 + l31;
                    const int en = e_st[t % 3][row], ep = e_st[(t + 2) % 3][row];
                    const int d = ep != kUnset && en != ep ? en - ep : 0;
                    if (wave_any(d != 0))
#pragma unroll
                        for (int a = 0; a < TNF; a++)
#pragma unroll
                            for (int q = 0; q < 16; q++) acc[a][b][q] = __builtin_amdgcn_ldexpf(acc[a][b][q], d);
                }
            }
        u32x4_t wraw[TNF];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            if (nb && ks < KS) {
#pragma unroll
                for (int i = ks * XPER; i < (ks + 1) * XPER; i++)
                    if (i < P::LX) issue_x(nb, i);
#pragma unroll
                for (int i = ks * WPER; i < (ks + 1) * WPER; i++)
                    if (i < P::LW) issue_w(nb, i);
            }
            half8_t xf[TMF], xl[TMF], wf[TNF];
#pragma unroll
            for (int b = 0; b < TMF; b++) {
                xf[b] = *(const half8_t *)(buf + xoff[ks] + b * 32 * XROWB);
                if constexpr (XF32) xl[b] = *(const half8_t *)(buf + xoff1[ks] + b * 32 * XROWB);
            }
#pragma unroll
            for (int a = 0; a < TNF; a++) {
                if constexpr (W8) {
                    if (ks % 2 == 0) wraw[a] = *(const u32x4_t *)(buf + woff[ks] + a * 32 * WROWB);
                    wf[a] = codes_to_f16(wraw[a][2 * (ks % 2)], wraw[a][2 * (ks % 2) + 1]);
                } else {
                    wf[a] = *(const half8_t *)(buf + woff[ks] + a * 32 * WROWB);
                }
            }
#pragma unroll
            for (int a = 0; a < TNF; a++)
#pragma unroll
                for (int b = 0; b < TMF; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[a], xf[b], acc[a][b], 0, 0, 0);
            if constexpr (XF32) {
#pragma unroll
                for (int a = 0; a < TNF; a++)
#pragma unroll
                    for (int b = 0; b < TMF; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[a], xl[b], acc[a][b], 0, 0, 0);
            }
        }
    };

    using RV = std::conditional_t<std::is_same<TC, float>::value, f32x4_t, half4_t>;


    auto epilogue = [&](int i) __attribute__((always_inline)) {
        const int m0 = unit_m0(i), n0 = unit_n0(i);
        const bool st32 = STAGED32 && cvec && n0 + BN <= n_valid;  // uniform
        // RS: the sums of token fragment b times 2^-e of its row (the
        // exponent of the unit's last stage)
        const int tl = (i + 1) * KT - 1;
        auto neg_e = [&](int b) __attribute__((always_inline)) {
            const int e = RS ? e_st[tl % 3][wm * TMF * 32 + b * 32 + l31] : 0;
            return e == kUnset ? 0 : -e;
        };
        auto unscale = [&](int b) __attribute__((always_inline)) {
            if constexpr (RS) {
                const int e = neg_e(b);
#pragma unroll
                for (int a = 0; a < TNF; a++)
#pragma unroll
                    for (int q = 0; q < 16; q++) acc[a][b][q] = __builtin_amdgcn_ldexpf(acc[a][b][q], e);
            }
        };
        if constexpr (!LN) {
#pragma unroll
            for (int b = 0; b < TMF; b++) {
                unscale(b);
                const int t = m0 + wm * TMF * 32 + b * 32 + l31;
#pragma unroll
                for (int a = 0; a < TNF; a++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int n = n0 + wn * TNF * 32 + a * 32 + 8 * g + 4 * half;
                        const f32x4_t s = *(const f32x4_t *)&par[0][n];
                        const f32x4_t bb = *(const f32x4_t *)&par[1][n];
                        float v[4];
                        using RV4 = std::conditional_t<std::is_same<TR, float>::value, f32x4_t, half4_t>;
                        RV4 res = {};
                        if constexpr (EPI == EPI_RES) {
                            res = *(const RV4 *)(R + (size_t)(t < M ? t : M - 1) * N + n);
                            vmem_load_issued();
                        }
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            v[q] = acc[a][b][4 * g + q] * s[q] + bb[q];  // sum * s + bias (matmul_w8a32.zig:55)
                            if (EPI == EPI_GELU) v[q] = gelu_fast(v[q]);
                            // input + (sum * s + bias), as the LayerNorm epilogue forms it
                            if (EPI == EPI_RES) v[q] = (float)res[q] + v[q];
                            if constexpr (STAGED || STAGED32) acc[a][b][4 * g + q] = v[q];
                        }
                        if constexpr (!STAGED)
                            if (!st32 && t < M && n < n_valid) {
                                // 16-byte stores where rows keep that alignment; more store
                                // instructions than the stage waits count only make them wait longer
                                if (cvec && n + 4 <= n_valid) {
                                    store4<TC>(C + (size_t)t * ldc + n, v[0], v[1], v[2], v[3]);
                                } else {
#pragma unroll
                                    for (int q = 0; q < 4; q++)
                                        if (n + q < n_valid) C[(size_t)t * ldc + n + q] = (TC)v[q];
                                }
                                vmem_store_issued();
                            }
                    }
                if constexpr (STAGED) {
                    const int t0 = m0 + wm * TMF * 32 + b * 32;
#pragma unroll
                    for (int a = 0; a < TNF; a++) {
                        float v[16];
#pragma unroll
                        for (int e = 0; e < 16; e++) v[e] = acc[a][b][e];
                        store_frag_f16(epi_ws + w * 2048, v, (_Float16 *)C + (size_t)t0 * ldc + n0 + wn * TNF * 32 + a * 32,
                                       ldc, M - t0);
                    }
                }
                if constexpr (STAGED32)
                    if (st32) {
                        const int t0 = m0 + wm * TMF * 32 + b * 32;
#pragma unroll
                        for (int a = 0; a < TNF; a++)
                            store_frag_f32(epi_ws + w * 4096, acc[a][b],
                                           (float *)C + (size_t)t0 * ldc + n0 + wn * TNF * 32 + a * 32, ldc, M - t0);
                    }
            }
        } else {
            float part[TMF];
#pragma unroll
            for (int b = 0; b < TMF; b++) {
                // the residual is loaded one weight fragment at a time so that
                // the live registers stay within budget (no scratch spills)
                int t = m0 + wm * TMF * 32 + b * 32 + l31;
                t = t < M ? t : M - 1;
                // RS: the sums times 2^-e of the fragment's row
                const int ne = neg_e(b);
                float sum = 0.0f;
#pragma unroll
                for (int a = 0; a < TNF; a++) {
                    RV res[4];
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        res[g] = *(const RV *)(R + (size_t)t * BN + wn * TNF * 32 + a * 32 + 8 * g + 4 * half);
                        vmem_load_issued();
                    }
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int n = wn * TNF * 32 + a * 32 + 8 * g + 4 * half;
                        const f32x4_t s = *(const f32x4_t *)&par[0][n];
                        const f32x4_t bb = *(const f32x4_t *)&par[1][n];
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            // input + (sum * s + bias)  (arctic.zig:720)
                            const float acc_v = RS ? __builtin_amdgcn_ldexpf(acc[a][b][4 * g + q], ne)
                                                   : acc[a][b][4 * g + q];
                            const float v = (float)res[g][q] + (acc_v * s[q] + bb[q]);
                            acc[a][b][4 * g + q] = v;
                            sum += v;
                        }
                    }
                }
                part[b] = sum + __shfl_xor(sum, 32, 64);
            }
            if (half == 0)
#pragma unroll
                for (int b = 0; b < TMF; b++) stat0[(wm * TMF * 32 + b * 32 + l31) * P::WN + wn] = part[b];
            lds_barrier();
            float mean[TMF];
#pragma unroll
            for (int b = 0; b < TMF; b++) {
                const float *sp = &stat0[(wm * TMF * 32 + b * 32 + l31) * P::WN];
                float tot = 0.0f;
#pragma unroll
                for (int j = 0; j < P::WN; j++) tot += sp[j];
                mean[b] = tot / (float)BN;
                float sq = 0.0f;
#pragma unroll
                for (int a = 0; a < TNF; a++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const float d = acc[a][b][e] - mean[b];
                        sq += d * d;
                    }
                part[b] = sq + __shfl_xor(sq, 32, 64);
            }
            if (half == 0)
#pragma unroll
                for (int b = 0; b < TMF; b++) stat1[(wm * TMF * 32 + b * 32 + l31) * P::WN + wn] = part[b];
            lds_barrier();
#pragma unroll
            for (int b = 0; b < TMF; b++) {
                const float *sp = &stat1[(wm * TMF * 32 + b * 32 + l31) * P::WN];
                float tot = 0.0f;
#pragma unroll
                for (int j = 0; j < P::WN; j++) tot += sp[j];
                const float inv_std = 1.0f / sqrtf(tot / (float)BN + eps);
                const int t = m0 + wm * TMF * 32 + b * 32 + l31;
#pragma unroll
                for (int a = 0; a < TNF; a++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const int n = wn * TNF * 32 + a * 32 + 8 * g + 4 * half;
                        const f32x4_t gg = *(const f32x4_t *)&par[2][n];
                        const f32x4_t bt = *(const f32x4_t *)&par[3][n];
                        float y[4];
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            y[q] = ((acc[a][b][4 * g + q] - mean[b]) * inv_std) * gg[q] + bt[q];
                            if constexpr (STAGED || STAGED32) acc[a][b][4 * g + q] = y[q];
                        }
                        if constexpr (!STAGED)
                            if (t < M) {
                                store4<TC>(C + (size_t)t * BN + n, y[0], y[1], y[2], y[3]);
                                vmem_store_issued();
                            }
                    }
                if constexpr (STAGED) {
                    const int t0 = m0 + wm * TMF * 32 + b * 32;
#pragma unroll
                    for (int a = 0; a < TNF; a++) {
                        float v[16];
#pragma unroll
                        for (int e = 0; e < 16; e++) v[e] = acc[a][b][e];
                        store_frag_f16(epi_ws + w * 2048, v, (_Float16 *)C + (size_t)t0 * BN + wn * TNF * 32 + a * 32,
                                       BN, M - t0);
                    }
                }

            }
        }
#pragma unroll
        for (int a = 0; a < TNF; a++)
#pragma unroll
            for (int b = 0; b < TMF; b++) acc[a][b] = f32x16_t{};
    };

    if (S == 0) return;
    set_unit(0);
    char *const bufs[4] = {st0, st1, st2, st3};
    // prologue: stages 0 .. NS-2
#pragma unroll
    for (int j = 0; j < NS - 1; j++)
        if (j < S) issue(bufs[j]);

    // The most recent epilogue issued, after the loads of stages up to
    // last_epi + NS - 1: its residual loads (one per lane, token fragment,
    // weight fragment and 4-column group; always issued, rows clamped to M)
    // and its stores (two 16-byte stores of staged f16 rows per token and
    // weight fragment, or one per 4-column group of f32), the stores all
    // issued exactly when the unit lies inside M (no lane of any store is
    // masked off), and only then counted.
    constexpr int EPI_LOADS = (LN || EPI == EPI_RES) ? TMF * TNF * 4 : 0;
    constexpr int EPI_STORES = TMF * TNF * (STAGED ? 2 : 4);
    int last_epi = -NS;
    bool last_full = false;
    // own loads of stage t landed (and own LDS reads done): at most the
    // loads of the stages issued after t and the epilogue ops issued after
    // them still outstanding
    auto wait_own = [&](int t) __attribute__((always_inline)) {
        wait_stage<NS - 2, P::L, EPI_LOADS, EPI_LOADS + EPI_STORES>(
            min(NS - 2, S - 1 - t), last_epi >= t - NS + 1 ? (last_full ? 2 : 1) : 0);
    };
    if constexpr (XF32) {
        wait_own(0);
        wave_lds_order();
        split_own(bufs[0], 0);
    }
    auto step = [&](auto jc, int s) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        if constexpr (XF32)
            __builtin_amdgcn_s_waitcnt(0xC07F);  // own split writes done (own loads of s waited for and split)
        else
            wait_own(s);
        lds_barrier_only();  // every wave's stage s landed (and split); stage s-1 fully read
        const int kt = s % KT;
        const bool more = s + NS - 1 < S;
        compute(bufs[j], more ? bufs[(j + NS - 1) % NS] : nullptr, s);
        if (more) advance();
        // (before this step's epilogue, whose stores the wait would
        // otherwise include, and whose registers the split would add to)
        if constexpr (XF32)
            if (s + 1 < S) {
                wait_own(s + 1);
                wave_lds_order();  // the lanes read slots their neighbours' loads wrote
                split_own(bufs[(j + 1) % NS], s + 1);
            }
        if (kt == KT - 1) {
            const int i = s / KT;
            epilogue(i);
            last_epi = s;
            last_full = unit_m0(i) + BM <= M && unit_n0(i) + BN <= n_valid;
        }
    };
    for (int s = 0; s < S; s += NS) {
        step(std::integral_constant<int, 0>{}, s);
        if (s + 1 < S) step(std::integral_constant<int, 1>{}, s + 1);
        if constexpr (NS > 2)
            if (s + 2 < S) step(std::integral_constant<int, 2>{}, s + 2);
        if constexpr (NS > 3)
            if (s + 3 < S) step(std::integral_constant<int, 3>{}, s + 3);
    }
}

// Tile shapes (tokens x output columns x k per stage, waves, stages), chosen
// by measurement on MI355X at the Arctic shapes (T = 67590 tokens), per
// activation type, for the weight format TZH_WF_W8T: biased int8 codes u =
// q + 128, stage-tiled in 384-row blocks (tile_codes_w8_kernel; n a
// multiple of 384).  Against f16 codes in row-major [n, k], half the weight
// bytes and one contiguous span per stage let a third stage fit in LDS:
// QKV 78 -> 73, FFN1 118 -> 114, FFN2 + LN 106 -> 98 us at T = 65536.
// 128 x 384 tiles halve the L2 -> LDS operand traffic of 128 x 128 ones.
// The pieces cut a partial last round of a LayerNorm GEMM (12, 6 or 3 per
// 128 x 384 tile; see launch_ln).  f32 activations double the X tile, so
// their configurations keep two stages of 128 x 384 x 64 (112 KiB).
constexpr int kWtBlock = 384;  // rows per stage-tiled weight block
template <int WF, int XE>
struct Cfgs;
template <>
struct Cfgs<TZH_WF_W8T, 2> {
    using Bias = PipeCfg<128, 384, 64, 2, 4, 3, true, kWtBlock>;
    using Narrow = Bias;  // n is always a multiple of 384
    using Ln = Bias;
    // short-k LayerNorm GEMMs (k <= 384): 64-row tiles of 4 waves, two
    // workgroups per CU.  One workgroup's epilogue then overlaps the other's
    // main loop, and a CU whose second workgroup has run out of tiles runs
    // the last one alone at full speed, so a partial last round costs
    // little.  Measured against Ln with the split last round: O-proj + LN
    // 0.67-0.98 of the time at T = 4096 .. 100000 (55 -> 43 us at the
    // headline's 67590); with k = 1536 it is slower at some sizes.
    using LnShortK = PipeCfg<64, 384, 64, 1, 4, 2, true, kWtBlock>;
    using Piece64 = PipeCfg<64, 64, 64, 2, 2, 4, true, kWtBlock>;
    using Piece128x64 = PipeCfg<128, 64, 64, 2, 2, 4, true, kWtBlock>;
    using Piece128 = PipeCfg<128, 128, 64, 2, 2, 4, true, kWtBlock>;
};
template <>
struct Cfgs<TZH_WF_W8T, 4> {
    using Bias = PipeCfg<128, 384, 64, 2, 4, 2, true, kWtBlock, 4>;
    using Ln = Bias;
    // k <= 384 (the O-projection): two 4-wave workgroups of 64 x 384 tiles
    // per CU, as for f16 activations; with f32 activations two of them fit
    // in LDS only with 32-wide k stages (3 x 20 KiB each).  99.9 -> 95.4 us
    // at the headline's T = 67590; for k = 1536 and the bias GEMMs the same
    // layout measured slower (FFN2 + LN 228 -> 232 us, FFN1 224 -> 257, QKV
    // 165 -> 187), so those keep the 8-wave 128-row tiles.
    using LnShortK = PipeCfg<64, 384, 32, 1, 4, 3, true, kWtBlock, 4>;
    using Narrow = Bias;
    using Piece64 = PipeCfg<64, 64, 64, 2, 2, 3, true, kWtBlock, 4>;
    using Piece128x64 = PipeCfg<128, 64, 64, 2, 2, 2, true, kWtBlock, 4>;
    using Piece128 = PipeCfg<128, 128, 64, 2, 2, 2, true, kWtBlock, 4>;
};
using LnCfg = Cfgs<TZH_WF_W8T, 2>::Ln;
static_assert(Cfgs<TZH_WF_W8T, 2>::LnShortK::WN == LnCfg::WN &&
                  Cfgs<TZH_WF_W8T, 2>::LnShortK::TNF == LnCfg::TNF && Cfgs<TZH_WF_W8T, 4>::Ln::WN == LnCfg::WN &&
                  Cfgs<TZH_WF_W8T, 4>::Ln::TNF == LnCfg::TNF && Cfgs<TZH_WF_W8T, 4>::Ln::BN == LnCfg::BN,
              "one LayerNorm epilogue layout (statistics order) for every configuration and ln_rows_kernel");
static_assert(Cfgs<TZH_WF_W8T, 2>::LnShortK::blocks_per_cu(true) == 2 &&
                  Cfgs<TZH_WF_W8T, 4>::LnShortK::blocks_per_cu(true) == 2,
              "two short-k LayerNorm workgroups per CU");
static_assert(Cfgs<TZH_WF_W8T, 4>::Bias::lds_bytes(false, true, true) <= 163840 &&
                  Cfgs<TZH_WF_W8T, 4>::Ln::lds_bytes(true, false) <= 163840,
              "f32-activation tiles with staged f32 output fit the 160 KiB of LDS");

template <typename T>
struct NoDeduce {
    using type = T;
};

template <int EPI, typename TC, typename P, typename TR = TC, typename TX>
int launch(hipStream_t st, int num_cus, const TX *x, const void *wc, const uint16_t *scale, const float *bias, TC *c,
           int M, int K, int N, const typename NoDeduce<TR>::type *res, const float *gamma, const float *beta,
           float eps, int ldc, int n_valid, bool rs) {
    const int nbm = (M + P::BM - 1) / P::BM;
    const int nbn = N / P::BN;
    constexpr bool f32_out = std::is_same<TC, float>::value && EPI != EPI_RES && EPI != EPI_LN;
    const int slots = num_cus * P::blocks_per_cu(EPI == EPI_LN, std::is_same<TC, _Float16>::value || f32_out, f32_out);
    // Persistent blocks.  Panel p goes to XCD p % 8 with its nbn units, so
    // 8 * ceil(panels / 8) * nbn blocks give every unit a block of its own
    // (blocks without a unit return at once); beyond that, one per slot.
    const int64_t spread = (int64_t)kXcds * ((nbm + kXcds - 1) / kXcds) * nbn;
    const int grid = spread < slots ? (int)spread : slots;
    // row scaling: every configuration but the 128-row LayerNorm tiles (whose
    // registers it would spill; launch_ln takes the 64-row ones instead)
    constexpr bool rs_ok = !(EPI == EPI_LN && P::BM == 128);
    if constexpr (sizeof(TX) == 4 && rs_ok) {
        if (rs) {
            hipLaunchKernelGGL((linear_pipe_kernel<EPI, TC, P, TR, TX, true>), dim3(grid), dim3(P::THREADS), 0, st, x,
                               wc, scale, bias, c, M, K, N, res, gamma, beta, eps, ldc, n_valid);
            TZH_LAUNCHED("linear_pipe_kernel");
            return TZH_OK;
        }
    }
    if (rs) return tzh_fail(TZH_ERR_INVALID_ARGS, "row scaling needs f32 activations and a tile that supports it");
    hipLaunchKernelGGL((linear_pipe_kernel<EPI, TC, P, TR, TX, false>), dim3(grid), dim3(P::THREADS), 0, st, x, wc,
                       scale, bias, c, M, K, N, res, gamma, beta, eps, ldc, n_valid);
    TZH_LAUNCHED("linear_pipe_kernel");
    return TZH_OK;
}

// LayerNorm of f32 pre-normalisation rows (residual already added) with the
// statistics summed in exactly the order of the LayerNorm epilogue of
// linear_pipe_kernel<EPI_LN, ., LnCfg>: the lane of wave column group wn and
// half-wave h sums its columns 96 wn + 32 a + 8 g + 4 h + q in (a, g, q)
// order, half-wave 1's sum is added to half-wave 0's, and the four groups
// are added in order from 0; the squared deviations likewise.  A row
// normalised here is therefore bit-identical to the same row normalised
// inside the GEMM.  One wave per 8 rows, lane = 8 r + 2 wn + h.
template <typename TO>
__global__ void __launch_bounds__(256) ln_rows_kernel(const float *__restrict__ V, int rows,
                                                      const float *__restrict__ gamma,
                                                      const float *__restrict__ beta, float eps,
                                                      TO *__restrict__ out) {
    constexpr int WN = LnCfg::WN, TNF = LnCfg::TNF, BN = LnCfg::BN;
    static_assert(WN == 4, "eight lanes per row");
    const int lane = threadIdx.x & 63;
    const int row = (int)(blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64) * 8 + lane / 8;
    const int wn = (lane & 7) >> 1, h = lane & 1, base = lane & ~7;
    const float *src = V + (size_t)(row < rows ? row : rows - 1) * BN;
    f32x4_t v[TNF][4];
#pragma unroll
    for (int a = 0; a < TNF; a++)
#pragma unroll
        for (int g = 0; g < 4; g++) v[a][g] = *(const f32x4_t *)(src + wn * TNF * 32 + a * 32 + 8 * g + 4 * h);
    // sum over this lane's 48 columns, then the row total in the GEMM's order
    auto row_total = [&](float own) __attribute__((always_inline)) {
        const float part = own + __shfl_xor(own, 1, 64);  // on h = 0 lanes: half 0 + half 1
        float tot = 0.0f;
#pragma unroll
        for (int j = 0; j < WN; j++) tot += __shfl(part, base + 2 * j, 64);
        return tot;
    };
    float sum = 0.0f;
#pragma unroll
    for (int a = 0; a < TNF; a++)
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int q = 0; q < 4; q++) sum += v[a][g][q];
    const float mean = row_total(sum) / (float)BN;
    float sq = 0.0f;
#pragma unroll
    for (int a = 0; a < TNF; a++)
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float d = v[a][g][q] - mean;
                sq += d * d;
            }
    const float inv_std = 1.0f / sqrtf(row_total(sq) / (float)BN + eps);
    if (row >= rows) return;
#pragma unroll
    for (int a = 0; a < TNF; a++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int n = wn * TNF * 32 + a * 32 + 8 * g + 4 * h;
            const f32x4_t gg = *(const f32x4_t *)(gamma + n);
            const f32x4_t bt = *(const f32x4_t *)(beta + n);
            float y[4];
#pragma unroll
            for (int q = 0; q < 4; q++) y[q] = ((v[a][g][q] - mean) * inv_std) * gg[q] + bt[q];
            store4<TO>(out + (size_t)row * BN + n, y[0], y[1], y[2], y[3]);
        }
}

// bias + residual + LayerNorm over 384-wide rows.  Tiled int8 weights with
// k <= 384, and row-scaled calls at any k, use the short-k configuration
// (two workgroups per CU, above).  Otherwise the 128-row tiles run in
// whole rounds of one tile per CU slot; when the rows left over for a
// partial last round would keep only a few CUs busy (at most slots / 3
// tiles), those tiles are instead cut into 64 x 64, 128 x 64 or 128 x 128
// pieces (the finest that fit one round), which store their pre-
// normalisation rows to ws (f32, ws_rows rows) for ln_rows_kernel.  Every
// output value comes out the same as it would from the whole-tile kernel:
// the pieces run the same MFMA sequence per element, and ln_rows_kernel
// sums the statistics in the tile epilogue's order.
template <int WF, typename TC, typename TX>
int launch_ln(hipStream_t st, int num_cus, const TX *x, const void *wc, const uint16_t *scale, const float *bias,
              TC *c, int M, int K, const TC *res, const float *gamma, const float *beta, float eps, float *ws,
              int64_t ws_rows, bool rs) {
    using C = Cfgs<WF, (int)sizeof(TX)>;
    constexpr int N = C::Ln::BN, BM = C::Ln::BM;
    constexpr bool f32_out = false;  // LayerNorm outputs are not staged when f32
    constexpr bool staged = std::is_same<TC, _Float16>::value && sizeof(TX) == 2;  // as the kernel decides
    if (K <= 384 || rs)  // row-scaled: the 64-row tiles at any k
        return launch<EPI_LN, TC, typename C::LnShortK>(st, num_cus, x, wc, scale, bias, c, M, K, N, res, gamma, beta,
                                                        eps, N, N, rs);
    const int slots = num_cus * C::Ln::blocks_per_cu(true, staged, f32_out);
    const int panels = (M + BM - 1) / BM;
    const int full = panels / slots * slots;
    const int rem = panels - full;
    const int tail_rows = M - full * BM;
    int per = 0;  // pieces per tile
    if (rem > 0 && ws && tail_rows <= ws_rows)
        for (int p : {12, 6, 3})
            if ((int64_t)rem * p <= slots) {
                per = p;
                break;
            }
    const int m_main = per ? full * BM : M;
    if (m_main > 0)
        TZH_TRY((launch<EPI_LN, TC, typename C::Ln>(st, num_cus, x, wc, scale, bias, c, m_main, K, N, res, gamma, beta,
                                                     eps, N, N, rs)));
    if (!per) return TZH_OK;
    const TX *xt = x + (size_t)m_main * K;
    const TC *rt = res + (size_t)m_main * N;
    if (per == 12)
        TZH_TRY((launch<EPI_RES, float, typename C::Piece64, TC>(st, num_cus, xt, wc, scale, bias, ws, tail_rows, K, N,
                                                                  rt, nullptr, nullptr, 0.f, N, N, rs)));
    else if (per == 6)
        TZH_TRY((launch<EPI_RES, float, typename C::Piece128x64, TC>(st, num_cus, xt, wc, scale, bias, ws, tail_rows, K,
                                                                      N, rt, nullptr, nullptr, 0.f, N, N, rs)));
    else
        TZH_TRY((launch<EPI_RES, float, typename C::Piece128, TC>(st, num_cus, xt, wc, scale, bias, ws, tail_rows, K, N,
                                                                   rt, nullptr, nullptr, 0.f, N, N, rs)));
    hipLaunchKernelGGL(ln_rows_kernel<TC>, dim3((unsigned)((tail_rows + 31) / 32)), dim3(256), 0, st, ws, tail_rows,
                       gamma, beta, eps, c + (size_t)m_main * N);
    TZH_LAUNCHED("ln_rows_kernel");
    return TZH_OK;
}

template <int WF, int EPI, typename TC, typename TX>
int launch_bias(hipStream_t st, int num_cus, const TX *x, const void *wc, const uint16_t *scale, const float *bias,
                TC *c, int M, int K, int N, int ldc, int n_valid, bool rs) {
    using C = Cfgs<WF, (int)sizeof(TX)>;
    if (N % C::Bias::BN == 0)
        return launch<EPI, TC, typename C::Bias>(st, num_cus, x, wc, scale, bias, c, M, K, N, nullptr, nullptr,
                                                 nullptr, 0.f, ldc, n_valid, rs);
    return launch<EPI, TC, typename C::Narrow>(st, num_cus, x, wc, scale, bias, c, M, K, N, nullptr, nullptr, nullptr,
                                               0.f, ldc, n_valid, rs);
}

// int8 codes q[r][j] (n rows of k) -> biased codes u = q + 128 stage-tiled
// for TZH_WF_W8T over the padded shape n_pad x k_pad (multiples of 384 and
// 64): u lands at ((r / 384 * (k_pad / 64) + j / 64) * 384 + r % 384) * 64 +
// j % 64; rows r >= n and columns j >= k hold code 0 (u = 128), which adds
// nothing to any sum.  One thread per 16 codes.
__global__ void tile_codes_w8_kernel(const int8_t *__restrict__ q, uint8_t *__restrict__ out, int n, int k,
                                     int n_pad, int k_pad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte group of the output
    const int kt_count = k_pad / 64;
    if (i >= (int64_t)n_pad * k_pad / 16) return;
    const int64_t o = i * 16;
    const int c = (int)(o % 64);
    const int64_t r_all = o / 64;  // row index inside the tiled layout (block, stage, row)
    const int r = (int)(r_all % kWtBlock);
    const int64_t bs = r_all / kWtBlock;
    const int kt = (int)(bs % kt_count);
    const int nb = (int)(bs / kt_count);
    const int row = nb * kWtBlock + r, j0 = kt * 64 + c;
    uint8_t v[16];
    if (row < n && j0 + 16 <= k) {
        const int8_t *src = q + (int64_t)row * k + j0;
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = (uint8_t)src[j] ^ 0x80u;
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = (row < n && j0 + j < k) ? (uint8_t)q[(int64_t)row * k + j0 + j] ^ 0x80u : 0x80u;
    }
    *(u32x4_t *)(out + o) = *(const u32x4_t *)v;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// int8 codes [n, k] -> the TZH_WF_W8T layout of the padded shape n_pad x
// k_pad (multiples of 384 and 64, at least n and k).
int tzh_tile_codes_w8_launch(hipStream_t st, const int8_t *q, uint8_t *out, int64_t n, int64_t k, int64_t n_pad,
                             int64_t k_pad) {
    if (n_pad % kWtBlock || k_pad % 64 || n <= 0 || k <= 0 || n > n_pad || k > k_pad)
        return tzh_fail(TZH_ERR_INVALID_ARGS, "tiled int8 weights need n_pad %% 384 == 0, k_pad %% 64 == 0");
    const int64_t groups = n_pad * k_pad / 16;
    hipLaunchKernelGGL(tile_codes_w8_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, q, out, (int)n,
                       (int)k, (int)n_pad, (int)k_pad);
    TZH_LAUNCHED("tile_codes_w8_kernel");
    return TZH_OK;
}

// Activations x (f16 or f32) x weight codes in format w_format (TZH_WF_W8T:
// tiled biased int8), output and residual both F16 or both F32.  The weight
// codes may be padded: n is the padded column count the code layout holds
// and n_valid <= n the columns that exist (scale and bias have n_valid
// entries; C rows are n_valid apart); the bias epilogues run n in chunks of
// up to 1536 columns.  ln_ws (f32, ln_ws_rows rows of 384; may be null) lets
// the LayerNorm epilogue split a partial last round of tiles (see
// launch_ln).  row_scale (f32 activations): each row scaled into the
// split's range by an exact power of two (see linear_pipe_kernel).
int tzh_linear_codes_launch(hipStream_t st, int num_cus, const void *x, int32_t x_dtype, const void *wc,
                            int32_t w_format, const uint16_t *scale, const float *bias, void *c, int32_t c_dtype,
                            int64_t m, int64_t k, int64_t n, int64_t n_valid, int32_t epilogue, const void *res,
                            const float *gamma, const float *beta, float eps, float *ln_ws, int64_t ln_ws_rows,
                            bool row_scale) {
    if (m < 0 || k <= 0 || n <= 0 || n_valid <= 0 || n_valid > n) return tzh_fail(TZH_ERR_INVALID_ARGS, "bad GEMM shape");
    if (m == 0) return TZH_OK;  // matmul_w8a32.zig:24
    if (m > (int64_t)1 << 30 || k > 65536 || n > 65536) return tzh_fail(TZH_ERR_TOO_LARGE, "GEMM shape too large");
    if (k % 64) return tzh_fail(TZH_ERR_INVALID_ARGS, "k=%lld must be a multiple of 64", (long long)k);
    if (!x || !wc || !scale || !c) return tzh_fail(TZH_ERR_INVALID_ARGS, "null operand");
    if (!aligned16(x) || !aligned16(wc) || (res && !aligned16(res)) || ((uintptr_t)c & 3) ||
        ((c_dtype == TZH_F16 || epilogue == TZH_EPI_BIAS_RES_LN) && !aligned16(c)))
        return tzh_fail(TZH_ERR_INVALID_ARGS, "operands must be 16-byte aligned");
    if (c_dtype != TZH_F16 && c_dtype != TZH_F32) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "output must be F16 or F32");
    if (x_dtype != TZH_F16 && x_dtype != TZH_F32)
        return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "activations must be F16 or F32");
    const int M = (int)m, K = (int)k, N = (int)n, NV = (int)n_valid;
    const bool c16 = c_dtype == TZH_F16, x32 = x_dtype == TZH_F32;
    if (w_format != TZH_WF_W8T) return tzh_fail(TZH_ERR_INVALID_ARGS, "unknown weight format %d", w_format);
    if (N % kWtBlock) return tzh_fail(TZH_ERR_INVALID_ARGS, "tiled int8 weights need n %% 384 == 0 (n=%d)", N);
    if (c16 && NV != N) return tzh_fail(TZH_ERR_INVALID_ARGS, "f16 output needs every column (n_valid == n)");
    if (row_scale && !x32) return tzh_fail(TZH_ERR_INVALID_ARGS, "row scaling needs f32 activations");
    // one call per (activation type, output type): f(x, c) with typed pointers
    auto typed = [&](auto &&f) -> int {
        if (x32)
            return c16 ? f((const float *)x, (_Float16 *)c) : f((const float *)x, (float *)c);
        return c16 ? f((const _Float16 *)x, (_Float16 *)c) : f((const _Float16 *)x, (float *)c);
    };
    if (epilogue == TZH_EPI_BIAS || epilogue == TZH_EPI_BIAS_GELU) {
        const bool gelu = epilogue == TZH_EPI_BIAS_GELU;
        // column chunks of up to 1536 (the parameters of a chunk sit in LDS)
        for (int j0 = 0; j0 < NV; j0 += 1536) {
            const int nc = N - j0 < 1536 ? N - j0 : 1536, nv = NV - j0 < nc ? NV - j0 : nc;
            const char *wj = (const char *)wc + (size_t)(j0 / kWtBlock) * K * kWtBlock;
            const uint16_t *sj = scale + j0;
            const float *bj = bias ? bias + j0 : nullptr;
            TZH_TRY(typed([&](auto xt, auto ct) {
                using TC = std::remove_pointer_t<decltype(ct)>;
                return gelu ? launch_bias<TZH_WF_W8T, EPI_GELU, TC>(st, num_cus, xt, wj, sj, bj, ct + j0, M, K, nc, NV,
                                                                    nv, row_scale)
                            : launch_bias<TZH_WF_W8T, EPI_BIAS, TC>(st, num_cus, xt, wj, sj, bj, ct + j0, M, K, nc, NV,
                                                                    nv, row_scale);
            }));
        }
        return TZH_OK;
    }
    if (epilogue == TZH_EPI_BIAS_RES_LN) {
        if (N != LnCfg::BN || NV != N)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "LayerNorm epilogue needs n == 384 (got %d)", NV);
        if (!res || !gamma || !beta) return tzh_fail(TZH_ERR_INVALID_ARGS, "null residual/gamma/beta");
        if (ln_ws && !aligned16(ln_ws)) return tzh_fail(TZH_ERR_INVALID_ARGS, "LayerNorm workspace must be 16-byte aligned");
        return typed([&](auto xt, auto ct) {
            using TC = std::remove_pointer_t<decltype(ct)>;
            return launch_ln<TZH_WF_W8T, TC>(st, num_cus, xt, wc, scale, bias, ct, M, K, (const TC *)res, gamma, beta,
                                             eps, ln_ws, ln_ws_rows, row_scale);
        });
    }
    return tzh_fail(TZH_ERR_INVALID_ARGS, "unknown epilogue %d", epilogue);
}
