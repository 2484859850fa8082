// gemm_mfma.hip — LDS-staged MFMA GEMM for the large-M (prefill) shapes.
//
// Replaces the arithmetic of reference src/quantized_gemm.cu:15-54 (INT8,
// int8_gemm_dp4a_kernel) and :99-118 (FP8, fp8_gemm_scaled_kernel) for M > 16.
//
// Workgroup tile 256x256, 4 waves (one per SIMD) in a 2x2 grid; each wave owns
// 128x128 outputs as 4x4 MFMA blocks of 32x32 (256 accumulator AGPRs).  The
// launch is persistent: one workgroup per CU (a multiple of the XCD count)
// walks its tiles without a relaunch between them.  A 128x128 tile (each wave
// 64x64 as 2x2 blocks, two workgroups per CU) serves shapes with fewer
// 256x256 tiles than CUs (tensor-parallel shards, short prefills); every
// output is still summed over K in the same order, so both tiles give
// identical results.
//   INT8: v_mfma_i32_32x32x32_i8   (exact int32 accumulation), 4 k steps/stage
//   FP8 : v_mfma_f32_32x32x64_f8f6f4 with E4M3 operands (fp32), 2 k steps/stage
// K advances 128 bytes per stage; two LDS stages of (256+256)x128 bytes
// (128 KiB of the CU's 160 KiB).  Both operands are copied global->LDS with
// 128-bit direct-to-LDS loads (buffer_load_dwordx4 ... lds) from per-lane
// 32-bit offsets computed once: A, and B stored [N,K], eight lanes per
// 128-byte row segment; B stored [K,N] row by row as it lies in memory, its
// fragments then read with the transposing ds_read_b64_tr_b8.
//
// Schedule of one stage, per wave (steps 0..n-1 of the stage are in LDS): n
// groups of 16 MFMAs.  Group 0 runs the previous stage's last step, carried
// across the barrier, while the reads of step 0 are issued; group g > 0 runs
// step g-1 while the reads of step g are issued.  The global->LDS copies of
// the next stage ride along in the first groups, one instruction per MFMA.
// The stage ends with a wait for this wave's reads and copies and a barrier.
// Fragment reads thus run one group ahead of their MFMAs and no memory
// instruction waits in a queue of its own; sched_barrier / sched_group_barrier
// keep the compiler to this order.
//
// LDS layout of a stage: row r (an M row of A or an N row of B) holds its 128
// K-bytes as eight 16-byte chunks; logical chunk c is stored at physical
// chunk c ^ swz(r), swz(r) = (q ^ (q >> 3)) & 7 with q = r mod 32.  A 128-bit
// fragment read by 8 (or 16) consecutive lanes of consecutive rows then
// touches every LDS bank once, whether the LDS serves 8 lanes x 16 B or 16
// lanes x 16 B per cycle; and because the swizzle repeats every 32 rows, all
// fragments of a k step share one address register plus immediate offsets.
//
// The per-row / per-column epilogue operands of the tile (scale_a, scale_b,
// bias) are staged once in LDS beside the two stages.
#include "fke_internal.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace fke {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BK = 128;  // bytes of K per stage
constexpr int NWAVES = 4;
constexpr int NTHREADS = NWAVES * 64;

// Workgroup tile: each of the 4 waves (2x2) owns NI x NJ MFMA blocks of 32x32
// (NI, NJ in {1, 2, 4}), with a ring of NS LDS stages (2 or 4: the copy of
// stage k + NS - 1 is issued while stage k runs).
template <int NI_, int NJ_, int NS_ = 2>
struct Tile {
    static constexpr int NI = NI_, NJ = NJ_, NS = NS_;
    static_assert(NS == 2 || NS == 4, "ring of 2 or 4 stages");
    static constexpr int BM = 64 * NI, BN = 64 * NJ;  // tile rows, B columns (B rows of [N,K])
    static constexpr int WM = 32 * NI, WN = 32 * NJ;  // one wave's rows, columns
    static constexpr int STAGE_A = BM * BK;           // A part of one LDS stage
    static constexpr int STAGE = (BM + BN) * BK;      // one LDS stage
    static constexpr int PWA = BM / 32, PWB = BN / 32;  // 1-KiB DMA loads per wave per stage
    static constexpr int NPIECE = NI * NJ;            // MFMAs per k step
    static constexpr int OCC = NS == 2 && NI * NJ <= 4 ? 2 : 1;  // workgroups per CU
    static_assert(NS * STAGE <= 128 * 1024, "the stages fit the CU's LDS beside the epilogue operands");
};
using T256 = Tile<4, 4>;
using T128 = Tile<2, 2>;
using T128R4 = Tile<2, 2, 4>;  // one workgroup per CU, three stages in flight
using T128x64R4 = Tile<2, 1, 4>;
using T64R4 = Tile<1, 1, 4>;

__device__ __forceinline__ int swz(int r) { return ((r & 31) ^ ((r & 31) >> 3)) & 7; }

// Workgroup -> output tile.  Consecutive workgroup ids are dispatched round
// robin over the 8 XCDs; give each XCD a contiguous range of tile ids and walk
// that range in groups of GROUP_M tile rows so the workgroups an XCD runs at
// once share A and B panels in its L2.
constexpr int GROUP_M = 4;
constexpr int NXCD = 8;

__device__ __forceinline__ void tile_of(int bid, int gm, int gn, int& tm, int& tn) {
    const int nwg = gm * gn;
    const int q = nwg / NXCD, rem = nwg % NXCD;
    const int xcd = bid % NXCD, local = bid / NXCD;
    const int tile = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + local;
    const int per_group = GROUP_M * gn;
    const int group = tile / per_group;
    const int first_m = group * GROUP_M;
    const int gsize = min(gm - first_m, GROUP_M);
    const int in_group = tile % per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Weight row held by column c (0..BN-1) of a SwiGLU tile whose BN/2 outputs
// start at column o0; B is [gate; up] with I = rows / 2.  Each wave's WN B
// columns are WN/2 gate columns then the WN/2 up columns of the same outputs,
// so MFMA block j (gate) and block j + NJ/2 (up) of a wave hold the two
// operands of one output in the same lane.
template <int NJ>
__device__ __forceinline__ int swiglu_b_row(int c, int o0, int I) {
    constexpr int WN = 32 * NJ, H = NJ / 2;
    const int jj = (c >> 5) % NJ;
    const int o = o0 + (c / WN) * (WN / 2) + (jj % H) * 32 + (c & 31);
    return jj >= H ? I + o : o;
}

// Direct-to-LDS copy plan of one (32*PW)-row x 128-byte K-contiguous panel (A,
// or B in [N,K] order).  Each wave issues PW loads of 1 KiB (8 rows x 128 B);
// lane l lands at byte 16*l of its KiB, so it fetches the logical chunk that
// the swizzle assigns to that physical slot.
//  * at_tile: the per-lane offsets are relative to the tile's first row and
//    the same for every tile (set once by init_lanes); the buffer resource
//    starts at that row and ends with the operand, so rows past the end read
//    zero (their outputs are never stored).  Moving to another tile is scalar
//    work only.
//  * init (SwiGLU B): panel row r holds weight row swiglu_b_row<NJ>(r, row0,
//    rows / 2), a per-tile lane offset over all of B; rows past `rows` re-read
//    the last valid row.
template <int PW>
struct Panel {
    __amdgpu_buffer_rsrc_t rsrc;  // from the tile's first row (init: the whole operand)
    uint32_t off[PW];             // byte offset of this lane's 16-byte source at k = 0
    __device__ void init_lanes(int ld, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int r = (wave * PW + i) * 8 + (lane >> 3);
            off[i] = static_cast<uint32_t>(r * ld + ((lane & 7) ^ swz(r)) * 16);
        }
    }
    __device__ __forceinline__ void at_tile(const int8_t* base, int ld, int row0, int rows) {
        rsrc = make_rsrc(base + static_cast<size_t>(row0) * ld, (rows - row0) * ld);
    }
    template <int NJ>
    __device__ void init_swiglu(const int8_t* base, int ld, int row0, int rows, int wave, int lane) {
        rsrc = make_rsrc(base, rows * ld);
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int r = (wave * PW + i) * 8 + (lane >> 3);
            const int lc = (lane & 7) ^ swz(r);
            const int src = swiglu_b_row<NJ>(r, row0, rows >> 1);  // (SwiGLU tiles have NJ >= 2)
            off[i] = static_cast<uint32_t>(min(src, rows - 1) * ld + lc * 16);
        }
    }
    // Load i of this wave for the stage at K byte k0 (uniform); AUX: cache policy.
    template <int AUX = 0>
    __device__ __forceinline__ void issue(int i, int k0, uint8_t* lds, int wave) const {
        dma16<AUX>(rsrc, off[i], k0, lds + (wave * PW + i) * 1024);
    }
};

// Chunk swizzle of a B [K,N] stage whose k rows hold BN bytes: logical
// 16-byte chunk c of row r sits at chunk c ^ kn_swz<BN>(r).  With it the
// transposed reads below touch every LDS bank once per 16-lane group (and,
// for 128- and 64-byte rows, once per 32-lane half), and it repeats every 8
// rows (16 for 256-byte rows), so other k steps are immediate offsets away.
template <int BN>
__device__ __forceinline__ int kn_swz(int r) {
    if constexpr (BN == 256) return r & 15;
    else if constexpr (BN == 128) return r & 7;
    else return (r >> 1) & 3;
}

// B stored [K,N]: a stage is 128 k rows of BN n bytes, copied as they lie in
// memory, 1024/BN rows per 1-KiB load, chunks swizzled by kn_swz.  The MFMA
// fragments (one column n per lane, k bytes consecutive) are then read with
// ds_read_b64_tr_b8, which transposes 8x8 byte blocks across lanes.  Columns
// past N read whatever follows them in memory (those outputs are never
// stored); reads past the end of B fall out of the buffer's range and return 0.
template <int BN>
struct KNPanel {
    static constexpr int PW = BN / 32;  // 1-KiB loads per wave per stage
    static constexpr int CH = BN / 16;  // 16-byte chunks per k row
    __amdgpu_buffer_rsrc_t rsrc;        // B from the tile's first column to its end
    uint32_t off[PW];                   // byte offset of this lane's 16-byte source at stage 0 (any tile)
    int stage_bytes;                    // BK rows of B
    __device__ void init_lanes(int N, int wave, int lane) {
        stage_bytes = BK * N;
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int r = (wave * PW + i) * (1024 / BN) + lane / CH;  // k row within the stage
            const int c = (lane % CH) ^ kn_swz<BN>(r);                // logical chunk landing at physical lane % CH
            off[i] = static_cast<uint32_t>(r * N + c * 16);
        }
    }
    __device__ __forceinline__ void at_tile(const int8_t* B, int N, int K, int n0) {
        rsrc = make_rsrc(B + n0, K * N - n0);
    }
    template <int AUX = 0>
    __device__ __forceinline__ void issue(int i, int kt, uint8_t* lds, int wave) const {
        dma16<AUX>(rsrc, off[i], kt * stage_bytes, lds + (wave * PW + i) * 1024);
    }
};

// ds_read_b64_tr_b8 (gfx950): within each 16-lane group, lane 8h+i receives
// byte i of the 8 bytes addressed by lanes 2b+h, b = 0..7, as its byte b.
typedef int v2i __attribute__((ext_vector_type(2)));
// The address-space cast keeps the pointer's provenance (lds0 or lds1), so
// the compiler can tell these reads from the DMA writes into the other stage.
__device__ __forceinline__ v2i ds_read_tr8(const uint8_t* p) {
    typedef v2i __attribute__((address_space(3))) * lptr;
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lptr)(p));
}

// Per-lane offsets (within a stage's B region) of the transposed reads of
// B block j, k rows 8*rr..8*rr+7 of the lane's half of the first step.
// Lane l = 16G + s reads row HS*(G>>1) + 8*rr + s/2 at column block
// wn*WN + 32j + 16*(G&1) + 8*(s&1), so that after the transpose lane l
// holds column wn*WN + 32j + l%32 with its k bytes in order.  The swizzle
// repeats every 8 rows, so other steps (and, for FP8, k rows 16..31 of the
// half) are immediate offsets away.
template <int ELEM, class TL>
__device__ __forceinline__ uint32_t kn_read_off(int lane, int wn, int j, int rr) {
    constexpr int HS = ELEM == ELEM_I8 ? 16 : 32;  // k bytes of one lane-half per step
    const int G = lane >> 4, sl = lane & 15, b = sl >> 1;
    const int row = HS * (G >> 1) + 8 * rr + b;
    const int chunk = (wn * (TL::WN / 16) + 2 * j + (G & 1)) ^ kn_swz<TL::BN>(row);
    return static_cast<uint32_t>(row * TL::BN + chunk * 16 + 8 * (sl & 1));
}

// Per element type: fragment and accumulator types, k steps per stage, and
// FB, the operand bytes per lane of one MFMA.  FB = 16 (INT8, fp16, bf16):
// lane l supplies row l%32 with bytes 16*(l/32)..+15 of a 32-byte k step
// (32 int8 or 16 fp16/bf16 values per row); FB = 32 (FP8): 32 codes per lane
// of a 64-byte step.
template <int ELEM>
struct Mma;
template <>
struct Mma<ELEM_I8> {
    using Frag = v4i;  // 16 k bytes per lane
    using AccT = v16i;
    static constexpr int KSTEPS = BK / 32;
    static constexpr int FB = 16;
};
template <>
struct Mma<ELEM_F8> {
    using Frag = v8i;  // 32 k codes per lane
    using AccT = v16f;
    static constexpr int KSTEPS = BK / 64;
    static constexpr int FB = 32;
};
template <int ELEM>
struct Mma16 {
    using Frag = v4i;  // 8 fp16 / bf16 k values per lane
    using AccT = v16f;
    static constexpr int KSTEPS = BK / 32;
    static constexpr int FB = 16;
};
template <>
struct Mma<ELEM_F16> : Mma16<ELEM_F16> {};
template <>
struct Mma<ELEM_BF16> : Mma16<ELEM_BF16> {};

template <int ELEM, class TL>
struct Frags {
    typename Mma<ELEM>::Frag a[TL::NI], b[TL::NJ];
};

// LDS reads of the wave's fragments of k step ks; read_piece issues read r
// (one instruction, nothing waits for the data).
//   A, and B in [N,K] order: ds_read_b128 of 16 k bytes.  INT8: r = 0..NI-1
//   A block r, NI..NI+NJ-1 B block r-NI.  FP8: r = 2f + h, f < NI A, f >= NI
//   B, h = which 16 of the lane's 32 codes.  Rows wm*WM + 32*i + lr (A) and
//   wn*WN + 32*j + lr (B^T) share swz(lr): one address plus immediates.
//   B in [K,N] order: ds_read_b64_tr_b8 of 8 k bytes.  INT8: r = NI + 2j + rr;
//   FP8: r = 2NI + 4j + rr, rr = which 8 of the lane's k bytes.
template <int ELEM, int BL, class TL>
struct Reads {
    static constexpr int PB = Mma<ELEM>::FB == 16 ? 1 : 2;  // reads per block and k step, [N,K]
    static constexpr int A = PB * TL::NI;
    static constexpr int N = A + (BL == FKE_B_NK ? PB : 2 * PB) * TL::NJ;
};

template <int ELEM, int BL, class TL>
__device__ __forceinline__ void read_piece(const uint8_t* buf, int ks, int wm, int wn, int lane,
                                           const uint32_t (&kn_off)[TL::NJ][2], Frags<ELEM, TL>& f, int r) {
    constexpr int NI = TL::NI;
    const int lr = lane & 31, lh = lane >> 5, sw = swz(lr);
    const uint8_t* Ab = buf + (wm * TL::WM + lr) * BK;
    const uint8_t* Bb = buf + TL::STAGE_A + (wn * TL::WN + lr) * BK;
    constexpr int RA = Reads<ELEM, BL, TL>::A;
    if constexpr (BL == FKE_B_KN) if (r >= RA) {
        constexpr int KSTEP = ELEM == ELEM_I8 ? 32 : 64;  // k rows per step
        const int p = r - RA;
        const int j = ELEM == ELEM_I8 ? p >> 1 : p >> 2, rr = ELEM == ELEM_I8 ? p & 1 : p & 3;
        const v2i x = ds_read_tr8(buf + TL::STAGE_A + kn_off[j][rr & 1] + (ks * KSTEP + (rr >> 1) * 16) * TL::BN);
        f.b[j][2 * rr] = x[0];
        f.b[j][2 * rr + 1] = x[1];
        return;
    }
    if constexpr (Mma<ELEM>::FB == 16) {
        const int co = ((ks * 2 + lh) ^ sw) << 4;  // this lane's 16-byte chunk of the 32-byte step
        if (r < NI) f.a[r] = *reinterpret_cast<const v4i*>(Ab + r * 32 * BK + co);
        else f.b[r - NI] = *reinterpret_cast<const v4i*>(Bb + (r - NI) * 32 * BK + co);
    } else {
        const int fi = r >> 1, h = r & 1;
        const int co = ((ks * 4 + lh * 2 + h) ^ sw) << 4;
        v8i& d = fi < NI ? f.a[fi] : f.b[fi - NI];
        const v4i x = *reinterpret_cast<const v4i*>((fi < NI ? Ab + fi * 32 * BK : Bb + (fi - NI) * 32 * BK) + co);
        if (h == 0) {
            d[0] = x[0]; d[1] = x[1]; d[2] = x[2]; d[3] = x[3];
        } else {
            d[4] = x[0]; d[5] = x[1]; d[6] = x[2]; d[7] = x[3];
        }
    }
}

// Clears the 0x7F/0xFF codes of an FP8 fragment (DMA-staged operands cannot
// be rewritten on the way into LDS).
__device__ __forceinline__ v8i sanitize8(v8i x) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(x[i])));
    return x;
}

// FP8: clear the 0x7F/0xFF codes of a fragment set.
template <int ELEM, class TL>
__device__ __forceinline__ void sanitize_frags(Frags<ELEM, TL>& f) {
    if constexpr (ELEM == ELEM_F8) {
#pragma unroll
        for (int i = 0; i < TL::NI; ++i) f.a[i] = sanitize8(f.a[i]);
#pragma unroll
        for (int j = 0; j < TL::NJ; ++j) f.b[j] = sanitize8(f.b[j]);
    }
}

// Element v of an accumulator block, as its 32 bits, read straight out of
// the AGPR that holds it (v_accvgpr_read_b32): the accumulators stay in AGPRs
// until the epilogue reads them one at a time, instead of being copied to
// VGPRs all at once when the K loop ends, which would take every VGPR and
// spill the rest of the epilogue's state to scratch.
template <class AccT>
__device__ __forceinline__ uint32_t acc_bits(const AccT& a, int v) {
    uint32_t x;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(a[v]));
    return x;
}

// MFMA (i, j) of one k step of the wave's WM x WN block.
template <int ELEM, class TL>
__device__ __forceinline__ void mfma_one(const Frags<ELEM, TL>& f, typename Mma<ELEM>::AccT (&acc)[TL::NI][TL::NJ],
                                         int i, int j) {
    typedef _Float16 v8h __attribute__((ext_vector_type(8)));
    typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
    if constexpr (ELEM == ELEM_I8)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
    else if constexpr (ELEM == ELEM_F8)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[i][j], 0, 0, 0, 0, 0, 0);
    else if constexpr (ELEM == ELEM_F16)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, f.a[i]),
                                                           __builtin_bit_cast(v8h, f.b[j]), acc[i][j], 0, 0, 0);
    else
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, f.a[i]),
                                                            __builtin_bit_cast(v8bf, f.b[j]), acc[i][j], 0, 0, 0);
}

// One lane's epilogue operands, read out of LDS with inline ds_reads and one
// wait: the compiler would order its own LDS reads after every LDS-DMA copy
// in flight (it cannot always tell the epilogue's arrays from the stages the
// next tile's copies fill), which would make the epilogue wait for those
// copies.  sa[i][g]: scale_a of tile rows WM*wm + 32i + 8g + 4*(lane/32) +
// 0..3; sb[j], bias[j]: scale_b and bias of tile column WN*wn + 32j + lane%32.
template <int NI, int NJ>
struct EpiOps {
    typedef float v4f __attribute__((ext_vector_type(4)));
    v4f sa[NI][4];
    float sb[NJ], bias[NJ];
    template <int WM, int WN>
    __device__ __forceinline__ void read(const float* esa, const float* esb, const float* ebias, int wm, int wn,
                                         int lane) {
        typedef __attribute__((address_space(3))) const float* lds_f;
        const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                asm volatile("ds_read_b128 %0, %1"
                             : "=v"(sa[i][g])
                             : "v"((lds_f)(esa + wm * WM + i * 32 + 8 * g + 4 * lh)));
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            asm volatile("ds_read_b32 %0, %1" : "=v"(sb[j]) : "v"((lds_f)(esb + wn * WN + j * 32 + lr)));
            asm volatile("ds_read_b32 %0, %1" : "=v"(bias[j]) : "v"((lds_f)(ebias + wn * WN + j * 32 + lr)));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // the registers are tied to the wait: nothing reads them before it
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) asm volatile("" : "+v"(sa[i][g]));
#pragma unroll
        for (int j = 0; j < NJ; ++j) asm volatile("" : "+v"(sb[j]), "+v"(bias[j]));
    }
};

// Output columns of one workgroup tile: BN, or BN/2 SwiGLU outputs (BN B rows).
template <bool SWI, class TL>
constexpr int tile_cols() { return SWI ? TL::BN / 2 : TL::BN; }

// BNT: the B panel is read exactly once (one row of tiles), so its copies are
// non-temporal (launch_t decides; A is re-read by every tile of the row).
template <int ELEM, int BL, int OUT, bool SWI, class TL, bool BNT = false>
__global__ __launch_bounds__(NTHREADS, TL::OCC) void gemm_mfma_kernel(GemmArgs p, SplitK sk) {
    static_assert(!SWI || (ELEM == ELEM_I8 && BL == FKE_B_NK && OUT != FKE_OUT_I32), "SwiGLU: INT8, B [N,K], float out");
    static_assert(!SWI || TL::NJ >= 2, "SwiGLU: each wave pairs gate and up blocks");
    constexpr int NKS = Mma<ELEM>::KSTEPS;
    constexpr int NI = TL::NI, NJ = TL::NJ, BM = TL::BM, NPIECE = TL::NPIECE;
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[TL::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[TL::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[TL::NS > 2 ? TL::STAGE : 16];  // NS = 4 only
    __shared__ __attribute__((aligned(1024))) uint8_t lds3[TL::NS > 2 ? TL::STAGE : 16];
    // Epilogue operands of two items (the one in its epilogue, the next one):
    // scale of each tile row, scale and bias of each tile column.
    __shared__ __attribute__((aligned(16))) float epi_sa[2][BM];
    __shared__ __attribute__((aligned(16))) float epi_sb[2][TL::BN];
    __shared__ __attribute__((aligned(16))) float epi_bias[2][TL::BN];
    __shared__ int redo;  // FP8: rerun with NaN codes cleared

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS/M0 math
    const int wm = wave >> 1, wn = wave & 1;                     // wave's WM x WN block

    const int M = p.M, N = p.N, K = p.K;
    constexpr int TC = tile_cols<SWI, TL>();
    const int NO = SWI ? N >> 1 : N;  // output columns
    const int gm = (M + BM - 1) / BM, gn = (NO + TC - 1) / TC;
    const int S = sk.S;
    const int items = gm * gn * S;
    // K stages of BK bytes; the last holds KREM bytes when K % BK != 0 (K a
    // multiple of 16): its chunks past K are cleared in LDS before it is read.
    const int KTT = (K + BK - 1) / BK, KREM = K % BK;
    const int8_t* A = static_cast<const int8_t*>(p.A);
    const int8_t* B = static_cast<const int8_t*>(p.B);

    // One output tile, or under a K split (S > 1) one K range of a tile: the S
    // splits of a tile are walked as S rows of tiles, item (split, tm, tn)
    // summing K stages [split * KS, split * KS + KT).
    struct Item {
        int m0, n0, split, kt0, KT;  // n0: first output column
    };
    auto item_of = [&](int slot) __attribute__((always_inline)) {
        int tm, tn;
        tile_of(slot, gm * S, gn, tm, tn);
        Item it;
        it.split = tm / gm;
        it.m0 = (tm - it.split * gm) * BM;
        it.n0 = tn * TC;
        it.kt0 = it.split * sk.KS;
        it.KT = S > 1 ? min(KTT - it.kt0, sk.KS) : KTT;
        return it;
    };

    // Copy plans.  The per-lane offsets are the same for every tile (SwiGLU's
    // B: set per tile); a tile's first row or column is scalar state.
    Panel<TL::PWA> pa;
    pa.init_lanes(K, wave, lane);
    using BPanel = typename std::conditional<BL == FKE_B_NK, Panel<TL::PWB>, KNPanel<TL::BN>>::type;
    BPanel pb;
    uint32_t kn_off[NJ][2] = {};
    if constexpr (BL == FKE_B_NK) {
        if constexpr (!SWI) pb.init_lanes(K, wave, lane);
    } else {
        pb.init_lanes(N, wave, lane);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) kn_off[j][rr] = kn_read_off<ELEM, TL>(lane, wn, j, rr);
    }
    int ckt0 = 0;  // first K stage of the item the copies are issued for
    auto at_item = [&](const Item& it) __attribute__((always_inline)) {
        pa.at_tile(A, K, it.m0, M);
        if constexpr (BL == FKE_B_NK) {
            if constexpr (SWI) pb.template init_swiglu<NJ>(B, K, it.n0, N, wave, lane);
            else pb.at_tile(B, K, it.n0, N);
        } else {
            pb.at_tile(B, N, K, it.n0);
        }
        ckt0 = it.kt0;
    };

    // Epilogue operands of an item into LDS set `set`, by dword LDS-DMA (no
    // registers wait for them; issued before the item's stage copies, they
    // have landed once stage 0 has): wave w fills entries 64w..64w+63 of each
    // array it covers, entries past M or N reading zero.  A missing scale or
    // bias is written as its constant.
    auto load_epi = [&](const Item& it, int set) __attribute__((always_inline)) {
        const int e = wave * 64 + lane;  // entry of this lane
        if (wave * 64 < BM) {
            if (p.scale_a) dma4(make_rsrc(p.scale_a, M * 4), static_cast<uint32_t>(it.m0 + e) * 4, 0, &epi_sa[set][wave * 64]);
            else epi_sa[set][e] = p.sa;
        }
        if (wave * 64 < TL::BN) {
            int n = it.n0 + e;  // B row of tile column e
            if constexpr (SWI) n = min(swiglu_b_row<NJ>(e, it.n0, NO), N - 1);
            const uint32_t off = static_cast<uint32_t>(n) * 4;
            if (p.scale_b) dma4(make_rsrc(p.scale_b, N * 4), off, 0, &epi_sb[set][wave * 64]);
            else epi_sb[set][e] = p.sb;
            if (p.bias) dma4(make_rsrc(p.bias, N * 4), off, 0, &epi_bias[set][wave * 64]);
            else epi_bias[set][e] = -0.0f;
        }
    };

    typename Mma<ELEM>::AccT acc[NI][NJ];
    int slot = blockIdx.x;
    if (slot >= items) return;  // (the grid never has more workgroups than items)
    Item cur = item_of(slot);
    int par = 0;  // epi_* set of item cur

    // Copy of stage kt into buffer b, slot q of NSLOT: slots 0..PWA-1 copy
    // A, the rest copy B, all buffer -> LDS.
    constexpr int PWA = TL::PWA;
    constexpr int NSLOT = PWA + TL::PWB;  // B [K,N] panels take BN/32 loads per wave too
    // kt counts from the first stage of the item at_item set last (ckt0).
    auto copy = [&](int q, int kt, uint8_t* b) __attribute__((always_inline)) {
        const int ka = ckt0 + kt;
        if (q < PWA) pa.issue(q, ka * BK, b, wave);
        else if constexpr (BL == FKE_B_NK) pb.template issue<BNT ? 2 : 0>(q - PWA, ka * BK, b + TL::STAGE_A, wave);
        else pb.template issue<BNT ? 2 : 0>(q - PWA, ka, b + TL::STAGE_A, wave);
    };
    // Stage kt of the current item, in `buf`, is the partial last stage of K:
    // every lane clears the 16-byte chunks past K that its own copies put
    // there (its copies have landed), then waits for its LDS writes, ahead of
    // the barrier after which the stage is read.  A, and B in [N,K] order:
    // the chunk's K offset is its logical chunk in the row; B in [K,N] order
    // needs nothing (its rows past K fall outside B and read zero).
    auto clear_tail = [&](uint8_t* buf, int kt) __attribute__((always_inline)) {
        if (KREM == 0 || ckt0 + kt != KTT - 1) return;
        const int rem = KREM >> 4;  // whole chunks of the stage inside K
        const int4 z = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < PWA; ++i) {
            const int r = (wave * PWA + i) * 8 + (lane >> 3);
            if (((lane & 7) ^ swz(r)) >= rem) *reinterpret_cast<int4*>(buf + (wave * PWA + i) * 1024 + 16 * lane) = z;
        }
        if constexpr (BL == FKE_B_NK) {
#pragma unroll
            for (int i = 0; i < TL::PWB; ++i) {
                const int r = (wave * TL::PWB + i) * 8 + (lane >> 3);
                if (((lane & 7) ^ swz(r)) >= rem)
                    *reinterpret_cast<int4*>(buf + TL::STAGE_A + (wave * TL::PWB + i) * 1024 + 16 * lane) = z;
            }
        }
        wait_lgkm0();
    };

    // A stage is NKS groups of NPIECE MFMAs (16 for the 256x256 tile).
    // Group g runs the MFMAs of one fragment set (g = 0: the previous stage's
    // last step, carried across the barrier; g > 0: step g-1) while the LDS
    // reads of step g fill the other set, and carries copy slots of the next
    // stage (INT8, fp16, bf16, 256x256: 6 / 6 / 4 / 0 over the four groups;
    // FP8: as many as the first of its two groups has MFMAs, the rest in the
    // second).  Within a group every memory instruction is paired with an
    // MFMA, so it issues in the MFMA's shadow instead of stalling the matrix
    // pipe.
    constexpr int PER_GROUP = (NSLOT + NKS - 2) / (NKS - 1);
    Frags<ELEM, TL> f0, f1;
    constexpr int NREAD = Reads<ELEM, BL, TL>::N;  // LDS reads per step
    auto group = [&](auto sanc, auto q0c, auto q1c, Frags<ELEM, TL>& use, Frags<ELEM, TL>& fill,
                     const uint8_t* cur, int rks, uint8_t* nxt, int kc) __attribute__((always_inline)) {
        constexpr bool SAN = decltype(sanc)::value;
        constexpr int Q0 = decltype(q0c)::value, Q1 = decltype(q1c)::value;
        constexpr int NQ = Q1 - Q0;
        fence();
        if constexpr (SAN) sanitize_frags<ELEM, TL>(use);
        // Piece t: MFMA (t/NJ, t%NJ), then the reads r = t (mod NPIECE) of
        // the next step, then copy slots Q0 + c, c = t (mod NPIECE) (one per
        // piece in its first pieces unless the group has more copies than
        // MFMAs; early in the group, so each copy has the rest of the stage to
        // land: 1.8 % faster at 8192^3 INT8 than the group's last pieces).
        // Each piece is fenced, so this is the issue order.
#pragma unroll
        for (int t = 0; t < NPIECE; ++t) {
            fence();
            mfma_one<ELEM, TL>(use, acc, t / NJ, t % NJ);
#pragma unroll
            for (int r = t; r < NREAD; r += NPIECE)
                read_piece<ELEM, BL, TL>(cur, rks, wm, wn, lane, kn_off, fill, r);
#pragma unroll
            for (int c = t; c < NQ; c += NPIECE) copy(Q0 + c, kc, nxt);
        }
        fence();
    };
    using I0 = std::integral_constant<int, 0>;
    using F = std::false_type;
    // Stage kt: MFMAs on `cur` while stage kt + NS - 1 is copied into `nxt`.
    // Past the end the last stage is copied again (into a buffer whose stage
    // is done), so the body has no data-dependent branch.
    constexpr int NS = TL::NS;
    // CLR: stage kt+1 may be the partial last stage (the last stages of the
    // loop), whose tail is cleared before the barrier.
    auto stage = [&](auto sanc, auto clrc, const uint8_t* cbuf, uint8_t* nxt, uint8_t* after, int kt)
                     __attribute__((always_inline)) {
        const int kc = min(kt + NS - 1, cur.KT - 1);
        using S = decltype(sanc);
        if constexpr (NKS == 4) {
            constexpr int P = PER_GROUP, P2 = 2 * P < NSLOT ? 2 * P : NSLOT;
            group(S{}, I0{}, std::integral_constant<int, P>{}, f1, f0, cbuf, 0, nxt, kc);
            group(S{}, std::integral_constant<int, P>{}, std::integral_constant<int, P2>{}, f0, f1, cbuf, 1, nxt, kc);
            group(S{}, std::integral_constant<int, P2>{}, std::integral_constant<int, NSLOT>{}, f1, f0, cbuf, 2, nxt, kc);
            group(S{}, std::integral_constant<int, NSLOT>{}, std::integral_constant<int, NSLOT>{}, f0, f1, cbuf, 3, nxt,
                  kc);
        } else {
            static_assert(NKS == 2, "k steps per stage");
            // FP8 steps are twice as long (64-cycle MFMAs): on the 256x256
            // tile all copies ride in the first group, one per MFMA, and the
            // whole second group (16 x 64 cycles) is left for them to land
            // before the stage's vmcnt(0).  Splitting them 8 / 8 left the
            // last copies one MFMA before that wait and measured 5 % slower
            // (438-444 us against 416-422 us at 8192^3, both B layouts).
            // Smaller tiles have more copies than MFMAs per group: half each.
            constexpr int P = NSLOT <= NPIECE ? NSLOT : (NSLOT + 1) / 2;
            group(S{}, I0{}, std::integral_constant<int, P>{}, f1, f0, cbuf, 0, nxt, kc);
            group(S{}, std::integral_constant<int, P>{}, std::integral_constant<int, NSLOT>{}, f0, f1, cbuf, 1, nxt,
                  kc);
        }
        wait_lgkm0();                  // last step's fragments in registers (f1): cbuf may be overwritten after the barrier
        wait_vm<(NS - 2) * NSLOT>();   // this wave's share of stage kt+1 has landed (later stages may be in flight)
        if constexpr (decltype(clrc)::value) clear_tail(after, kt + 1);  // stage kt+1 is in `after`
        barrier();
    };

    // Stages 0..NS-2 of the item at_item set last, into lds0.. (issued, not
    // waited for).
    auto prologue_copies = [&](int KT) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < NSLOT; ++q) copy(q, 0, lds0);
        if constexpr (NS == 4) {
#pragma unroll
            for (int q = 0; q < NSLOT; ++q) copy(q, min(1, KT - 1), lds1);
#pragma unroll
            for (int q = 0; q < NSLOT; ++q) copy(q, min(2, KT - 1), lds2);
        }
    };
    // VMEM instructions a wave issues after its stage-0 copies and before the
    // K loop waits for them: the copies of stages 1..NS-2, and, when the
    // copies were issued ahead of the previous item's epilogue, that
    // epilogue's stores (counted as a quarter of them, should the compiler
    // pair stores).  vmcnt retires in issue order and counts to 63 at most,
    // so waiting down to this many waits for stage 0 and not for the stores
    // issued after it.
    constexpr int NSTORE = (SWI ? NI * (NJ / 2) : NI * NJ) * 16;
    constexpr int WAIT0 = (NS - 2) * NSLOT;
    constexpr int WAIT0_AFTER_EPI = WAIT0 + NSTORE / 4 < 63 ? WAIT0 + NSTORE / 4 : 63;

    // The whole K loop of item `cur`, whose first NS-1 stages have been
    // issued (after_epi: ahead of the previous item's epilogue).  Buffer
    // roles are static (lds0..lds3 are distinct objects, so the compiler sees
    // that a stage's DMA never aliases another stage's reads), hence NS
    // stages per iteration; the body has no data-dependent branches, so the
    // accumulators stay in AGPRs.  On return no copy is in flight in any wave
    // and no wave reads the stages any more: the next item's copies may start.
    auto k_loop = [&](auto sanc, bool after_epi) __attribute__((always_inline)) {
        using S = decltype(sanc);
        wait_lgkm0();
        if (after_epi) wait_vm<WAIT0_AFTER_EPI>();  // stage 0 has landed
        else wait_vm<WAIT0>();
        clear_tail(lds0, 0);
        barrier();
        // f1 (the carried set) starts at zero.
#pragma unroll
        for (int i = 0; i < NI; ++i) f1.a[i] = typename Mma<ELEM>::Frag{};
#pragma unroll
        for (int j = 0; j < NJ; ++j) f1.b[j] = typename Mma<ELEM>::Frag{};
        const int KT = cur.KT;
        int kt = 0;
        using T = std::true_type;
        // The loop runs the stages whose next stage is not the item's last;
        // the last few stages follow it, with the partial-stage check.
        if constexpr (NS == 2) {
            for (; kt + 4 <= KT; kt += 2) {
                stage(S{}, F{}, lds0, lds1, lds1, kt);
                stage(S{}, F{}, lds1, lds0, lds0, kt + 1);
            }
            if (kt < KT) stage(S{}, T{}, lds0, lds1, lds1, kt);
            if (kt + 1 < KT) stage(S{}, T{}, lds1, lds0, lds0, kt + 1);
            if (kt + 2 < KT) stage(S{}, T{}, lds0, lds1, lds1, kt + 2);
        } else {
            for (; kt + 6 <= KT; kt += 4) {
                stage(S{}, F{}, lds0, lds3, lds1, kt);
                stage(S{}, F{}, lds1, lds0, lds2, kt + 1);
                stage(S{}, F{}, lds2, lds1, lds3, kt + 2);
                stage(S{}, F{}, lds3, lds2, lds0, kt + 3);
            }
            if (kt < KT) stage(S{}, T{}, lds0, lds3, lds1, kt);
            if (kt + 1 < KT) stage(S{}, T{}, lds1, lds0, lds2, kt + 1);
            if (kt + 2 < KT) stage(S{}, T{}, lds2, lds1, lds3, kt + 2);
            if (kt + 3 < KT) stage(S{}, T{}, lds3, lds2, lds0, kt + 3);
            if (kt + 4 < KT) stage(S{}, T{}, lds0, lds3, lds1, kt + 4);
            wait_vm0();  // the re-copies of the last stage have landed, in every wave
            barrier();
        }
        // the last stage's carried step
        if constexpr (S::value) sanitize_frags<ELEM, TL>(f1);
#pragma unroll
        for (int t = 0; t < NPIECE; ++t) mfma_one<ELEM, TL>(f1, acc, t / NJ, t % NJ);
    };

    // Fused epilogue of item `cur` (its tile's scale_a, scale_b and bias in
    // set `par` of epi_*).
    auto epilogue = [&]() __attribute__((always_inline)) {
        // 32x32 block layout of the accumulator: lane l holds
        // column l%32 and rows 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.
        // y = fma(acc, sa_m*sb_n, bias_n) with bias_n = -0.0 when there is no
        // bias, which is exactly acc*s (signed zeros included).
        // The tile is written through a buffer resource based at row m0 whose
        // range ends at the last valid row, so stores to rows >= M fall out of
        // range and are dropped; a lane whose column is >= N adds 2^31 to its
        // offsets and drops all of its stores.  One code path serves full and
        // edge tiles.  Stores are non-temporal: the output is written once and
        // should not evict the operand panels other workgroups still stream
        // through L2.
        const int lr = lane & 31, lh = lane >> 5;
        if constexpr (!SWI) {
            if (S > 1) {
                // K split: the item's raw sums to part[split][m][n] (int32 / fp32),
                // through a buffer resource based at row m0 of the split whose
                // range ends at the last valid row, as the fused epilogue below.
                const uint32_t prow = static_cast<uint32_t>(N) * 4;
                const __amdgpu_buffer_rsrc_t rp =
                    make_rsrc(static_cast<char*>(sk.part) + (static_cast<size_t>(cur.split) * M + cur.m0) * prow,
                              min(M - cur.m0, BM) * static_cast<int>(prow));
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int cn = wn * TL::WN + j * 32 + lr;
                    const uint32_t lane_off =
                        cur.n0 + cn < N ? static_cast<uint32_t>(wm * TL::WM + 4 * lh) * prow + static_cast<uint32_t>(cur.n0 + cn) * 4
                                    : 0x80000000u;
#pragma unroll
                    for (int i = 0; i < NI; ++i) {
                        fence();
#pragma unroll
                        for (int g = 0; g < 4; ++g)
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int voff = static_cast<int>(lane_off + static_cast<uint32_t>(i * 32 + 8 * g + e) * prow);
                                const int v = 4 * g + e;
                                uint32_t bits;
                                bits = acc_bits(acc[i][j], v);
                                __builtin_amdgcn_raw_buffer_store_b32(bits, rp, voff, 0, 0);
                            }
                    }
                }
                return;
            }
        }
        constexpr int OB = OUT == FKE_OUT_BF16 ? 2 : 4;  // output bytes per element
        const uint32_t row_bytes = static_cast<uint32_t>(NO) * OB;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(static_cast<char*>(p.C) + static_cast<size_t>(cur.m0) * row_bytes,
                                                    min(M - cur.m0, BM) * static_cast<int>(row_bytes));
        // This lane's epilogue operands, out of LDS into registers in one go:
        // sa[i][g] = scale_a of tile rows wm*WM + 32i + 8g + 4*lh + 0..3, and
        // scale_b / bias of tile column wn*WN + 32j + lane%32.
        EpiOps<NI, NJ> eo;
        eo.template read<TL::WM, TL::WN>(epi_sa[par], epi_sb[par], epi_bias[par], wm, wn, lane);
        if constexpr (SWI) {
            // SwiGLU: block j (gate) and j + NJ/2 (up) of the wave hold output
            // column n0 + wn*WN/2 + 32*j + lane%32; h = swiglu_pair(g, u) of the
            // two canonical epilogue values.
            constexpr int WN = TL::WN;
#pragma unroll
            for (int j = 0; j < NJ / 2; ++j) {
                // tile columns wn*WN + 32j + lr (gate) and that + WN/2 (up)
                const float sbg = eo.sb[j], sbu = eo.sb[j + NJ / 2];
                const float bg = eo.bias[j], bu = eo.bias[j + NJ / 2];
                const int o = cur.n0 + wn * (WN / 2) + j * 32 + lr;
                const uint32_t lane_off = o < NO
                    ? static_cast<uint32_t>(wm * TL::WM + 4 * lh) * row_bytes + static_cast<uint32_t>(o) * OB
                    : 0x80000000u;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    fence();
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const float sav[4] = {eo.sa[i][g][0], eo.sa[i][g][1], eo.sa[i][g][2], eo.sa[i][g][3]};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int v = 4 * g + e;
                            const int voff =
                                static_cast<int>(lane_off + static_cast<uint32_t>(i * 32 + 8 * g + e) * row_bytes);
                            const float yg = __builtin_fmaf(static_cast<float>(static_cast<int32_t>(acc_bits(acc[i][j], v))),
                                                            sav[e] * sbg, bg);
                            const float yu = __builtin_fmaf(
                                static_cast<float>(static_cast<int32_t>(acc_bits(acc[i][j + NJ / 2], v))), sav[e] * sbu, bu);
                            const float h = swiglu_pair(yg, yu);
                            if constexpr (OUT == FKE_OUT_F32)
                                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(h), rc, voff, 0, 2);
                            else
                                __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_rne(h), rc, voff, 0, 2);
                        }
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int cn = wn * TL::WN + j * 32 + lr;  // column within the tile
            const float sbn = eo.sb[j];
            const float bn = eo.bias[j];
            const uint32_t lane_off = cur.n0 + cn < N
                ? static_cast<uint32_t>(wm * TL::WM + 4 * lh) * row_bytes + static_cast<uint32_t>(cur.n0 + cn) * OB
                : 0x80000000u;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                fence();
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float sav[4] = {eo.sa[i][g][0], eo.sa[i][g][1], eo.sa[i][g][2], eo.sa[i][g][3]};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int v = 4 * g + e;
                        const int voff = static_cast<int>(lane_off + static_cast<uint32_t>(i * 32 + 8 * g + e) * row_bytes);
                        float y;
                        int32_t a = 0;
                        if constexpr (ELEM == ELEM_I8) {
                            a = static_cast<int32_t>(acc_bits(acc[i][j], v));
                            y = __builtin_fmaf(static_cast<float>(a), sav[e] * sbn, bn);
                        } else if constexpr (ELEM == ELEM_F8) {
                            y = __builtin_fmaf(__uint_as_float(acc_bits(acc[i][j], v)), p.sa * p.sb, bn);
                        } else {
                            y = __builtin_fmaf(__uint_as_float(acc_bits(acc[i][j], v)), sav[e] * sbn, bn);
                        }
                        if constexpr (OUT == FKE_OUT_F32)
                            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), rc, voff, 0, 2);
                        else if constexpr (OUT == FKE_OUT_BF16)
                            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_rne(y), rc, voff, 0, 2);
                        else
                            __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(a), rc, voff, 0, 2);
                    }
                }
            }
        }
    };

    // Persistent walk: workgroup b takes items b, b + G, b + 2G, ... (G = grid
    // size, a multiple of the XCD count, so every tile of a workgroup stays on
    // its XCD and each XCD walks its tile range in the same order as a
    // one-tile-per-workgroup launch would).  The next item's first stages and
    // epilogue operands are requested as soon as this item's K loop is done,
    // ahead of its epilogue: they arrive while the epilogue runs, and the next
    // K loop does not wait behind the epilogue's stores.
    at_item(cur);
    load_epi(cur, par);  // (issued before the stage copies: waited for with stage 0)
    prologue_copies(cur.KT);
    if (tid == 0) redo = 0;  // visible after the K loop's first barrier
    bool after_epi = false;
    for (;;) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

        if constexpr (ELEM != ELEM_F8) {
            k_loop(F{}, after_epi);
        } else {
            // E4M3 0x7F/0xFF are NaN to the MFMA but 0.0 to the reference.
            // Clearing them costs ~5 VALU per operand word, more than the MFMAs
            // can hide, and real quantizers never emit them (they saturate at
            // 448).  So run the K loop on the raw codes first: every product is
            // finite and no sum can overflow, so a NaN accumulator proves a
            // NaN code in the tile's rows or columns.  Only then does the
            // workgroup run the loop again with the codes cleared.
            k_loop(F{}, after_epi);
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) t += __uint_as_float(acc_bits(acc[i][j], v));
            if (__builtin_isnan(t)) redo = 1;  // benign race: every writer stores 1
            wait_lgkm0();
            barrier();
            if (redo) {
#pragma unroll
                for (int i = 0; i < NI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
                prologue_copies(cur.KT);  // the copy plans still point at this item
                k_loop(std::true_type{}, false);
            }
        }

        const int next = slot + static_cast<int>(gridDim.x);
        const bool more = next < items;
        Item nx = cur;
        if (more) {
            nx = item_of(next);
            at_item(nx);
            load_epi(nx, par ^ 1);
            prologue_copies(nx.KT);
        }
        epilogue();
        if (!more) break;
        barrier();  // every wave has read this item's redo flag
        // redo = 0 for the next item, written by an inline ds_write: the compiler
        // would hold its own LDS store until the copies in flight had landed
        if (tid == 0) asm volatile("ds_write_b32 %0, %1" ::"v"((__attribute__((address_space(3))) int*)&redo), "v"(0)
                                   : "memory");
        cur = nx;
        slot = next;
        par ^= 1;
        after_epi = true;
    }
}


// The second kernel of a K split: the thread of output (m, n) (grid: column
// blocks x M) adds the S partial sums of idx = m * N + n in the order
// s = 0..S-1 (INT8: exact int32; FP8: fp32 in that fixed order) and applies
// the fused epilogue's arithmetic:
// y = fmaf(sum, sa_m * sb_n, bias_n) (FP8: fmaf(sum, sa * sb, bias_n)), bias_n
// = -0.0 without a bias, as the fused epilogue does.
template <int ELEM, int OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs p, SplitK sk) {
    using AccE = typename std::conditional<ELEM == ELEM_I8, int32_t, float>::type;
    const int64_t mn = static_cast<int64_t>(p.M) * p.N;
    const int m = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;  // grid: column blocks x M
    if (n >= p.N) return;
    const int64_t idx = static_cast<int64_t>(m) * p.N + n;
    const AccE* part = static_cast<const AccE*>(sk.part);
    AccE v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = t < sk.S ? part[t * mn + idx] : AccE(0);
    AccE sum = v[0];
#pragma unroll
    for (int t = 1; t < 8; ++t)
        if (t < sk.S) sum += v[t];
    const float bn = p.bias ? p.bias[n] : -0.0f;
    float y;
    int32_t a = 0;
    if constexpr (ELEM == ELEM_I8) {
        a = sum;
        const float sam = p.scale_a ? p.scale_a[m] : p.sa, sbn = p.scale_b ? p.scale_b[n] : p.sb;
        y = __builtin_fmaf(static_cast<float>(a), sam * sbn, bn);
    } else {
        y = __builtin_fmaf(sum, p.sa * p.sb, bn);
    }
    store_out<OUT>(p.C, static_cast<size_t>(idx), y, a);
}

template <int ELEM, int BL, int OUT, bool SWI, class TL>
hipError_t launch_t(const GemmArgs& p, hipStream_t stream, int cus, const SplitK& sk) {
    constexpr int TC = tile_cols<SWI, TL>();
    const int gm = (p.M + TL::BM - 1) / TL::BM, gn = ((SWI ? p.N / 2 : p.N) + TC - 1) / TC;
    const int grid = min(gm * gn * sk.S, cus / NXCD * NXCD * TL::OCC);
    if (sk.S > 1 && (SWI || elem_bytes(ELEM) != 1 || sk.part == nullptr)) return hipErrorInvalidValue;
    GemmArgs a = p;
    SplitK k = sk;
    void* args[] = {&a, &k};
    // One row of tiles reads each B byte once: non-temporal B copies (8-bit
    // operands on the ring tiles, the batched-decode shapes).  Measured at
    // N = 14336, K = 4096, cold weights: M = 64 on the 64x64 ring 16.6 -> 15.4
    // us, M = 128 on the 128x64 ring 19.7 -> 19.2; with more tile rows the
    // panel is re-read from L2 and non-temporal copies lose (4096x1376x4096:
    // 27.6 against 46.6 us).
    const void* f = reinterpret_cast<const void*>(&gemm_mfma_kernel<ELEM, BL, OUT, SWI, TL>);
    if constexpr (TL::NS == 4 && elem_bytes(ELEM) == 1)
        if (gm == 1) f = reinterpret_cast<const void*>(&gemm_mfma_kernel<ELEM, BL, OUT, SWI, TL, true>);
    const hipError_t e = hipLaunchKernel(f, dim3(grid), dim3(NTHREADS), args, 0, stream);
    if (e != hipSuccess || sk.S == 1) return e;
    if constexpr (!SWI && elem_bytes(ELEM) == 1) {
        // (a split plan has at most one ring tile per CU and split: M is far below grid.y's 65536)
        return hipLaunchKernel(reinterpret_cast<const void*>(&splitk_reduce_kernel<ELEM, OUT>),
                               dim3((p.N + 255) / 256, p.M), dim3(256), args, 0, stream);
    }
    return hipErrorInvalidValue;  // not reached: checked before the launch
}

template <int ELEM, int BL, int OUT, bool SWI = false>
hipError_t launch_tile(const GemmArgs& p, hipStream_t s, int tile, int cus, const SplitK& sk) {
    switch (tile) {
        case MFMA_TILE_128x128: return launch_t<ELEM, BL, OUT, SWI, T128>(p, s, cus, sk);
        case MFMA_TILE_128x128_RING4: return launch_t<ELEM, BL, OUT, SWI, T128R4>(p, s, cus, sk);
        case MFMA_TILE_128x64_RING4:
            if constexpr (!SWI) return launch_t<ELEM, BL, OUT, SWI, T128x64R4>(p, s, cus, sk);
            return hipErrorInvalidValue;
        case MFMA_TILE_64x64_RING4:
            if constexpr (!SWI) return launch_t<ELEM, BL, OUT, SWI, T64R4>(p, s, cus, sk);
            return hipErrorInvalidValue;
        default: return launch_t<ELEM, BL, OUT, SWI, T256>(p, s, cus, sk);
    }
}

template <int ELEM, int BL>
hipError_t launch_out(const GemmArgs& p, hipStream_t s, int tile, int cus, const SplitK& sk) {
    switch (p.out_dtype) {
        case FKE_OUT_F32: return launch_tile<ELEM, BL, FKE_OUT_F32>(p, s, tile, cus, sk);
        case FKE_OUT_BF16: return launch_tile<ELEM, BL, FKE_OUT_BF16>(p, s, tile, cus, sk);
        default:
            if constexpr (ELEM == ELEM_I8) return launch_tile<ELEM, BL, FKE_OUT_I32>(p, s, tile, cus, sk);
            return hipErrorInvalidValue;
    }
}

}  // namespace

// Read once per device and kept (0: not read yet).
int device_cus() {
    static std::atomic<int> known[64];
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (dev >= 0 && dev < 64 && (cus = known[dev].load(std::memory_order_relaxed)) > 0) return cus;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < NXCD)
        return 256;
    if (dev >= 0 && dev < 64) known[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

bool mfma_supports(const GemmArgs& p, int elem) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    const int64_t kb = static_cast<int64_t>(p.K) * elem_bytes(elem);  // K bytes per row
    // rows start 16-byte aligned; a last stage shorter than BK is cleared past K
    if (p.M < 1 || p.N < 1 || kb < 16 || kb % 16 != 0) return false;
    if ((a | b) & 15) return false;
    // per-lane DMA offsets are 32-bit: (rows - 1) * K + K must fit
    if (p.M * kb > INT32_MAX) return false;
    if (p.N * kb > INT32_MAX) return false;
    // 16-bit operands: B [N,K] only (the transposed LDS reads are byte-wise)
    if (elem_bytes(elem) == 2 && p.b_layout != FKE_B_NK) return false;
    if (p.b_layout == FKE_B_KN && (p.N % 16 != 0)) return false;
    if (p.swiglu && (elem != ELEM_I8 || p.b_layout != FKE_B_NK)) return false;
    // epilogue offsets are 32-bit: 256 output rows plus the 2^31 drop offset
    if (p.N > (1 << 20)) return false;
    return true;
}

// Tile for a shape on `cus` CUs (`bench.py --tile-sweep`: 23 shapes, INT8,
// FP8 and bf16, weights cache-warm and cold, B [N,K]; times below are INT8,
// cold weights, bf16 out).
// - The tiles fit the CUs one each: a 4-stage ring, the smallest tile whose
//   count fits (64x64, else 128x64, else 128x128; SwiGLU pairs need 128
//   columns).  A lone tile is bound by the bytes its CU loads, (BM + BN) * K,
//   at about 45 GB/s per CU, and waits on every stage's copy unless several
//   are in flight: 512x1792x4096 runs 12.0 us on 64x64, 14.6 on 128x64, 19.8
//   on 128x128, 30.2 on 128x128 with two stages; 128x14336x4096 (64x64 would
//   be 448 tiles) 20.3 on 128x64 against 26.5 on 128x128.
// - Fewer 256x256 tiles than CUs, and 128x128 tiles that fit one round of
//   two per CU: 128x128 with two stages, two workgroups per CU
//   (4096x1376x4096: 37.9 us against 41.2 on the 128x64 ring, 42.5 on the
//   128x128 ring and 51.3 on 256x256).
// - Everything else: 256x256, which reads the fewest operand bytes per MFMA
//   (3072x4096x4096: 55.8 against 60.3 us; 4096x11008x4096: 181 against
//   243).  That includes short K: two 128x128 workgroups per CU hide a short
//   tile's prologue and epilogue, but fetch each weight panel twice as often,
//   which loses once the weights come from HBM (8192x8192x1024: 105 against
//   120 us cold, though 99 against 103 warm).
// - One row of tiles with more tiles than CUs (decode batches against a large
//   N, e.g. an LM head): the smallest tile height that holds M, over several
//   rounds, rather than 256x256 rows of mostly padding.  M <= 64: the 64x64
//   ring (64x65536x4096: 59.9 us against 89.6 on 256x256; 64x128256: 116.7
//   against 152.3), unless one round of the 128x128 ring leaves an eighth of
//   the CUs or more idle (64x16896: 23.5 against 27.5 on 64x64, but
//   64x32768: 35.0 against 31.8).  M <= 128: 128x128 tiles at two per CU
//   (128x49152: 58.1 against 70.3; 128x65536: 72.0 against 82.3).  Past 128
//   rows 256x256 stays ahead (256x65536: 86.6 against 104.5 on 128x128).
// A 256x128 tile (one workgroup per CU) measured slower than 128x128 on every
// few-tile shape, INT8, FP8 and bf16.  B [K,N] uses the same rule.
int mfma_pick_tile(const GemmArgs& p, int cus) {
    const int64_t NO = p.swiglu ? p.N / 2 : p.N;
    auto tiles = [&](int64_t bm, int64_t bn) {
        const int64_t tc = p.swiglu ? bn / 2 : bn;
        return (p.M + bm - 1) / bm * ((NO + tc - 1) / tc);
    };
    if (!p.swiglu && tiles(64, 64) <= cus) return MFMA_TILE_64x64_RING4;
    const int64_t t128 = tiles(128, 128);
    if (!p.swiglu && p.M <= 64)
        return t128 * 8 <= static_cast<int64_t>(cus) * 7 ? MFMA_TILE_128x128_RING4 : MFMA_TILE_64x64_RING4;
    if (!p.swiglu && tiles(128, 64) <= cus) return MFMA_TILE_128x64_RING4;
    if (t128 <= cus) return MFMA_TILE_128x128_RING4;
    if (!p.swiglu && p.M <= 128) return MFMA_TILE_128x128;
    if (tiles(256, 256) < cus && t128 <= 2 * static_cast<int64_t>(cus)) return MFMA_TILE_128x128;
    return MFMA_TILE_256x256;
}

// Time (us) of the MFMA GEMM on an 8-bit B [N,K] shape, for the choice
// between it and the streamed decode kernel (cold weights, bf16 out; fitted on
// N = 1792..14336, K = 4096 and 14336, M = 16..512, within about 20 %).
// Ring tiles: the larger of the bytes one CU loads, (BM + BN) * K per round of
// tiles, at 44 GB/s and the weights at 4.2 TB/s (4.5 TB/s past two rounds:
// 64x65536x4096 ran 59.9 us, 64x128256x4096 116.7), plus 1 us.  128x128 with two stages: about
// 1 us per stage per round of two tiles per CU.  256x256: 1.35 us per stage
// and 11 us per round of tiles.
namespace {

double mfma_unsplit_estimate_us(const GemmArgs& p, int cus) {
    const double kt = p.K / 128.0;
    const int64_t NO = p.swiglu ? p.N / 2 : p.N;
    auto ring = [&](int64_t bm, int64_t bn) {
        const int64_t tc = p.swiglu ? bn / 2 : bn;
        const double rounds = static_cast<double>(((p.M + bm - 1) / bm * ((NO + tc - 1) / tc) + cus - 1) / cus);
        return std::max(static_cast<double>(bm + bn) * p.K * rounds / 44.0e3,
                        static_cast<double>(p.N) * p.K / (rounds > 2 ? 4.5e6 : 4.2e6)) + 1.0;
    };
    switch (mfma_pick_tile(p, cus)) {
        case MFMA_TILE_64x64_RING4: return ring(64, 64);
        case MFMA_TILE_128x64_RING4: return ring(128, 64);
        case MFMA_TILE_128x128_RING4: return ring(128, 128);
        case MFMA_TILE_128x128: {
            const int64_t tc = p.swiglu ? 64 : 128;
            const double t = static_cast<double>((int64_t{p.M} + 127) / 128 * ((NO + tc - 1) / tc));
            return 1.05 * kt + 6.0 * t / cus;
        }
        default: {
            const int64_t tc = p.swiglu ? 128 : 256;
            const int64_t t = (int64_t{p.M} + 255) / 256 * ((NO + tc - 1) / tc);
            return static_cast<double>((t + cus - 1) / cus) * (1.35 * kt + 11.0);
        }
    }
}

constexpr int kSplitMax = 8;                            // splits of one tile's K range
constexpr int kSplitMinStages = 4;                      // BK stages per split, at least
constexpr size_t kSplitMaxBytes = FKE_SPLIT_SLOT_BYTES; // partial sums of all splits: one split-pool slot

// One round of bm x bn ring tiles (count <= CUs), each summing ks_bytes of
// K, measured on one-round shapes (cold weights, bf16 out): the bytes one CU
// loads, (bm + bn) * ks_bytes, at 80 GB/s when two or more tile rows share
// each B panel in L2 and 52 GB/s for one tile row (B [K,N]: 48 GB/s); a K
// split's items at 55 and 42 GB/s (shorter K ranges, more of them in flight);
// the weights at 4.2 TB/s, half as much again with two or more tile rows (the
// rows' workgroups do not share every panel in L2); plus 1 us.  Unsplit
// 64x64: 64x4096x14336 36.5 us, 128x4096x14336 24.6, 128x8192x28672 80.8;
// split: 64x4096x14336 20.3 (64x64, 3 splits), 128x8192x28672 65.6 (128x128,
// 3 splits), 100x1000x14720 10.9 (64x64, 8 splits).
double ring_round_us(const GemmArgs& p, int bm, int bn, int64_t ks_bytes, bool split) {
    const int64_t gm = (int64_t{p.M} + bm - 1) / bm;
    const double rate = split ? (gm >= 2 ? 55.0e3 : 42.0e3)
                              : (p.b_layout == FKE_B_KN ? 48.0e3 : (gm >= 2 ? 80.0e3 : 52.0e3));
    const double weights = static_cast<double>(p.N) * p.K * (gm >= 2 ? 1.5 : 1.0) / 4.2e6;
    return std::max(static_cast<double>(bm + bn) * ks_bytes / rate, weights) + 1.0;
}

// Time (us) of a K split on ring tiles bm x bn: the first kernel's round, then
// the partial sums written and read back once at about 4 TB/s, the output
// written, and 3 us for the second launch.
double split_estimate_us(const GemmArgs& p, int bm, int bn, int S, int KS) {
    const double mn = static_cast<double>(p.M) * p.N;
    return ring_round_us(p, bm, bn, static_cast<int64_t>(KS) * BK, true) + 3.0 +
           (2.0 * S * mn * 4.0 + mn * (p.out_dtype == FKE_OUT_BF16 ? 2 : 4)) / 4.0e6;
}

int ring_bm(int tile) { return tile == MFMA_TILE_64x64_RING4 ? 64 : 128; }
int ring_bn(int tile) { return tile == MFMA_TILE_128x128_RING4 ? 128 : 64; }

}  // namespace

size_t mfma_split_bytes(const GemmArgs& p, int S) {
    return static_cast<size_t>(S) * static_cast<size_t>(p.M) * static_cast<size_t>(p.N) * 4;
}

// K split of an 8-bit GEMM with few tiles and a long K: a ring tile whose
// count, times S, still fits one round of the CUs, each item summing KS of
// the K stages.  Every ring tile and S = 2..8 (at least four stages a split,
// at most 32 MiB of partial sums) is priced by split_estimate_us; the best is
// taken when it is under 0.85 of the unsplit time (ring_round_us for one
// round of ring tiles).
MfmaPlan mfma_plan(const GemmArgs& p, int elem, int cus) {
    MfmaPlan pl{mfma_pick_tile(p, cus), 1, 0};
    if (p.swiglu || elem_bytes(elem) != 1) return pl;
    const int KT = static_cast<int>((static_cast<int64_t>(p.K) * elem_bytes(elem) + BK - 1) / BK);
    double base = mfma_unsplit_estimate_us(p, cus);
    if (pl.tile == MFMA_TILE_64x64_RING4 || pl.tile == MFMA_TILE_128x64_RING4 || pl.tile == MFMA_TILE_128x128_RING4) {
        const int bm = ring_bm(pl.tile), bn = ring_bn(pl.tile);
        if ((int64_t{p.M} + bm - 1) / bm * ((int64_t{p.N} + bn - 1) / bn) <= cus)
            base = ring_round_us(p, bm, bn, p.K, false);
    }
    double best = 0.85 * base;
    const struct { int tile, bm, bn; } rings[] = {{MFMA_TILE_64x64_RING4, 64, 64},
                                                  {MFMA_TILE_128x64_RING4, 128, 64},
                                                  {MFMA_TILE_128x128_RING4, 128, 128}};
    for (const auto& r : rings) {
        const int64_t t = (int64_t{p.M} + r.bm - 1) / r.bm * ((int64_t{p.N} + r.bn - 1) / r.bn);
        for (int S = 2; S <= kSplitMax && t * S <= cus; ++S) {
            const int KS = (KT + S - 1) / S;
            if (KS < kSplitMinStages) break;
            const int s = (KT + KS - 1) / KS;  // splits that have stages
            if (mfma_split_bytes(p, s) > kSplitMaxBytes) break;
            const double e = split_estimate_us(p, r.bm, r.bn, s, KS);
            if (e < best) {
                best = e;
                pl = MfmaPlan{r.tile, s, KS};
            }
        }
    }
    return pl;
}

double mfma_time_estimate_us(const GemmArgs& p, int cus) {
    const MfmaPlan pl = mfma_plan(p, ELEM_I8, cus);
    if (pl.S == 1) return mfma_unsplit_estimate_us(p, cus);
    return split_estimate_us(p, ring_bm(pl.tile), ring_bn(pl.tile), pl.S, pl.KS);
}

hipError_t launch_mfma(const GemmArgs& p, int elem, hipStream_t s, int tile, const SplitK& sk) {
    const int cus = device_cus();
    if (tile == MFMA_TILE_AUTO) tile = mfma_pick_tile(p, cus);
    if (sk.S < 1 || sk.S > kSplitMax) return hipErrorInvalidValue;
    if (sk.S > 1) {  // every split has stages: the last starts before K ends
        if (p.swiglu || elem_bytes(elem) != 1 || sk.part == nullptr || sk.KS < 1) return hipErrorInvalidValue;
        if (static_cast<int64_t>(sk.S - 1) * sk.KS >= (p.K + BK - 1) / BK) return hipErrorInvalidValue;
    }
    if (elem == ELEM_F16 || elem == ELEM_BF16) {
        GemmArgs q = p;
        q.K = 2 * p.K;  // the kernel walks K bytes
        return elem == ELEM_F16 ? launch_out<ELEM_F16, FKE_B_NK>(q, s, tile, cus, sk)
                                : launch_out<ELEM_BF16, FKE_B_NK>(q, s, tile, cus, sk);
    }
    if (p.swiglu)
        return p.out_dtype == FKE_OUT_F32 ? launch_tile<ELEM_I8, FKE_B_NK, FKE_OUT_F32, true>(p, s, tile, cus, sk)
                                          : launch_tile<ELEM_I8, FKE_B_NK, FKE_OUT_BF16, true>(p, s, tile, cus, sk);
    if (elem == ELEM_I8)
        return p.b_layout == FKE_B_NK ? launch_out<ELEM_I8, FKE_B_NK>(p, s, tile, cus, sk)
                                      : launch_out<ELEM_I8, FKE_B_KN>(p, s, tile, cus, sk);
    return p.b_layout == FKE_B_NK ? launch_out<ELEM_F8, FKE_B_NK>(p, s, tile, cus, sk)
                                  : launch_out<ELEM_F8, FKE_B_KN>(p, s, tile, cus, sk);
}

}  // namespace fke
