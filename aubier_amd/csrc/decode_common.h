// decode_common.h -- the parts shared by the split-K kernels over an f16 cache (kqkv_decode.hip,
// and in part the prefill and 8-bit cache kernels): the KV slice geometry and its LDS slot layout,
// the slice DMA, the q staging prologue, the Q.K^T step, P.V and the end of a split.
//
// A split is a run of whole 64-key tiles; wave w of the workgroup owns keys 16 w .. 16 w + 15 of
// every tile (its "slice") and streams them into its own slot of a two-stage LDS ring by bounds-
// checked LDS DMA (buffer_load_dwordx4 ... lds: no staging registers; rows at or past n_kv read as
// zeros).  The workgroup covers a 32-head group; q enters Q.K^T as f16 fragments held in VGPRs.
#pragma once

#include <type_traits>

#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {
namespace decode {

constexpr int TK = 64;          // keys per split tile (splits are whole tiles)
constexpr int NWAVE = 4;
constexpr int NTHR = 64 * NWAVE;
constexpr int WK = TK / NWAVE;  // keys per wave slice
constexpr int HG = 32;          // heads per workgroup
constexpr float LAZY = 15.0f;   // log2 slack before a reference max moves: P = 2^(s - m) <= 2^15,
                                // exact in f16 (max 65504); a move rescales every accumulator
// The lazily moved reference max of a head with no live key yet: below every finite score, so a
// live key always moves it and exp2(s - M_NONE) of a masked key (s = -inf) is 0 without a special
// case; a head still at M_NONE after the split had no live key (recorded as -inf).
constexpr float M_NONE = -3.402823466e38f;      // -FLT_MAX
constexpr half2 ONE2 = {1.0f16, 1.0f16};

template <int DK>
struct SliceGeom {
    static_assert(DK % 64 == 0, "geometry");
    static constexpr int CH = DK * 2 / 16;              // 16-byte chunks per cache row
    static_assert(CH % 8 == 0, "1 KB slot blocks of 8 rows x 8 chunks");
    static constexpr int DMA_N = WK * CH / 64;          // 16-byte DMA instructions per slice
    static constexpr int ROWS_BYTES = WK * DK * 2;
    static constexpr int STAGE = ROWS_BYTES + 256;      // 16 K rows + the mask slot
    static constexpr int RING = 2 * NWAVE * STAGE;
    static constexpr int QSTEPS = DK / 32;              // K-steps of the 16x16x32 MFMA
    static constexpr int QC = DK / 4;                   // 16-byte f32 chunks per q row
    static constexpr int QD = HG * QC / 64 / NWAVE;     // q DMA instructions per wave
    static_assert(QC % 16 == 0 && (HG * QC) % (64 * NWAVE) == 0, "q staging swizzle, whole q DMA instructions");
    static_assert(HG * DK * 4 <= NWAVE * STAGE, "the f32 q staging fits stage 1 of the ring");
    static_assert(QSTEPS == DMA_N, "one DMA block per Q.K^T step");
};

// Slot layout (one wave slice, 16 cache rows of CH 16-byte chunks): 1 KB blocks b = 0 .. CH/4 - 1,
// block b holding rows 8 (b & 1) .. +7 and chunks 8 (b >> 1) .. +7 -- one 128-byte segment of each
// of 8 rows, row r at 128 (r & 7), its chunk c at slot (c ^ r) & 7 of the segment.  DMA instruction
// b fills block b (lane l -> slot l), so quarter-wave qq fetches rows 2 qq, 2 qq + 1 as two whole
// 128-byte segments: whole cache lines per request (a layout that splits each line over two
// instructions streams ~20% slower per CU).  The XOR by the row was chosen by measurement on gfx950
// (LDS read probes with the bank-conflict counters): Q.K^T's 16-row operand reads run at the rate of
// linear ds_read_b128 (192 vs 196 B/clk per CU; a permuted-row swizzle that is conflict-free in a
// plain 64-bank model reached 128) and the P.V transpose reads at 128 B/clk (linear: 141).  Chunk
// c + 4 of a row (c & 4 == 0) is at the byte offset of chunk c XOR 64, chunk c + 8 at + 2048.
__device__ __forceinline__ int row_sw(int r) { return r & 7; }
__device__ __forceinline__ int slot_byte(int r, int c) {
    return 1024 * (2 * (c >> 3) + (r >> 3)) + 128 * (r & 7) + 16 * ((c & 7) ^ row_sw(r));
}

// Where the V^T / V operand of P.V comes from: two transpose reads per 32-column tile, in 16-lane
// group g lane j supplying row 8 (g >> 1) + (j >> 2) (then + 4) of a slice, 4 columns at
// 32 i + 16 (g & 1) + 4 (j & 3).  Lane l then holds column 32 i + (l & 31), keys 8 (l >> 5) .. +7.
struct PvAddr {
    int lo, hi;                              // tile 0 (chunks 0 .. 3)
    __device__ __forceinline__ explicit PvAddr(int lane) {
        const int g = lane >> 4, j16 = lane & 15;
        const int r0 = 8 * (g >> 1) + (j16 >> 2);
        const int cq = 2 * (g & 1) + ((j16 & 3) >> 1);
        lo = slot_byte(r0, cq) + 8 * (j16 & 1);
        hi = slot_byte(r0 + 4, cq) + 8 * (j16 & 1);
    }
    // the operand of 32-column tile i (chunks 4 i .. 4 i + 3) of the slice at sb
    __device__ __forceinline__ half8 load(const char * sb, int i) const {
        const int x = 64 * (i & 1), o = 2048 * (i >> 1);
        const half4 l4 = lds_read_tr16(reinterpret_cast<const half_t *>(sb + (lo ^ x) + o));
        const half4 h4 = lds_read_tr16(reinterpret_cast<const half_t *>(sb + (hi ^ x) + o));
        return half8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
    }
};

struct SliceDma { i32x4 krs, mrs; uint32_t sb; };

// The wave's view of its split: tile range, DMA of its slice of tile k into stage s.
template <int DK>
struct SliceStream {
    using G = SliceGeom<DK>;
    const char * kc;
    int64_t kc_nb1;
    const float * mrow;     // this token's mask row (or any valid pointer when there is none)
    bool has_mask;
    int n_kv, n_tiles, t0, n_my, w;
    uint32_t ring_lds, kvoff0, kvoff1, mvoff;  // lane offsets of even / odd row blocks, of the mask

    __device__ __forceinline__ SliceStream(const DecodeArgs & a, int sp, int t, int w_, uint32_t ring_lds_, int lane) {
        kc = a.kc;
        kc_nb1 = a.kc_nb1;
        has_mask = a.mask != nullptr;
        mrow = has_mask ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1) : a.q;
        n_kv = a.n_kv;
        n_tiles = a.n_tiles;
        // balanced partition of whole 64-key tiles over the splits
        const int base_t = a.n_tiles / a.n_split;
        const int rem = a.n_tiles % a.n_split;
        t0 = sp * base_t + min(sp, rem);
        n_my = base_t + (sp < rem ? 1 : 0);
        w = w_;
        ring_lds = ring_lds_;
        // lane l = 16 qq + 8 h + x of block b: row 8 (b & 1) + 2 qq + h, chunk 8 (b >> 1) + (x ^ row_sw(row))
        const int r0 = 2 * (lane >> 4) + ((lane >> 3) & 1);
        kvoff0 = (uint32_t)(r0 * kc_nb1) + 16u * (uint32_t)((lane & 7) ^ row_sw(r0));
        kvoff1 = (uint32_t)((r0 + 8) * kc_nb1) + 16u * (uint32_t)((lane & 7) ^ row_sw(r0 + 8));
        mvoff = 4u * (uint32_t)(lane & 15);
    }
    __device__ __forceinline__ int stage_off(int s, int v) const { return (s * NWAVE + v) * G::STAGE; }
    // The resources are rebased on the slice, num_records = bytes up to the end of row n_kv - 1, so
    // rows (and mask entries) at or past n_kv come back as zeros.  k is clamped into the split (a
    // split with no tile re-reads a valid one and never uses it).
    __device__ __forceinline__ SliceDma plan(int s, int k) const {
        const int tile = min(t0 + min(k, n_my - 1), n_tiles - 1);
        const int key0 = tile * TK + WK * w;
        const int left = n_kv - key0;                    // rows of this slice that exist (may be <= 0)
        SliceDma d;
        d.krs = make_rsrc(kc + (int64_t)key0 * kc_nb1, left > 0 ? (uint32_t)((int64_t)(left - 1) * kc_nb1 + DK * 2) : 0u);
        d.mrs = make_rsrc(mrow + key0, (has_mask && left > 0) ? (uint32_t)left * 4u : 0u);
        d.sb = ring_lds + (uint32_t)stage_off(s, w);
        return d;
    }
    // instruction i < DMA_N: block i of the rows (NT: streaming cache policy); i == DMA_N: the mask
    // slot (float l = key key0 + (l & 15))
    template <bool NT = true>
    __device__ __forceinline__ void put(const SliceDma & d, int i) const {
        if (i < G::DMA_N) {
            const uint32_t vo = (i & 1) ? kvoff1 : kvoff0, so = 128u * (uint32_t)(i >> 1);
            if constexpr (NT) dma16_nt(d.krs, vo, so, d.sb + (uint32_t)(1024 * i));
            else dma16(d.krs, vo, so, d.sb + (uint32_t)(1024 * i));
        } else {
            dma4(d.mrs, mvoff, 0u, d.sb + (uint32_t)G::ROWS_BYTES);
        }
    }
};

constexpr int LIVE_ROUND_TILES = 6;  // tiles per round trip of the row-liveness check
constexpr int ROWS_MAX = 16;         // rows (tokens) per workgroup of the decode kernels

// Workgroups along the row axis of a decode launch: rows t = z, z + Z, ... share a workgroup, Z as
// small as keeps ~256 workgroups in flight (one, at 256 splits: batch-of-N decode over per-sequence
// regions then has one live row per split), and at most ROWS_MAX rows per workgroup.
inline int decode_row_groups(const DecodeArgs & a, int n_hgroups) {
    const int per_row = a.n_split * n_hgroups;
    int z = (256 + per_row - 1) / per_row;
    z = z < 1 ? 1 : z;
    const int zmin = (a.nt + ROWS_MAX - 1) / ROWS_MAX;
    z = z < zmin ? zmin : z;
    return z < a.nt ? z : a.nt;
}

// Liveness of this workgroup's rows in split sp: bit i set when row blockIdx.z + i gridDim.z has a
// key with mask > -inf below n_kv in the split.  Wave w checks rows w, w + 4, w + 8, w + 12, MAXT
// tiles of the split per round trip (every load of a round issued before its first compare), until
// the split ends or every row it checks has been found live.
template <int MAXT>
__device__ __forceinline__ uint32_t live_rows_of_wave(const DecodeArgs & a, int sp, int w, int lane) {
    constexpr int RW = ROWS_MAX / NWAVE;
    const int base_t = a.n_tiles / a.n_split, rem = a.n_tiles % a.n_split;
    const int t0 = sp * base_t + min(sp, rem);
    const int n_my = base_t + (sp < rem ? 1 : 0);
    const int k0 = t0 * TK, k1 = min((t0 + n_my) * TK, a.n_kv);
    uint32_t rows = 0;                       // the rows this wave checks
#pragma unroll
    for (int r = 0; r < RW; ++r)
        if ((int)blockIdx.z + (w + NWAVE * r) * (int)gridDim.z < a.nt) rows |= 1u << (w + NWAVE * r);
    uint32_t bits = 0;
    for (int kb = k0; kb < k1 && bits != rows; kb += TK * MAXT) {
        float v[RW][MAXT];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int t = (int)blockIdx.z + (w + NWAVE * r) * (int)gridDim.z;
            const float * row = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) +
                                                                (size_t)min(t, a.nt - 1) * a.mask_nb1);
#pragma unroll
            for (int j = 0; j < MAXT; ++j) {
                const int k = kb + lane + 64 * j;
                v[r][j] = (t < a.nt && k < k1) ? row[k] : -INFINITY;
            }
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            bool live = false;
#pragma unroll
            for (int j = 0; j < MAXT; ++j) live |= v[r][j] != -INFINITY;
            if (__builtin_amdgcn_ballot_w64(live) != 0) bits |= 1u << (w + NWAVE * r);
        }
    }
    return bits;
}

// Whether token t has a live key (mask > -inf, key < n_kv) in the split's tiles: the mask row
// read over the split's range (cached loads, one key per lane per step), OR-ed over the wavefront.
// Every wave of the workgroup computes the same answer.  Without a mask every key below n_kv is live.
template <int DK>
__device__ __forceinline__ bool split_live(const DecodeArgs & a, const SliceStream<DK> & ss, int t, int lane) {
    const int k0 = ss.t0 * TK, k1 = min((ss.t0 + ss.n_my) * TK, a.n_kv);
    if (a.mask == nullptr) return k0 < k1;
    const float * row = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1);
    bool live = false;
    for (int k = k0 + lane; k < k1; k += 64) live |= row[k] != -INFINITY;
    return __builtin_amdgcn_ballot_w64(live) != 0;
}

// The (m, l) pairs of a split with no live key: m = -inf, l = 0 for the record's 32 heads; its o
// block is left unwritten (the merge reads o only where m > -inf).  Lanes 0..31 of one wave.
__device__ __forceinline__ void write_empty_pairs(const DecodeArgs & a, int g, int t, int sp, int dv, int lane) {
    if (lane < HG) {
        char * rec = part_record(a.part, g, a.nt, t, a.n_split, dv, 2);
        *reinterpret_cast<f32x2 *>(rec + part_ml_off(a.n_split, lane, sp)) = f32x2{-INFINITY, 0.0f};
    }
}

// q block DMA: this wave's share of the 32 heads x DK f32 q rows of token t into the staging area
// at LDS address qsb, f32 chunk c of head h at slot h * QC + (c ^ (h & 15)) (so that the fragment
// reads of q_convert, 16 heads at one chunk, hit distinct banks); heads past n_head read as zeros.
// QD instructions per wave.
template <int DK>
__device__ __forceinline__ void q_dma(const DecodeArgs & a, uint32_t qsb, int hg0, int t, int w, int lane) {
    using G = SliceGeom<DK>;
    const int nh = min(HG, a.n_head - hg0);
    const i32x4 qrs = make_rsrc(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 + (size_t)hg0 * a.q_nb1,
                                (uint32_t)((int64_t)(nh - 1) * a.q_nb1 + DK * 4));
#pragma unroll
    for (int i = 0; i < G::QD; ++i) {
        const int p = (w * G::QD + i) * 64 + lane;
        const int h = p / G::QC;
        const int c = (p - h * G::QC) ^ (h & 15);
        dma16(qrs, (uint32_t)(h * a.q_nb1) + 16u * (uint32_t)c, 0u, qsb + (uint32_t)((w * G::QD + i) * 1024));
    }
}

// The staged q block (q_dma's layout at qs) -> f16 B fragments in registers: qreg[n][s] = head
// 16 n + j16, d = 32 s + 8 g .. +7.
template <int DK>
__device__ __forceinline__ void q_convert(const char * qs_lds, int lane, half8 (&qreg)[2][SliceGeom<DK>::QSTEPS]) {
    using G = SliceGeom<DK>;
    const int g = lane >> 4, j16 = lane & 15;
    // reads in batches of QB fragments ahead of their conversion (a read-convert chain per
    // fragment would serialise on the LDS latency)
    constexpr int QB = G::QSTEPS % 6 == 0 ? 6 : (G::QSTEPS % 5 == 0 ? 5 : 2);
    static_assert(G::QSTEPS % QB == 0, "whole batches");
    const float * qs = reinterpret_cast<const float *>(qs_lds);
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        const float * row = qs + 4 * (16 * n + j16) * G::QC;
#pragma unroll
        for (int s0 = 0; s0 < G::QSTEPS; s0 += QB) {
            f32x4 x[QB][2];
#pragma unroll
            for (int b = 0; b < QB; ++b) {
                x[b][0] = *reinterpret_cast<const f32x4 *>(row + 4 * ((8 * (s0 + b) + 2 * g) ^ j16));
                x[b][1] = *reinterpret_cast<const f32x4 *>(row + 4 * ((8 * (s0 + b) + 2 * g + 1) ^ j16));
            }
#pragma unroll
            for (int b = 0; b < QB; ++b) {
                half8 h = {to_half(x[b][0][0]), to_half(x[b][0][1]), to_half(x[b][0][2]), to_half(x[b][0][3]),
                           to_half(x[b][1][0]), to_half(x[b][1][1]), to_half(x[b][1][2]), to_half(x[b][1][3])};
                // materialise the f16 fragment here: left alone, the compiler keeps the f32
                // values (twice the registers) and re-converts them at every use in the loop
                asm volatile("" : "+v"(h));
                qreg[n][s0 + b] = h;
            }
        }
    }
}

// q block (32 heads x DK f32) -> stage 1 of the ring by DMA, tile 0's slice -> stage 0 behind it,
// then f16 B fragments in registers (q_convert).  Ends with a barrier after which stage 1 is free;
// the slice DMA of tile 0 (DMA_N + 1 instructions) may still be in flight.
template <int DK>
__device__ __forceinline__ void stage_q(const DecodeArgs & a, const SliceStream<DK> & ss, char * ring, int hg0, int t,
                                        int lane, half8 (&qreg)[2][SliceGeom<DK>::QSTEPS]) {
    using G = SliceGeom<DK>;
    q_dma<DK>(a, ss.ring_lds + (uint32_t)(NWAVE * G::STAGE), hg0, t, ss.w, lane);
    {
        const SliceDma d0 = ss.plan(0, 0);
#pragma unroll
        for (int i = 0; i <= G::DMA_N; ++i) ss.put(d0, i);
    }
    wait_vm<G::DMA_N + 1>();                 // this wave's part of q has landed
    __syncthreads();
    q_convert<DK>(ring + NWAVE * G::STAGE, lane, qreg);
    __syncthreads();                         // the q staging in stage 1 is free again
}

// acc += a . b (v_mfma_f32_16x16x32_f16; first: acc = a . b).  VACC keeps acc in VGPRs through
// inline asm: in the kernels whose output accumulators fill all 256 AGPRs the compiler selects the
// AGPR form for every MFMA and would move an output tile out to VGPRs and back around each Q.K^T
// (48 v_accvgpr moves per slice).  Inline asm is outside the compiler's hazard tracking, so the
// caller covers the MFMA -> VALU read distance (vacc_settle) before it reads the result.
template <bool VACC>
__device__ __forceinline__ void mfma16(f32x4 & acc, const half8 & a, const half8 & b, bool first) {
    if constexpr (VACC) {
        if (first) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b));
        else asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
    } else {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, first ? f32x4{0.f, 0.f, 0.f, 0.f} : acc, 0, 0, 0);
    }
}
// 24 wait states after the last MFMA writing acc0..acc3, ahead of any VALU read of them (the
// operands tie the reads to this point)
__device__ __forceinline__ void vacc_settle(f32x4 & acc0, f32x4 & acc1, f32x4 & acc2, f32x4 & acc3) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(acc0), "+v"(acc1), "+v"(acc2), "+v"(acc3));
}

// S^T = K . Q^T for the wave's 16 keys of the slice at sb (C rows = keys 4 g + r, C cols = heads
// j16 (acc0) and 16 + j16 (acc1)).  DMA accounting (instructions complete in issue order): the
// slice is DMA_N blocks then the mask, step s reading blocks 2 (s >> 1) and 2 (s >> 1) + 1; before
// that read, the blocks after them, the mask and the next slice's instructions issued so far (one
// per completed step) may still be in flight.
// With DMA, the next slice's DMA (dn, streaming cache policy) is spread over the steps.  Operand
// reads run QPF steps ahead of their MFMAs; the scheduling barriers keep the compiler from sinking
// them back next to their use.  Two accumulator chains per head tile (even / odd steps) keep
// consecutive MFMAs independent.  Returns with the slice's mask slot landed.  WAIT = false: the
// slice is known to be in LDS already (no DMA accounting, no next-slice DMA).
template <int DK, bool DMA, bool WAIT = true>
__device__ __forceinline__ void qk_slice(const SliceStream<DK> & ss, const SliceDma & dn, const char * sb, int lane,
                                         const half8 (&qreg)[2][SliceGeom<DK>::QSTEPS], f32x4 & s0, f32x4 & s1) {
    static_assert(WAIT || !DMA, "a slice already in LDS comes with no DMA to spread");
    using G = SliceGeom<DK>;
    constexpr int QPF = 4;
    const int g = lane >> 4, j16 = lane & 15;
    f32x4 acc0, acc1, acc2, acc3;
    static_assert(QPF % 2 == 0, "operand reads ahead by whole block pairs");
    // row j16, chunk 4 s + g: step s at (a0 ^ 64 (s & 1)) + 2048 (s >> 1)
    const int a0 = slot_byte(j16, g);
    auto arow = [&](int st) { return reinterpret_cast<const half8 *>(sb + (a0 ^ (64 * (st & 1))) + 2048 * (st >> 1)); };
    half8 abuf[QPF];
    if constexpr (WAIT) wait_vm<G::DMA_N + 1 - QPF>();      // blocks 0 .. QPF - 1
#pragma unroll
    for (int s = 0; s < QPF; ++s) abuf[s] = *arow(s);
#pragma unroll
    for (int s = 0; s < G::QSTEPS; ++s) {
        const half8 av = abuf[s % QPF];
        if (s + QPF < G::QSTEPS) {
            // blocks 0 .. 2 ((s + QPF) >> 1) + 1 landed; s instructions of the next slice issued
            const int later = G::DMA_N - 1 - 2 * ((s + QPF) >> 1);
            if constexpr (DMA) wait_vm_le(later + s);
            else if constexpr (WAIT) wait_vm_le(later);
            abuf[s % QPF] = *arow(s + QPF);
        }
        if (s & 1) {
            mfma16<false>(acc2, av, qreg[0][s], s == 1);
            mfma16<false>(acc3, av, qreg[1][s], s == 1);
        } else {
            mfma16<false>(acc0, av, qreg[0][s], s == 0);
            mfma16<false>(acc1, av, qreg[1][s], s == 0);
        }
        if constexpr (DMA) ss.put(dn, s);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (DMA) {
        ss.put(dn, G::DMA_N);
        wait_vm<G::DMA_N + 1>();             // the mask slot (the next slice's DMA_N + 1 may be in flight)
    } else if constexpr (WAIT) {
        wait_vm<0>();
    }
    s0 = acc0 + acc2;
    s1 = acc1 + acc3;
}

// Q.K^T of a slice already in LDS (no DMA accounting; the prefill's tiles land before a barrier),
// accumulators in VGPRs.  Operand block st of the wave's rows is read QPF_LANDED steps ahead; the
// first QPF_LANDED come in `abuf` (qk_operands, which the caller may issue early so that their LDS
// latency passes under other work).  hook(s) runs after step s's MFMAs: the caller's DMA of the
// next tile, spread over the steps.
constexpr int QPF_LANDED = 4;
template <int DK>
__device__ __forceinline__ void qk_operands(const char * sb, int lane, half8 (&abuf)[QPF_LANDED]) {
    const int a0 = slot_byte(lane & 15, lane >> 4);
#pragma unroll
    for (int st = 0; st < QPF_LANDED; ++st)
        abuf[st] = *reinterpret_cast<const half8 *>(sb + (a0 ^ (64 * (st & 1))) + 2048 * (st >> 1));
}
template <int DK, typename H>
__device__ __forceinline__ void qk_slice_landed(const char * sb, int lane, const half8 (&qreg)[2][SliceGeom<DK>::QSTEPS],
                                                half8 (&abuf)[QPF_LANDED], f32x4 & s0, f32x4 & s1, H && hook) {
    using G = SliceGeom<DK>;
    constexpr int QPF = QPF_LANDED;
    const int a0 = slot_byte(lane & 15, lane >> 4);
    auto arow = [&](int st) { return reinterpret_cast<const half8 *>(sb + (a0 ^ (64 * (st & 1))) + 2048 * (st >> 1)); };
    f32x4 acc0, acc1, acc2, acc3;
#pragma unroll
    for (int s = 0; s < G::QSTEPS; ++s) {
        const half8 av = abuf[s % QPF];
        if (s + QPF < G::QSTEPS) abuf[s % QPF] = *arow(s + QPF);
        if (s & 1) {
            mfma16<true>(acc2, av, qreg[0][s], s == 1);
            mfma16<true>(acc3, av, qreg[1][s], s == 1);
        } else {
            mfma16<true>(acc0, av, qreg[0][s], s == 0);
            mfma16<true>(acc1, av, qreg[1][s], s == 0);
        }
        hook(s);
        __builtin_amdgcn_sched_barrier(0);
    }
    vacc_settle(acc0, acc1, acc2, acc3);
    s0 = acc0 + acc2;
    s1 = acc1 + acc3;
}

// the mask values of keys 4 g .. 4 g + 3 of the slice at sb (its mask slot)
template <int DK>
__device__ __forceinline__ f32x4 slice_mask(const char * sb, int lane) {
    return *reinterpret_cast<const f32x4 *>(sb + SliceGeom<DK>::ROWS_BYTES + 16 * (lane >> 4));
}

// Scores in log2 units of keys kbase + 4 g + r for heads j16 (sc[0]) and 16 + j16 (sc[1]); masked,
// padded and out-of-range keys are -inf.  mk = the mask values of those 4 keys (zeros without a
// mask).  mx = the slice's max per head over its 16 keys (ACROSS), or over this lane's 4 keys.
template <bool ACROSS = true>
__device__ __forceinline__ void slice_scores(const DecodeArgs & a, const f32x4 & mk, int kbase, int lane, const f32x4 & s0,
                                             const f32x4 & s1, float (&sc)[2][4], float (&mx)[2]) {
    const int g = lane >> 4;
    mx[0] = -INFINITY;
    mx[1] = -INFINITY;
    const int kq = kbase + 4 * g;                    // this lane's first key
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        // a key past n_kv (its K row reads as zeros, so its raw score is 0) takes a -inf mask
        const float mb = (kq + r < a.n_kv) ? mk[r] * LOG2E : -INFINITY;     // mk: zeros without a mask
        sc[0][r] = s0[r] * a.scale_log2 + mb;
        sc[1][r] = s1[r] * a.scale_log2 + mb;
        mx[0] = fmaxf(mx[0], sc[0][r]);
        mx[1] = fmaxf(mx[1], sc[1][r]);
    }
    if constexpr (ACROSS) {
#pragma unroll
        for (int n = 0; n < 2; ++n) mx[n] = rows4_max(mx[n]);
    }
}

// Whether a head's lazily moved reference max m (M_NONE before its first live key) must move for
// scores whose max is x: x exceeds m by more than 2^LAZY (any live key, while m = M_NONE).  A
// head's slice max exceeds the bound iff one of its four lanes' own maxima does, so the kernels
// test the lanes' own maxima first and take the cross-lane max only on the (rare) path where some
// reference moves.
__device__ __forceinline__ bool ref_moves(float m, float x) { return x > m + LAZY; }

// ---------------------------------------------------------------- the decode kernels
// (kqkv_decode.hip, and the 8-bit cache kernel of kqkv_decode_q8.hip)

// byte offset of wave slot v of ring stage s
template <int DK>
__device__ __forceinline__ constexpr int stage_byte(int s, int v) { return (s * NWAVE + v) * SliceGeom<DK>::STAGE; }

template <int DK, int DV>
struct DecodeCfg {
    using G = SliceGeom<DK>;
    static_assert(DV % 128 == 0 && DV <= DK, "geometry");
    static constexpr int DVQ = DV / NWAVE;              // output columns per wave
    static constexpr int NTQ = DVQ / 32;                // 32-column output tiles per wave
    static constexpr int PROW = TK + 8;                 // P exchange row pitch (halves)
    static constexpr int OPITCH = DVQ * 2 + 16;         // f16 output staging row pitch (bytes)
    static constexpr int CPR = DVQ / 8;                 // 16-byte output chunks per head row
    static_assert(HG * OPITCH <= G::ROWS_BYTES, "a wave's output staging fits its slot of a stage");
    static_assert(CPR % 2 == 0, "whole rounds of 64 chunks");
    static_assert(NWAVE * NTQ - 1 < 64, "P.V operand offsets fit the DS immediate");
};

// LDS of the kernel: the slice ring, the P exchange and the slice maxima, by tile parity
template <int DK, int DV>
struct DecodeLds {
    __attribute__((aligned(16))) char ring[SliceGeom<DK>::RING];       // [stage][wave] K rows + mask
    __attribute__((aligned(16))) half_t px[2][HG * DecodeCfg<DK, DV>::PROW];
    __attribute__((aligned(16))) float red[2][HG][NWAVE];              // [head][wave]
};

// O^T[own columns, heads] += V^T . P^T over the tile's 64 keys (4 slices x 16), for wave w's
// quarter of the columns: the V operand (column, 8 keys per lane) and the P rows (head, 8 keys per
// lane) are the A and B operands of the 32x32x16 MFMA.  The operands of slice ks + 1 are read
// while the MFMAs of slice ks run.  l_acc sums the f16 P values the MFMAs consume (head lane & 31,
// keys 8 (lane >> 5) .. +7 of each slice).
template <int DK, int DV>
__device__ __forceinline__ void pv_tile(const char * ring, const half_t * pxv, int par, int w, int lane, const PvAddr & pv,
                                        f32x16 (&o)[DecodeCfg<DK, DV>::NTQ], float & l_acc) {
    using C = DecodeCfg<DK, DV>;
    {
        half8 pa[2], vb[2][C::NTQ];
        auto load = [&](int ks, int b) {
            pa[b] = *reinterpret_cast<const half8 *>(&pxv[(lane & 31) * C::PROW + WK * ks + 8 * (lane >> 5)]);
            const char * vs = ring + stage_byte<DK>(par, ks);
#pragma unroll
            for (int i = 0; i < C::NTQ; ++i) vb[b][i] = pv.load(vs, C::NTQ * w + i);
        };
        load(0, 0);
#pragma unroll
        for (int ks = 0; ks < NWAVE; ++ks) {
            if (ks + 1 < NWAVE) load(ks + 1, (ks + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < C::NTQ; ++i)
                o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb[ks & 1][i], pa[ks & 1], o[i], 0, 0, 0);
            const half8 pp = pa[ks & 1];
#pragma unroll
            for (int e = 0; e < 8; e += 2) l_acc = __builtin_amdgcn_fdot2(half2{pp[e], pp[e + 1]}, ONE2, l_acc, false);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The end of a split (every tile's P.V done, this wave's DMA drained): l per head from the P sums,
// then o / l -- in f32 to dst with a single split, else the split's partial record ((m, l) pairs
// by wave 0, o / l in f16 through this wave's slot of the ring stage the last tile did not use).
// No workgroup barrier: every wave holds its own heads' l.
template <int DK, int DV>
__device__ __forceinline__ void decode_epilogue(const DecodeArgs & a, char * stg, int w, int tid, int t, int hg0,
                                                int sp, f32x16 (&o)[DecodeCfg<DK, DV>::NTQ], float l_acc,
                                                const float (&m_ref)[2]) {
    using C = DecodeCfg<DK, DV>;
    // thread indices re-derived through an opaque move, so that the epilogue's address arithmetic
    // is computed here rather than before the loop and kept alive (or spilled) across it
    int tid_e;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid_e) : "v"(tid));
    const int lane_e = tid_e & 63;

    // ---- per head: l over all keys of the split, relative to the common reference m_ref ----
    // Every wave summed the whole P exchange for its heads, so each finishes on its own: no
    // workgroup barrier from here on.  The header is (m_ref, l): m_ref lies within 2^15 below the
    // split's max, which the merge's algebra does not care about (only m + ln l enters it).
    const float L = halves_sum(l_acc);         // head lane_e & 31
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const int hl = lane_e & 31, hi4 = 4 * (lane_e >> 5);

    const bool direct = a.dst != nullptr;                 // single split: final f32 output to dst
    if (direct) {
        const int h = hg0 + hl;
        if (h < a.n_head) {
            float * d = a.dst + ((size_t)h * a.nt + t) * DV + C::DVQ * w + hi4;
#pragma unroll
            for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                    *reinterpret_cast<f32x4 *>(d + 32 * i + 8 * q4) =
                        f32x4{o[i][4 * q4] * inv, o[i][4 * q4 + 1] * inv, o[i][4 * q4 + 2] * inv, o[i][4 * q4 + 3] * inv};
        }
        return;
    }
    char * rec = part_record(a.part, blockIdx.y, a.nt, t, a.n_split, DV, 2);
    char * blk = rec + part_o_off(a.n_split, sp, DV, 2);
    if (w == 0 && lane_e < HG) {
        const float mr = m_ref[(lane_e >> 4) & 1];        // lane_e's head 16 ((lane_e >> 4) & 1) + j16
        *reinterpret_cast<f32x2 *>(rec + part_ml_off(a.n_split, lane_e, sp)) =
            f32x2{(mr == M_NONE) ? -INFINITY : mr * LN2, L};                      // m in natural-log units
    }
    // o / l in f16 through stg, LDS of this wave's own that no wave reads any more (at least
    // HG * OPITCH bytes), as [32 heads][DVQ] rows; then 16-byte chunks out, 4 head rows of 2 * DVQ
    // bytes per instruction (whole cache lines).  Write and read are the same wave's, in LDS order.
#pragma unroll
    for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const half4 hv = {to_half(o[i][4 * q4] * inv), to_half(o[i][4 * q4 + 1] * inv), to_half(o[i][4 * q4 + 2] * inv),
                              to_half(o[i][4 * q4 + 3] * inv)};
            *reinterpret_cast<half4 *>(stg + hl * C::OPITCH + (32 * i + 8 * q4 + hi4) * 2) = hv;
        }
#pragma unroll
    for (int it = 0; it < C::CPR / 2; ++it) {
        const int q = 64 * it + lane_e;
        const int row = q / C::CPR, ch = q % C::CPR;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + row * C::OPITCH + 16 * ch);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(blk + ((size_t)row * DV + C::DVQ * w + 8 * ch) * 2));
    }
}

}  // namespace decode
}  // namespace mla
