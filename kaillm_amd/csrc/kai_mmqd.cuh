// Persistent paired-tile GEMM for decode activations (kai_fused_mmvq above the GEMV's rows):
// Y[j, r] = inverse[j] * sum_b dot(W[r, b], q8[j, b]) over the decode path's Q8_1 blocks
// (block_q8_1 [m][k/32], m <= 8, k % 256 == 0), with the paired tile's decode arithmetic
// (kai_mmq.cuh, paired_step: two 32-value blocks per v_mfma_i32_16x16x64_i8).
//
// Design for gfx950. The tiled kernel stages each K step's activation behind a workgroup
// barrier, so each wave holds one weight step in flight and a launch of 8 decode rows waits on
// HBM latency (2 waves per SIMD, two thirds of their cycles waiting). Here:
//   * one workgroup of MMQD_WAVES waves per CU owns a contiguous range of 16-row weight sets
//     (the ranges differ by at most one set);
//   * it stages the activation of a K chunk (the whole K where the LDS holds it) once, in the
//     paired LDS layout, converting the Q8_1 blocks in registers as the tiled kernel does
//     (stage_block), behind one barrier;
//   * the chunk's (row set, K step) pairs of the workgroup are cut into equal contiguous runs,
//     one per wave; each wave streams its run's weights through the small-M kernel's ring
//     (MmqsStream units into the wave's LDS transpose buffer, DEPTH steps in flight, no
//     barrier), crossing row sets without draining it;
//   * each piece of a row set (the part of one wave's run inside it) goes to an LDS slot; after
//     the last chunk the workgroup adds the slots in chunk and piece order (deterministic),
//     times inverse, into the output.
// kai_fused_mmvq takes no scratch, so nothing but the output leaves the workgroup.
#pragma once

#include "kai_mmqs.cuh"

namespace kai {

// 12 waves and two steps in flight each: 16 waves spill at the 128 registers of four waves per
// SIMD; measured on MI355X against 8 waves with 2 / 3 / 4 steps in flight (Q4_K 34816 x 5120 at
// 8 rows 29.2 us against 29.4 / 31.7 / 30.7), and two workgroups per CU of one row set each
// against one (20-60 % slower on 5120 to 34816 rows).
constexpr int MMQD_WAVES = 12, MMQD_DEPTH = 2;
constexpr int MMQD_SLOT = 8 * 16;  // floats of one piece: 8 activation rows x 16 weight rows

template <int TYPE>
constexpr int mmqd_step_bytes() {  // one K step of 8 activation rows in the paired layout
    return 8 * (8 * 32 + 8 * 4 + MmqW<TYPE>::NTERM * 4);
}
template <int TYPE>
constexpr int mmqd_stream_bytes() {  // a wave's transpose buffer: 16 rows and a spare unit
    return 16 * MmqsStream<TYPE>::SBP + 16;
}

// The work split of a launch (host and device agree on it).
struct MmqdSplit {
    int wgs;            // workgroups: workgroup g owns row sets [g * rowsets / wgs, (g + 1) * rowsets / wgs)
    int sets;           // row sets a workgroup owns at most
    int chunks, chunk;  // K chunks of `chunk` steps (the last may be shorter)
    int qmax;           // piece slots per (chunk, row set)
};
// Positions of a chunk of sc steps: sc rounded up to a multiple of the ring's depth (the
// added steps have zero activation), and a wave's run over nr row sets of sce positions each
// (also a multiple of the depth), so that every piece of a row set starts and ends on a whole
// turn of the ring.
__host__ __device__ inline int mmqd_positions(int sc, int depth) { return (sc + depth - 1) / depth * depth; }
__host__ __device__ inline int mmqd_run(int nr, int sce, int waves, int depth) {
    return mmqd_positions((nr * sce + waves - 1) / waves, depth);
}
// Pieces of local row set i (positions [i*sce, (i+1)*sce) cut by runs of `run`).
__host__ __device__ inline int mmqd_pieces(int i, int sce, int run) {
    return (i * sce + sce - 1) / run - (i * sce) / run + 1;
}

template <int TYPE, int DEPTH, int WAVES>
__global__ __launch_bounds__(WAVES * WAVE) void mmqd_kernel(
    const uint8_t *weight, int64_t row_bytes, int n, int k, const block_q8_1 *__restrict__ act, int m,
    const float *__restrict__ inverse, MmqdSplit split, void *__restrict__ dst, int64_t stride_dst, int dst_bf16) {
    constexpr int THREADS = WAVES * WAVE;
    // `weight` is not __restrict__: its loads must stay ordered by the compiler fences of the
    // ring below (loads through a restrict pointer are treated as invariant and move freely)
    using W = MmqLoad<TYPE>;
    using S = MmqsStream<TYPE>;
    constexpr int BUF = mmqd_step_bytes<TYPE>();
    extern __shared__ __align__(16) uint8_t kai_mmqd_lds[];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];

    const int tid = threadIdx.x, lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);  // uniform: the run's control is scalar
    const int col = lane % 16, oct = lane / 16;
    const int nb = k / QK8_1, steps = k / MMQ_STEP;
    const int rowsets = (n + 15) / 16;
    const int r0 = static_cast<int>(int64_t(blockIdx.x) * rowsets / split.wgs);
    const int nr = static_cast<int>(int64_t(blockIdx.x + 1) * rowsets / split.wgs) - r0;
    if constexpr (TYPE == IQ3_S) {
        for (int i = tid; i < 512; i += THREADS) grid_lds[i] = mmq_iq3s_grid[i];
    }
    // LDS: the chunk's activation steps, the waves' transpose buffers, the piece slots
    const int act_bytes = mmqd_positions(split.chunk, DEPTH) * BUF;
    lds_u8 *tb = (lds_u8 *)kai_mmqd_lds + act_bytes + wave * mmqd_stream_bytes<TYPE>();
    float *slots = reinterpret_cast<float *>(kai_mmqd_lds + act_bytes + WAVES * mmqd_stream_bytes<TYPE>());

    // ---- the lane's units (row u / U, unit u % U of a row set) as 32-bit byte offsets (the
    // launcher checks that the matrix is below 4 GiB); a lane with no unit in a group re-reads
    // the set's first unit into a spare slot. A wave whose run reaches the matrix's last row
    // set, when its rows can end inside a unit (rows not a multiple of 16, superblocks that
    // are not whole units), clamps each unit start to the matrix's last 16 bytes and moves the
    // unit's LDS position back by as many bytes (0 for a unit wholly past the end, whose rows
    // are never stored), so no load leaves the matrix; that wave runs its own copy of the loop.
    uint32_t ug[S::UPL];
    int uoff[S::UPL];
#pragma unroll
    for (int i = 0; i < S::UPL; ++i) {
        const int u = lane + WAVE * i, r = u / S::U, c = u % S::U;
        const bool real = u < 16 * S::U;
        ug[i] = real ? static_cast<uint32_t>(r) * static_cast<uint32_t>(row_bytes) + 16 * c : 0u;
        uoff[i] = real ? r * S::SBP + 16 * c : 16 * S::SBP;
    }
    const bool ragged = n % 16 != 0 || S::SB % 16 != 0;
    const uint32_t tail = static_cast<uint32_t>(int64_t(n) * row_bytes - 16);
    const uint32_t set_bytes = 16u * static_cast<uint32_t>(row_bytes);
    const int aoct = W::act_pos(oct) / 8;
    struct Slot {
        uint4 v[S::UPL];
        uint32_t back;  // careful: 4 bits per unit, the bytes its load start was moved back
    };

    for (int ch = 0; ch < split.chunks; ++ch) {
        const int s0 = ch * split.chunk, sc = min(split.chunk, steps - s0);
        const int sce = mmqd_positions(sc, DEPTH), run = mmqd_run(nr, sce, WAVES, DEPTH), total = nr * sce;
        const int t0 = min(wave * run, total), t1 = min(t0 + run, total);
        const bool careful = ragged && t1 > t0 && r0 + (t1 - 1) / sce == rowsets - 1;  // uniform

        Slot wr[DEPTH];
        // the next position to load (local row set lr, position lj); the ring's run-ahead past
        // the run's end repeats its last position, and a chunk's zero step re-reads its last step
        int lt = t0, lr = t1 > t0 ? t0 / sce : 0, lj = t1 > t0 ? t0 % sce : 0;
        auto wload = [&](Slot &sl, auto careful_tag) {
            const uint32_t lbase = static_cast<uint32_t>(r0 + lr) * set_bytes +
                                   static_cast<uint32_t>(s0 + min(lj, sc - 1)) * S::SB;
            if constexpr (decltype(careful_tag)::value) {
                sl.back = 0;
#pragma unroll
                for (int i = 0; i < S::UPL; ++i) {
                    const uint32_t g = ug[i] + lbase, a = min(g, tail), back = g - a;
                    sl.v[i] = load_unaligned<uint4>(weight + a);
                    sl.back |= (back < 16u ? back : 0u) << (4 * i);
                }
            } else {
                const uint8_t *b = weight + lbase;
#pragma unroll
                for (int i = 0; i < S::UPL; ++i) sl.v[i] = load_unaligned<uint4>(b + ug[i]);
            }
            const int adv = lt < t1 - 1 ? 1 : 0;  // scalar selects: a branch would split the loop body
            lt += adv;
            lj += adv;
            const int wrap = lj == sce ? 1 : 0;
            lj = wrap ? 0 : lj;
            lr += wrap;
        };
        if (t1 > t0) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                wload(wr[d], std::true_type{});
                __asm__ volatile("" ::: "memory");  // the loop's order: its waits then count the slots in flight
            }
        }

        // ---- the chunk's activation -> LDS: (step j, block b, row r) items, rows past m zero;
        // four items a thread in flight
        const int items = sc * 64;
        for (int i0 = tid; i0 < items; i0 += 4 * THREADS) {
            uint4 q0[4], q1[4];
            uint32_t ds[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int it = i0 + u * THREADS, r = it % 8, b = (it / 8) % 8, j = it / 64;
                q0[u] = q1[u] = make_uint4(0, 0, 0, 0);
                ds[u] = 0;
                if (it < items && r < m) {
                    const uint8_t *src = reinterpret_cast<const uint8_t *>(act + int64_t(r) * nb + 8 * (s0 + j) + b);
                    ds[u] = load_unaligned<uint32_t>(src);
                    q0[u] = load_unaligned<uint4>(src + 4);
                    q1[u] = load_unaligned<uint4>(src + 20);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int it = i0 + u * THREADS;
                if (it < items) {
                    const float d8 = half_bits_to_float(ds[u] & 0xffffu);
                    float t[2] = {0.0f, 0.0f};
                    act_terms<TYPE>(q0[u], q1[u], ds[u], d8, t);
                    stage_block<TYPE, 8>(kai_mmqd_lds + (it / 64) * BUF, it % 8, (it / 8) % 8, q0[u], q1[u], d8, t);
                }
            }
        }
        if (sce > sc) {  // the zero steps that round the chunk up to whole turns of the ring
            for (int u = tid; u < (sce - sc) * BUF / 16; u += THREADS)
                *reinterpret_cast<uint4 *>(kai_mmqd_lds + sc * BUF + 16 * u) = make_uint4(0, 0, 0, 0);
        }
        __syncthreads();

        // ---- the run: DEPTH steps in flight, straight-line loads and waits; a piece of a row
        // set ends at its last step or the run's, and goes to its slot
        auto store = [&](v4f_t acc, int rl) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += __shfl_xor(acc[i], 32);  // odd blocks' sums (D rows 8-15)
            const int q = wave - (rl * sce) / run;
            if (oct < 2) {
                float *p = slots + ((ch * split.sets + rl) * split.qmax + q) * MMQD_SLOT + 4 * oct * 16 + col;
#pragma unroll
                for (int i = 0; i < 4; ++i) p[16 * i] = acc[i];
            }
        };
        auto loop = [&](auto careful_tag) {
#pragma unroll 1
            for (int pa = t0; pa < t1;) {  // one piece of a row set: positions [pa, pb), whole ring turns
                const int rl = pa / sce, pb = min(t1, (rl + 1) * sce);
                v4f_t acc[1] = {{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll 1
                for (int j = pa - rl * sce; j < pb - rl * sce; j += DEPTH) {
#pragma unroll
                    for (int d = 0; d < DEPTH; ++d) {
                        const Slot &sl = wr[d];
#pragma unroll
                        for (int i = 0; i < S::UPL; ++i) {
                            if constexpr (decltype(careful_tag)::value)
                                store_unaligned(tb + uoff[i] - int((sl.back >> (4 * i)) & 15u), sl.v[i]);
                            else
                                store16(tb + uoff[i], sl.v[i]);
                        }
                        typename W::Raw w[1];
                        W::load(w[0], tb + col * S::SBP, oct, 8);
                        W::fix(w[0]);
                        paired_step<TYPE, 1, true>(w, kai_mmqd_lds + (j + d) * BUF, acc, col, oct, aoct, grid_lds);
                        wload(wr[d], careful_tag);
                        // keep the refill here and each step's work in its own section: without
                        // these fences the loads are sunk to their use and the next slot's decode
                        // is hoisted into this one, and the waits drain the ring every step
                        __asm__ volatile("" ::: "memory");
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                store(acc[0], rl);
                pa = pb;
            }
        };
        if (t1 > t0) {
            // Q8_0 and Q4_0 (whose raw fields are many small pieces) run every wave on the
            // clamped copy: two copies of their loop do not fit the registers without spilling
            if constexpr (LazyLoad<MmqW<TYPE>>::value) {
                loop(std::true_type{});
            } else {
                if (careful) loop(std::true_type{});
                else loop(std::false_type{});
            }
        }
        __syncthreads();  // the slots are written; the next chunk may overwrite the activation
    }

    // ---- out[j][16 (r0 + rl) + c] = inverse[j] * the slots of (rl, j, c) in chunk, then piece order
    for (int e = tid; e < nr * MMQD_SLOT; e += THREADS) {
        const int rl = e / MMQD_SLOT, j = (e / 16) % 8, c = 16 * (r0 + rl) + e % 16;
        if (j >= m || c >= n) continue;
        float s = 0.0f;
        for (int ch = 0; ch < split.chunks; ++ch) {
            const int sce = mmqd_positions(min(split.chunk, steps - ch * split.chunk), DEPTH);
            const int np = mmqd_pieces(rl, sce, mmqd_run(nr, sce, WAVES, DEPTH));
            const float *p = slots + (ch * split.sets + rl) * split.qmax * MMQD_SLOT + e % MMQD_SLOT;
            for (int q = 0; q < np; ++q) s += p[q * MMQD_SLOT];
        }
        const float v = s * inverse[j];
        const int64_t idx = int64_t(j) * stride_dst + c;
        if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
        else static_cast<float *>(dst)[idx] = v;
    }
}

// The split: one workgroup per CU (fewer for matrices of fewer row sets), K in as few chunks as
// the LDS holds with the transpose buffers and the slots. It depends only on the type and shape.
template <int TYPE>
inline MmqdSplit mmqd_split(int64_t n, int64_t k, int cus) {
    constexpr int BUF = mmqd_step_bytes<TYPE>();
    constexpr size_t FIXED = size_t(MMQD_WAVES) * mmqd_stream_bytes<TYPE>() + (TYPE == IQ3_S ? 2048 : 0);
    const int steps = static_cast<int>(k / MMQ_STEP), rowsets = static_cast<int>((n + 15) / 16);
    MmqdSplit p;
    p.wgs = std::max(1, std::min(rowsets, cus));
    p.sets = (rowsets + p.wgs - 1) / p.wgs;
    const int fewest = rowsets / p.wgs;  // the other workgroups' count (when it differs)
    for (int want = 1;; ++want) {
        p.chunk = (steps + want - 1) / want;
        p.chunks = (steps + p.chunk - 1) / p.chunk;
        p.qmax = 1;
        for (int c = 0; c < p.chunks; ++c) {
            const int sce = mmqd_positions(std::min(p.chunk, steps - c * p.chunk), MMQD_DEPTH);
            for (int nr = std::max(1, fewest); nr <= p.sets; ++nr)
                for (int i = 0; i < nr; ++i)
                    p.qmax = std::max(p.qmax, mmqd_pieces(i, sce, mmqd_run(nr, sce, MMQD_WAVES, MMQD_DEPTH)));
        }
        const size_t lds = size_t(mmqd_positions(p.chunk, MMQD_DEPTH)) * BUF + FIXED +
                           size_t(p.chunks) * p.sets * p.qmax * MMQD_SLOT * sizeof(float);
        if (lds <= size_t(MMQS_LDS_BUDGET)) return p;
        if (p.chunk <= 2) {  // does not fit: wgs = 0
            p.wgs = 0;
            return p;
        }
    }
}
// Whether an n x k matrix suits the persistent paired GEMM: k % 256 == 0, its split fits the
// LDS, and whole row sets per workgroup keep the workgroups busy for at least 90 % of the
// longest one's time (a workgroup owns rowsets / wgs sets, rounded up or down). Measured on
// MI355X at 5 to 8 rows against the tiled paired kernel: 2176 row sets (34816 x 5120: Q4_K 28.6
// against 36.2 us, Q2_K 28.2 / 35.5, IQ3_S 42.9 / 54.8), 1024 (Q4_0 16384 x 2048, 15.0 / 24.5)
// and 128 (Q4_0 2048 x 8192, 15.7 / 30.0) gain; 448 (87.5 % busy: Q4_K 7168 x 5120, 12.8 / 12.1)
// and 320 (62.5 %: Q6_K 5120 x 6144, 18.0 / 16.3) lose.
template <int TYPE>
inline bool mmqd_suits(int64_t n, int64_t k, int cus) {
    if (n < 1 || k < MMQ_STEP || k % MMQ_STEP || k > INT_MAX || n > INT_MAX ||
        n * ((k / block_elems(TYPE)) * block_bytes(TYPE)) >= (int64_t(1) << 32))
        return false;
    const int64_t rowsets = (n + 15) / 16, wgs = std::min<int64_t>(rowsets, cus), most = (rowsets + wgs - 1) / wgs;
    return rowsets * 10 >= 9 * wgs * most && mmqd_split<TYPE>(n, k, cus).wgs > 0;
}
template <int TYPE>
inline size_t mmqd_lds_bytes(const MmqdSplit &p) {
    return size_t(mmqd_positions(p.chunk, MMQD_DEPTH)) * mmqd_step_bytes<TYPE>() +
           size_t(MMQD_WAVES) * mmqd_stream_bytes<TYPE>() +
           size_t(p.chunks) * p.sets * p.qmax * MMQD_SLOT * sizeof(float);
}

template <int TYPE>
void launch_mmqd(const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y, const float *inverse,
                 void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if (m < 1 || m > 8) throw Error("The persistent paired GEMM takes 1..8 activation rows");
    if (n < 1 || k < MMQ_STEP || k % MMQ_STEP) throw Error("The persistent paired GEMM needs k to be a multiple of 256");
    const int64_t row_bytes = (k / block_elems(TYPE)) * block_bytes(TYPE);
    if (n * row_bytes >= (int64_t(1) << 32)) throw Error("The persistent paired GEMM takes matrices below 4 GiB");
    const MmqdSplit p = mmqd_split<TYPE>(n, k, device_cu_count());
    const size_t lds = mmqd_lds_bytes<TYPE>(p);
    if (p.wgs < 1 || lds + (TYPE == IQ3_S ? 2048 : 0) > size_t(MMQS_LDS_BUDGET))
        throw Error("The persistent paired GEMM's split does not fit the LDS");
    auto kernel = mmqd_kernel<TYPE, MMQD_DEPTH, MMQD_WAVES>;
    static DeviceFlags lds_raised;
    raise_dynamic_lds(reinterpret_cast<const void *>(kernel), MMQS_LDS_BUDGET - (TYPE == IQ3_S ? 2048 : 0), lds_raised,
                      "Cannot raise the persistent paired GEMM's dynamic LDS limit");
    kernel<<<dim3(static_cast<unsigned>(p.wgs)), MMQD_WAVES * WAVE, lds, stream>>>(
        static_cast<const uint8_t *>(weight), row_bytes, static_cast<int>(n), static_cast<int>(k), y,
        static_cast<int>(m), inverse, p, dst, stride_dst, dst_bf16 ? 1 : 0);
}

}  // namespace kai
