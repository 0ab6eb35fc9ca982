// Persistent GEMM over whole weight row sets per workgroup, for two activations:
//   * decode (kai_fused_mmvq above the GEMV's rows): Y[j, r] = inverse[j] * sum_b dot(W[r, b],
//     q8[j, b]) over the decode path's Q8_1 blocks (block_q8_1 [m][k/32], m <= 8,
//     k % 256 == 0), with the paired tile's decode arithmetic (kai_mmq.cuh, paired_step: two
//     32-value blocks per v_mfma_i32_16x16x64_i8);
//   * IMAGE (kai_fused_mmq_run, 9 to 16 rows): the batched path's small-M image of the
//     type's layout (kai_launch.h), with the small-M GEMM's block arithmetic (kai_mmqs.cuh,
//     mmqs_step; EXACT: the legacy MMQ's exact weight products).
//
// Design for gfx950. The tiled kernel stages each K step's activation behind a workgroup
// barrier, so each wave holds one weight step in flight and a launch of 8 decode rows waits on
// HBM latency (2 waves per SIMD, two thirds of their cycles waiting). Here:
//   * one workgroup of MMQD_WAVES waves per CU owns a contiguous range of 16-row weight sets
//     (the ranges differ by at most one set);
//   * it stages the activation of a K chunk (the whole K where the LDS holds it) once, behind
//     one barrier: decode Q8_1 blocks converted in registers to the paired LDS layout as the
//     tiled kernel does (stage_block), or the image copied straight to the LDS
//     (global_load_lds_dwordx4, no registers);
//   * the chunk's (row set, K step) pairs of the workgroup are cut into equal contiguous runs,
//     one per wave; each wave streams its run's weights through the small-M kernel's ring
//     (MmqsStream units into the wave's LDS transpose buffer, DEPTH steps in flight, no
//     barrier), crossing row sets without draining it;
//   * each piece of a row set (the part of one wave's run inside it) goes to an LDS slot; after
//     the last chunk the workgroup adds the slots in chunk and piece order (deterministic),
//     times inverse, into the output.
// Nothing but the output leaves the workgroup: kai_fused_mmvq takes no scratch, and the
// batched path needs neither the small-M GEMM's partial-sum scratch nor its reduction launch.
#pragma once

#include "kai_mmqs.cuh"

namespace kai {

// 12 waves and two steps in flight each: 16 waves spill at the 128 registers of four waves per
// SIMD; measured on MI355X against 8 waves with 2 / 3 / 4 steps in flight (Q4_K 34816 x 5120 at
// 8 rows 29.2 us against 29.4 / 31.7 / 30.7), and two workgroups per CU of one row set each
// against one (20-60 % slower on 5120 to 34816 rows).
constexpr int MMQD_WAVES = 12, MMQD_DEPTH = 2;

template <int TYPE, bool IMAGE>
constexpr int mmqd_step_bytes() {  // one K step: 8 rows in the paired layout, or 16 (IMAGE)
    return IMAGE ? mmqs_step_bytes<TYPE>() : 8 * (8 * 32 + 8 * 4 + MmqW<TYPE>::NTERM * 4);
}
template <bool IMAGE>
constexpr int mmqd_slot() {  // floats of one piece: 8 (16) activation rows x 16 weight rows
    return (IMAGE ? 16 : 8) * 16;
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

template <int TYPE, int DEPTH, int WAVES, bool IMAGE, bool EXACT>
__global__ __launch_bounds__(WAVES * WAVE) void mmqd_kernel(
    const uint8_t *weight, int64_t row_bytes, int n, int k, const void *__restrict__ act, int m,
    const float *__restrict__ inverse, MmqdSplit split, void *__restrict__ dst, int64_t stride_dst, int dst_bf16) {
    static_assert(IMAGE || !EXACT, "the decode arithmetic is exact already");
    constexpr int THREADS = WAVES * WAVE;
    // `weight` is not __restrict__: its loads must stay ordered by the compiler fences of the
    // ring below (loads through a restrict pointer are treated as invariant and move freely)
    using W = MmqLoad<TYPE>;
    using S = MmqsStream<TYPE>;
    constexpr int BUF = mmqd_step_bytes<TYPE, IMAGE>(), SLOT = mmqd_slot<IMAGE>(), MT = IMAGE ? 16 : 8;
    extern __shared__ __align__(16) uint8_t kai_mmqd_lds[];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];

    const int tid = threadIdx.x, lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);  // uniform: the run's control is scalar
    const int col = lane % 16, oct = lane / 16;
    const int nb = k / QK8_1, steps = (k + MMQ_STEP - 1) / MMQ_STEP;
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
    // set, when its rows or runs can end inside a unit (rows not a multiple of 16, superblocks
    // that are not whole units, a short last step), clamps each unit start to the matrix's
    // last 16 bytes and moves the unit's LDS position back by as many bytes (0 for a unit
    // wholly past the end, whose rows are never stored), so no load leaves the matrix; that
    // wave runs its own copy of the loop.
    uint32_t ug[S::UPL];
    int uoff[S::UPL];
#pragma unroll
    for (int i = 0; i < S::UPL; ++i) {
        const int u = lane + WAVE * i, r = u / S::U, c = u % S::U;
        const bool real = u < 16 * S::U;
        ug[i] = real ? static_cast<uint32_t>(r) * static_cast<uint32_t>(row_bytes) + 16 * c : 0u;
        uoff[i] = real ? r * S::SBP + 16 * c : 16 * S::SBP;
    }
    const bool ragged = n % 16 != 0 || S::SB % 16 != 0 || k % MMQ_STEP != 0;
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
        // the ring's first DEPTH steps: decode, right after the activation's first loads (vector
        // loads retire in order, so the activation's wait then leaves the weights in flight:
        // Q4_K 34816x5120 at 8 rows -0.4 us, Q2_K -1.0 us); image, before the copies (after
        // them, 0.2-0.5 us slower)
        auto prologue = [&]() {
            if (t1 > t0) {
#pragma unroll
                for (int d = 0; d < DEPTH; ++d) {
                    wload(wr[d], std::true_type{});
                    __asm__ volatile("" ::: "memory");  // the loop's order: its waits then count the slots in flight
                }
            }
        };

        if constexpr (IMAGE) {
            prologue();
            // ---- the chunk's image -> LDS, 16 bytes a lane, a wave's 64 lanes filling 1 KiB in
            // lane order. Q4_0 takes its terms from the image's second term array.
            constexpr int IMG = mmqs_image_step(mmq_layout(TYPE)), UNITS = BUF / 16;
            const uint8_t *img = static_cast<const uint8_t *>(act) + int64_t(s0) * IMG;
            const int units = sc * UNITS;
            for (int u0 = wave * WAVE; u0 < units; u0 += THREADS) {
                const int u = u0 + lane, j = u / UNITS, o = (u % UNITS) * 16;
                if (u < units) {
                    const int src = TYPE == Q4_0 && o >= MMQS_CODE_BYTES + MMQS_D8_BYTES ? o + MMQS_D8_BYTES : o;
                    __builtin_amdgcn_global_load_lds(static_cast<const void *>(img + j * IMG + src),
                                                     (__attribute__((address_space(3))) uint8_t *)kai_mmqd_lds + u0 * 16,
                                                     16, 0, 0);
                }
            }
        } else {
            // ---- the chunk's Q8_1 blocks -> LDS: (step j, block b, row r) items, rows past m
            // zero; four items a thread in flight, in rounds every wave runs (the ring's
            // prologue follows the first round's loads)
            const block_q8_1 *y = static_cast<const block_q8_1 *>(act);
            const int items = sc * 64;
            for (int round = 0; round == 0 || round * 4 * THREADS < items; ++round) {
                uint4 q0[4], q1[4];
                uint32_t ds[4];
                const int i0 = tid + round * 4 * THREADS;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int it = i0 + u * THREADS, r = it % 8, b = (it / 8) % 8, j = it / 64;
                    q0[u] = q1[u] = make_uint4(0, 0, 0, 0);
                    ds[u] = 0;
                    if (it < items && r < m) {
                        const uint8_t *src = reinterpret_cast<const uint8_t *>(y + int64_t(r) * nb + 8 * (s0 + j) + b);
                        ds[u] = load_unaligned<uint32_t>(src);
                        q0[u] = load_unaligned<uint4>(src + 4);
                        q1[u] = load_unaligned<uint4>(src + 20);
                    }
                }
                if (round == 0) prologue();
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
        }
        if (sce > sc) {  // the zero steps that round the chunk up to whole turns of the ring
            for (int u = tid; u < (sce - sc) * BUF / 16; u += THREADS)
                *reinterpret_cast<uint4 *>(kai_mmqd_lds + sc * BUF + 16 * u) = make_uint4(0, 0, 0, 0);
        }
        __syncthreads();

        // ---- the run: DEPTH steps in flight, straight-line loads and waits; a piece of a row
        // set ends at its last step or the run's, and goes to its slot
        auto store = [&](v4f_t acc, int rl) {
            if constexpr (!IMAGE) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] += __shfl_xor(acc[i], 32);  // odd blocks' sums (D rows 8-15)
            }
            const int q = wave - (rl * sce) / run;
            if (IMAGE || oct < 2) {  // slot [activation row 4 oct + i][weight row col]
                float *p = slots + ((ch * split.sets + rl) * split.qmax + q) * SLOT + 4 * oct * 16 + col;
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
                        if constexpr (IMAGE) {
                            mmqs_step<TYPE, EXACT>(tb + col * S::SBP, min(8, nb - 8 * (s0 + min(j + d, sc - 1))),
                                                   kai_mmqd_lds + (j + d) * BUF, acc[0], col, oct, aoct, grid_lds);
                        } else {
                            typename W::Raw w[1];
                            W::load(w[0], tb + col * S::SBP, oct, 8);
                            W::fix(w[0]);
                            paired_step<TYPE, 1, true>(w, kai_mmqd_lds + (j + d) * BUF, acc, col, oct, aoct, grid_lds);
                        }
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
    for (int e = tid; e < nr * SLOT; e += THREADS) {
        const int rl = e / SLOT, j = (e / 16) % MT, c = 16 * (r0 + rl) + e % 16;
        if (j >= m || c >= n) continue;
        float s = 0.0f;
        for (int ch = 0; ch < split.chunks; ++ch) {
            const int sce = mmqd_positions(min(split.chunk, steps - ch * split.chunk), DEPTH);
            const int np = mmqd_pieces(rl, sce, mmqd_run(nr, sce, WAVES, DEPTH));
            const float *p = slots + (ch * split.sets + rl) * split.qmax * SLOT + e % SLOT;
            for (int q = 0; q < np; ++q) s += p[q * SLOT];
        }
        const float v = s * inverse[j];
        const int64_t idx = int64_t(j) * stride_dst + c;
        if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
        else static_cast<float *>(dst)[idx] = v;
    }
}

// The split: one workgroup per CU (fewer for matrices of fewer row sets), K in as few chunks as
// the LDS holds with the transpose buffers and the slots. It depends only on the type and shape.
template <int TYPE, bool IMAGE>
inline size_t mmqd_lds_bytes(const MmqdSplit &p) {
    return size_t(mmqd_positions(p.chunk, MMQD_DEPTH)) * mmqd_step_bytes<TYPE, IMAGE>() +
           size_t(MMQD_WAVES) * mmqd_stream_bytes<TYPE>() +
           size_t(p.chunks) * p.sets * p.qmax * mmqd_slot<IMAGE>() * sizeof(float);
}
template <int TYPE, bool IMAGE>
inline MmqdSplit mmqd_split(int64_t n, int64_t k, int cus) {
    const int steps = static_cast<int>((k + MMQ_STEP - 1) / MMQ_STEP), rowsets = static_cast<int>((n + 15) / 16);
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
        if (mmqd_lds_bytes<TYPE, IMAGE>(p) + (TYPE == IQ3_S ? 2048 : 0) <= size_t(MMQS_LDS_BUDGET)) return p;
        if (p.chunk <= MMQD_DEPTH) {  // does not fit: wgs = 0
            p.wgs = 0;
            return p;
        }
    }
}
// Whether an n x k matrix suits the persistent GEMM: the activation's K (decode: k % 256 == 0;
// IMAGE: whole blocks of the type), a split that fits the LDS, and whole row sets per
// workgroup keeping the workgroups busy for at least 90 % (IMAGE: 85 %) of the longest one's
// time (a workgroup owns rowsets / wgs sets, rounded up or down). Measured on MI355X at 5 to 8
// decode rows against the tiled paired kernel: 2176 row sets (34816 x 5120: Q4_K 28.6 against
// 36.2 us, Q2_K 28.2 / 35.5, IQ3_S 42.9 / 54.8), 1024 (Q4_0 16384 x 2048, 15.0 / 24.5) and 128
// (Q4_0 2048 x 8192, 15.7 / 30.0) gain; 448 (87.5 % busy: Q4_K 7168 x 5120, 12.8 / 12.1) and
// 320 (62.5 %: Q6_K 5120 x 6144, 18.0 / 16.3) lose. At 9 to 16 rows against the small-M GEMM
// and its reduction (whole calls): 2176 row sets (Q4_K 41.0 / 37.8, Q2_K 51.0 / 48.6, IQ3_S
// 55.6 / 52.8), 128 (Q8_0 2048 x 2048 28.0 / 13.4) and 448 (Q4_K 7168 x 5120 22.4 / 18.2) gain;
// 320 (Q6_K 5120 x 6144 27.5 / 26.8, 5120 x 17408 38.7 / 68.8) does not.
template <int TYPE, bool IMAGE>
inline bool mmqd_suits(int64_t n, int64_t k, int cus) {
    const bool k_ok = IMAGE ? k >= MMQ_STEP / 8 && k % block_elems(TYPE) == 0 : k >= MMQ_STEP && k % MMQ_STEP == 0;
    if (n < 1 || !k_ok || k > INT_MAX || n > INT_MAX ||
        n * ((k / block_elems(TYPE)) * block_bytes(TYPE)) >= (int64_t(1) << 32))
        return false;
    const int64_t rowsets = (n + 15) / 16, wgs = std::min<int64_t>(rowsets, cus), most = (rowsets + wgs - 1) / wgs;
    return rowsets * 20 >= (IMAGE ? 17 : 18) * wgs * most && mmqd_split<TYPE, IMAGE>(n, k, cus).wgs > 0;
}

template <int TYPE, bool IMAGE, bool EXACT>
void launch_mmqd_kernel(const void *weight, int64_t n, int64_t k, int64_t m, const void *act, const float *inverse,
                        void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if (m < 1 || m > (IMAGE ? MMQS_MAX_ROWS : 8)) throw Error("Too many activation rows for the persistent GEMM");
    if (!mmqd_suits<TYPE, IMAGE>(n, k, device_cu_count()))
        throw Error("The persistent GEMM does not take this matrix shape");
    const int64_t row_bytes = (k / block_elems(TYPE)) * block_bytes(TYPE);
    const MmqdSplit p = mmqd_split<TYPE, IMAGE>(n, k, device_cu_count());
    auto kernel = mmqd_kernel<TYPE, MMQD_DEPTH, MMQD_WAVES, IMAGE, EXACT>;
    static DeviceFlags lds_raised;
    raise_dynamic_lds(reinterpret_cast<const void *>(kernel), MMQS_LDS_BUDGET - (TYPE == IQ3_S ? 2048 : 0), lds_raised,
                      "Cannot raise the persistent GEMM's dynamic LDS limit");
    kernel<<<dim3(static_cast<unsigned>(p.wgs)), MMQD_WAVES * WAVE, mmqd_lds_bytes<TYPE, IMAGE>(p), stream>>>(
        static_cast<const uint8_t *>(weight), row_bytes, static_cast<int>(n), static_cast<int>(k), act,
        static_cast<int>(m), inverse, p, dst, stride_dst, dst_bf16 ? 1 : 0);
}

// Decode Q8_1 blocks, up to 8 rows.
template <int TYPE>
void launch_mmqd(const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y, const float *inverse,
                 void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    launch_mmqd_kernel<TYPE, false, false>(weight, n, k, m, y, inverse, dst, dst_bf16, stride_dst, stream);
}
// The small-M image of the type's layout, up to MMQS_MAX_ROWS rows (EXACT: the legacy MMQ's
// weight products).
template <int TYPE, bool EXACT = false>
void launch_mmqd_image(const void *weight, int64_t n, int64_t k, int64_t m, const uint8_t *image, const float *inverse,
                       void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    launch_mmqd_kernel<TYPE, true, EXACT>(weight, n, k, m, image, inverse, dst, dst_bf16, stride_dst, stream);
}

}  // namespace kai
