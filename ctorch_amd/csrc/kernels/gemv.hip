// Host dispatch of the projections: the GEMV (gemv_impl.h) for one or two activation rows (or shapes the matrix
// cores do not take), the matrix-core kernel (gemm_rows.h) for a batch of decode rows, and the tiled matrix-core
// kernel (gemm_tiles.h) for prefill chunks large enough to fill the device; all instantiated per epilogue in
// gemv_*.hip.
//
// The grid is persistent: one wave per row group, capped at the number of waves the chosen kernel keeps
// resident on the device (its occupancy times the CU count), so every wave streams from the start and none
// waits for another to retire.  LOGITS launches write one sampling candidate per work-group.
#include "kernels/gemm_tiles.h"

#include <mutex>
#include <unordered_map>

namespace {

using dlk::gemv::Kernel;

Kernel resolve(const dlk_gemv_params& p, int mt) {
    switch (p.epilogue) {
    case DLK_EPI_STORE: return dlk_gemv_kernel_store(p, mt);
    case DLK_EPI_RESIDUAL: return dlk_gemv_kernel_residual(p, mt);
    case DLK_EPI_QKV: return dlk_gemv_kernel_qkv(p, mt);
    case DLK_EPI_SWIGLU: return dlk_gemv_kernel_swiglu(p, mt);
    case DLK_EPI_LOGITS: return dlk_gemv_kernel_logits(p, mt);
    default: return {};
    }
}

int activation_tile(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : 4; }

Kernel resolve_gemm(const dlk_gemv_params& p, int mt, int nc) {
    switch (p.epilogue) {
    case DLK_EPI_STORE: return dlk_gemm_kernel_store(p, mt, nc);
    case DLK_EPI_RESIDUAL: return dlk_gemm_kernel_residual(p, mt, nc);
    case DLK_EPI_QKV: return dlk_gemm_kernel_qkv(p, mt, nc);
    case DLK_EPI_SWIGLU: return dlk_gemm_kernel_swiglu(p, mt, nc);
    case DLK_EPI_LOGITS: return dlk_gemm_kernel_logits(p, mt, nc);
    default: return {};
    }
}

Kernel resolve_reduce(const dlk_gemv_params& p) {
    switch (p.epilogue) {
    case DLK_EPI_STORE: return dlk_gemm_reduce_store(p);
    case DLK_EPI_RESIDUAL: return dlk_gemm_reduce_residual(p);
    case DLK_EPI_QKV: return dlk_gemm_reduce_qkv(p);
    case DLK_EPI_SWIGLU: return dlk_gemm_reduce_swiglu(p);
    case DLK_EPI_LOGITS: return dlk_gemm_reduce_logits(p);
    default: return {};
    }
}

Kernel resolve_tiles(const dlk_gemv_params& p) {
    switch (p.epilogue) {
    case DLK_EPI_STORE: return dlk_tiles_kernel_store(p);
    case DLK_EPI_RESIDUAL: return dlk_tiles_kernel_residual(p);
    case DLK_EPI_QKV: return dlk_tiles_kernel_qkv(p);
    case DLK_EPI_SWIGLU: return dlk_tiles_kernel_swiglu(p);
    default: return {};
    }
}

int launch_prepare(const dlk_gemv_params& p, hipStream_t stream);

// Tiled path: prepare_rows splits the activation rows into the staging workspace (unless the caller says it
// already holds them), then the tiled projection.
int launch_tiles(const dlk_gemv_params& p, hipStream_t stream) {
    using namespace dlk::tiles;
    const Kernel narrow = dlk_tiles_kernel_narrow(p);
    const Kernel kernel = narrow.fn ? narrow : resolve_tiles(p);
    if (!kernel.fn) return static_cast<int>(hipErrorInvalidValue);
    const int status = launch_prepare(p, stream);
    if (status != 0) return status;
    void* args[] = {const_cast<dlk_gemv_params*>(&p)};
    if (narrow.fn) {
        const int waves = (p.M + 15) / 16;
        return static_cast<int>(hipLaunchKernel(kernel.fn, dim3((waves + kNarrowWaves - 1) / kNarrowWaves),
                                                dim3(kNarrowWaves * dlk::kWave), args, 0, stream));
    }
    const int blocks = col_blocks(p) * row_blocks(p);
    return static_cast<int>(hipLaunchKernel(kernel.fn, dim3(blocks), dim3(kThreads), args, kernel.lds, stream));
}

int launch_prepare(const dlk_gemv_params& p, hipStream_t stream) {
    using namespace dlk::tiles;
    if (p.stage_ready) return 0;
    void* args[] = {const_cast<dlk_gemv_params*>(&p)};
    const bool norm = p.apply_norm && p.epilogue != DLK_EPI_RESIDUAL;
    const void* prep = norm ? reinterpret_cast<const void*>(&prepare_rows<true>)
                            : reinterpret_cast<const void*>(&prepare_rows<false>);
    return static_cast<int>(
        hipLaunchKernel(prep, dim3((p.M + 15) / 16, prep_chunks(p.K)), dim3(kPrepThreads), args, 0, stream));
}

int launch_gemm(const dlk_gemv_params& params, hipStream_t stream) {
    using namespace dlk::gemm;
    const int blocks = blocks_of(params);
    if (params.epilogue == DLK_EPI_LOGITS && params.sample_mode != 0 && params.partial_blocks != blocks)
        return static_cast<int>(hipErrorInvalidValue);
    dlk_gemv_params p = params;
    for (int m0 = 0; m0 < params.M; m0 += kMaxRows) {
        p.M = std::min(kMaxRows, params.M - m0);
        p.x = params.x + static_cast<int64_t>(m0) * params.ldx;
        p.m_base = params.m_base + m0;
        if (params.epilogue != DLK_EPI_QKV) p.y = params.y ? params.y + static_cast<int64_t>(m0) * params.ldy : nullptr;
        if (params.residual) p.residual = params.residual + static_cast<int64_t>(m0) * params.ldres;
        p.bump_position = m0 + kMaxRows >= params.M ? params.bump_position : nullptr;
        const bool wide_parts = wide_parts_eligible(p);
        if (wide_parts || wide_eligible(p)) {
            // few weight tiles: one launch, K split over the waves of each tile's work-group
            const int parts = wide_parts ? (p.M + 15) / 16 : 1;
            p.row_parts = parts;
            const Kernel wide = resolve_gemm(p, wide_parts ? 1 : row_tiles(p.M), -1);
            if (!wide.fn) return static_cast<int>(hipErrorInvalidValue);
            void* wargs[] = {&p};
            const hipError_t status = hipLaunchKernel(wide.fn, dim3(tiles_of(p), parts),
                                                      dim3(kWideWaves * dlk::kWave), wargs, 0, stream);
            p.row_parts = 0;
            if (status != hipSuccess) return static_cast<int>(status);
            continue;
        }
        // SwiGLU over two or more 16-row tiles with tile groups for a quarter of the CUs or more: split over the
        // rows rather than the keys.  The row parts of a tile group run on one XCD (consecutive work-group ids go
        // to the 8 XCDs in turn and the grid is a multiple of 8 wide), where they share its weights in the L2, and
        // no reduce launch follows (measured on MI355X at batch 32, 1B: gate/up 19.2 -> 16.5 us a layer, the
        // C3 step 1.326 -> 1.280 ms)
        const int parts = (p.M + 15) / 16;
        if (p.epilogue == DLK_EPI_SWIGLU && parts > 1 && blocks >= 64 && blocks * parts <= 256 && blocks % 8 == 0) {
            p.row_parts = parts;
            // parts of 16 rows: the deep pipeline when the weights come repacked
            const Kernel kernel = resolve_gemm(p, 1, loop_variant(p.K / chunk_k(1), repacked(p)));
            if (!kernel.fn) return static_cast<int>(hipErrorInvalidValue);
            void* args[] = {&p};
            const hipError_t status =
                hipLaunchKernel(kernel.fn, dim3(blocks, parts), dim3(kThreads), args, kernel.lds, stream);
            if (status != hipSuccess) return static_cast<int>(status);
            p.row_parts = 0;
            continue;
        }
        // key slices when the tiles leave CUs idle and the caller gave room for the partials
        int splits = splits_of(p, p.M);
        if (splits > 1 && (!p.split_partial || p.split_capacity < split_floats(p, splits, p.M))) splits = 1;
        // the reduce addresses the partials with 32-bit byte offsets
        if (splits > 1 && split_floats(p, kMaxSplits, p.M) * 4 > INT32_MAX) splits = 1;
        // a deferred reduce leaves one row block's QKV partials for the attention
        if (p.defer_reduce && (splits == 1 || p.epilogue != DLK_EPI_QKV || params.M > kMaxRows))
            return static_cast<int>(hipErrorInvalidValue);
        const int mt = row_tiles(p.M);
        const bool deep = repacked(p) && p.M >= 16;
        const Kernel kernel = resolve_gemm(p, mt, loop_variant(p.K / splits / chunk_k(mt), deep));
        if (!kernel.fn) return static_cast<int>(hipErrorInvalidValue);
        const int64_t* bump = p.bump_position;
        if (splits > 1) p.bump_position = nullptr; // the reduce launch advances the length
        void* args[] = {&p};
        hipError_t status = hipLaunchKernel(kernel.fn, dim3(blocks, splits), dim3(kThreads), args, kernel.lds, stream);
        if (status != hipSuccess) return static_cast<int>(status);
        if (p.defer_reduce) continue; // the attention finishes the projection
        if (splits > 1) {
            p.bump_position = const_cast<int64_t*>(bump);
            const Kernel reduce = resolve_reduce(p);
            if (!reduce.fn) return static_cast<int>(hipErrorInvalidValue);
            const int64_t threads = static_cast<int64_t>(p.M) * tiles_of(p) * 4;
            void* rargs[] = {&p, &splits};
            status = hipLaunchKernel(reduce.fn,
                                     dim3(static_cast<unsigned>((threads + kReduceThreads - 1) / kReduceThreads)),
                                     dim3(kReduceThreads), rargs, 0, stream);
            if (status != hipSuccess) return static_cast<int>(status);
        }
    }
    return 0;
}

// resident waves of a kernel on the current device (0 on error)
int resident_waves(const Kernel& kernel) {
    static std::mutex mutex;
    static std::unordered_map<uint64_t, int> cache;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 0;
    const uint64_t key = reinterpret_cast<uint64_t>(kernel.fn) ^ (static_cast<uint64_t>(kernel.lds) << 48) ^
                         (static_cast<uint64_t>(device) << 40);
    {
        std::lock_guard<std::mutex> lock(mutex);
        auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel.fn, dlk::gemv::kThreads, kernel.lds) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return 0;
    const int waves = per_cu * cus * dlk::gemv::kWavesPerBlock;
    std::lock_guard<std::mutex> lock(mutex);
    cache[key] = waves;
    return waves;
}

// waves of every launch of this call (sized for the widest activation tile, the lowest occupancy); 0 on error.
// Launches of many row groups give each wave two: the wave loads its activation row once for both, and the
// second group's weights are in flight while the first is reduced.  Measured on MI355X under graph replay at
// the 1B decode shapes (groups 1536 / 2816 / 2048 for QKV, gate/up, down): 6.04 -> 5.62, 10.83 -> 10.14 and
// 7.31 -> 6.26 us; with 1024 groups (O projection) one per wave stays faster (3.76 vs 4.45 us).  Three or four
// groups per wave were slower (a C2 step 541 -> 553 / 591 us), and so were work-groups of two waves instead of four
// (543 -> 558 us).
int launch_waves(const dlk_gemv_params& p) {
    using namespace dlk::gemv;
    constexpr int kPairedGroups = 1536;
    const Plan plan = plan_of(p.K, p.w_bf16 != 0, p.epilogue);
    const Kernel widest = resolve(p, activation_tile(std::min(p.M, plan.mt_max)));
    if (!widest.fn) return 0;
    const int resident = resident_waves(widest);
    if (resident <= 0) return 0;
    const int groups = groups_of(p, plan.rows, p.epilogue == DLK_EPI_SWIGLU);
    const int wanted = groups >= kPairedGroups ? (groups + 1) / 2 : groups;
    return std::max(1, std::min({wanted, kMaxWaves, resident}));
}

} // namespace

namespace {

// One thread per 16-byte piece of the output: piece (tile t, k step s, lane l) = row l % 16 of tile t, columns
// 32 s + 8 (l / 16) .. +8.
__global__ __launch_bounds__(256) void pack_tiles(const uint16_t* w0, const uint16_t* w1, int swiglu, int64_t tiles,
                                                  int64_t K, uint16_t* out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t steps = K / 32;
    if (i >= tiles * steps * dlk::kWave) return;
    const int lane = static_cast<int>(i % dlk::kWave);
    const int64_t block = i / dlk::kWave, t = block / steps, s = block % steps;
    const int r = lane % 16, q = lane / 16;
    const uint16_t* row = swiglu ? (r & 1 ? w1 : w0) + (8 * t + r / 2) * K : w0 + (16 * t + r) * K;
    *reinterpret_cast<uint4*>(out + block * 512 + 8 * lane) = *reinterpret_cast<const uint4*>(row + 32 * s + 8 * q);
}

} // namespace

extern "C" int dlk_pack_tiles(const void* w0, const void* w1, int swiglu, int64_t rows, int64_t K, void* out,
                              dlh_stream stream) {
    const int64_t per_tile = swiglu ? 8 : 16;
    if (!w0 || !out || (swiglu && !w1) || rows <= 0 || K <= 0 || K % 32 != 0 || rows % per_tile != 0)
        return static_cast<int>(hipErrorInvalidValue);
    const int64_t pieces = rows / per_tile * (K / 32) * dlk::kWave;
    const int64_t blocks = (pieces + 255) / 256;
    if (blocks > INT32_MAX) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(pack_tiles, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w0),
                       static_cast<const uint16_t*>(w1), swiglu, rows / per_tile, K, static_cast<uint16_t*>(out));
    return static_cast<int>(hipGetLastError());
}

extern "C" int dlk_gemv_uses_rows(const dlk_gemv_params* p) {
    // both matrix-core kernels of the batched path (gemm_rows, gemm_wide) read the repacked weights
    return !dlk::tiles::eligible(*p) && dlk::gemm::eligible(*p) ? 1 : 0;
}

extern "C" int dlk_gemv_folds_lora(const dlk_gemv_params* p) {
    return !dlk::tiles::eligible(*p) && dlk::gemm::eligible(*p) && dlk::gemm::lora_fold_eligible(*p) ? 1 : 0;
}

extern "C" int64_t dlk_gemv_split_floats(const dlk_gemv_params* p) {
    if (dlk::tiles::eligible(*p)) return 0;
    if (!dlk::gemm::eligible(*p)) return 0;
    const int rows = std::min(p->M, dlk::gemm::kMaxRows);
    return dlk::gemm::split_floats(*p, dlk::gemm::splits_of(*p, rows), rows);
}

extern "C" int dlk_gemv_split_count(const dlk_gemv_params* p) {
    using namespace dlk::gemm;
    if (dlk::tiles::eligible(*p) || !eligible(*p) || p->M > kMaxRows || wide_eligible(*p) || wide_parts_eligible(*p))
        return 1;
    int splits = splits_of(*p, p->M);
    if (splits > 1 && (!p->split_partial || p->split_capacity < split_floats(*p, splits, p->M))) splits = 1;
    if (splits > 1 && split_floats(*p, kMaxSplits, p->M) * 4 > INT32_MAX) splits = 1;
    return splits;
}

extern "C" int64_t dlk_gemv_stage_bytes(const dlk_gemv_params* p) {
    return dlk::tiles::shape_eligible(*p) ? dlk::tiles::stage_bytes(*p) : 0;
}

extern "C" int dlk_gemv_blocks(const dlk_gemv_params* p) {
    // LOGITS: one sampling candidate per work-group of the launch
    if (dlk::gemm::eligible(*p)) return dlk::gemm::blocks_of(*p);
    const int waves = launch_waves(*p);
    return waves > 0 ? (waves + dlk::gemv::kWavesPerBlock - 1) / dlk::gemv::kWavesPerBlock : -1;
}

extern "C" int dlk_gemv(const dlk_gemv_params* params, dlh_stream stream_handle) {
    using namespace dlk::gemv;
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    const int chunk = params->w_bf16 ? 8 : 4;
    if (params->K <= 0 || params->K % chunk != 0 || params->M <= 0 || params->nseg < 1 || params->nseg > 3)
        return static_cast<int>(hipErrorInvalidValue);
    if (params->K > kLdsXL * kThreads * 4 || static_cast<size_t>(params->K) * sizeof(float) > kLdsBytes)
        return static_cast<int>(hipErrorInvalidValue);
    if (params->apply_norm && params->epilogue == DLK_EPI_RESIDUAL) return static_cast<int>(hipErrorInvalidValue);
    if (params->epilogue == DLK_EPI_SWIGLU && (params->nseg != 2 || params->seg_rows[0] != params->seg_rows[1]))
        return static_cast<int>(hipErrorInvalidValue);
    if (params->epilogue == DLK_EPI_QKV)
        for (int s = 0; s < params->nseg; ++s)
            if (params->seg_rows[s] % 2 != 0 || params->head_dim % 2 != 0) return static_cast<int>(hipErrorInvalidValue);
    // the staged SwiGLU output exists only on the tiled path
    if (params->stage_out && (params->epilogue != DLK_EPI_SWIGLU || !dlk::tiles::eligible(*params) ||
                              params->seg_rows[0] % 32 != 0 || reinterpret_cast<uintptr_t>(params->stage_out) % 16 != 0))
        return static_cast<int>(hipErrorInvalidValue);
    if (params->defer_reduce && (dlk::tiles::eligible(*params) || !dlk::gemm::eligible(*params) ||
                                 dlk::gemm::wide_eligible(*params)))
        return static_cast<int>(hipErrorInvalidValue);
    // only the wide kernel applies LoRA down rows
    if ((params->lora_down[0] || params->lora_down[1] || params->lora_down[2]) && !dlk_gemv_folds_lora(params))
        return static_cast<int>(hipErrorInvalidValue);
    if (dlk::tiles::eligible(*params)) return launch_tiles(*params, stream);
    if (dlk::gemm::eligible(*params)) return launch_gemm(*params, stream);
    const int waves = launch_waves(*params);
    if (waves <= 0) return static_cast<int>(hipErrorInvalidValue);
    const int blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    if (params->epilogue == DLK_EPI_LOGITS && params->sample_mode != 0 && params->partial_blocks != blocks)
        return static_cast<int>(hipErrorInvalidValue);
    const int max_rows = plan_of(params->K, params->w_bf16 != 0, params->epilogue).mt_max;
    dlk_gemv_params p = *params;
    // activation rows are processed max_rows at a time (weights re-streamed per chunk of rows)
    for (int m0 = 0; m0 < params->M; m0 += max_rows) {
        p.M = std::min(max_rows, params->M - m0);
        p.x = params->x + static_cast<int64_t>(m0) * params->ldx;
        p.m_base = params->m_base + m0;
        if (params->epilogue != DLK_EPI_QKV) p.y = params->y ? params->y + static_cast<int64_t>(m0) * params->ldy : nullptr;
        if (params->residual) p.residual = params->residual + static_cast<int64_t>(m0) * params->ldres;
        p.bump_position = m0 + max_rows >= params->M ? params->bump_position : nullptr;
        const Kernel kernel = resolve(p, activation_tile(p.M));
        if (!kernel.fn) return static_cast<int>(hipErrorInvalidValue);
        void* args[] = {&p};
        const hipError_t status = hipLaunchKernel(kernel.fn, dim3(blocks), dim3(kThreads), args, kernel.lds, stream);
        if (status != hipSuccess) return static_cast<int>(status);
    }
    return 0;
}
