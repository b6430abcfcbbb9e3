// The C ABI (include/tgx.h) over the runtime: argument checks, the thread's error message, and
// nothing else.
#include "handles.hpp"

namespace tgx {
const char* last_error();
}


using namespace tgx;

extern "C" {

const char* tgx_last_error(void) { return last_error(); }

tgx_status tgx_context_create(int device, tgx_context** out) {
    clear_error();
    if (!out) return fail(TGX_E_ARG, "null output");
    Context* ctx = nullptr;
    TGX_TRY(context_create(device, &ctx));
    *out = new tgx_context{ctx};
    return TGX_OK;
}

void tgx_context_destroy(tgx_context* ctx) {
    if (!ctx) return;
    context_destroy(ctx->ctx);
    delete ctx;
}

tgx_status tgx_context_report(const tgx_context* ctx, tgx_device_report* out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    const hipDeviceProp_t& p = ctx->ctx->prop;
    *out = tgx_device_report{};
    std::snprintf(out->name, sizeof out->name, "%s", p.name);
    std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bytes = p.totalGlobalMem;
    out->wavefront = p.warpSize;
    return TGX_OK;
}

tgx_status tgx_stream_read(tgx_context* ctx, size_t bytes, int times, float* best_ms, float* mean_ms) {
    clear_error();
    if (!ctx || !best_ms || !mean_ms) return fail(TGX_E_ARG, "null context or output");
    const size_t unit = stream_read_unit();
    if (bytes < unit || times <= 0) return fail(TGX_E_ARG, "stream read of " + std::to_string(bytes) + " bytes " + std::to_string(times) + " times");
    bytes -= bytes % unit;
    Context* c = ctx->ctx;
    TGX_HIP(hipSetDevice(c->device));
    void* data = nullptr;
    uint32_t* out = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    auto done = [&](tgx_status st) {
        if (data) hipFree(data);
        if (out) hipFree(out);
        if (a) hipEventDestroy(a);
        if (b) hipEventDestroy(b);
        return st;
    };
    auto check = [&](hipError_t e, const char* what) {
        return e == hipSuccess ? TGX_OK : fail(TGX_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
    };
    tgx_status st = check(hipMalloc(&data, bytes), "hipMalloc");
    if (st == TGX_OK) st = check(hipMalloc((void**)&out, bytes / unit * 4 * sizeof(uint32_t)), "hipMalloc");
    if (st == TGX_OK) st = check(hipMemsetAsync(data, 0x5a, bytes, c->stream), "hipMemsetAsync");
    if (st == TGX_OK) st = check(hipEventCreate(&a), "hipEventCreate");
    if (st == TGX_OK) st = check(hipEventCreate(&b), "hipEventCreate");
    if (st == TGX_OK) st = check(launch_stream_read(data, bytes, out, c->stream), "stream_read");  // warm
    float best = 0.f, total = 0.f;
    for (int i = 0; i < times && st == TGX_OK; ++i) {
        st = check(hipEventRecord(a, c->stream), "hipEventRecord");
        if (st == TGX_OK) st = check(launch_stream_read(data, bytes, out, c->stream), "stream_read");
        if (st == TGX_OK) st = check(hipEventRecord(b, c->stream), "hipEventRecord");
        if (st == TGX_OK) st = check(hipEventSynchronize(b), "hipEventSynchronize");
        float ms = 0.f;
        if (st == TGX_OK) st = check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
        total += ms;
        if (i == 0 || ms < best) best = ms;
    }
    if (st == TGX_OK) {
        *best_ms = best;
        *mean_ms = total / times;
    }
    return done(st);
}

tgx_status tgx_shape_check(const tgx_shape* shape, const tgx_batch* batch) {
    clear_error();
    Shape s;
    TGX_TRY(check_shape(shape, &s));
    return check_batch(s, batch);
}

tgx_status tgx_batch_placement(int slots, int capacity, const tgx_row* rows, int nrows, uint32_t* words) {
    clear_error();
    if (!rows || !words || nrows < 0) return fail(TGX_E_ARG, "null rows or words");
    return placement(slots, capacity, rows, nrows, words);
}

tgx_status tgx_decoder_create(tgx_context* ctx, const tgx_shape* shape, const tgx_batch* batch, tgx_decoder** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    Decoder* d = nullptr;
    TGX_TRY(decoder_create(ctx->ctx, shape, batch, &d));
    *out = new tgx_decoder{d};
    return TGX_OK;
}

void tgx_decoder_destroy(tgx_decoder* dec) {
    if (!dec || dec->borrowed) return;
    decoder_destroy(dec->dec);
    delete dec;
}

#define DEC(d) ((d) ? (d)->dec : nullptr)

tgx_status tgx_decoder_load(tgx_decoder* dec, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    clear_error();
    return decoder_load(DEC(dec), name, data, dtype, count);
}

tgx_status tgx_decoder_set_rows(tgx_decoder* dec, const tgx_row* rows, int nrows, const float* x) {
    clear_error();
    return decoder_set_rows(DEC(dec), rows, nrows, x);
}

tgx_status tgx_decoder_start(tgx_decoder* dec) {
    clear_error();
    return decoder_start(DEC(dec));
}

tgx_status tgx_decoder_wait(tgx_decoder* dec) {
    clear_error();
    return decoder_wait(DEC(dec));
}

tgx_status tgx_decoder_output(tgx_decoder* dec, float* out) {
    clear_error();
    return decoder_output(DEC(dec), out);
}

tgx_status tgx_decoder_step_rows(tgx_decoder* dec, const tgx_row* rows, int nrows, const float* x, float* out) {
    clear_error();
    TGX_TRY(decoder_set_rows(DEC(dec), rows, nrows, x));
    TGX_TRY(decoder_start(DEC(dec)));
    TGX_TRY(decoder_wait(DEC(dec)));
    return decoder_output(DEC(dec), out);
}

tgx_status tgx_decoder_step(tgx_decoder* dec, uint32_t position, const float* x, float* out) {
    clear_error();
    if (!dec) return fail(TGX_E_ARG, "null decoder");
    if (dec->dec->rows != 1) return fail(TGX_E_SHAPE, "a step at batch 1 on a batch of " + std::to_string(dec->dec->rows));
    const tgx_row row{position, 0};
    return tgx_decoder_step_rows(dec, &row, 1, x, out);
}

tgx_status tgx_decoder_release_slot(tgx_decoder* dec, uint32_t slot) {
    clear_error();
    return decoder_release_slot(DEC(dec), slot);
}

tgx_status tgx_decoder_reserve(tgx_decoder* dec, uint32_t slot, uint32_t positions) {
    clear_error();
    return decoder_reserve(DEC(dec), slot, positions);
}

tgx_status tgx_decoder_free_blocks(const tgx_decoder* dec, int* out) {
    clear_error();
    if (!dec || !out) return fail(TGX_E_ARG, "null decoder or output");
    *out = (int)dec->dec->free_list.size();
    return TGX_OK;
}

tgx_status tgx_decoder_launch(tgx_decoder* dec, int times, int advance) {
    clear_error();
    return decoder_launch(DEC(dec), times, advance);
}

tgx_status tgx_decoder_elapsed_ms(const tgx_decoder* dec, float* out) {
    clear_error();
    if (!dec || !out) return fail(TGX_E_ARG, "null decoder or output");
    if (dec->dec->pending) return fail(TGX_E_BUSY, "a step is under way");
    TGX_HIP(hipEventElapsedTime(out, dec->dec->ev_start, dec->dec->ev_end));
    return TGX_OK;
}

tgx_status tgx_decoder_set_timed(tgx_decoder* dec, int timed) {
    clear_error();
    if (!dec) return fail(TGX_E_ARG, "null decoder");
    if (dec->dec->pending) return fail(TGX_E_BUSY, "a step is under way");
    dec->dec->timed = timed != 0;
    return TGX_OK;
}

tgx_status tgx_decoder_set_graph(tgx_decoder* dec, int use_graph) {
    clear_error();
    if (!dec) return fail(TGX_E_ARG, "null decoder");
    if (dec->dec->pending) return fail(TGX_E_BUSY, "a step is under way");
    dec->dec->use_graph = use_graph != 0;
    return TGX_OK;
}

tgx_status tgx_decoder_timings(tgx_decoder* dec, int max, tgx_timing* out, int* n) {
    clear_error();
    return decoder_timings(DEC(dec), max, out, n);
}

tgx_status tgx_decoder_dispatches(const tgx_decoder* dec, int* out) {
    clear_error();
    if (!dec || !out) return fail(TGX_E_ARG, "null decoder or output");
    *out = dec->dec->dispatches;
    return TGX_OK;
}

tgx_status tgx_decoder_device_bytes(const tgx_decoder* dec, size_t* out) {
    clear_error();
    if (!dec || !out) return fail(TGX_E_ARG, "null decoder or output");
    *out = dec->dec->device_bytes + prefill_bytes(dec->dec);
    return TGX_OK;
}

tgx_status tgx_decoder_read_cache(tgx_decoder* dec, uint32_t slot, uint32_t positions, float* k, float* v) {
    clear_error();
    return decoder_read_cache(DEC(dec), slot, positions, k, v);
}

tgx_status tgx_prefill_run(tgx_decoder* dec, uint32_t slot, uint32_t start, uint32_t len, const float* x, float* out) {
    clear_error();
    const tgx_run run{slot, start, len};
    return prefill_runs(DEC(dec), &run, 1, x, out);
}

tgx_status tgx_prefill_runs(tgx_decoder* dec, const tgx_run* runs, int nruns, const float* x, float* out) {
    clear_error();
    return prefill_runs(DEC(dec), runs, nruns, x, out);
}

tgx_status tgx_prefill_launch(tgx_decoder* dec, int times) {
    clear_error();
    return prefill_launch(DEC(dec), times);
}

tgx_status tgx_prefill_runs_noalloc(tgx_decoder* dec, const tgx_run* runs, int nruns, const float* x, float* out) {
    clear_error();
    return prefill_runs_noalloc(DEC(dec), runs, nruns, x, out);
}

}  // extern "C"
