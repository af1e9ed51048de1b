// HIP runtime behind the engine-level C ABI (include/dinov3_engine.h). It
// replaces the HRX surface used by the reference's src/engine.rs:
// Device::open + target check (engine.rs:40-59), Stream::allocate/upload
// (60-70, 191-202), graph record (87-129), replay (203-214), pinned readback
// (215-269), the graph-vs-direct benchmark (130-190) and poison-on-failure.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/dinov3_engine.h"
#include "engine_internal.hpp"
#include "errors.hpp"
#include "host_copy.hpp"
#include "kernels/launch.hpp"

namespace {

constexpr char kPoisoned[] = "session is unusable after a GPU failure";

struct Recorded {
    hipGraphExec_t exec = nullptr;
    std::vector<dhx_launch> launches;  // the branches' lists back to back
    std::vector<uint64_t> counts;      // launches per branch
};

}  // namespace

struct dhx_engine {
    int device = 0;
    hipStream_t stream = nullptr;
    // Extra streams and events for plans with several branches: branch 0
    // runs on `stream`, branch i on aux[i-1], forked from and joined back
    // into `stream` with events (created on first use; default priority).
    std::vector<hipStream_t> aux;
    hipEvent_t fork = nullptr;
    std::vector<hipEvent_t> join;
    std::vector<void*> buffers;
    std::vector<uint64_t> sizes;
    std::vector<char> owned;  // 0: an external slot (engine_external), never freed here
    std::map<uint64_t, Recorded> graphs;
    void* readback = nullptr;
    uint64_t readback_bytes = 0;
    // Pipelined transfers: per slot a pinned input and output staging buffer
    // and events marking the end of its upload, graph and readback.
    hipStream_t up = nullptr, down = nullptr;
    void* pin_in[DHX_STAGING_SLOTS] = {};
    void* pin_out[DHX_STAGING_SLOTS] = {};
    uint64_t pin_in_bytes = 0, pin_out_bytes = 0;
    hipEvent_t in_done[DHX_STAGING_SLOTS] = {}, graph_done[DHX_STAGING_SLOTS] = {},
               out_done[DHX_STAGING_SLOTS] = {};
    bool failed = false;
    bool fail_next = false;
    std::string error;
};

namespace {

// Every HIP call goes through here: a failure (or an injected one) poisons
// the engine, as any failed HRX call does in engine.rs.
void hip_check(dhx_engine* e, hipError_t err, const char* what) {
    if (e->fail_next) {
        e->fail_next = false;
        err = hipErrorUnknown;
    }
    if (err != hipSuccess) {
        e->failed = true;
        throw dhx::Error(std::string(what) + ": " + hipGetErrorString(err));
    }
}

void ensure_usable(const dhx_engine* e) {
    if (e->failed) throw dhx::Error(kPoisoned);
}

void* region_ptr(const dhx_engine* e, const dhx_region& r) {
    return static_cast<char*>(e->buffers[r.buffer]) + r.offset;
}

void check_region(const dhx_engine* e, const dhx_region& r) {
    if (r.buffer >= e->buffers.size()) throw dhx::Error("region names an unknown buffer");
    if (r.offset > e->sizes[r.buffer] || r.bytes > e->sizes[r.buffer] - r.offset)
        throw dhx::Error("region exceeds its buffer");
}

using dhx::kHidden;

struct Need {
    uint32_t bindings;
    std::vector<uint64_t> bytes;
};

uint64_t tokens_for(uint32_t grid) { return (uint64_t)grid * grid + dhx::kPrefix; }

// Bytes of an f16 activation matrix in fragment order (rows padded to 32).
uint64_t frag(uint64_t rows, uint64_t k) { return (rows + 31) / 32 * 32 * k * 2; }

// The shapes each kernel reads and writes, from its scalars; recording and
// dispatch refuse any binding smaller than this (so no kernel can run past a
// buffer) and any misaligned binding (kernels use 16-byte vector accesses).
Need required(const dhx_launch& l) {
    const uint32_t* s = l.scalars;
    const uint64_t H = kHidden;
    auto positive = [](uint64_t v, const char* what) {
        if (v == 0) throw dhx::Error(std::string(what) + " must be positive");
    };
    const uint64_t S = dhx::kStatFloats * 4;  // stats bytes per row
    switch (l.kernel) {
        case DHX_K_PATCH_EMBED:
        case DHX_K_PATCH_EMBED_STATS: {
            positive(s[0], "images");
            positive(s[1], "grid");
            const uint64_t side = 16ull * s[1], T = tokens_for(s[1]);
            const uint64_t px = s[0] * 3 * side * side * 4, x = frag(s[0] * T, H);
            if (l.kernel == DHX_K_PATCH_EMBED) return {5, {px, H * 768 * 2, H * 4, 5 * H * 4, x}};
            return {7, {px, H * 768 * 2, H * 4, 5 * H * 4, 5 * S, x, s[0] * T * S}};
        }
        case DHX_K_LAYERNORM:
        case DHX_K_LAYERNORM_F32: {
            positive(s[0], "rows");
            const uint64_t out = l.kernel == DHX_K_LAYERNORM ? frag(s[0], H) : s[0] * H * 4;
            return {4, {frag(s[0], H), H * 4, H * 4, out}};
        }
        case DHX_K_QKV_ROPE:
        case DHX_K_QKV_ROPE_LN:
        case DHX_K_ATTENTION: {
            positive(s[0], "images");
            positive(s[1], "grid");
            const uint64_t T = tokens_for(s[1]), P = (uint64_t)s[1] * s[1];
            if (s[2] % 128 != 0 || s[2] < T) throw dhx::Error("tpad must be a multiple of 128 covering every token");
            const uint64_t heads = s[0] * dhx::kHeads * (uint64_t)s[2] * dhx::kHeadDim * 2;
            if (l.kernel == DHX_K_ATTENTION) return {4, {heads, heads, heads, frag(s[0] * T, H)}};
            if (l.kernel == DHX_K_QKV_ROPE)
                return {8, {frag(s[0] * T, H), 3 * H * H * 2, 3 * H * 4, P * 64 * 4, P * 64 * 4, heads, heads, heads}};
            return {10, {frag(s[0] * T, H), s[0] * T * S, 3 * H * H * 2, 3 * H * 4, 3 * H * 4, P * 64 * 4, P * 64 * 4,
                         heads, heads, heads}};
        }
        case DHX_K_RESID:
        case DHX_K_RESID_STATS: {
            positive(s[0], "rows");
            if (s[1] == 0 || s[1] % 384 != 0) throw dhx::Error("k must be a positive multiple of 384");
            std::vector<uint64_t> b = {frag(s[0], s[1]), H * s[1] * 2, H * 4, H * 4, frag(s[0], H)};
            if (l.kernel == DHX_K_RESID_STATS) b.push_back(s[0] * S);
            return {(uint32_t)b.size(), b};
        }
        case DHX_K_SWIGLU:
            positive(s[0], "rows");
            return {4, {frag(s[0], H), 2ull * dhx::kFF * H * 2, 2ull * dhx::kFF * 4, frag(s[0], dhx::kFF)}};
        case DHX_K_SWIGLU_LN:
            positive(s[0], "rows");
            return {6, {frag(s[0], H), s[0] * S, 2ull * dhx::kFF * H * 2, 2ull * dhx::kFF * 4, 2ull * dhx::kFF * 4,
                        frag(s[0], dhx::kFF)}};
        case DHX_K_SPLITK: {
            positive(s[0], "rows");
            positive(s[2], "splits");
            if (s[1] == 0 || s[1] % (384ull * s[2]) != 0) throw dhx::Error("k must split into multiples of 384");
            return {3, {frag(s[0], s[1]), H * s[1] * 2, (uint64_t)s[2] * s[0] * H * 4}};
        }
        case DHX_K_SPLITK_REDUCE:
        case DHX_K_SPLITK_REDUCE_STATS: {
            positive(s[0], "rows");
            positive(s[1], "splits");
            std::vector<uint64_t> b = {(uint64_t)s[1] * s[0] * H * 4, H * 4, H * 4, frag(s[0], H)};
            if (l.kernel == DHX_K_SPLITK_REDUCE_STATS) b.push_back(s[0] * S);
            return {(uint32_t)b.size(), b};
        }
        default:
            throw dhx::Error("unknown kernel id " + std::to_string(l.kernel));
    }
}

void validate(const dhx_engine* e, const dhx_launch& l) {
    const Need need = required(l);
    if (l.n_bindings != need.bindings)
        throw dhx::Error("kernel " + std::to_string(l.kernel) + " takes " + std::to_string(need.bindings) +
                         " bindings, got " + std::to_string(l.n_bindings));
    for (uint32_t i = 0; i < l.n_bindings; ++i) {
        const dhx_region& r = l.bindings[i];
        check_region(e, r);
        if (r.offset % 16 != 0) throw dhx::Error("binding " + std::to_string(i) + " is not 16-byte aligned");
        if (r.bytes < need.bytes[i])
            throw dhx::Error("kernel " + std::to_string(l.kernel) + " binding " + std::to_string(i) + " needs " +
                             std::to_string(need.bytes[i]) + " bytes, region has " + std::to_string(r.bytes));
    }
}

hipError_t launch_one(dhx_engine* e, const dhx_launch& l, hipStream_t stream) {
    using namespace dhx;
    auto P = [&](int i) { return region_ptr(e, l.bindings[i]); };
    auto F = [&](int i) { return static_cast<const float*>(P(i)); };
    auto Hf = [&](int i) { return static_cast<half_t*>(P(i)); };
    const uint32_t* s = l.scalars;
    auto Fm = [&](int i) { return static_cast<float*>(P(i)); };
    switch (l.kernel) {
        case DHX_K_PATCH_EMBED:
            return launch_patch_embed({F(0), Hf(1), F(2), F(3), Hf(4), (int)s[0], (int)s[1]}, stream);
        case DHX_K_PATCH_EMBED_STATS:
            return launch_patch_embed({F(0), Hf(1), F(2), F(3), Hf(5), (int)s[0], (int)s[1], F(4), Fm(6)}, stream);
        case DHX_K_LAYERNORM:
        case DHX_K_LAYERNORM_F32:
            return launch_layernorm({Hf(0), F(1), F(2), P(3), (int)s[0], l.kernel == DHX_K_LAYERNORM_F32}, stream);
        case DHX_K_QKV_ROPE:
            return launch_qkv_rope({Hf(0), Hf(1), F(2), F(3), F(4), Hf(5), Hf(6), Hf(7), (int)s[0], (int)s[1], (int)s[2]},
                                   stream);
        case DHX_K_QKV_ROPE_LN:
            return launch_qkv_rope({Hf(0), Hf(2), F(4), F(5), F(6), Hf(7), Hf(8), Hf(9), (int)s[0], (int)s[1], (int)s[2],
                                    F(1), F(3)},
                                   stream);
        case DHX_K_ATTENTION:
            return launch_attention({Hf(0), Hf(1), Hf(2), Hf(3), (int)s[0], (int)tokens_for(s[1]), (int)s[2]}, stream);
        case DHX_K_RESID:
            return launch_resid({Hf(0), Hf(1), F(2), F(3), Hf(4), (int)s[0], (int)s[1]}, stream);
        case DHX_K_RESID_STATS:
            return launch_resid({Hf(0), Hf(1), F(2), F(3), Hf(4), (int)s[0], (int)s[1], Fm(5)}, stream);
        case DHX_K_SWIGLU:
            return launch_swiglu({Hf(0), Hf(1), F(2), Hf(3), (int)s[0]}, stream);
        case DHX_K_SWIGLU_LN:
            return launch_swiglu({Hf(0), Hf(2), F(4), Hf(5), (int)s[0], F(1), F(3)}, stream);
        case DHX_K_SPLITK:
            return launch_splitk({Hf(0), Hf(1), (float*)P(2), (int)s[0], (int)s[1], (int)s[2]}, stream);
        case DHX_K_SPLITK_REDUCE:
            return launch_splitk_reduce({F(0), F(1), F(2), Hf(3), (int)s[0], (int)s[1]}, stream);
        case DHX_K_SPLITK_REDUCE_STATS:
            return launch_splitk_reduce({F(0), F(1), F(2), Hf(3), (int)s[0], (int)s[1], Fm(4)}, stream);
        default:
            return hipErrorInvalidValue;
    }
}

// Streams and events for `branches` concurrent lists.
void ensure_branch_streams(dhx_engine* e, uint32_t branches) {
    if (!e->fork) hip_check(e, hipEventCreateWithFlags(&e->fork, hipEventDisableTiming), "hipEventCreate");
    while (e->aux.size() + 1 < branches) {
        hipStream_t s = nullptr;
        hip_check(e, hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        e->aux.push_back(s);
        hipEvent_t ev = nullptr;
        hip_check(e, hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate");
        e->join.push_back(ev);
    }
}

// Queues the branches of a plan: branch 0 on the engine stream, the others
// forked from it onto the auxiliary streams and joined back, so work queued
// on the engine stream afterwards waits for every branch. Used both under
// stream capture (the fork/join become graph edges) and for direct dispatch.
// Returns the first launch error; the fork/join structure is completed even
// then so that a capture can still be ended.
hipError_t queue_branches(dhx_engine* e, const Recorded& r) {
    const size_t n = r.counts.size();
    hipError_t err = hipSuccess;
    auto keep = [&](hipError_t x) {
        if (err == hipSuccess) err = x;
    };
    if (n > 1) {
        keep(hipEventRecord(e->fork, e->stream));
        for (size_t i = 1; i < n; ++i) keep(hipStreamWaitEvent(e->aux[i - 1], e->fork, 0));
    }
    size_t first = 0;
    for (size_t i = 0; i < n; ++i) {
        hipStream_t s = i == 0 ? e->stream : e->aux[i - 1];
        for (size_t j = first; j < first + r.counts[i] && err == hipSuccess; ++j) keep(launch_one(e, r.launches[j], s));
        first += r.counts[i];
    }
    for (size_t i = 1; i < n; ++i) {
        keep(hipEventRecord(e->join[i - 1], e->aux[i - 1]));
        keep(hipStreamWaitEvent(e->stream, e->join[i - 1], 0));
    }
    return err;
}

void set_device(dhx_engine* e) { hip_check(e, hipSetDevice(e->device), "hipSetDevice"); }

double percentile_sorted(const std::vector<double>& t, int pct) {
    // engine.rs:177-183: median = t[n/2], p95 = t[ceil(n*95/100) - 1].
    if (pct == 50) return t[t.size() / 2];
    return t[(t.size() * pct + 99) / 100 - 1];
}

template <class F>
int guarded(dhx_engine* e, F&& f) {
    try {
        if (!e) throw dhx::Error("null engine");
        f();
        return 0;
    } catch (const std::exception& ex) {
        if (e) e->error = ex.what();
        else dhx::set_global_error(ex.what());
        return 1;
    }
}

void release_staging(dhx_engine* e) {
    for (hipStream_t* st : {&e->up, &e->down})
        if (*st) {
            (void)hipStreamSynchronize(*st);
            (void)hipStreamDestroy(*st);
            *st = nullptr;
        }
    for (int i = 0; i < DHX_STAGING_SLOTS; ++i) {
        for (hipEvent_t* ev : {&e->in_done[i], &e->graph_done[i], &e->out_done[i]})
            if (*ev) {
                (void)hipEventDestroy(*ev);
                *ev = nullptr;
            }
        if (e->pin_in[i]) (void)hipHostFree(e->pin_in[i]);
        if (e->pin_out[i]) (void)hipHostFree(e->pin_out[i]);
        e->pin_in[i] = e->pin_out[i] = nullptr;
    }
    e->pin_in_bytes = e->pin_out_bytes = 0;
}

void check_slot(const dhx_engine* e, uint32_t slot) {
    if (slot >= DHX_STAGING_SLOTS) throw dhx::Error("staging slot must be 0 or 1");
    if (!e->up) throw dhx::Error("staging was not reserved");
}

}  // namespace

namespace dhx {

// memcpy split over host threads: pageable <-> pinned copies of tens of MB
// run at a few GB/s on one core, far below the PCIe link.
uint32_t engine_external(dhx_engine* e, void* ptr, uint64_t bytes) {
    e->buffers.push_back(ptr);
    e->sizes.push_back(bytes);
    e->owned.push_back(0);
    return (uint32_t)(e->buffers.size() - 1);
}

void engine_rebind(dhx_engine* e, uint32_t buffer, void* ptr, uint64_t bytes) {
    if (buffer >= e->buffers.size() || e->owned[buffer]) throw Error("not an external buffer slot");
    e->buffers[buffer] = ptr;
    e->sizes[buffer] = bytes;
}

void engine_queue(dhx_engine* e, const dhx_launch* launches, size_t n, hipStream_t stream) {
    ensure_usable(e);
    for (size_t i = 0; i < n; ++i) validate(e, launches[i]);
    set_device(e);
    for (size_t i = 0; i < n; ++i) hip_check(e, launch_one(e, launches[i], stream), "kernel launch");
}

void* engine_staging_in(dhx_engine* e, uint32_t slot) {
    check_slot(e, slot);
    return e->pin_in[slot];
}

void* engine_staging_out(dhx_engine* e, uint32_t slot) {
    check_slot(e, slot);
    return e->pin_out[slot];
}

uint64_t engine_staging_in_bytes(const dhx_engine* e) { return e->pin_in_bytes; }

uint64_t engine_staging_out_bytes(const dhx_engine* e) { return e->pin_out_bytes; }

void engine_wait_upload(dhx_engine* e, uint32_t slot) {
    ensure_usable(e);
    check_slot(e, slot);
    set_device(e);
    hip_check(e, hipEventSynchronize(e->in_done[slot]), "upload wait");
}

void engine_upload(dhx_engine* e, dhx_region dst, uint64_t n, uint32_t slot) {
    ensure_usable(e);
    check_slot(e, slot);
    check_region(e, dst);
    if (n > dst.bytes) throw Error("input exceeds allocated region");
    if (n > e->pin_in_bytes) throw Error("input exceeds reserved staging");
    set_device(e);
    // dst is the slot's device input, which the graph last replayed for this
    // slot may still be reading.
    hip_check(e, hipStreamWaitEvent(e->up, e->graph_done[slot], 0), "hipStreamWaitEvent");
    hip_check(e, hipMemcpyAsync(region_ptr(e, dst), e->pin_in[slot], n, hipMemcpyHostToDevice, e->up), "upload");
    hip_check(e, hipEventRecord(e->in_done[slot], e->up), "hipEventRecord");
}

void engine_wait_readback(dhx_engine* e, uint32_t slot) {
    ensure_usable(e);
    check_slot(e, slot);
    set_device(e);
    hip_check(e, hipEventSynchronize(e->out_done[slot]), "readback wait");
}

hipStream_t engine_stream(const dhx_engine* e) { return e->stream; }

int engine_device(const dhx_engine* e) { return e->device; }

void engine_check(dhx_engine* e, hipError_t err, const char* what) { hip_check(e, err, what); }

void engine_ensure_usable(const dhx_engine* e) { ensure_usable(e); }

}  // namespace dhx

extern "C" {

int dhx_engine_open(int32_t device, dhx_engine** out) {
    try {
        if (!out) throw dhx::Error("null output pointer");
        *out = nullptr;
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw dhx::Error("no HIP device is available");
        if (device < 0 || device >= count)
            throw dhx::Error("device " + std::to_string(device) + " does not exist (" + std::to_string(count) +
                             " visible)");
        if (hipSetDevice(device) != hipSuccess) throw dhx::Error("cannot select device " + std::to_string(device));
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, device) != hipSuccess) throw dhx::Error("cannot query device properties");
        const std::string arch = prop.gcnArchName;
        if (arch.rfind("gfx950", 0) != 0)
            throw dhx::Error("these kernels are validated for gfx950, found " + arch);
        auto* e = new dhx_engine();
        e->device = device;
        if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
            delete e;
            throw dhx::Error("cannot create a HIP stream");
        }
        *out = e;
        return 0;
    } catch (const std::exception& ex) {
        dhx::set_global_error(ex.what());
        return 1;
    }
}

void dhx_engine_free(dhx_engine* e) {
    if (!e) return;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    release_staging(e);  // waits for the transfer streams before their buffers go
    for (auto& kv : e->graphs)
        if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    for (size_t i = 0; i < e->buffers.size(); ++i)
        if (e->owned[i]) (void)hipFree(e->buffers[i]);
    if (e->readback) (void)hipHostFree(e->readback);
    for (hipStream_t s : e->aux) {
        (void)hipStreamSynchronize(s);
        (void)hipStreamDestroy(s);
    }
    for (hipEvent_t ev : e->join) (void)hipEventDestroy(ev);
    if (e->fork) (void)hipEventDestroy(e->fork);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

const char* dhx_last_error(const dhx_engine* e) { return e ? e->error.c_str() : dhx::global_error(); }

int dhx_allocate(dhx_engine* e, uint64_t bytes, dhx_region* out) {
    return guarded(e, [&] {
        ensure_usable(e);
        if (!out) throw dhx::Error("null output region");
        set_device(e);
        void* p = nullptr;
        hip_check(e, hipMalloc(&p, std::max<uint64_t>(bytes, 16)), "hipMalloc");
        e->buffers.push_back(p);
        e->sizes.push_back(bytes);
        e->owned.push_back(1);
        // Zero once: padded rows of q/k/v are never written and must stay finite.
        // The engine's stream does not synchronise with the legacy default
        // stream, so the fill is queued on it and waited for: a later upload or
        // kernel on that stream can never overtake it.
        hip_check(e, hipMemsetAsync(p, 0, std::max<uint64_t>(bytes, 16), e->stream), "hipMemsetAsync");
        hip_check(e, hipStreamSynchronize(e->stream), "allocation synchronize");
        *out = dhx_region{(uint32_t)(e->buffers.size() - 1), 0, bytes};
    });
}

int dhx_weight(dhx_engine* e, const void* bytes, uint64_t n, dhx_region* out) {
    return guarded(e, [&] {
        if (dhx_allocate(e, n, out) != 0) throw dhx::Error(e->error);
        hip_check(e, hipMemcpyAsync(region_ptr(e, *out), bytes, n, hipMemcpyHostToDevice, e->stream), "weight upload");
        hip_check(e, hipStreamSynchronize(e->stream), "weight upload synchronize");
    });
}

int dhx_upload(dhx_engine* e, dhx_region r, const void* bytes, uint64_t n) {
    return guarded(e, [&] {
        ensure_usable(e);
        check_region(e, r);
        if (n > r.bytes) throw dhx::Error("input exceeds allocated region");
        set_device(e);
        hip_check(e, hipMemcpyAsync(region_ptr(e, r), bytes, n, hipMemcpyHostToDevice, e->stream), "upload");
        hip_check(e, hipStreamSynchronize(e->stream), "upload synchronize");
    });
}

int dhx_record_branches(dhx_engine* e, uint64_t batch, const dhx_launch* launches, const uint64_t* counts,
                        uint32_t branches) {
    return guarded(e, [&] {
        ensure_usable(e);
        if (e->graphs.count(batch)) return;
        if (branches < 1 || branches > DHX_MAX_BRANCHES)
            throw dhx::Error("branches must be 1.." + std::to_string(DHX_MAX_BRANCHES));
        if (!counts) throw dhx::Error("null branch counts");
        Recorded rec;
        rec.counts.assign(counts, counts + branches);
        uint64_t n = 0;
        for (uint64_t c : rec.counts) n += c;
        if (n && !launches) throw dhx::Error("null launch list");
        rec.launches.assign(launches, launches + n);
        for (const dhx_launch& l : rec.launches) validate(e, l);  // before any GPU work
        set_device(e);
        ensure_branch_streams(e, branches);
        // Within a branch each node follows its predecessor, covering every
        // read-before-write on reused buffers (engine.rs:110-111); branches
        // are forked from and joined back into the capturing stream.
        hip_check(e, hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "begin capture");
        const hipError_t launch_err = queue_branches(e, rec);
        hipGraph_t graph = nullptr;
        const hipError_t end_err = hipStreamEndCapture(e->stream, &graph);
        if (launch_err != hipSuccess || end_err != hipSuccess) {
            if (graph) (void)hipGraphDestroy(graph);
            hip_check(e, launch_err != hipSuccess ? launch_err : end_err, "graph capture");
        }
        hipGraphExec_t exec = nullptr;
        const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        hip_check(e, inst, "graph instantiate");
        rec.exec = exec;
        e->graphs[batch] = std::move(rec);
    });
}

int dhx_record(dhx_engine* e, uint64_t batch, const dhx_launch* launches, uint64_t n) {
    return dhx_record_branches(e, batch, launches, &n, 1);
}

int dhx_has_graph(const dhx_engine* e, uint64_t batch) { return e && e->graphs.count(batch) ? 1 : 0; }

int dhx_replay(dhx_engine* e, uint64_t batch) {
    return guarded(e, [&] {
        ensure_usable(e);
        auto it = e->graphs.find(batch);
        if (it == e->graphs.end()) throw dhx::Error("batch has not been prepared");
        set_device(e);
        hip_check(e, hipGraphLaunch(it->second.exec, e->stream), "graph launch");
    });
}

int dhx_dispatch(dhx_engine* e, uint64_t batch) {
    return guarded(e, [&] {
        ensure_usable(e);
        auto it = e->graphs.find(batch);
        if (it == e->graphs.end()) throw dhx::Error("batch has not been prepared");
        set_device(e);
        hip_check(e, queue_branches(e, it->second), "kernel launch");
    });
}

int dhx_synchronize(dhx_engine* e) {
    return guarded(e, [&] {
        ensure_usable(e);
        set_device(e);
        hip_check(e, hipStreamSynchronize(e->stream), "synchronize");
    });
}

int dhx_reserve_readback(dhx_engine* e, uint64_t bytes) {
    return guarded(e, [&] {
        ensure_usable(e);
        set_device(e);
        if (e->readback) {
            hip_check(e, hipHostFree(e->readback), "hipHostFree");
            e->readback = nullptr;
            e->readback_bytes = 0;
        }
        hip_check(e, hipHostMalloc(&e->readback, std::max<uint64_t>(bytes, 16), hipHostMallocDefault), "hipHostMalloc");
        e->readback_bytes = bytes;
    });
}

int dhx_read(dhx_engine* e, dhx_region r, void* out, uint64_t n) {
    return guarded(e, [&] {
        ensure_usable(e);
        if (!e->readback) throw dhx::Error("readback was not reserved");
        if (n > e->readback_bytes) throw dhx::Error("readback exceeds reserved capacity");
        check_region(e, r);
        if (n > r.bytes) throw dhx::Error("output exceeds allocated region");
        set_device(e);
        hip_check(e, hipMemcpyAsync(e->readback, region_ptr(e, r), n, hipMemcpyDeviceToHost, e->stream), "readback copy");
        hip_check(e, hipStreamSynchronize(e->stream), "readback synchronize");
        std::memcpy(out, e->readback, n);
    });
}

int dhx_fragment_order(const uint16_t* rows_in, uint64_t rows, uint64_t k, uint16_t* frag_out) {
    try {
        if (k % 16 != 0 || (rows && (!rows_in || !frag_out))) throw dhx::Error("fragment order needs k % 16 == 0");
        const uint64_t padded = (rows + 31) / 32 * 32;
        std::memset(frag_out, 0, padded * k * 2);
        for (uint64_t m = 0; m < rows; ++m)
            for (uint64_t c = 0; c < k; c += 8) {
                const uint64_t o = ((m / 32) * (k / 16) + c / 16) * 512 + ((c / 8) % 2 * 32 + m % 32) * 8;
                std::memcpy(frag_out + o, rows_in + m * k + c, 16);
            }
        return 0;
    } catch (const std::exception& ex) {
        dhx::set_global_error(ex.what());
        return 1;
    }
}

int dhx_row_order(const uint16_t* frag_in, uint64_t rows, uint64_t k, uint16_t* rows_out) {
    try {
        if (k % 16 != 0 || (rows && (!frag_in || !rows_out))) throw dhx::Error("fragment order needs k % 16 == 0");
        for (uint64_t m = 0; m < rows; ++m)
            for (uint64_t c = 0; c < k; c += 8) {
                const uint64_t o = ((m / 32) * (k / 16) + c / 16) * 512 + ((c / 8) % 2 * 32 + m % 32) * 8;
                std::memcpy(rows_out + m * k + c, frag_in + o, 16);
            }
        return 0;
    } catch (const std::exception& ex) {
        dhx::set_global_error(ex.what());
        return 1;
    }
}

int dhx_reserve_staging(dhx_engine* e, uint64_t in_bytes, uint64_t out_bytes) {
    return guarded(e, [&] {
        ensure_usable(e);
        set_device(e);
        release_staging(e);
        hip_check(e, hipStreamCreateWithFlags(&e->up, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(e, hipStreamCreateWithFlags(&e->down, hipStreamNonBlocking), "hipStreamCreate");
        for (int i = 0; i < DHX_STAGING_SLOTS; ++i) {
            hip_check(e, hipHostMalloc(&e->pin_in[i], std::max<uint64_t>(in_bytes, 16), hipHostMallocDefault),
                      "hipHostMalloc");
            hip_check(e, hipHostMalloc(&e->pin_out[i], std::max<uint64_t>(out_bytes, 16), hipHostMallocDefault),
                      "hipHostMalloc");
            for (hipEvent_t* ev : {&e->in_done[i], &e->graph_done[i], &e->out_done[i]})
                hip_check(e, hipEventCreateWithFlags(ev, hipEventDisableTiming), "hipEventCreate");
            // Completed events, so the first use of each slot waits for nothing.
            hip_check(e, hipEventRecord(e->in_done[i], e->up), "hipEventRecord");
            hip_check(e, hipEventRecord(e->graph_done[i], e->stream), "hipEventRecord");
            hip_check(e, hipEventRecord(e->out_done[i], e->down), "hipEventRecord");
        }
        e->pin_in_bytes = in_bytes;
        e->pin_out_bytes = out_bytes;
    });
}

int dhx_copy_in(dhx_engine* e, dhx_region dst, const void* src, uint64_t n, uint32_t slot) {
    return guarded(e, [&] {
        if (n && !src) throw dhx::Error("null input");
        dhx::engine_wait_upload(e, slot);  // staging buffer free again
        dhx::parallel_copy(e->pin_in[slot], src, n);
        dhx::engine_upload(e, dst, n, slot);
    });
}

int dhx_replay_slot(dhx_engine* e, uint64_t batch, uint32_t slot) {
    return guarded(e, [&] {
        ensure_usable(e);
        check_slot(e, slot);
        auto it = e->graphs.find(batch);
        if (it == e->graphs.end()) throw dhx::Error("batch has not been prepared");
        set_device(e);
        hip_check(e, hipStreamWaitEvent(e->stream, e->in_done[slot], 0), "hipStreamWaitEvent");
        hip_check(e, hipStreamWaitEvent(e->stream, e->out_done[slot], 0), "hipStreamWaitEvent");
        hip_check(e, hipGraphLaunch(it->second.exec, e->stream), "graph launch");
        hip_check(e, hipEventRecord(e->graph_done[slot], e->stream), "hipEventRecord");
    });
}

int dhx_copy_out(dhx_engine* e, dhx_region src, uint64_t n, uint32_t slot) {
    return guarded(e, [&] {
        ensure_usable(e);
        check_slot(e, slot);
        check_region(e, src);
        if (n > src.bytes) throw dhx::Error("output exceeds allocated region");
        if (n > e->pin_out_bytes) throw dhx::Error("output exceeds reserved staging");
        set_device(e);
        hip_check(e, hipStreamWaitEvent(e->down, e->graph_done[slot], 0), "hipStreamWaitEvent");
        hip_check(e, hipMemcpyAsync(e->pin_out[slot], region_ptr(e, src), n, hipMemcpyDeviceToHost, e->down),
                  "readback copy");
        hip_check(e, hipEventRecord(e->out_done[slot], e->down), "hipEventRecord");
    });
}

int dhx_copy_out_finish(dhx_engine* e, void* dst, uint64_t n, uint32_t slot) {
    return guarded(e, [&] {
        if (n > e->pin_out_bytes) throw dhx::Error("output exceeds reserved staging");
        if (n && !dst) throw dhx::Error("null output");
        dhx::engine_wait_readback(e, slot);
        dhx::parallel_copy(dst, e->pin_out[slot], n);
    });
}

int dhx_benchmark(dhx_engine* e, uint64_t batch, uint64_t samples, dhx_timings* out) {
    return guarded(e, [&] {
        if (samples < 10) throw dhx::Error("use at least ten timing samples");
        ensure_usable(e);
        auto it = e->graphs.find(batch);
        if (it == e->graphs.end()) throw dhx::Error("batch has not been prepared");
        set_device(e);
        std::vector<double> times[2];
        for (uint64_t i = 0; i < samples + 10; ++i) {
            const int order[2] = {(int)(i % 2), (int)(1 - i % 2)};
            for (int mode : order) {
                const auto start = std::chrono::steady_clock::now();
                if (mode == 0) hip_check(e, hipGraphLaunch(it->second.exec, e->stream), "graph launch");
                else hip_check(e, queue_branches(e, it->second), "kernel launch");
                hip_check(e, hipStreamSynchronize(e->stream), "synchronize");
                const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
                if (i >= 10) times[mode].push_back(ms);
            }
        }
        for (auto& t : times) std::sort(t.begin(), t.end());
        out->samples = samples;
        out->graph = dhx_distribution{percentile_sorted(times[0], 50), percentile_sorted(times[0], 95)};
        out->direct = dhx_distribution{percentile_sorted(times[1], 50), percentile_sorted(times[1], 95)};
    });
}

int dhx_launch_timings(dhx_engine* e, uint64_t batch, uint32_t iters, double* ms_out, uint32_t* kernel_out,
                       uint64_t capacity, uint64_t* count) {
    return guarded(e, [&] {
        ensure_usable(e);
        auto it = e->graphs.find(batch);
        if (it == e->graphs.end()) throw dhx::Error("batch has not been prepared");
        const auto& list = it->second.launches;
        if (count) *count = list.size();
        if (capacity < list.size()) throw dhx::Error("timing output too small");
        if (iters == 0) throw dhx::Error("iters must be positive");
        set_device(e);
        hipEvent_t a, b;
        hip_check(e, hipEventCreate(&a), "hipEventCreate");
        hip_check(e, hipEventCreate(&b), "hipEventCreate");
        for (size_t i = 0; i < list.size(); ++i) {
            hip_check(e, launch_one(e, list[i], e->stream), "kernel launch");  // warm
            hip_check(e, hipEventRecord(a, e->stream), "hipEventRecord");
            for (uint32_t k = 0; k < iters; ++k) hip_check(e, launch_one(e, list[i], e->stream), "kernel launch");
            hip_check(e, hipEventRecord(b, e->stream), "hipEventRecord");
            hip_check(e, hipEventSynchronize(b), "hipEventSynchronize");
            float ms = 0.f;
            hip_check(e, hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
            ms_out[i] = ms / iters;
            if (kernel_out) kernel_out[i] = list[i].kernel;
        }
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    });
}

int dhx_test_fail_next_call(dhx_engine* e) {
    return guarded(e, [&] { e->fail_next = true; });
}

}  // extern "C"
