// The C++ mirror of the crate's public API (src/lib.rs): DINOv3 with
// load / from_pretrained / forward / cls / patch_mean / benchmark, batch
// chunking, the buffer plan and the per-batch launch plan (`prepare`),
// built on the engine C ABI exactly as lib.rs builds on HRX.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <sys/stat.h>
#include <thread>
#include <vector>

#include "../../include/dinov3.h"
#include "engine_internal.hpp"
#include "errors.hpp"
#include "host_copy.hpp"
#include "kernels/launch.hpp"
#include "weights.hpp"

namespace dhx {

namespace {
thread_local std::string g_error;
}
void set_global_error(const std::string& message) { g_error = message; }
const char* global_error() { return g_error.c_str(); }

namespace {

constexpr uint64_t kHiddenU = 384;
constexpr uint32_t kSplits = 4;
// Smallest image group worth its own branch of the plan.
constexpr uint64_t kMinBranchImages = 4;

// hub.rs:7-11
constexpr char kRepoOwner[] = "facebook";
constexpr char kRepoName[] = "dinov3-vits16plus-pretrain-lvd1689m";
constexpr char kRevision[] = "c93d816fc9e567563bc068f01475bec89cc634a6";
constexpr char kFile[] = "model.safetensors";

void check_max_batch(uint64_t b) {
    if (b < 1 || b > 64) throw Error("max_batch must be 1..=64");
}

uint32_t image_size_of(const dinov3_options& o) {
    const uint32_t s = o.image_size == 0 ? 224 : o.image_size;
    if (s % 16 != 0 || s < 16 || s > 1024) throw Error("image_size must be a multiple of 16 in 16..=1024");
    return s;
}

bool exists(const std::string& p) {
    struct stat st;
    return ::stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

// hub.rs:17-54 with downloads unavailable: the pinned snapshot in the
// Hugging Face cache (HF_HUB_CACHE, else HF_HOME/hub, else
// ~/.cache/huggingface/hub), laid out as the hub client writes it.
std::string hub_weights() {
    std::string cache;
    if (const char* c = std::getenv("HF_HUB_CACHE"); c && *c) cache = c;
    else if (const char* h = std::getenv("HF_HOME"); h && *h) cache = std::string(h) + "/hub";
    else if (const char* home = std::getenv("HOME"); home && *home) cache = std::string(home) + "/.cache/huggingface/hub";
    else throw Error("cannot read the Hugging Face cache: no HF_HUB_CACHE, HF_HOME or HOME");
    const std::string path = cache + "/models--" + kRepoOwner + "--" + kRepoName + "/snapshots/" + kRevision + "/" + kFile;
    if (!exists(path))
        throw Error(std::string(kRepoOwner) + "/" + kRepoName + " at " + kRevision + ": " + kFile +
                    " is not cached and model downloads are disabled");
    return path;
}

void check(int rc, dhx_engine* e) {
    if (rc != 0) throw Error(dhx_last_error(e));
}

// The allocation-free forward's intermediate buffers: one array per GPU,
// loaded with the library's code object and held until the process ends.
// Host code never uses the name as an address (on the host it is only a
// handle for the symbol lookup): scratch_address() asks the runtime for
// each device's copy once, with that device current.
constexpr uint64_t kScratchBytes = DINOV3_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// Restores the calling thread's current device when it goes out of scope.
class DeviceGuard {
public:
    DeviceGuard() {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    }
    ~DeviceGuard() {
        if (prev_ >= 0) (void)hipSetDevice(prev_);
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int prev_ = -1;
};

// Per device: the array's address on that device, and an event recorded
// after the launches of the last allocation-free call queued there. Each
// call's stream waits for that event before its first launch, so calls on
// one GPU run one after another whatever their streams, threads or models.
// Both are created once (the first model load on the device) and kept
// until the process ends, like the array.
struct ScratchSlot {
    void* ptr = nullptr;
    hipEvent_t last = nullptr;
};
std::mutex g_scratch_mutex;  // guards g_scratch and orders the queueing of calls
ScratchSlot g_scratch[kMaxDevices];

// Callers hold g_scratch_mutex. Leaves the caller's current device as it was.
ScratchSlot& scratch_slot_locked(int device) {
    if (device < 0 || device >= kMaxDevices) throw Error("device id out of range for the scratch table");
    ScratchSlot& s = g_scratch[device];
    if (!s.ptr) {
        DeviceGuard keep;
        hipError_t err = hipSetDevice(device);
        void* p = nullptr;
        if (err == hipSuccess) err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p)
            throw Error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
        hipEvent_t ev = nullptr;
        err = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (err != hipSuccess) throw Error(std::string("hipEventCreateWithFlags: ") + hipGetErrorString(err));
        s.ptr = p;
        s.last = ev;
    }
    return s;
}

void* scratch_address(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    return scratch_slot_locked(device).ptr;
}

constexpr uint64_t align256(uint64_t v) { return (v + 255) & ~255ull; }

// Finite check of the whole input before any GPU work (lib.rs validates
// every pixel first), split over host threads for large batches.
bool all_finite(const float* p, uint64_t n) {
    auto scan = [p](uint64_t a, uint64_t b) {
        bool ok = true;
        for (uint64_t i = a; i < b; ++i) ok &= std::isfinite(p[i]);
        return ok;
    };
    constexpr uint64_t kChunk = 1ull << 20;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned threads = (unsigned)std::min<uint64_t>(std::min(16u, hw), (n + kChunk - 1) / kChunk);
    if (threads <= 1) return scan(0, n);
    std::vector<std::thread> pool;
    std::vector<char> ok(threads, 1);
    const uint64_t per = (n + threads - 1) / threads;
    for (unsigned t = 0; t < threads; ++t)
        pool.emplace_back([&, t] { ok[t] = scan(t * per, std::min(n, (t + 1) * per)); });
    for (auto& th : pool) th.join();
    for (char v : ok)
        if (!v) return false;
    return true;
}

}  // namespace

class Model {
public:
    Model(const std::string& path, const dinov3_options& opts) : opts_(opts) {
        check_max_batch(opts.max_batch);
        size_ = image_size_of(opts);
        grid_ = size_ / 16;
        patches_ = (uint64_t)grid_ * grid_;
        tokens_ = patches_ + 5;
        tpad_ = (tokens_ + 127) / 128 * 128;
        image_elems_ = 3ull * size_ * size_;
        // Validation and packing finish before the device is opened.
        Packed packed = load_weights(path, grid_);
        dhx_engine* e = nullptr;
        if (dhx_engine_open(opts.device, &e) != 0) throw Error(dhx_last_error(nullptr));
        engine_.reset(e);
        for (auto& kv : packed) {
            dhx_region r;
            check(dhx_weight(e, kv.second.data(), kv.second.size(), &r), e);
            weights_[kv.first] = r;
        }
        const uint64_t B = opts.max_batch, r = B * tokens_;
        const uint64_t heads = B * 6 * tpad_ * 64 * 2;
        // Activations in fragment order: each image group starts on a 32-row
        // block, so up to 32 padding rows per group.
        const uint64_t rf = r + 32ull * DHX_MAX_BRANCHES;
        // x, h, attn and act are f16 in fragment order, and so is each
        // (image, head) [tpad][64] matrix of q/k/v (padded rows stay zero); out, the NCHW images, the split-K slabs and the
        // LayerNorm row statistics of x are f32. The images and out exist
        // twice (one per transfer slot) so that consecutive chunks of a
        // forward overlap their uploads and readbacks with each other's graph.
        const uint64_t sizes[kBuffers] = {rf * kHiddenU * 2, rf * kHiddenU * 2, heads, heads, heads, rf * kHiddenU * 2,
                                          rf * 1536 * 2,     r * kHiddenU * 4, B * image_elems_ * 4,
                                          (uint64_t)kSplits * r * kHiddenU * 4, r * 12 * 4,
                                          r * kHiddenU * 4, B * image_elems_ * 4};
        for (int i = 0; i < kBuffers; ++i) check(dhx_allocate(e, sizes[i], &a_[i]), e);
        check(dhx_reserve_staging(e, B * image_elems_ * 4, r * kHiddenU * 4), e);
        // The allocation-free forward: this device's scratch array and three
        // external buffer slots (scratch, caller input, caller output). A
        // failed lookup only disables that entry point (it reports why).
        try {
            ext_scratch_ = dhx::engine_external(e, scratch_address(opts.device), kScratchBytes);
            ext_in_ = dhx::engine_external(e, nullptr, 0);
            ext_out_ = dhx::engine_external(e, nullptr, 0);
            noalloc_launches_.reserve(128);
        } catch (const Error& ex) {
            noalloc_error_ = ex.what();
        }
    }

    dhx_engine* engine() { return engine_.get(); }
    uint64_t image_elements() const { return image_elems_; }
    uint64_t tokens() const { return tokens_; }

    void set_splitk(int mode) {
        if (mode != 0 && mode != 1) throw Error("split-K mode must be 0 or 1");
        splitk_ = mode;  // graphs are keyed by (batch, variant); see key()
    }

    void set_layernorm_fusion(int on) {
        if (on != 0 && on != 1) throw Error("layernorm fusion must be 0 or 1");
        fused_ln_ = on;
    }

    void set_branches(uint32_t n) {
        if (n < 1 || n > DHX_MAX_BRANCHES) throw Error("branches must be 1.." + std::to_string(DHX_MAX_BRANCHES));
        branches_ = n;
    }

    // lib.rs:90-114: chunks of max_batch images, pipelined over the two
    // transfer slots: chunk i uses slot i % 2. This thread issues every HIP
    // call (uploads, graph launches, readbacks); with more than one chunk a
    // Copier thread does the host copies into and out of the pinned staging
    // buffers, each handed over as soon as its buffer is free: chunk i+1's
    // input copy and chunk i-1's output copy run while chunk i is launched
    // and computed. Results are those of the chunks run one at a time.
    void forward(const float* pixels, uint64_t n, float* out, uint64_t out_floats) {
        check_input(pixels, n);
        const uint64_t batch = n / image_elems_;
        const uint64_t per_image = tokens_ * kHiddenU;
        if (out_floats < batch * per_image) throw Error("output buffer holds fewer than images*tokens*384 floats");
        if (batch == 0) return;
        dhx_engine* e = engine_.get();
        const uint64_t chunks = (batch + opts_.max_batch - 1) / opts_.max_batch;
        auto size_of = [&](uint64_t i) { return std::min<uint64_t>(opts_.max_batch, batch - i * opts_.max_batch); };
        for (uint64_t i = 0; i < std::min<uint64_t>(chunks, 2); ++i) prepare(size_of(i), (uint32_t)(i & 1));
        if (chunks > 2) prepare(size_of(chunks - 1), (uint32_t)((chunks - 1) & 1));  // the tail chunk
        auto in_bytes = [&](uint64_t i) { return size_of(i) * image_elems_ * 4; };
        auto out_bytes = [&](uint64_t i) { return size_of(i) * per_image * 4; };
        if (in_bytes(0) > dhx::engine_staging_in_bytes(e) || out_bytes(0) > dhx::engine_staging_out_bytes(e))
            throw Error("chunk exceeds reserved staging");
        std::vector<uint64_t> filled(chunks), drained(chunks);
        Copier copier(chunks > 1);
        // Chunk i's pixels into slot i % 2's input staging, once the slot's
        // previous upload has left it.
        auto fill = [&](uint64_t i) {
            const uint32_t slot = (uint32_t)(i & 1);
            dhx::engine_wait_upload(e, slot);
            filled[i] = copier.submit(dhx::engine_staging_in(e, slot), pixels + i * opts_.max_batch * image_elems_,
                                      in_bytes(i));
        };
        // Chunk i's tokens out of slot i % 2's output staging, once its
        // readback has landed there.
        auto drain = [&](uint64_t i) {
            const uint32_t slot = (uint32_t)(i & 1);
            dhx::engine_wait_readback(e, slot);
            drained[i] = copier.submit(out + i * opts_.max_batch * per_image, dhx::engine_staging_out(e, slot),
                                       out_bytes(i));
        };
        fill(0);
        if (chunks > 1) fill(1);
        for (uint64_t i = 0; i < chunks; ++i) {
            const uint32_t slot = (uint32_t)(i & 1);
            copier.wait(filled[i]);
            dhx::engine_upload(e, a_[image_buffer(slot)], in_bytes(i), slot);
            if (i >= 2) copier.wait(drained[i - 2]);  // the slot's output staging is read out
            check(dhx_replay_slot(e, key(size_of(i), slot), slot), e);
            check(dhx_copy_out(e, a_[out_buffer(slot)], out_bytes(i), slot), e);
            if (i >= 1 && i + 1 < chunks) fill(i + 1);  // its slot last held chunk i-1, uploaded by now
            if (i >= 1) drain(i - 1);
        }
        drain(chunks - 1);
        copier.wait(drained[chunks - 1]);
    }

    // Upload one chunk and replay its graph (recording it on first use).
    void stage(const float* pixels, uint64_t b) {
        prepare(b);
        check(dhx_upload(engine_.get(), region(kImage), pixels, b * image_elems_ * 4), engine_.get());
        replay(b);
    }

    void replay(uint64_t b) { check(dhx_replay(engine_.get(), key(b)), engine_.get()); }

    void check_input(const float* pixels, uint64_t n) const {
        if (n % image_elems_ != 0)
            throw Error("input must contain complete 3×" + std::to_string(size_) + "×" + std::to_string(size_) + " images");
        if (!all_finite(pixels, n)) throw Error("input must be finite");
    }

    // lib.rs:116-124
    void benchmark(const float* pixels, uint64_t n, uint64_t samples, dinov3_timings* out) {
        if (n == 0 || n > opts_.max_batch * image_elems_) throw Error("benchmark requires one nonempty batch");
        check_input(pixels, n);
        std::vector<float> tmp(n / image_elems_ * tokens_ * kHiddenU);
        forward(pixels, n, tmp.data(), tmp.size());
        check(dhx_benchmark(engine_.get(), key(n / image_elems_), samples, out), engine_.get());
    }

    // lib.rs:149-263 (prepare): one launch plan per batch size, recorded as
    // one graph. The batch is cut into `branches_` groups of images (for
    // b >= 2 * kMinBranchImages) that run as independent chains, each over
    // its own slice of every buffer: the kernels of one group fill the last,
    // partial wave of workgroups of the other's. A row's arithmetic does not
    // depend on the group it is in, so results are bitwise the same. The down
    // projection is the residual GEMM, or split-K slabs + reduce when selected
    // (the reference takes split-K at batch 1, lib.rs:218-225; here the
    // residual GEMM is faster at batch 1 too, one launch instead of two per
    // block, and keeps every image's result independent of the batch size).
    // By default LayerNorm is folded
    // into the QKV and gate/up GEMMs, fed by row statistics that the
    // producers of x write (62 launches per group at b > 1); the unfused plan
    // runs LayerNorm kernels as the reference does (86).
    void prepare(uint64_t b, uint32_t slot = 0) {
        if (dhx_has_graph(engine_.get(), key(b, slot))) return;
        const uint32_t nb = groups(b);
        std::vector<dhx_launch> l;
        std::vector<uint64_t> counts;
        uint64_t frag_row0 = 0;  // first 32-row block of the group in the fragment-order buffers
        for (uint32_t g = 0; g < nb; ++g) {
            const uint64_t first = b * g / nb, end = b * (g + 1) / nb;
            const size_t before = l.size();
            plan(first, end - first, b, slot, frag_row0, l, a_);
            counts.push_back(l.size() - before);
            frag_row0 += ((end - first) * tokens_ + 31) / 32 * 32;
        }
        check(dhx_record_branches(engine_.get(), key(b, slot), l.data(), counts.data(), nb), engine_.get());
    }

    // The launches for images [first, first + n) of a batch of b.
    void plan(uint64_t first, uint64_t n, uint64_t b, uint32_t slot, uint64_t frag_row0, std::vector<dhx_launch>& l,
              const dhx_region* bufs) const {
        const uint32_t r = (uint32_t)(n * tokens_);
        const uint32_t B = (uint32_t)n, G = grid_, TP = (uint32_t)tpad_;
        auto add = [&](uint32_t kernel, std::initializer_list<uint32_t> s, std::initializer_list<dhx_region> bind) {
            dhx_launch x{};
            x.kernel = kernel;
            int i = 0;
            for (uint32_t v : s) x.scalars[i++] = v;
            x.n_bindings = 0;
            for (const dhx_region& g : bind) x.bindings[x.n_bindings++] = g;
            l.push_back(x);
        };
        auto w = [&](const std::string& name) { return weights_.at(name); };
        // This group's slice of a buffer holding `per_image` bytes per image.
        auto part = [&](int buf, uint64_t per_image) {
            dhx_region g = bufs[buf];
            g.offset += first * per_image;
            g.bytes = n * per_image;
            return g;
        };
        // This group's rows of a fragment-order activation buffer of width k.
        auto frag_part = [&](int buf, uint64_t k) {
            dhx_region g = bufs[buf];
            g.offset += frag_row0 * k * 2;
            g.bytes = (n * tokens_ + 31) / 32 * 32 * k * 2;
            return g;
        };
        const uint64_t row = tokens_ * kHiddenU;
        const uint64_t heads = 6 * tpad_ * 64 * 2;
        const dhx_region X = frag_part(kX, kHiddenU), H = frag_part(kH, kHiddenU), S = part(kStats, tokens_ * 12 * 4);
        const dhx_region Q = part(kQ, heads), K = part(kK, heads), V = part(kV, heads);
        const dhx_region A = frag_part(kAttn, kHiddenU), F = frag_part(kAct, 1536);
        const dhx_region O = part(out_buffer(slot), row * 4), I = part(image_buffer(slot), image_elems_ * 4);
        const dhx_region SL = part(kPartials, (uint64_t)kSplits * row * 4);  // [splits][rows][384] per group
        const bool split = splitk_ == 1;
        if (fused_ln_) {
            add(DHX_K_PATCH_EMBED_STATS, {B, G}, {I, w("patch_w"), w("patch_b"), w("prefix"), w("prefix_stats"), X, S});
        } else {
            add(DHX_K_PATCH_EMBED, {B, G}, {I, w("patch_w"), w("patch_b"), w("prefix"), X});
            add(DHX_K_LAYERNORM, {r}, {X, w("l0_norm1_w"), w("l0_norm1_b"), H});
        }
        for (int i = 0; i < 12; ++i) {
            const std::string p = "l" + std::to_string(i) + "_";
            const bool last = i == 11;
            if (fused_ln_)
                add(DHX_K_QKV_ROPE_LN, {B, G, TP},
                    {X, S, w(p + "qkv_wln"), w(p + "qkv_wsum"), w(p + "qkv_t"), w("rope_cos"), w("rope_sin"), Q, K, V});
            else
                add(DHX_K_QKV_ROPE, {B, G, TP},
                    {H, w(p + "qkv_w"), w(p + "qkv_b"), w("rope_cos"), w("rope_sin"), Q, K, V});
            add(DHX_K_ATTENTION, {B, G, TP}, {Q, K, V, A});
            if (fused_ln_) {
                add(DHX_K_RESID_STATS, {r, 384}, {A, w(p + "o_w"), w(p + "o_b"), w(p + "ls1"), X, S});
                add(DHX_K_SWIGLU_LN, {r}, {X, S, w(p + "gateup_wln"), w(p + "gateup_wsum"), w(p + "gateup_t"), F});
            } else {
                add(DHX_K_RESID, {r, 384}, {A, w(p + "o_w"), w(p + "o_b"), w(p + "ls1"), X});
                add(DHX_K_LAYERNORM, {r}, {X, w(p + "norm2_w"), w(p + "norm2_b"), H});
                add(DHX_K_SWIGLU, {r}, {H, w(p + "gateup_w"), w(p + "gateup_b"), F});
            }
            // The last block's statistics would have no reader (the final
            // LayerNorm computes its own).
            const bool stats = fused_ln_ && !last;
            if (split) {
                add(DHX_K_SPLITK, {r, 1536, kSplits}, {F, w(p + "down_w"), SL});
                if (stats)
                    add(DHX_K_SPLITK_REDUCE_STATS, {r, kSplits}, {SL, w(p + "down_b"), w(p + "ls2"), X, S});
                else
                    add(DHX_K_SPLITK_REDUCE, {r, kSplits}, {SL, w(p + "down_b"), w(p + "ls2"), X});
            } else if (stats) {
                add(DHX_K_RESID_STATS, {r, 1536}, {F, w(p + "down_w"), w(p + "down_b"), w(p + "ls2"), X, S});
            } else {
                add(DHX_K_RESID, {r, 1536}, {F, w(p + "down_w"), w(p + "down_b"), w(p + "ls2"), X});
            }
            if (!fused_ln_ && !last) {
                const std::string nx = "l" + std::to_string(i + 1) + "_";
                add(DHX_K_LAYERNORM, {r}, {X, w(nx + "norm1_w"), w(nx + "norm1_b"), H});
            }
        }
        add(DHX_K_LAYERNORM_F32, {r}, {X, w("norm_w"), w("norm_b"), O});
    }

    // dinov3_forward_noalloc: the plan of one image group over the scratch
    // array (laid out for this batch, 256-byte aligned pieces) and the
    // caller's device input and output, queued on `stream` after a fill of
    // the q/k/v padding rows. The same launches and arithmetic per row as
    // forward(), so the same bits. Allocates nothing and does not wait.
    void forward_noalloc(const float* pixels, uint64_t images, float* out, hipStream_t stream) {
        dhx_engine* e = engine_.get();
        dhx::engine_ensure_usable(e);
        if (!noalloc_error_.empty()) throw Error("the allocation-free forward is unavailable: " + noalloc_error_);
        if (images == 0) return;
        if (!pixels || !out) throw Error("null device pointer");
        if ((reinterpret_cast<uintptr_t>(pixels) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
            throw Error("device input and output must be 16-byte aligned");
        if (images > 64) throw Error("the allocation-free forward takes at most 64 images per call");
        const uint64_t r = images * tokens_, rf = (r + 31) / 32 * 32;
        const uint64_t heads = images * 6 * tpad_ * 64 * 2;
        const bool split = splitk_ == 1;
        uint64_t need[kBuffers] = {};
        need[kX] = rf * kHiddenU * 2;
        need[kH] = fused_ln_ ? 0 : rf * kHiddenU * 2;
        need[kQ] = need[kK] = need[kV] = heads;
        need[kAttn] = rf * kHiddenU * 2;
        need[kAct] = rf * 1536 * 2;
        need[kStats] = fused_ln_ ? r * 12 * 4 : 0;
        need[kPartials] = split ? (uint64_t)kSplits * r * kHiddenU * 4 : 0;
        dhx_region bufs[kBuffers] = {};
        uint64_t at = 0;
        for (int i = 0; i < kBuffers; ++i) {
            if (i == kOut || i == kOut1 || i == kImage || i == kImage1) continue;
            bufs[i] = dhx_region{ext_scratch_, at, need[i]};
            at += align256(need[i]);
        }
        if (at > kScratchBytes)
            throw Error("the allocation-free forward of " + std::to_string(images) + " images needs " +
                        std::to_string(at) + " bytes of scratch, more than its " + std::to_string(kScratchBytes));
        // One call at a time binds, plans and queues its launches on this
        // GPU (the lock also keeps two threads of one model from rebinding
        // each other's input and output), and each call's stream waits for
        // the previous call's launches (its event), so overlapping calls
        // from other streams, threads or models run in turn instead of
        // racing on the array. Under stream capture the wait and the record
        // are left out (the graph's launches are ordered by whoever launches
        // the graph), and nothing else changes.
        DeviceGuard keep;
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        ScratchSlot& slot = scratch_slot_locked(dhx::engine_device(e));
        const uint64_t in_bytes = images * image_elems_ * 4, out_bytes = r * kHiddenU * 4;
        dhx::engine_rebind(e, ext_in_, const_cast<float*>(pixels), in_bytes);
        dhx::engine_rebind(e, ext_out_, out, out_bytes);
        bufs[kImage] = bufs[kImage1] = dhx_region{ext_in_, 0, in_bytes};
        bufs[kOut] = bufs[kOut1] = dhx_region{ext_out_, 0, out_bytes};
        noalloc_launches_.clear();  // capacity reserved at load: no reallocation
        plan(0, images, images, 0, 0, noalloc_launches_, bufs);
        char* const base = static_cast<char*>(slot.ptr);
        const dhx::PadRowsArgs pad{reinterpret_cast<dhx::half_t*>(base + bufs[kQ].offset),
                                   reinterpret_cast<dhx::half_t*>(base + bufs[kK].offset),
                                   reinterpret_cast<dhx::half_t*>(base + bufs[kV].offset), (int)images, (int)tokens_,
                                   (int)tpad_};
        if (!stream) stream = dhx::engine_stream(e);
        dhx::engine_check(e, hipSetDevice(dhx::engine_device(e)), "hipSetDevice");
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        dhx::engine_check(e, hipStreamIsCapturing(stream, &capture), "hipStreamIsCapturing");
        const bool ordered = capture == hipStreamCaptureStatusNone;
        if (ordered) dhx::engine_check(e, hipStreamWaitEvent(stream, slot.last, 0), "hipStreamWaitEvent");
        dhx::engine_check(e, dhx::launch_zero_pad_rows(pad, stream), "kernel launch");
        dhx::engine_queue(e, noalloc_launches_.data(), noalloc_launches_.size(), stream);
        if (ordered) dhx::engine_check(e, hipEventRecord(slot.last, stream), "hipEventRecord");
    }

    // Number of image groups run side by side for a batch of b.
    uint32_t groups(uint64_t b) const {
        return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(branches_, b / kMinBranchImages));
    }

    // Graph key: batch size plus one bit per plan variant.
    uint64_t key(uint64_t b, uint32_t slot = 0) const {
        return b | (splitk_ ? (1ull << 32) : 0) | (fused_ln_ ? 0 : (1ull << 33)) |
               ((uint64_t)(groups(b) - 1) << 34) | ((uint64_t)slot << 36);
    }

private:
    enum { kX, kH, kQ, kK, kV, kAttn, kAct, kOut, kImage, kPartials, kStats, kOut1, kImage1, kBuffers };
    static int image_buffer(uint32_t slot) { return slot ? kImage1 : kImage; }
    static int out_buffer(uint32_t slot) { return slot ? kOut1 : kOut; }
    struct EngineFree {
        void operator()(dhx_engine* e) const { dhx_engine_free(e); }
    };
    dhx_region region(int i) const { return a_[i]; }

    dinov3_options opts_;
    uint32_t size_ = 224, grid_ = 14;
    uint64_t patches_ = 196, tokens_ = 201, tpad_ = 256, image_elems_ = 0;
    int splitk_ = 0;
    int fused_ln_ = 1;
    uint32_t branches_ = 2;
    std::unique_ptr<dhx_engine, EngineFree> engine_;
    std::map<std::string, dhx_region> weights_;
    dhx_region a_[kBuffers];
    uint32_t ext_scratch_ = 0, ext_in_ = 0, ext_out_ = 0;
    std::vector<dhx_launch> noalloc_launches_;
    std::string noalloc_error_;
};

}  // namespace dhx

struct dinov3_model {
    std::unique_ptr<dhx::Model> model;
    std::string error;
};

namespace {

template <class F>
int guarded(dinov3_model* m, F&& f) {
    try {
        if (!m || !m->model) throw dhx::Error("null model");
        f(*m->model);
        return 0;
    } catch (const std::exception& ex) {
        if (m) m->error = ex.what();
        else dhx::set_global_error(ex.what());
        return 1;
    }
}

template <class F>
int guarded_global(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& ex) {
        dhx::set_global_error(ex.what());
        return 1;
    }
}

}  // namespace

extern "C" {

void dinov3_options_default(dinov3_options* out) {
    if (out) *out = dinov3_options{0, 32, 224};
}

int dinov3_load(const char* path, const dinov3_options* options, dinov3_model** out) {
    return guarded_global([&] {
        if (!options || !out) throw dhx::Error("null argument");
        *out = nullptr;
        dhx::check_max_batch(options->max_batch);  // before any file I/O
        auto m = std::make_unique<dinov3_model>();
        m->model = std::make_unique<dhx::Model>(path ? path : "", *options);
        *out = m.release();
    });
}

int dinov3_from_pretrained(const dinov3_options* options, dinov3_model** out) {
    return guarded_global([&] {
        if (!options || !out) throw dhx::Error("null argument");
        *out = nullptr;
        dhx::check_max_batch(options->max_batch);
        const std::string path = dhx::hub_weights();
        auto m = std::make_unique<dinov3_model>();
        m->model = std::make_unique<dhx::Model>(path, *options);
        *out = m.release();
    });
}

int dinov3_hub_weights(char* path_out, uint64_t capacity) {
    return guarded_global([&] {
        const std::string p = dhx::hub_weights();
        if (!path_out || capacity < p.size() + 1) throw dhx::Error("path buffer too small");
        std::memcpy(path_out, p.c_str(), p.size() + 1);
    });
}

int dinov3_forward(dinov3_model* m, const float* pixels, uint64_t n, float* out, uint64_t out_floats) {
    return guarded(m, [&](dhx::Model& x) { x.forward(pixels, n, out, out_floats); });
}

int dinov3_forward_noalloc(dinov3_model* m, const float* pixels, uint64_t images, float* out, void* stream) {
    return guarded(m, [&](dhx::Model& x) { x.forward_noalloc(pixels, images, out, static_cast<hipStream_t>(stream)); });
}

int dinov3_cls(dinov3_model* m, const float* pixels, uint64_t n, float* out, uint64_t out_floats) {
    return guarded(m, [&](dhx::Model& x) {
        x.check_input(pixels, n);
        const uint64_t images = n / x.image_elements(), per = x.tokens() * 384;
        if (out_floats < images * 384) throw dhx::Error("output buffer holds fewer than images*384 floats");
        std::vector<float> all(images * per);
        x.forward(pixels, n, all.data(), all.size());
        for (uint64_t i = 0; i < images; ++i) std::memcpy(out + i * 384, all.data() + i * per, 384 * sizeof(float));
    });
}

int dinov3_patch_mean(dinov3_model* m, const float* pixels, uint64_t n, float* out, uint64_t out_floats) {
    return guarded(m, [&](dhx::Model& x) {
        x.check_input(pixels, n);
        const uint64_t images = n / x.image_elements(), T = x.tokens(), per = T * 384;
        if (out_floats < images * 384) throw dhx::Error("output buffer holds fewer than images*384 floats");
        std::vector<float> all(images * per);
        x.forward(pixels, n, all.data(), all.size());
        const float patches = (float)(T - 5);
        for (uint64_t i = 0; i < images; ++i) {
            float* o = out + i * 384;
            for (int c = 0; c < 384; ++c) o[c] = 0.f;
            // lib.rs:139-144: float32 `+= v / 196` in token order.
            for (uint64_t t = 5; t < T; ++t) {
                const float* row = all.data() + i * per + t * 384;
                for (int c = 0; c < 384; ++c) o[c] += row[c] / patches;
            }
        }
    });
}

int dinov3_benchmark(dinov3_model* m, const float* pixels, uint64_t n, uint64_t samples, dinov3_timings* out) {
    return guarded(m, [&](dhx::Model& x) {
        if (!out) throw dhx::Error("null timings");
        x.benchmark(pixels, n, samples, out);
    });
}

const char* dinov3_last_error(const dinov3_model* m) { return m ? m->error.c_str() : dhx::global_error(); }

void dinov3_free(dinov3_model* m) { delete m; }

uint64_t dinov3_image_elements(const dinov3_model* m) { return m && m->model ? m->model->image_elements() : 0; }

uint64_t dinov3_tokens(const dinov3_model* m) { return m && m->model ? m->model->tokens() : 0; }

dhx_engine* dinov3_engine(dinov3_model* m) { return m && m->model ? m->model->engine() : nullptr; }

int dinov3_stage(dinov3_model* m, const float* pixels, uint64_t n) {
    return guarded(m, [&](dhx::Model& x) {
        x.check_input(pixels, n);
        const uint64_t b = n / x.image_elements();
        if (b == 0) throw dhx::Error("stage requires one nonempty batch");
        x.stage(pixels, b);
    });
}

int dinov3_replay(dinov3_model* m, uint64_t images) {
    return guarded(m, [&](dhx::Model& x) { x.replay(images); });
}

int dinov3_set_splitk(dinov3_model* m, int mode) {
    return guarded(m, [&](dhx::Model& x) { x.set_splitk(mode); });
}

int dinov3_set_layernorm_fusion(dinov3_model* m, int on) {
    return guarded(m, [&](dhx::Model& x) { x.set_layernorm_fusion(on); });
}

int dinov3_set_branches(dinov3_model* m, uint32_t n) {
    return guarded(m, [&](dhx::Model& x) { x.set_branches(n); });
}

int dinov3_launch_timings(dinov3_model* m, uint64_t images, uint32_t iters, double* ms_out, uint32_t* kernel_out,
                          uint64_t capacity, uint64_t* count) {
    return guarded(m, [&](dhx::Model& x) {
        if (dhx_launch_timings(x.engine(), x.key(images), iters, ms_out, kernel_out, capacity, count) != 0)
            throw dhx::Error(dhx_last_error(x.engine()));
    });
}

int dinov3_write_random_weights(const char* path, uint64_t seed, int preset) {
    return guarded_global([&] {
        if (!path) throw dhx::Error("null path");
        dhx::write_random_weights(path, seed, preset);
    });
}

int dinov3_random_pixels(uint64_t seed, uint64_t images, uint32_t image_size, float* out) {
    return guarded_global([&] {
        if (image_size == 0 || !out) throw dhx::Error("bad arguments");
        dhx::random_pixels(seed, images, image_size, out);
    });
}

int dinov3_patchify(const float* pixels, uint64_t images, uint32_t image_size, float* out) {
    return guarded_global([&] {
        if (image_size % 16 != 0 || image_size == 0) throw dhx::Error("image_size must be a multiple of 16");
        dhx::patchify(pixels, images, image_size, out);
    });
}

int dinov3_pack_f16(const char* name, const float* values, uint64_t n, uint16_t* out) {
    return guarded_global([&] {
        const std::vector<uint8_t> b = dhx::pack_f16(name ? name : "", values, n);
        std::memcpy(out, b.data(), b.size());
    });
}

}  // extern "C"
