// Plan-time selection of rank-1 lowerings: the static gfx950 model, replay
// from the user selection cache, or on-device measurement of every candidate
// (reference src/c_api.cpp:722-764 for the cache, 1420-1885 for the searches).
//
// The cache is a text file of `key<TAB>algorithm` records, appended under an
// exclusive flock and read under a shared one; the last record for a key
// wins and an unterminated final line (a writer that died mid-record) is
// ignored. Keys name the device (architecture, CU count), this library's
// selection version and every field of the rank-1 request that changes the
// kernels run, so a record is replayed only for the same work on the same
// kind of device.
#include "planner.hpp"

#include <fcntl.h>
#include <sys/file.h>
#include <unistd.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <fstream>
#include <limits>
#include <vector>

#include "json.hpp"

namespace cbw {
namespace {

class CacheLock {
  public:
    CacheLock(const std::string& path, bool write)
        : fd_(::open(path.c_str(), write ? (O_RDWR | O_CREAT) : O_RDONLY, 0600)) {
        if (fd_ < 0) {
            if (write) throw std::runtime_error("cannot open the selection cache " + path);
            return;  // no file yet: nothing to replay
        }
        if (::flock(fd_, write ? LOCK_EX : LOCK_SH) != 0) {
            ::close(fd_);
            fd_ = -1;
            throw std::runtime_error("cannot lock the selection cache " + path);
        }
    }
    ~CacheLock() {
        if (fd_ >= 0) {
            ::flock(fd_, LOCK_UN);
            ::close(fd_);
        }
    }
    CacheLock(const CacheLock&) = delete;
    CacheLock& operator=(const CacheLock&) = delete;

  private:
    int fd_;
};

std::string device_identity() {
    int device = 0;
    hipDeviceProp_t prop{};
    if (hipGetDevice(&device) != hipSuccess || hipGetDeviceProperties(&prop, device) != hipSuccess) {
        (void)hipGetLastError();
        return "no-device";
    }
    return std::string(prop.gcnArchName) + "|cu" + std::to_string(prop.multiProcessorCount);
}

// Priority of the reference's combined_source (src/c_api.cpp:1887-1901).
int rank_of(cubutterflySelectionSource_t s) {
    switch (s) {
        case CUBUTTERFLY_SELECTION_UNMEASURED_FALLBACK: return 5;
        case CUBUTTERFLY_SELECTION_RUNTIME_MEASURED: return 4;
        case CUBUTTERFLY_SELECTION_USER_CACHE: return 3;
        case CUBUTTERFLY_SELECTION_EXPLICIT: return 2;
        case CUBUTTERFLY_SELECTION_MEASURED_TABLE: return 1;
        default: return 0;
    }
}

void note(Selection& sel, const std::string& text) {
    if (!sel.notes.empty()) sel.notes += "; ";
    sel.notes += text;
}

struct DeviceScratch {
    void* ptr = nullptr;
    explicit DeviceScratch(std::size_t bytes) {
        if (bytes && hipMalloc(&ptr, bytes) != hipSuccess) {
            ptr = nullptr;
            (void)hipGetLastError();
            throw std::bad_alloc();
        }
    }
    ~DeviceScratch() {
        if (ptr) (void)hipFree(ptr);
    }
    DeviceScratch(DeviceScratch&& o) noexcept : ptr(o.ptr) { o.ptr = nullptr; }
    DeviceScratch(const DeviceScratch&) = delete;
    DeviceScratch& operator=(const DeviceScratch&) = delete;
    DeviceScratch& operator=(DeviceScratch&&) = delete;
};

struct Event {
    hipEvent_t e = nullptr;
    Event() { hip_check(hipEventCreate(&e), "MEASURE event"); }
    ~Event() {
        if (e) (void)hipEventDestroy(e);
    }
    Event(const Event&) = delete;
    Event& operator=(const Event&) = delete;
};

// CUBUTTERFLY_PLAN_TRACE = 1 | stderr | <path>: one JSON line per search
// event (schema cubutterfly-plan-search-trace-v1, reference
// src/plan_search_trace.hpp:17-60). Tracing never changes the search: a sink
// that cannot be written disables it with a note on stderr.
class SearchTrace {
  public:
    SearchTrace() {
        const char* dest = std::getenv("CUBUTTERFLY_PLAN_TRACE");
        if (!dest || !*dest || std::string(dest) == "0") return;
        static std::atomic<std::uint64_t> next_id{0};
        id_ = ++next_id;
        if (std::string(dest) == "1" || std::string(dest) == "stderr") {
            sink_ = stderr;
        } else {
            sink_ = std::fopen(dest, "a");
            owns_ = sink_ != nullptr;
            if (!sink_) std::fprintf(stderr, "cuButterfly: CUBUTTERFLY_PLAN_TRACE disabled: cannot open %s\n", dest);
        }
    }
    ~SearchTrace() {
        if (owns_) std::fclose(sink_);
    }
    SearchTrace(const SearchTrace&) = delete;
    SearchTrace& operator=(const SearchTrace&) = delete;
    // `fields`: the members after the common ones, as JSON text without braces.
    void event(const char* phase, const std::string& fields) {
        if (!sink_) return;
        const std::string line = "{\"schema\":\"cubutterfly-plan-search-trace-v1\",\"search_id\":" +
                                 std::to_string(id_) + ",\"phase\":" + json::quote(phase) +
                                 (fields.empty() ? "" : "," + fields) + "}\n";
        if (std::fwrite(line.data(), 1, line.size(), sink_) != line.size() || std::fflush(sink_) != 0) {
            std::fprintf(stderr, "cuButterfly: CUBUTTERFLY_PLAN_TRACE disabled: write failed\n");
            if (owns_) std::fclose(sink_);
            sink_ = nullptr;
            owns_ = false;
        }
    }

  private:
    std::FILE* sink_ = nullptr;
    bool owns_ = false;
    std::uint64_t id_ = 0;
};

// Milliseconds per execution of each candidate, over `sets` rotating input /
// output buffers (in_place: the input buffers only). Every candidate first
// runs kWarmup untimed calls; then kRounds rounds each time one block of
// kCalls calls per candidate, in candidate order, between two events on the
// selection stream; a candidate's figure is its median block / kCalls.
// Interleaving gives every candidate the same clock state: on MI355X the
// first few hundred calls after an idle gap run up to 12% slower than the
// sustained rate (a power / clock transient), which timing the candidates
// one after another would charge to whichever came first.
constexpr int kWarmup = 3, kRounds = 7, kCalls = 10;
std::vector<double> time_executors(const std::vector<std::unique_ptr<Executor>>& es,
                                   const std::vector<DeviceScratch>& in, const std::vector<DeviceScratch>& out,
                                   bool in_place, void* ws, hipStream_t stream) {
    const std::size_t sets = in.size();
    auto run = [&](Executor& e, int i) {
        const std::size_t k = std::size_t(i) % sets;
        e.execute(in[k].ptr, in_place ? in[k].ptr : out[k].ptr, ws, stream);
    };
    for (const auto& e : es)
        for (int i = 0; i < kWarmup; ++i) run(*e, i);
    std::vector<std::vector<double>> blocks(es.size());
    Event start, stop;
    for (int round = 0; round < kRounds; ++round) {
        for (std::size_t c = 0; c < es.size(); ++c) {
            hip_check(hipEventRecord(start.e, stream), "MEASURE event record");
            for (int i = 0; i < kCalls; ++i) run(*es[c], round * kCalls + i);
            hip_check(hipEventRecord(stop.e, stream), "MEASURE event record");
            hip_check(hipEventSynchronize(stop.e), "MEASURE synchronize");
            float ms = 0.0f;
            hip_check(hipEventElapsedTime(&ms, start.e, stop.e), "MEASURE elapsed time");
            blocks[c].push_back(double(ms) / kCalls);
        }
    }
    std::vector<double> result;
    for (auto& b : blocks) {
        std::sort(b.begin(), b.end());
        result.push_back(b[b.size() / 2]);
    }
    return result;
}

}  // namespace

void note_selection(Selection& sel, const std::string& text) { note(sel, text); }

void require_no_capture(const Selection& sel) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(sel.stream, &capture), "MEASURE capture query");
    supported(capture == hipStreamCaptureStatusNone, "MEASURE cannot time candidates during stream capture");
}

void combine_source(Selection& sel, cubutterflySelectionSource_t next) {
    if (rank_of(next) > rank_of(sel.source)) sel.source = next;
}

std::string lookup_cache(const std::string& path, const std::string& key) {
    if (path.empty()) return {};
    CacheLock lock(path, false);
    std::ifstream input(path);
    std::string line, match;
    while (std::getline(input, line)) {
        if (input.eof()) break;  // unterminated final record
        const auto tab = line.find('\t');
        if (tab == key.size() && line.compare(0, tab, key) == 0) match = line.substr(tab + 1);
    }
    return match;
}

void store_cache(const std::string& path, const std::string& key, const std::string& algorithm) {
    if (path.empty()) return;
    require(key.find('\n') == std::string::npos && algorithm.find_first_of("\t\n") == std::string::npos,
            "selection cache records are single lines");
    CacheLock lock(path, true);
    std::ofstream output(path, std::ios::app);
    if (!output) throw std::runtime_error("cannot open the selection cache " + path + " for writing");
    output << key << '\t' << algorithm << '\n';
    output.flush();
    if (!output) throw std::runtime_error("cannot persist the selection cache record");
}

std::string selection_key(const Request& r) {
    json::Writer w;
    w.begin_object()
        .field("op", int(r.op))
        .field("storage", int(r.storage))
        .field("log_n", r.log_n)
        .field("batch", r.batch)
        .field("inverse", r.inverse)
        .field("normalize", r.normalize)
        .field("in_place", r.in_place)
        .field("fp16_final", r.fp16_final)
        .field("allow_mma", r.allow_mma)
        .field("output_scale", double(r.output_scale))
        .field("modulus", r.modulus)
        .field("word_bits", r.word_bits)
        .field("negacyclic", r.negacyclic)
        .field("psi", r.psi)
        .field("input_bit_reversed", r.input_bit_reversed)
        .field("output_bit_reversed", r.output_bit_reversed)
        .field("pitched", r.pitched)
        .field("input_batch_stride", r.pitched ? r.in_batch_stride : 0)
        .field("output_batch_stride", r.pitched ? r.out_batch_stride : 0)
        .end_object();
    return "cubutterfly-gfx950-selection-v2|" + device_identity() + "|" + w.str();
}

std::unique_ptr<Executor> build_leaf(const Request& r) {
    switch (r.op) {
        case Op::Fwht: return make_fwht_executor(r);
        case Op::Fft: return make_fft_executor(r);
        case Op::Ntt: return make_ntt_executor(r);
    }
    throw NotSupported("operator has no MI355X lowering");
}

std::vector<std::string> leaf_candidates(const Request& r) {
    switch (r.op) {
        case Op::Fwht: return fwht_candidates(r);
        case Op::Fft: return fft_candidates(r);
        case Op::Ntt: return ntt_candidates(r);
    }
    return {};
}

// MEASURE over built executors of one request, with the search trace of the
// caller: times them on rotating scratch buffers, records the fastest under
// `key` and notes the figures. Returns the fastest's index, or built.size()
// when the scratch could not be allocated (the caller keeps its static choice).
static std::size_t measure_traced(const Request& r, const std::string& key,
                                  const std::vector<std::unique_ptr<Executor>>& built, Selection& sel,
                                  std::size_t candidate_count, SearchTrace& trace);

std::unique_ptr<Executor> select_leaf(const Request& r, Selection* sel) {
    if (sel == nullptr || sel->policy == CUBUTTERFLY_ALGORITHM_EXPLICIT) {
        if (r.policy != CUBUTTERFLY_ALGORITHM_EXPLICIT) return build_leaf(r);
        Request v = r;
        v.variant = r.explicit_algorithm;
        return build_leaf(v);
    }
    const std::string key = selection_key(r);
    if (sel->policy == CUBUTTERFLY_ALGORITHM_DEFAULT) {
        const std::string cached = lookup_cache(sel->cache_path, key);
        if (!cached.empty()) {
            Request v = r;
            v.variant = cached;
            try {
                auto e = build_leaf(v);
                combine_source(*sel, CUBUTTERFLY_SELECTION_USER_CACHE);
                note(*sel, "replayed '" + cached + "' from the selection cache");
                return e;
            } catch (const NotSupported&) {
                note(*sel, "ignored cache record '" + cached + "' (not a lowering of this request)");
            }
        }
        return build_leaf(r);
    }
    // MEASURE: every candidate on the device, on shared scratch buffers
    // (refused before any candidate allocates its tables on a capturing
    // stream).
    require_no_capture(*sel);
    SearchTrace trace;
    const auto names = leaf_candidates(r);
    std::vector<std::unique_ptr<Executor>> built;
    for (const auto& name : names) {
        Request v = r;
        v.variant = name;
        try {
            built.push_back(build_leaf(v));
        } catch (const NotSupported& e) {  // not a lowering here after all: skip it
            trace.event("result", "\"candidate\":" + json::quote(name) + ",\"status\":\"rejected\",\"reason\":" +
                                      json::quote(e.what()));
        }
    }
    require(!built.empty(), "no candidate lowering to measure");
    const std::size_t best = measure_traced(r, key, built, *sel, names.size(), trace);
    if (best == built.size()) return build_leaf(r);
    return std::move(built[best]);
}

std::size_t measure_executors(const Request& r, const std::string& key,
                              const std::vector<std::unique_ptr<Executor>>& built, Selection& sel) {
    SearchTrace trace;
    return measure_traced(r, key, built, sel, built.size(), trace);
}

static std::size_t measure_traced(const Request& r, const std::string& key,
                                  const std::vector<std::unique_ptr<Executor>>& built, Selection& sel,
                                  std::size_t candidate_count, SearchTrace& trace) {
    require_no_capture(sel);
    require(!built.empty(), "no candidate lowering to measure");
    // Scratch sides span what the kernels address: a pitched leaf reads and
    // writes row b at b * batch stride, up to (batch - 1) * pitch + n elements.
    const std::size_t in_bytes = r.in_place ? std::max(r.span_bytes(true), r.span_bytes(false)) : r.span_bytes(true);
    const std::size_t out_bytes = r.in_place ? 0 : r.span_bytes(false);
    const std::size_t footprint = in_bytes + out_bytes;
    // Buffer sets: transforms of 16 MiB or more rotate over enough sets that
    // their inputs alone exceed twice the 256 MB Infinity Cache (nontemporal
    // output stores do not evict earlier inputs from it; at most 16 sets, so
    // below 32 MiB of input part of the data stays cached), so candidates
    // are timed at HBM speed as in steady use over large data. The search
    // stays within max(512 MiB, min(2 GiB, free / 4)) of scratch (the
    // reference's tuning budget); beyond it, fewer sets.
    constexpr std::size_t kCacheBytes = std::size_t{256} << 20;
    std::size_t sets = r.data_bytes() >= (std::size_t{16} << 20)
                           ? std::min<std::size_t>(16, (2 * kCacheBytes) / std::max<std::size_t>(in_bytes, 1) + 1)
                           : 1;
    std::size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess) {
        (void)hipGetLastError();
        free_bytes = 0;
    }
    const std::size_t budget = std::max(std::size_t{512} << 20, std::min(std::size_t{2} << 30, free_bytes / 4));
    std::size_t ws_bytes = 0;
    for (const auto& e : built) ws_bytes = std::max(ws_bytes, e->workspace_bytes());
    while (sets > 1 && sets * footprint + ws_bytes > budget) --sets;
    trace.event("inventory", "\"key\":" + json::quote(key) + ",\"candidate_count\":" +
                                 std::to_string(candidate_count) +
                                 ",\"timing_protocol\":\"interleaved-rounds\",\"warmup\":" +
                                 std::to_string(kWarmup) + ",\"rounds\":" + std::to_string(kRounds) +
                                 ",\"calls_per_round\":" + std::to_string(kCalls) + "," +
                                 "\"buffer_sets\":" + std::to_string(sets) + ",\"input_bytes\":" +
                                 std::to_string(in_bytes) + ",\"output_bytes\":" + std::to_string(out_bytes) +
                                 ",\"workspace_bytes\":" + std::to_string(ws_bytes) + ",\"scratch_bytes\":" +
                                 std::to_string(sets * footprint + ws_bytes));
    std::vector<DeviceScratch> in, out;
    std::unique_ptr<DeviceScratch> ws;
    try {
        in.reserve(sets);
        out.reserve(sets);
        for (std::size_t k = 0; k < sets; ++k) {
            in.emplace_back(in_bytes);
            out.emplace_back(out_bytes);
            hip_check(hipMemsetAsync(in.back().ptr, 0, in_bytes, sel.stream), "MEASURE input fill");
        }
        ws = std::make_unique<DeviceScratch>(ws_bytes);
    } catch (const std::bad_alloc&) {
        // Not enough device memory to time the candidates: keep the static
        // model's lowering and say so, instead of failing the plan.
        trace.event("selected", "\"algorithm\":null,\"reason\":\"scratch allocation failed\"");
        note(sel, "MEASURE skipped: could not allocate " + std::to_string(sets * footprint + ws_bytes) +
                      " bytes of scratch; static model used");
        return built.size();
    }
    std::size_t best = 0;
    double best_ms = std::numeric_limits<double>::infinity();
    std::string results;
    const std::vector<double> times = time_executors(built, in, out, r.in_place, ws->ptr, sel.stream);
    for (std::size_t i = 0; i < built.size(); ++i) {
        const double ms = times[i];
        char text[64];
        std::snprintf(text, sizeof text, "=%.4f ms", ms);
        results += (i ? ", " : "") + built[i]->algorithm + text;
        trace.event("result", "\"candidate\":" + json::quote(built[i]->algorithm) +
                                  ",\"status\":\"accepted\",\"kernel_ms\":" + std::to_string(ms));
        if (ms < best_ms) {
            best_ms = ms;
            best = i;
        }
    }
    trace.event("selected", "\"algorithm\":" + json::quote(built[best]->algorithm) +
                                ",\"kernel_ms\":" + std::to_string(best_ms));
    store_cache(sel.cache_path, key, built[best]->algorithm);
    combine_source(sel, CUBUTTERFLY_SELECTION_RUNTIME_MEASURED);
    note(sel, "measured " + results);
    return best;
}

}  // namespace cbw
