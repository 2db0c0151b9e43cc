// C ABI of libcubutterfly (include/cubutterfly/cubutterfly.h). Every entry is
// an exception firewall: C++ exceptions become status codes plus a
// thread-local detail string (reference behaviour: src/c_api.cpp:121-163).
#include "../../include/cubutterfly/cubutterfly.h"
#include "../../include/cubutterfly/cubutterfly_mi355x.h"
#include "descriptor.hpp"
#include "json.hpp"
#include "planner.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>

struct cubutterflyHandle {
    hipStream_t stream = nullptr;
    cubutterflyLogCallback_t logger = nullptr;
    void* logger_data = nullptr;
    std::string cache_path;
};

struct cubutterflyPlan {
    cubutterflyDescriptor descriptor;
    cbw::Request request;
    std::unique_ptr<cbw::Executor> executor;
    std::size_t input_bytes = 0, output_bytes = 0, workspace_bytes = 0;
    void* workspace = nullptr;
    hipStream_t bound_stream = nullptr;
    bool bound = false;
    cubutterflySelectionSource_t source = CUBUTTERFLY_SELECTION_STATIC_MODEL;
};

namespace {

thread_local std::string last_error;

template <class F>
cubutterflyStatus_t protect(F&& body) noexcept {
    try {
        last_error.clear();
        body();
        return CUBUTTERFLY_STATUS_SUCCESS;
    } catch (const cbw::NotSupported& e) {
        last_error = e.what();
        return CUBUTTERFLY_STATUS_NOT_SUPPORTED;
    } catch (const cbw::HipError& e) {
        last_error = e.what();
        return CUBUTTERFLY_STATUS_CUDA_ERROR;
    } catch (const std::invalid_argument& e) {
        last_error = e.what();
        return CUBUTTERFLY_STATUS_INVALID_VALUE;
    } catch (const std::overflow_error& e) {
        last_error = e.what();
        return CUBUTTERFLY_STATUS_INVALID_VALUE;
    } catch (const std::bad_alloc&) {
        last_error = "allocation failed";
        return CUBUTTERFLY_STATUS_ALLOC_FAILED;
    } catch (const std::logic_error& e) {
        last_error = e.what();
        return CUBUTTERFLY_STATUS_INTERNAL_ERROR;
    } catch (const std::runtime_error& e) {
        last_error = e.what();
        return CUBUTTERFLY_STATUS_BACKEND_ERROR;
    } catch (...) {
        last_error = "unrecognized exception";
        return CUBUTTERFLY_STATUS_INTERNAL_ERROR;
    }
}

using cbw::require;

// Two-call string query: text == NULL stores the size (with NUL) in *bytes;
// a short buffer is INVALID_VALUE with *bytes updated.
void copy_text(const std::string& value, char* text, size_t* bytes) {
    require(bytes != nullptr, "size pointer must be non-null");
    const std::size_t needed = value.size() + 1;
    const std::size_t capacity = *bytes;
    *bytes = needed;
    if (text == nullptr) return;
    require(capacity >= needed, "string buffer is too small");
    std::memcpy(text, value.c_str(), needed);
}

void log_event(cubutterflyHandle_t handle, cubutterflyLogLevel_t level, const char* event, const std::string& message) {
    if (handle && handle->logger) handle->logger(level, event, message.c_str(), handle->logger_data);
}

void check_execution(cubutterflyHandle_t handle, cubutterflyPlan_t plan, const void* input, void* output) {
    require(handle != nullptr && plan != nullptr && input != nullptr && output != nullptr,
            "execution arguments must be non-null");
    require(plan->request.in_place ? input == output : input != output,
            plan->request.in_place ? "in-place execution requires identical pointers"
                                   : "out-of-place execution requires distinct pointers");
}

void execute_plan(cubutterflyHandle_t handle, cubutterflyPlan_t plan, const void* input, void* output) {
    check_execution(handle, plan, input, output);
    require(plan->workspace_bytes == 0 || plan->workspace != nullptr,
            "plan requires a workspace; bind one with cubutterflyPlanSetWorkspace");
    plan->executor->execute(input, output, plan->workspace, handle->stream);
    plan->bound_stream = handle->stream;
    plan->bound = true;
}

}  // namespace

namespace cbw {

cubutterflyStatus_t guarded_call(void (*body)(void*), void* context) noexcept {
    return protect([&] { body(context); });
}

void execute_plan_with_workspace(cubutterflyHandle_t handle, cubutterflyPlan_t plan, const void* input, void* output,
                                 void* workspace, std::size_t capacity, const char* what) {
    check_execution(handle, plan, input, output);
    if (plan->workspace_bytes > capacity)
        throw std::invalid_argument("plan needs " + std::to_string(plan->workspace_bytes) + " bytes of workspace; " +
                                    what + " holds " + std::to_string(capacity));
    plan->executor->execute(input, output, plan->workspace_bytes ? workspace : nullptr, handle->stream);
}

}  // namespace cbw

extern "C" {

const char* cubutterflyGetLastErrorString(void) { return last_error.c_str(); }

const char* cubutterflyGetStatusString(cubutterflyStatus_t status) {
    switch (status) {
        case CUBUTTERFLY_STATUS_SUCCESS: return "success";
        case CUBUTTERFLY_STATUS_INVALID_VALUE: return "invalid value";
        case CUBUTTERFLY_STATUS_INVALID_TYPE: return "invalid type";
        case CUBUTTERFLY_STATUS_NOT_SUPPORTED: return "not supported";
        case CUBUTTERFLY_STATUS_ALLOC_FAILED: return "allocation failed";
        case CUBUTTERFLY_STATUS_CUDA_ERROR: return "HIP error";
        case CUBUTTERFLY_STATUS_BACKEND_ERROR: return "backend error";
        case CUBUTTERFLY_STATUS_INTERNAL_ERROR: return "internal error";
    }
    return "unknown status";
}

cubutterflyStatus_t cubutterflyGetVersion(int* major, int* minor, int* patch) {
    return protect([&] {
        require(major && minor && patch, "version pointers must be non-null");
        *major = CUBUTTERFLY_VERSION_MAJOR;
        *minor = CUBUTTERFLY_VERSION_MINOR;
        *patch = CUBUTTERFLY_VERSION_PATCH;
    });
}

cubutterflyStatus_t cubutterflyCreate(cubutterflyHandle_t* handle) {
    return protect([&] {
        require(handle != nullptr, "handle pointer must be non-null");
        *handle = new cubutterflyHandle;
    });
}
cubutterflyStatus_t cubutterflyDestroy(cubutterflyHandle_t handle) {
    delete handle;
    return CUBUTTERFLY_STATUS_SUCCESS;
}
cubutterflyStatus_t cubutterflySetStream(cubutterflyHandle_t handle, hipStream_t stream) {
    return protect([&] {
        require(handle != nullptr, "handle must be non-null");
        handle->stream = stream;
    });
}
cubutterflyStatus_t cubutterflyGetStream(cubutterflyHandle_t handle, hipStream_t* stream) {
    return protect([&] {
        require(handle && stream, "handle and stream pointer must be non-null");
        *stream = handle->stream;
    });
}
cubutterflyStatus_t cubutterflySetLogCallback(cubutterflyHandle_t handle, cubutterflyLogCallback_t callback,
                                              void* user_data) {
    return protect([&] {
        require(handle != nullptr, "handle must be non-null");
        handle->logger = callback;
        handle->logger_data = user_data;
    });
}
cubutterflyStatus_t cubutterflySetCachePath(cubutterflyHandle_t handle, const char* path) {
    return protect([&] {
        require(handle != nullptr, "handle must be non-null");
        handle->cache_path = path ? path : "";
    });
}

int cubutterflyPackRealFp32(const float*, void*, size_t, float, uint64_t) {
    last_error = "real-FFT packing adapters are not part of the MI355X butterfly path";
    return CUBUTTERFLY_STATUS_NOT_SUPPORTED;
}
int cubutterflyExpandHermitianFp32(const void*, void*, uint32_t, uint32_t, size_t, uint64_t) {
    last_error = "real-FFT expansion adapters are not part of the MI355X butterfly path";
    return CUBUTTERFLY_STATUS_NOT_SUPPORTED;
}

// ---- descriptor ------------------------------------------------------------

cubutterflyStatus_t cubutterflyCreateDescriptor(cubutterflyDescriptor_t* descriptor) {
    return protect([&] {
        require(descriptor != nullptr, "descriptor pointer must be non-null");
        *descriptor = new cubutterflyDescriptor;
    });
}
cubutterflyStatus_t cubutterflyDestroyDescriptor(cubutterflyDescriptor_t descriptor) {
    delete descriptor;
    return CUBUTTERFLY_STATUS_SUCCESS;
}

#define CBW_DESCRIPTOR_SETTER(body)                                    \
    return protect([&] {                                               \
        require(descriptor != nullptr, "descriptor must be non-null"); \
        body;                                                          \
    })

cubutterflyStatus_t cubutterflySetOperator(cubutterflyDescriptor_t descriptor, cubutterflyOperator_t op) {
    CBW_DESCRIPTOR_SETTER(descriptor->op = op);
}
cubutterflyStatus_t cubutterflySetDataType(cubutterflyDescriptor_t descriptor, cubutterflyDataType_t storage,
                                           cubutterflyComputeType_t compute) {
    CBW_DESCRIPTOR_SETTER(descriptor->storage = storage; descriptor->compute = compute);
}
cubutterflyStatus_t cubutterflySetShape(cubutterflyDescriptor_t descriptor, uint32_t rank, const size_t* extents,
                                        size_t batch) {
    return protect([&] {
        require(descriptor && extents, "descriptor and extents must be non-null");
        require(rank >= 1, "rank must be positive");
        require(batch != 0, "batch must be positive");
        std::vector<std::size_t> shape(extents, extents + rank);
        std::size_t count = batch;
        for (auto e : shape) {
            require(e != 0, "extents must be positive");
            require(count <= std::numeric_limits<std::size_t>::max() / e, "shape element count overflows size_t");
            count *= e;
        }
        descriptor->rank = rank;
        descriptor->extents = std::move(shape);
        descriptor->batch = batch;
        descriptor->stage_matrices.resize(std::max<std::size_t>(rank, descriptor->stage_matrices.size()));
    });
}
cubutterflyStatus_t cubutterflySetExecutionMode(cubutterflyDescriptor_t descriptor, cubutterflyExecutionMode_t mode) {
    CBW_DESCRIPTOR_SETTER(require(mode >= CUBUTTERFLY_EXECUTION_AUTO && mode <= CUBUTTERFLY_EXECUTION_COMPOSITE,
                                  "unknown execution mode");
                          descriptor->execution_mode = mode);
}
cubutterflyStatus_t cubutterflySetFftTransformType(cubutterflyDescriptor_t descriptor,
                                                   cubutterflyFftTransformType_t type) {
    CBW_DESCRIPTOR_SETTER(require(type >= CUBUTTERFLY_FFT_C2C && type <= CUBUTTERFLY_FFT_C2R,
                                  "unknown FFT transform type");
                          descriptor->fft_type = type);
}
cubutterflyStatus_t cubutterflySetFftOutputScale(cubutterflyDescriptor_t descriptor, double scale) {
    CBW_DESCRIPTOR_SETTER(require(std::isfinite(scale), "FFT scale must be finite");
                          descriptor->fft_output_scale = scale);
}
cubutterflyStatus_t cubutterflySetOutputScale(cubutterflyDescriptor_t descriptor, double scale) {
    CBW_DESCRIPTOR_SETTER(require(std::isfinite(scale), "output scale must be finite");
                          descriptor->output_scale = scale);
}
cubutterflyStatus_t cubutterflySetArithmeticPolicy(cubutterflyDescriptor_t descriptor,
                                                   cubutterflyArithmeticPolicy_t policy) {
    CBW_DESCRIPTOR_SETTER(require(policy == CUBUTTERFLY_ARITHMETIC_STRICT ||
                                      policy == CUBUTTERFLY_ARITHMETIC_ALLOW_FP16_MMA,
                                  "invalid arithmetic policy");
                          descriptor->arithmetic_policy = policy);
}
cubutterflyStatus_t cubutterflySetOutputRounding(cubutterflyDescriptor_t descriptor,
                                                 cubutterflyOutputRounding_t rounding) {
    CBW_DESCRIPTOR_SETTER(require(rounding == CUBUTTERFLY_ROUNDING_STAGE_STORAGE ||
                                      rounding == CUBUTTERFLY_ROUNDING_FINAL_STORAGE,
                                  "invalid output rounding");
                          descriptor->output_rounding = rounding);
}
cubutterflyStatus_t cubutterflySetStrides(cubutterflyDescriptor_t descriptor, const size_t* input_strides,
                                          size_t input_batch_stride, const size_t* output_strides,
                                          size_t output_batch_stride) {
    CBW_DESCRIPTOR_SETTER(
        descriptor->input_strides.assign(input_strides ? input_strides : nullptr,
                                         input_strides ? input_strides + descriptor->rank : nullptr);
        descriptor->output_strides.assign(output_strides ? output_strides : nullptr,
                                          output_strides ? output_strides + descriptor->rank : nullptr);
        descriptor->input_batch_stride = input_batch_stride; descriptor->output_batch_stride = output_batch_stride);
}
cubutterflyStatus_t cubutterflySetLogicalOrders(cubutterflyDescriptor_t descriptor,
                                                const cubutterflyLogicalOrder_t* input_orders,
                                                const cubutterflyLogicalOrder_t* output_orders) {
    return protect([&] {
        require(descriptor != nullptr, "descriptor must be non-null");
        std::vector<cubutterflyLogicalOrder_t> in(descriptor->rank, CUBUTTERFLY_ORDER_NATURAL), out = in;
        if (input_orders) std::copy(input_orders, input_orders + descriptor->rank, in.begin());
        if (output_orders) std::copy(output_orders, output_orders + descriptor->rank, out.begin());
        for (const auto* side : {&in, &out})
            for (auto o : *side)
                require(o == CUBUTTERFLY_ORDER_NATURAL || o == CUBUTTERFLY_ORDER_BIT_REVERSED,
                        "unknown logical order");
        descriptor->input_orders = std::move(in);
        descriptor->output_orders = std::move(out);
        descriptor->input_ntt_layout = descriptor->output_ntt_layout = CUBUTTERFLY_NTT_LAYOUT_NATURAL;
    });
}
cubutterflyStatus_t cubutterflySetDirection(cubutterflyDescriptor_t descriptor, cubutterflyDirection_t direction,
                                            int normalize_inverse) {
    CBW_DESCRIPTOR_SETTER(descriptor->direction = direction; descriptor->normalize_inverse = normalize_inverse != 0);
}
cubutterflyStatus_t cubutterflySetPlacement(cubutterflyDescriptor_t descriptor, cubutterflyPlacement_t placement) {
    CBW_DESCRIPTOR_SETTER(descriptor->placement = placement);
}
cubutterflyStatus_t cubutterflySetLengthMode(cubutterflyDescriptor_t descriptor, cubutterflyLengthMode_t mode) {
    CBW_DESCRIPTOR_SETTER(descriptor->length_mode = mode);
}
cubutterflyStatus_t cubutterflySetAlgorithmPolicy(cubutterflyDescriptor_t descriptor,
                                                  cubutterflyAlgorithmPolicy_t policy,
                                                  const char* explicit_algorithm) {
    CBW_DESCRIPTOR_SETTER(
        require(policy != CUBUTTERFLY_ALGORITHM_EXPLICIT || (explicit_algorithm && explicit_algorithm[0]),
                "explicit policy requires an algorithm name");
        descriptor->algorithm_policy = policy;
        descriptor->explicit_algorithm = explicit_algorithm ? explicit_algorithm : "");
}
cubutterflyStatus_t cubutterflySetModulus(cubutterflyDescriptor_t descriptor, uint64_t modulus, uint32_t word_bits) {
    CBW_DESCRIPTOR_SETTER(require(word_bits == 32 || word_bits == 64, "word width must be 32 or 64");
                          descriptor->modulus = modulus; descriptor->word_bits = word_bits);
}
cubutterflyStatus_t cubutterflySetNttLayouts(cubutterflyDescriptor_t descriptor, cubutterflyNttLayout_t input_layout,
                                             cubutterflyNttLayout_t output_layout) {
    CBW_DESCRIPTOR_SETTER(
        require(input_layout >= CUBUTTERFLY_NTT_LAYOUT_NATURAL && input_layout <= CUBUTTERFLY_NTT_LAYOUT_BIT_REVERSED &&
                    output_layout >= CUBUTTERFLY_NTT_LAYOUT_NATURAL &&
                    output_layout <= CUBUTTERFLY_NTT_LAYOUT_BIT_REVERSED,
                "unknown NTT layout");
        descriptor->input_ntt_layout = input_layout; descriptor->output_ntt_layout = output_layout;
        descriptor->input_orders.clear(); descriptor->output_orders.clear());
}
cubutterflyStatus_t cubutterflySetStageMatrices(cubutterflyDescriptor_t descriptor, uint32_t axis,
                                                const cubutterflyMatrix2x2_t* matrices, size_t count) {
    return protect([&] {
        require(descriptor && matrices && count, "matrix arguments must be non-null and non-empty");
        require(axis < descriptor->rank, "matrix axis must be in the descriptor rank");
        if (descriptor->stage_matrices.size() <= axis) descriptor->stage_matrices.resize(axis + 1);
        descriptor->stage_matrices[axis].assign(matrices, matrices + count);
    });
}
cubutterflyStatus_t cubutterflySetNttRing(cubutterflyDescriptor_t descriptor, cubutterflyNttRing_t ring,
                                          uint64_t psi) {
    CBW_DESCRIPTOR_SETTER(
        require(ring == CUBUTTERFLY_NTT_RING_CYCLIC || ring == CUBUTTERFLY_NTT_RING_NEGACYCLIC, "unknown NTT ring");
        require(ring == CUBUTTERFLY_NTT_RING_NEGACYCLIC || psi == 0, "psi requires the negacyclic ring");
        descriptor->ring = ring; descriptor->psi = psi);
}

cubutterflyStatus_t cubutterflyDescriptorValidate(cubutterflyDescriptor_t descriptor) {
    CBW_DESCRIPTOR_SETTER(cbw::validate_descriptor(*descriptor));
}
cubutterflyStatus_t cubutterflyDescriptorGetJson(cubutterflyDescriptor_t descriptor, char* json, size_t* bytes) {
    CBW_DESCRIPTOR_SETTER(copy_text(cbw::descriptor_json(*descriptor), json, bytes));
}
cubutterflyStatus_t cubutterflyDescriptorSetJson(cubutterflyDescriptor_t descriptor, const char* json) {
    return protect([&] {
        require(descriptor && json, "descriptor and JSON must be non-null");
        *descriptor = cbw::descriptor_from_json(json);  // atomic: replaced only on success
    });
}
cubutterflyStatus_t cubutterflyDescriptorGetCapabilities(cubutterflyDescriptor_t descriptor, char* json,
                                                         size_t* bytes) {
    CBW_DESCRIPTOR_SETTER(copy_text(cbw::capabilities_json(*descriptor), json, bytes));
}

// ---- plan ------------------------------------------------------------------

cubutterflyStatus_t cubutterflyCreatePlan(cubutterflyHandle_t handle, cubutterflyDescriptor_t descriptor,
                                          cubutterflyPlan_t* plan) {
    return protect([&] {
        require(handle && descriptor && plan, "plan arguments must be non-null");
        *plan = nullptr;
        auto created = std::make_unique<cubutterflyPlan>();
        created->descriptor = *descriptor;
        created->request = cbw::lower_request(*descriptor);
        // Selection (reference src/c_api.cpp:4329-4420): EXPLICIT builds the
        // named lowering, DEFAULT replays the selection cache where it holds a
        // record, MEASURE times every candidate of each rank-1 plan and records
        // the fastest.
        cbw::Selection selection;
        selection.policy = created->request.policy;
        selection.cache_path = handle->cache_path;
        selection.stream = handle->stream;
        created->executor = cbw::plan_executor(created->request, &selection);
        if (created->request.policy == CUBUTTERFLY_ALGORITHM_EXPLICIT) {
            cbw::supported(created->executor->algorithm == created->request.explicit_algorithm,
                           "explicit algorithm '" + created->request.explicit_algorithm +
                               "' is not a lowering of this descriptor (available: " +
                               created->executor->algorithm + ")");
            created->source = CUBUTTERFLY_SELECTION_EXPLICIT;
        } else {
            created->source = selection.source;
        }
        if (!selection.notes.empty()) {
            created->executor->reason += "; " + selection.notes;
            if (created->request.policy == CUBUTTERFLY_ALGORITHM_MEASURE)
                log_event(handle, CUBUTTERFLY_LOG_INFO, "measure-complete",
                          selection.notes + "; algorithm=" + created->executor->algorithm);
        }
        created->input_bytes = created->request.span_bytes(true);
        created->output_bytes = created->request.span_bytes(false);
        created->workspace_bytes = created->executor->workspace_bytes();
        // The reference's log events (src/c_api.cpp:4526-4529, 4782;
        // docs/c_api.md:193-198): every plan reports its selection, and a
        // DEFAULT plan that took the static model -- no measured or cached
        // mapping for this exact workload -- warns and recommends MEASURE.
        log_event(handle, CUBUTTERFLY_LOG_INFO, "algorithm-selection",
                  created->executor->reason + "; algorithm=" + created->executor->algorithm);
        if (created->request.policy == CUBUTTERFLY_ALGORITHM_DEFAULT &&
            (created->source == CUBUTTERFLY_SELECTION_STATIC_MODEL ||
             created->source == CUBUTTERFLY_SELECTION_UNMEASURED_FALLBACK))
            log_event(handle, CUBUTTERFLY_LOG_WARNING, "workload-profile-miss",
                      "no measured or cached mapping for this workload on gfx950; " +
                          cbw::selection_key(created->request) + "; " + created->executor->reason + "; using " +
                          created->executor->algorithm + "; set MEASURE with a cache path to calibrate this workload");
        *plan = created.release();
    });
}
cubutterflyStatus_t cubutterflyDestroyPlan(cubutterflyPlan_t plan) {
    delete plan;
    return CUBUTTERFLY_STATUS_SUCCESS;
}
cubutterflyStatus_t cubutterflyPlanGetDescriptorJson(cubutterflyPlan_t plan, char* json, size_t* bytes) {
    return protect([&] {
        require(plan != nullptr, "plan must be non-null");
        copy_text(cbw::descriptor_json(plan->descriptor), json, bytes);
    });
}
cubutterflyStatus_t cubutterflyPlanGetWorkspaceSize(cubutterflyPlan_t plan, size_t* bytes) {
    return protect([&] {
        require(plan && bytes, "plan and output must be non-null");
        *bytes = plan->workspace_bytes;
    });
}
cubutterflyStatus_t cubutterflyPlanGetInputSize(cubutterflyPlan_t plan, size_t* bytes) {
    return protect([&] {
        require(plan && bytes, "plan and output must be non-null");
        *bytes = plan->input_bytes;
    });
}
cubutterflyStatus_t cubutterflyPlanGetOutputSize(cubutterflyPlan_t plan, size_t* bytes) {
    return protect([&] {
        require(plan && bytes, "plan and output must be non-null");
        *bytes = plan->output_bytes;
    });
}
cubutterflyStatus_t cubutterflyPlanGetPhysicalExtents(cubutterflyPlan_t plan, size_t* extents, uint32_t capacity) {
    return protect([&] {
        require(plan && extents, "plan and extents must be non-null");
        const auto& r = plan->request;
        const std::uint32_t rank = plan->descriptor.rank;
        require(capacity >= rank, "extent capacity is too small");
        if (rank == 1) extents[0] = r.n;  // a factored FWHT reports its one axis
        else std::copy(r.extents.begin(), r.extents.end(), extents);
    });
}
cubutterflyStatus_t cubutterflyPlanGetSelectionSource(cubutterflyPlan_t plan, cubutterflySelectionSource_t* source) {
    return protect([&] {
        require(plan && source, "plan and output must be non-null");
        *source = plan->source;
    });
}
cubutterflyStatus_t cubutterflyPlanGetAlgorithmName(cubutterflyPlan_t plan, char* name, size_t* bytes) {
    return protect([&] {
        require(plan != nullptr, "plan must be non-null");
        copy_text(plan->executor->algorithm, name, bytes);
    });
}
cubutterflyStatus_t cubutterflyPlanGetSelectionReason(cubutterflyPlan_t plan, char* reason, size_t* bytes) {
    return protect([&] {
        require(plan != nullptr, "plan must be non-null");
        copy_text(plan->executor->reason, reason, bytes);
    });
}
cubutterflyStatus_t cubutterflyPlanGetMappingJson(cubutterflyPlan_t plan, char* json, size_t* bytes) {
    return protect([&] {
        require(plan != nullptr, "plan must be non-null");
        copy_text(plan->executor->mapping_json, json, bytes);
    });
}
cubutterflyStatus_t cubutterflyPlanGetNttLayoutInfo(cubutterflyPlan_t plan, cubutterflyNttLayoutInfo_t* info) {
    return protect([&] {
        require(plan && info, "plan and info must be non-null");
        cbw::supported(false, "APPT layout information is not produced by MI355X NTT plans");
    });
}
cubutterflyStatus_t cubutterflyPlanSetWorkspace(cubutterflyPlan_t plan, void* workspace, size_t bytes) {
    return protect([&] {
        require(plan != nullptr, "plan must be non-null");
        if (workspace == nullptr) {
            plan->workspace = nullptr;
            return;
        }
        require(bytes >= plan->workspace_bytes, "workspace is smaller than PlanGetWorkspaceSize");
        require(reinterpret_cast<std::uintptr_t>(workspace) % 16 == 0, "workspace must be 16-byte aligned");
        plan->workspace = workspace;
    });
}
cubutterflyStatus_t cubutterflyExecute(cubutterflyHandle_t handle, cubutterflyPlan_t plan, const void* input,
                                       void* output) {
    return protect([&] { execute_plan(handle, plan, input, output); });
}
cubutterflyStatus_t cubutterflyExecuteSteady(cubutterflyHandle_t handle, cubutterflyPlan_t plan, const void* input,
                                             void* output) {
    // Plans bind no child state to streams, so the steady path is the same
    // submission; it exists for ABI compatibility (reference :5390-5411).
    return protect([&] { execute_plan(handle, plan, input, output); });
}

}  // extern "C"
