// C-ABI plumbing: thread-local error messages, launch checks, version and the
// demand-staging copy (A7, expertbench/executor.py:341-363).
#include "common.h"

#include <cstring>

namespace pd {

static thread_local std::string g_error;

void set_error(const std::string &msg) { g_error = msg; }

int fail(int code, const std::string &msg) {
    g_error = msg;
    return code;
}

int check_launch(const char *what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(kEHip, std::string(what) + ": " + hipGetErrorString(err));
    return kOk;
}

}  // namespace pd

using namespace pd;

PD_API const char *pdscope_last_error(void) { return g_error.c_str(); }

PD_API const char *pdscope_version(void) { return "pdscope_moe gfx950 0.1"; }

PD_API int pdscope_stage_expert(void *dst_slot, const void *pinned_src, size_t bytes, void *event,
                                void *stream) {
    if (!dst_slot || !pinned_src || bytes == 0) return fail(kEInval, "stage_expert: bad arguments");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t err = hipMemcpyAsync(dst_slot, pinned_src, bytes, hipMemcpyHostToDevice, s);
    if (err != hipSuccess) return fail(kEHip, std::string("hipMemcpyAsync(stage_expert): ") + hipGetErrorString(err));
    if (event) {
        err = hipEventRecord(reinterpret_cast<hipEvent_t>(event), s);
        if (err != hipSuccess) return fail(kEHip, std::string("hipEventRecord: ") + hipGetErrorString(err));
    }
    return kOk;
}

// Host half of the native decode dispatch (native/native_layer_dispatch.cpp:34-40,
// 59-67): `rows` copies of one activation row into the packed block, expert ids
// into `selected`, unit coefficients and the row count, ready for the CPU
// expert queue's forward_task.
PD_API int pdscope_dispatch_pack(const void *row, int64_t rows, int64_t row_bytes, void *packed, int32_t *count,
                                 int64_t *selected, float *coeff, const int64_t *ids) {
    if (rows < 1 || row_bytes < 2 || row_bytes % 2 != 0) return fail(kEInval, "invalid decode pack shape");
    if (!row || !packed || !count || !selected || !coeff || !ids) return fail(kEInval, "dispatch_pack: null pointer");
    char *dst = static_cast<char *>(packed);
    for (int64_t r = 0; r < rows; ++r) {
        selected[r] = ids[r];
        coeff[r] = 1.0f;
        std::memcpy(dst + r * row_bytes, row, static_cast<size_t>(row_bytes));
    }
    *count = static_cast<int32_t>(rows);
    return kOk;
}
