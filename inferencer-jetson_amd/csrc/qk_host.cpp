// qk_host.cpp - status codes, thread-local error text, argument validation
// and cached device properties shared by every entry point of libqk.so.
#include "qk_internal.h"

#include <mutex>
#include <vector>

namespace qk {

namespace {
thread_local std::string g_last_error;
}

int fail(int status, const std::string &message) {
    g_last_error = message;
    return status;
}

int ok() {
    g_last_error.clear();
    return QK_OK;
}

int launch_status(const char *where) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(QK_ERR_DEVICE, std::string(where) + ": " + hipGetErrorString(err));
    return ok();
}

int block_bytes(int type) {
    return type == QK_TYPE_Q4_K ? 144 : type == QK_TYPE_Q6_K || type == QK_TYPE_Q6_K_SPLIT ? 210 : 0;
}

int64_t row_bytes(int type, int nb) {
    const int64_t raw = static_cast<int64_t>(nb) * block_bytes(type);
    return type == QK_TYPE_Q6_K_SPLIT ? (raw + 15) / 16 * 16 : raw;
}

int check_weights(const char *where, int type, const void *w, int cols, int rows) {
    // Mirrors FastGPU::matvec's checks (inferencer.cu:1157-1158) and the
    // quantized shape rule (inferencer.cu:254-256), plus the alignment the
    // GGUF data section guarantees (inferencer.cu:270-272).
    if (!block_bytes(type))
        return fail(QK_ERR_TYPE, std::string(where) + ": unsupported storage type " + std::to_string(type));
    if (cols <= 0 || cols % 256 != 0 || rows < 1)
        return fail(QK_ERR_SHAPE, std::string(where) + ": unexpected quantized matrix shape " +
                                      std::to_string(cols) + " x " + std::to_string(rows));
    if (!w) return fail(QK_ERR_INVALID_ARG, std::string(where) + ": null weight pointer");
    if (!aligned(w, 16)) return fail(QK_ERR_ALIGN, std::string(where) + ": weight base not 16-byte aligned");
    return QK_OK;
}

const DeviceInfo &device_info() {
    // A fixed table: the references handed out stay valid.
    constexpr int kDevicesMax = 64;
    static std::mutex mutex;
    static DeviceInfo cache[kDevicesMax];
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kDevicesMax) device = 0;
    std::lock_guard<std::mutex> lock(mutex);
    DeviceInfo &info = cache[device];
    if (info.device < 0) {
        hipDeviceProp_t prop{};
        if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
            info.cus = prop.multiProcessorCount;
            info.max_threads = prop.maxThreadsPerBlock;
        } else {
            info.cus = 256;
        }
        info.device = device;
    }
    return info;
}


// Resident workgroups of a kernel on the current device, cached per
// (device, kernel, block size, LDS bytes): the occupancy query costs
// microseconds of host time, more than a small GEMV runs.
int resident_blocks(const void *kernel, int block, size_t lds) {
    struct Key {
        int device;
        const void *kernel;
        int block;
        size_t lds;
        bool operator==(const Key &o) const {
            return device == o.device && kernel == o.kernel && block == o.block && lds == o.lds;
        }
    };
    static std::mutex mutex;
    static std::vector<std::pair<Key, int>> cache;
    const Key key{device_info().device, kernel, block, lds};
    {
        std::lock_guard<std::mutex> lock(mutex);
        for (const auto &e : cache)
            if (e.first == key) return e.second;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int total = per_cu * device_info().cus;
    std::lock_guard<std::mutex> lock(mutex);
    cache.emplace_back(key, total);
    return total;
}

}  // namespace qk

extern "C" {

const char *qk_status_string(int status) {
    switch (status) {
        case QK_OK: return "ok";
        case QK_ERR_INVALID_ARG: return "invalid argument";
        case QK_ERR_SHAPE: return "unexpected quantized matrix shape";
        case QK_ERR_TYPE: return "unsupported storage type";
        case QK_ERR_ALIGN: return "misaligned pointer or leading dimension";
        case QK_ERR_DEVICE: return "HIP device error";
        case QK_ERR_LIMIT: return "size beyond kernel limits";
        case QK_ERR_FORMAT: return "malformed or unsupported GGUF file";
        case QK_ERR_IO: return "file cannot be opened or mapped";
        default: return "unknown status";
    }
}

const char *qk_last_error(void) { return qk::g_last_error.c_str(); }

int qk_block_bytes(int type) { return qk::block_bytes(type); }

int64_t qk_tensor_bytes(int type, int64_t cols, int64_t rows) {
    int bpb = qk::block_bytes(type);
    if (!bpb || cols <= 0 || cols % 256 || rows < 0 || cols / 256 > (1 << 24)) return -1;
    return qk::row_bytes(type, static_cast<int>(cols / 256)) * rows;
}

}  // extern "C"
