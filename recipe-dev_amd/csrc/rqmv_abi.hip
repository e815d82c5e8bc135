// C-ABI entry points of librqmv (declared in include/rqmv.h).
#include <stdlib.h>

#include <memory>
#include <mutex>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/rqmv.h"
#include "act.h"
#include "kernels.h"
#include "decode.h"
#include "gguf.h"
#include "moe.h"
#include "repack.h"
#include "requant.h"

struct rqmv_weight {
    int fmt;
    int64_t rows;     // rows of one matrix (of one expert)
    int64_t cols;
    int64_t experts;  // 1 for a plain weight
    int64_t row_bytes;
    int64_t nch;
    uint8_t* dev;
    size_t dev_bytes;
    int device;
    bool glu = false;  // rows are (gate, up) pairs (rqmv_glu_weight_create)
};

struct rqmv_gguf {
    std::unique_ptr<rq::GgufFile> file;
};

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(RQMV_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

struct DeviceInfo {
    bool ready = false;
    int cus = 0;
    size_t lds_limit = 0;
    void* scratch = nullptr;  // this device's copy of `scratch` (rqmv_moe_batch_noalloc)
};

// The workspace of rqmv_moe_batch_noalloc, for callers that cannot allocate:
// one copy per GPU, held until the process ends. Host code never passes the
// array's name to a kernel (on the host it names no device address); it uses
// each device's address from hipGetSymbolAddress (DeviceInfo::scratch).
constexpr size_t kMoeScratchBytes = size_t(1) << 20;
__device__ __align__(256) uint8_t scratch[kMoeScratchBytes];

std::mutex g_mutex;
DeviceInfo g_devices[64];

int current_device(DeviceInfo* out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(RQMV_ESTATE, "device index out of range");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_devices[dev].ready) return fail(RQMV_ESTATE, "rqmv_init was not called for device " + std::to_string(dev));
    *out = g_devices[dev];
    return dev;
}

rq::Planes planes_of(const rqmv_weight* w, int64_t first_row) {
    rq::Planes P;
    P.base = w->dev + first_row * w->row_bytes;
    P.row_bytes = w->row_bytes;
    P.nch = (int)w->nch;
    P.bytes = (uint32_t)(w->dev_bytes - (size_t)(first_row * w->row_bytes));
    return P;
}

int env_int(const char* name, int fallback) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : fallback;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

int create(int format, int64_t experts, int64_t rows, int64_t cols, const void* bytes, size_t nbytes, rqmv_weight** out) {
    if (!out) return fail(RQMV_EINVAL, "out is NULL");
    *out = nullptr;
    if (!rq::format_supported(format) || format == rq::F32) return fail(RQMV_EINVAL, "unsupported format " + std::to_string(format));
    if (experts <= 0 || rows <= 0 || cols <= 0) return fail(RQMV_EINVAL, "shape must be positive");
    if (cols > rq::kMaxCols) return fail(RQMV_EINVAL, "cols too large");
    int64_t total_rows;
    if (__builtin_mul_overflow(experts, rows, &total_rows) || total_rows > rq::kMaxRows)
        return fail(RQMV_EINVAL, "experts x rows must stay below 2^31 rows");
    const int64_t want = rq::gguf_bytes(format, total_rows, cols);
    if (want < 0)
        return fail(RQMV_EINVAL, "cols is not a whole number of blocks for this format (a multiple of 32, and of "
                                 "256 for Q4_K/Q6_K and 64 for F16), or the shape's size overflows");
    if (!bytes || (size_t)want != nbytes)
        return fail(RQMV_EINVAL, "expected " + std::to_string(want) + " GGUF bytes, got " + std::to_string(nbytes));
    DeviceInfo info;
    int dev = current_device(&info);
    if (dev < 0) return dev;
    const int64_t layout = rq::layout_bytes(format, total_rows, cols);
    if (layout >= (int64_t)rq::kOobOffset)
        return fail(RQMV_EINVAL, "a weight's repacked bytes must stay below 4 GiB - 256 B; split the tensor");
    std::vector<uint8_t> host((size_t)layout);
    if (rq::repack(format, total_rows, cols, static_cast<const uint8_t*>(bytes), host.data()) != 0)
        return fail(RQMV_EINVAL, "repack failed");
    uint8_t* d = nullptr;
    hipError_t e = hipMalloc(&d, host.size());
    if (e != hipSuccess) return fail(RQMV_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    e = hipMemcpy(d, host.data(), host.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "hipMemcpy");
    }
    rqmv_weight* w = new rqmv_weight;
    w->fmt = format;
    w->rows = rows;
    w->cols = cols;
    w->experts = experts;
    w->row_bytes = rq::row_bytes(format, cols);
    w->nch = rq::chunks_per_row(format, cols);
    w->dev = d;
    w->dev_bytes = host.size();
    w->device = dev;
    *out = w;
    return RQMV_OK;
}

int check_launch(const rqmv_weight* w, DeviceInfo* info) {
    if (!w) return fail(RQMV_EINVAL, "weight is NULL");
    int dev = current_device(info);
    if (dev < 0) return dev;
    if (dev != w->device) return fail(RQMV_ESTATE, "weight lives on another device than the current one");
    return RQMV_OK;
}

// Runs y = W x over rows [first_row, first_row + rows) of a weight, M rows of x
// at a time in blocks the VALU kernels take (8, 4, 2, 1; 16 for F16 weights)
// and LDS can hold.
int matvec_rows(const rqmv_weight* w, int64_t first_row, int64_t rows, const void* x, int xtype, int m, int64_t ldx,
                float* y, int64_t ldy, hipStream_t stream, const DeviceInfo& info, hipEvent_t ev0 = nullptr,
                hipEvent_t ev1 = nullptr, const rqmv_weight* extra_row = nullptr) {
    if (!x || !y) return fail(RQMV_EINVAL, "x or y is NULL");
    if (xtype != RQMV_DTYPE_F16 && xtype != RQMV_DTYPE_F32) return fail(RQMV_EINVAL, "x_dtype must be F16 or F32");
    if (m <= 0) return fail(RQMV_EINVAL, "m must be positive");
    const size_t esize = xtype == RQMV_DTYPE_F16 ? 2 : 4;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (m > 1 && ((size_t)ldx * esize) % 16 != 0))
        return fail(RQMV_EINVAL, "x rows must start 16-byte aligned (x and ldx * element size)");
    rq::MvParams p;
    p.P = planes_of(w, first_row);
    p.P2 = p.P;
    p.split = rows;
    if (extra_row) {  // one more output row from a second F16 weight of the same width
        if (w->fmt != rq::F16 || extra_row->fmt != rq::F16 || extra_row->cols != w->cols)
            return fail(RQMV_EINVAL, "an extra row needs two F16 weights of one width");
        p.P2 = planes_of(extra_row, 0);
        rows += 1;
    }
    if (m > 1 && (ldx < w->cols || ldy < rows)) return fail(RQMV_EINVAL, "ldx < cols or ldy < rows");
    p.rows = rows;
    p.K = (int)w->cols;
    p.ldx = ldx;
    p.ldy = ldy;
    int done = 0;
    // Three or more activation rows of a quantized weight go to the matrix
    // cores, up to 32 rows per launch (at two the vector kernels are as fast),
    // except three or four rows of Q8_0 and three of Q6_K in the
    // two-waves-per-tile form, which measured faster (Q8_0 5120x5120 at four
    // rows 16.2 -> 13.6 us, Q6_K 5120->25600 at three 38.8 -> 33.6).
    const int mfma_min = env_int("RQMV_MFMA_MIN", 3);
    const bool k2_few = (m == 3 || m == 4) && (w->fmt == rq::Q8_0 || w->fmt == rq::Q6_K) && env_int("RQMV_K2_FEW", 1) &&
                        rq::k2_takes(w->fmt, rows, w->cols, m, xtype, info.cus);
    if (w->fmt != rq::F16 && m >= mfma_min && !k2_few) {
        while (done < m) {
            const int mb = m - done > 32 ? 32 : m - done;
            if (rq::mfma_lds_bytes(w->fmt, xtype, mb, rows, info.cus) > info.lds_limit)
                return fail(RQMV_EINVAL, "LDS too small");
            p.x = static_cast<const char*>(x) + (size_t)done * (size_t)ldx * esize;
            p.y = y + (int64_t)done * ldy;
            const bool first = done == 0, last = done + mb >= m;
            hipError_t e = rq::launch_matvec_mfma(w->fmt, xtype, mb, p, info.cus, stream, first ? ev0 : nullptr,
                                                  last ? ev1 : nullptr);
            if (e != hipSuccess) return hip_fail(e, "matvec launch");
            done += mb;
        }
        return RQMV_OK;
    }
    while (done < m) {
        int mb = w->fmt == rq::F16 ? 16 : 8;  // F16 (routers) takes sixteen rows per launch
        while (mb > m - done) mb >>= 1;
        if (k2_few && done == 0) mb = m;  // (three or four rows in one launch)
        while (mb > 1 && rq::matvec_lds_bytes(w->fmt, xtype, mb, (int)w->cols) > info.lds_limit) mb >>= 1;
        if (rq::matvec_lds_bytes(w->fmt, xtype, mb, (int)w->cols) > info.lds_limit)
            return fail(RQMV_EINVAL, "cols too large for one LDS stage");
        p.x = static_cast<const char*>(x) + (size_t)done * (size_t)ldx * esize;
        p.y = y + (int64_t)done * ldy;
        rq::LaunchShape s = rq::plan_matvec(w->fmt, rows, w->cols, mb, xtype, info.cus);
        p.G = s.G;
        const bool first = done == 0, last = done + mb >= m;
        hipError_t e = hipSuccess;
        // (the burst form, for products of at most 20 MB, except where the
        // two-waves-per-tile form measured faster: Q8_0 4096x4096 with fp32 x
        // 6.36 -> 6.20 us; Q4_K 4096x4096 with fp16 x stays in the burst form,
        // 4.91 against 5.02)
        if (!extra_row && !(s.k2 && w->fmt == rq::Q8_0) &&
            rq::try_launch_burst(w->fmt, xtype, mb, p, info.cus, stream, first ? ev0 : nullptr, last ? ev1 : nullptr,
                                 &e)) {
            if (e != hipSuccess) return hip_fail(e, "matvec launch");
            done += mb;
            continue;
        }
        e = rq::launch_matvec(w->fmt, xtype, mb, p, s, stream, first ? ev0 : nullptr, last ? ev1 : nullptr);
        if (e != hipSuccess) return hip_fail(e, "matvec launch");
        done += mb;
    }
    return RQMV_OK;
}

}  // namespace

extern "C" {

int rqmv_init(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count || device >= 64) return fail(RQMV_EINVAL, "no such device");
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    int cus = 0, lds = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    e = hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_devices[device].scratch) {  // this device's address of the no-alloc workspace (with it current)
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        g_devices[device].scratch = ptr;
    }
    g_devices[device].cus = cus > 0 ? cus : 1;
    g_devices[device].lds_limit = lds > 0 ? (size_t)lds : 65536;
    g_devices[device].ready = true;
    g_error.clear();
    return RQMV_OK;
}

const char* rqmv_last_error(void) { return g_error.c_str(); }

int rqmv_weight_create(int format, int64_t rows, int64_t cols, const void* gguf_bytes, size_t nbytes, rqmv_weight** out) {
    return create(format, 1, rows, cols, gguf_bytes, nbytes, out);
}

int rqmv_expert_bank_create(int format, int64_t experts, int64_t rows, int64_t cols, const void* gguf_bytes,
                            size_t nbytes, rqmv_weight** out) {
    return create(format, experts, rows, cols, gguf_bytes, nbytes, out);
}

// The gfx950 row of recipe's capability table (recipe.rs:2646-2738): per
// compute format, the vector and matrix instructions this library runs it on.
namespace {
struct Capability {
    const char* format;
    const char* vector;
    const char* matrix;
};
const Capability kGfx950[] = {
    {"int4", nullptr, nullptr},
    {"int8", "v_dot4_i32_i8 on Q8 activation records (rqmv_matvec_int8)", nullptr},
    {"int16", nullptr, nullptr},
    {"int32", nullptr, nullptr},
    {"fp8", nullptr, nullptr},
    {"fp16",
     "v_dot8_i32_i4 / v_dot4_i32_i8 on exactly encoded activations, v_dot2_f32_f16 for F16 weights (rqmv_matvec)",
     "v_mfma_f32_16x16x32_f16 on exact fp16 weight codes (rqmv_matvec, M >= 3)"},
    {"fp32", "v_dot8_i32_i4 / v_dot4_i32_i8 on exactly encoded activations, fp32 fma for F16 weights (rqmv_matvec)",
     "v_mfma_f32_16x16x32_f16 on exact fp16 weight codes, activations as fp16 high and low parts (rqmv_matvec, M >= 3)"},
    {"fp64", nullptr, nullptr},
    {"bf16", nullptr, nullptr},
    {"tf32", nullptr, nullptr},
};
}  // namespace

int rqmv_capability(const char* format, const char** vector, const char** matrix) {
    if (!format || !vector || !matrix) return fail(RQMV_EINVAL, "capability: NULL argument");
    *vector = nullptr;
    *matrix = nullptr;
    for (const Capability& c : kGfx950) {
        if (std::strcmp(c.format, format) != 0) continue;
        if (!c.vector && !c.matrix) {
            std::string vectors, matrices;
            for (const Capability& e : kGfx950) {
                if (e.vector) vectors += std::string(vectors.empty() ? "" : " ") + e.format;
                if (e.matrix) matrices += std::string(matrices.empty() ? "" : " ") + e.format;
            }
            return fail(RQMV_EINVAL, std::string("gfx950 has no ") + format + " instruction. Vector: " +
                                         (vectors.empty() ? "none" : vectors) + ". Matrix: " +
                                         (matrices.empty() ? "none" : matrices) + ".");
        }
        *vector = c.vector;
        *matrix = c.matrix;
        return RQMV_OK;
    }
    return fail(RQMV_EINVAL, std::string("gfx950 has no ") + format + " capability entry");
}

int rqmv_requantize_q8_0_host(int format, int64_t rows, int64_t cols, const void* gguf_bytes, size_t nbytes,
                              void* out) {
    if (!gguf_bytes || !out) return fail(RQMV_EINVAL, "requantize: NULL argument");
    if (!rq::requantizable_to_q8_0(format)) return fail(RQMV_EINVAL, "requantize: the source must be F16, Q8_0, Q4_0 or Q6_K");
    const int64_t want = rq::gguf_bytes(format, rows, cols);
    if (want < 0 || cols % 32 != 0) return fail(RQMV_EINVAL, "requantize: cols is not a whole number of blocks");
    if ((size_t)want != nbytes)
        return fail(RQMV_EINVAL, "requantize: expected " + std::to_string(want) + " GGUF bytes, got " + std::to_string(nbytes));
    if (rq::requantize_q8_0(format, rows, cols, static_cast<const uint8_t*>(gguf_bytes), static_cast<uint8_t*>(out)) != 0)
        return fail(RQMV_EINVAL, "requantize failed");
    return RQMV_OK;
}

int rqmv_weight_create_int8(int format, int64_t experts, int64_t rows, int64_t cols, const void* gguf_bytes,
                            size_t nbytes, rqmv_weight** out) {
    if (!out) return fail(RQMV_EINVAL, "out is NULL");
    *out = nullptr;
    if (format == rq::Q4_K || format == rq::Q8_0) return create(format, experts, rows, cols, gguf_bytes, nbytes, out);
    if (experts <= 0 || rows <= 0) return fail(RQMV_EINVAL, "shape must be positive");
    int64_t total;
    if (__builtin_mul_overflow(experts, rows, &total) || total > rq::kMaxRows)
        return fail(RQMV_EINVAL, "experts x rows must stay below 2^31 rows");
    std::vector<uint8_t> q8;
    const int64_t q8_bytes = rq::gguf_bytes(rq::Q8_0, total, cols);
    if (q8_bytes < 0) return fail(RQMV_EINVAL, "cols is not a whole number of Q8_0 blocks");
    q8.resize((size_t)q8_bytes);
    const int rc = rqmv_requantize_q8_0_host(format, total, cols, gguf_bytes, nbytes, q8.data());
    if (rc != RQMV_OK) return rc;
    return create(rq::Q8_0, experts, rows, cols, q8.data(), q8.size(), out);
}

int rqmv_glu_weight_create(int format, int64_t rows, int64_t cols, const void* gate_gguf, const void* up_gguf,
                           size_t nbytes_each, rqmv_weight** out) {
    if (!gate_gguf || !up_gguf || !out) return fail(RQMV_EINVAL, "NULL argument");
    if (format == rq::F16 || format == rq::F32) return fail(RQMV_EINVAL, "a GLU pair must be quantized");
    const int64_t want = rq::gguf_bytes(format, rows, cols);
    if (rows <= 0 || want < 0 || (size_t)want != nbytes_each)
        return fail(RQMV_EINVAL, "gate and up must each hold rows x cols GGUF blocks");
    if (rows > rq::kMaxRows / 2) return fail(RQMV_EINVAL, "2 x rows must stay below 2^31 rows");
    // rows interleaved: row 2i = gate row i, row 2i + 1 = up row i
    const size_t rb = (size_t)want / (size_t)rows;
    std::vector<uint8_t> pairs(2 * (size_t)want);
    const uint8_t* g = static_cast<const uint8_t*>(gate_gguf);
    const uint8_t* u = static_cast<const uint8_t*>(up_gguf);
    for (int64_t i = 0; i < rows; ++i) {
        std::memcpy(pairs.data() + (2 * i) * rb, g + i * rb, rb);
        std::memcpy(pairs.data() + (2 * i + 1) * rb, u + i * rb, rb);
    }
    int rc = create(format, 1, 2 * rows, cols, pairs.data(), pairs.size(), out);
    if (rc == RQMV_OK) (*out)->glu = true;
    return rc;
}

int rqmv_weight_destroy(rqmv_weight* w) {
    if (!w) return RQMV_OK;
    hipError_t e = hipFree(w->dev);
    delete w;
    if (e != hipSuccess) return hip_fail(e, "hipFree");
    return RQMV_OK;
}

int rqmv_weight_info(const rqmv_weight* w, int* format, int64_t* rows, int64_t* cols, int64_t* experts,
                     size_t* device_bytes) {
    if (!w) return fail(RQMV_EINVAL, "weight is NULL");
    if (format) *format = w->fmt;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (experts) *experts = w->experts;
    if (device_bytes) *device_bytes = w->dev_bytes;
    return RQMV_OK;
}

int rqmv_weight_unpack(const rqmv_weight* w, void* gguf_bytes, size_t nbytes) {
    if (!w || !gguf_bytes) return fail(RQMV_EINVAL, "NULL argument");
    const int64_t total_rows = w->rows * w->experts;
    const int64_t want = rq::gguf_bytes(w->fmt, total_rows, w->cols);
    if ((size_t)want != nbytes) return fail(RQMV_EINVAL, "nbytes does not match the GGUF size");
    std::vector<uint8_t> host(w->dev_bytes);
    hipError_t e = hipMemcpy(host.data(), w->dev, w->dev_bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy");
    if (rq::unpack(w->fmt, total_rows, w->cols, host.data(), static_cast<uint8_t*>(gguf_bytes)) != 0)
        return fail(RQMV_EINVAL, "unpack failed");
    return RQMV_OK;
}

int rqmv_weight_dequantize(const rqmv_weight* w, float* out_dev, void* stream) {
    DeviceInfo info;
    int rc = check_launch(w, &info);
    if (rc != RQMV_OK) return rc;
    if (!out_dev) return fail(RQMV_EINVAL, "out is NULL");
    hipError_t e = rq::launch_dequant(w->fmt, planes_of(w, 0), w->rows * w->experts, (int)w->cols, out_dev,
                                      static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return RQMV_OK;
}

int rqmv_matvec(const rqmv_weight* w, const void* x_dev, int x_dtype, int m, int64_t ldx, float* y_dev, int64_t ldy,
                void* stream) {
    DeviceInfo info;
    int rc = check_launch(w, &info);
    if (rc != RQMV_OK) return rc;
    return matvec_rows(w, 0, w->rows * w->experts, x_dev, x_dtype, m, ldx, y_dev, ldy,
                       static_cast<hipStream_t>(stream), info);
}

int rqmv_matvec_timed(const rqmv_weight* w, const void* x_dev, int x_dtype, int m, int64_t ldx, float* y_dev,
                      int64_t ldy, void* stream, void* start_event, void* stop_event) {
    DeviceInfo info;
    int rc = check_launch(w, &info);
    if (rc != RQMV_OK) return rc;
    return matvec_rows(w, 0, w->rows * w->experts, x_dev, x_dtype, m, ldx, y_dev, ldy,
                       static_cast<hipStream_t>(stream), info, static_cast<hipEvent_t>(start_event),
                       static_cast<hipEvent_t>(stop_event));
}

int rqmv_matvec_fused(const rqmv_weight* w, const float* x_dev, float* y_dev, const rqmv_fusion* f, void* stream) {
    DeviceInfo info;
    int rc = check_launch(w, &info);
    if (rc != RQMV_OK) return rc;
    if (!f || !x_dev) return fail(RQMV_EINVAL, "fused: NULL argument");
    if (w->fmt == rq::F16 || w->experts != 1) return fail(RQMV_EINVAL, "fused: a plain quantized weight is required");
    if (reinterpret_cast<uintptr_t>(x_dev) % 16 != 0) return fail(RQMV_EINVAL, "fused: x must be 16-byte aligned");
    rq::MvParams p;
    p.P = planes_of(w, 0);
    p.P2 = p.P;
    p.rows = w->rows;
    p.split = p.rows;
    p.K = (int)w->cols;
    p.x = x_dev;
    p.ldx = w->cols;
    p.y = y_dev;
    p.ldy = w->rows;
    if (rq::matvec_lds_bytes(w->fmt, RQMV_DTYPE_F32, 1, (int)w->cols) > info.lds_limit)
        return fail(RQMV_EINVAL, "fused: cols too large for one LDS stage");
    if (!y_dev) return fail(RQMV_EINVAL, "fused: y is NULL");
    const rq::LaunchShape s = rq::plan_fused(w->fmt, w->rows, w->cols, info.cus, f->epilogue == RQMV_EPI_GLU,
                                             f->norm_weight != nullptr);
    p.G = s.G;
    switch (f->epilogue) {
        case RQMV_EPI_PLAIN: break;
        case RQMV_EPI_GLU:
            if (!w->glu) return fail(RQMV_EINVAL, "fused: the GLU epilogue needs a GLU weight");
            p.epi = rq::kEpiGlu;
            break;
        default: return fail(RQMV_EINVAL, "fused: unknown epilogue");
    }
    if (f->norm_weight) {
        if (!(f->eps >= 0.f)) return fail(RQMV_EINVAL, "fused: eps must be >= 0");
        if (((uintptr_t)f->norm_weight | (uintptr_t)f->delta | (uintptr_t)f->x_out) & 15)
            return fail(RQMV_EINVAL, "fused: norm weight, delta and x_out must be 16-byte aligned");
        if (f->x_out && (f->x_out == x_dev || f->x_out == f->delta))
            return fail(RQMV_EINVAL, "fused: x_out must be a buffer other than x and delta");
        p.norm_w = f->norm_weight;
        p.delta = f->delta;
        p.x_out = f->x_out;
        p.eps = f->eps;
    } else if (f->delta || f->x_out) {
        return fail(RQMV_EINVAL, "fused: delta and x_out come with the norm prologue");
    }
    hipError_t e = rq::launch_matvec_fused(w->fmt, p, s, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "fused matvec launch");
}

int rqmv_expert_matvec(const rqmv_weight* bank, int64_t expert, const void* x_dev, int x_dtype, int m, int64_t ldx,
                       float* y_dev, int64_t ldy, void* stream) {
    DeviceInfo info;
    int rc = check_launch(bank, &info);
    if (rc != RQMV_OK) return rc;
    if (expert < 0 || expert >= bank->experts) return fail(RQMV_EINVAL, "expert index out of range");
    return matvec_rows(bank, expert * bank->rows, bank->rows, x_dev, x_dtype, m, ldx, y_dev, ldy,
                       static_cast<hipStream_t>(stream), info);
}

}  // extern "C"

namespace {

// Validates the gguf_moe operands (Builder::expert_planes shape rules,
// recipe.rs:18274-18316) and fills the kernel-side description.
int moe_dims(const rqmv_moe_params* p, rq::MoeDims* d, const DeviceInfo& info) {
    (void)info;
    if (!p) return fail(RQMV_EINVAL, "params is NULL");
    if (!p->router || !p->gate_exps || !p->up_exps || !p->down_exps) return fail(RQMV_EINVAL, "router and banks are required");
    const rqmv_weight *r = p->router, *g = p->gate_exps, *u = p->up_exps, *dn = p->down_exps;
    if (r->fmt != rq::F16 || r->experts != 1) return fail(RQMV_EINVAL, "router must be a plain F16 weight");
    const int64_t E = r->rows, D = r->cols;
    if (g->fmt != u->fmt || g->fmt != dn->fmt) return fail(RQMV_EINVAL, "gate, up and down banks must share a format");
    if (g->fmt == rq::F16) return fail(RQMV_EINVAL, "expert banks must be quantized");
    if (g->experts != E || u->experts != E || dn->experts != E) return fail(RQMV_EINVAL, "bank expert count differs from the router rows");
    const int64_t H = g->rows;
    if (g->cols != D || u->cols != D || u->rows != H) return fail(RQMV_EINVAL, "gate/up banks must be experts x hidden x d_model");
    if (dn->rows != D || dn->cols != H) return fail(RQMV_EINVAL, "down bank must be experts x d_model x hidden");
    const int cw = rq::format_info(g->fmt).chunk_values;
    if (H % cw != 0 || D % cw != 0) return fail(RQMV_EINVAL, "hidden and d_model must be multiples of the format's chunk");
    if (p->top_k < 1 || p->top_k > 64 || p->top_k > E) return fail(RQMV_EINVAL, "top_k must be in 1..min(64, experts)");
    if (E > 2048) return fail(RQMV_EINVAL, "at most 2048 experts");
    if (p->scoring != RQMV_SCORE_SOFTMAX && p->scoring != RQMV_SCORE_SIGMOID) return fail(RQMV_EINVAL, "bad scoring");
    if (!rq::act_known(p->activation) || !rq::act_known(p->shared_gate_activation))
        return fail(RQMV_EINVAL, "unknown activation code (rqmv_activation)");
    // Scale's constant and PReLU's slope must be finite (lower_activation's
    // Scale arm, recipe.rs:22717-22721)
    const bool uses_factor = p->activation == rq::kActScale || p->activation == rq::kActPrelu ||
                             p->shared_gate_activation == rq::kActScale || p->shared_gate_activation == rq::kActPrelu;
    if (uses_factor && !(p->activation_factor - p->activation_factor == 0.f))
        return fail(RQMV_EINVAL, "scale factor must be finite");
    if (!(p->scale == p->scale) || p->scale - p->scale != 0.f) return fail(RQMV_EINVAL, "moe routed scale must be finite");
    if (reinterpret_cast<uintptr_t>(p->selection_bias) % 4 != 0)
        return fail(RQMV_EINVAL, "selection_bias must be 4-byte aligned");
    int64_t HS = 0;
    const bool any_shared = p->gate_shexp || p->up_shexp || p->down_shexp;
    if (any_shared) {
        const rqmv_weight *gs = p->gate_shexp, *us = p->up_shexp, *ds = p->down_shexp;
        if (!gs || !us || !ds) return fail(RQMV_EINVAL, "shared expert needs gate, up and down");
        if (gs->fmt != g->fmt || us->fmt != g->fmt || ds->fmt != g->fmt) return fail(RQMV_EINVAL, "shared expert format differs from the banks");
        if (gs->experts != 1 || us->experts != 1 || ds->experts != 1) return fail(RQMV_EINVAL, "shared expert weights must be plain");
        HS = gs->rows;
        if (gs->cols != D || us->cols != D || us->rows != HS || ds->rows != D || ds->cols != HS)
            return fail(RQMV_EINVAL, "shared expert shapes must be hidden_shared x d_model and d_model x hidden_shared");
        if (HS % cw != 0) return fail(RQMV_EINVAL, "hidden_shared must be a multiple of the format's chunk");
        if (p->shared_gate_inp) {
            const rqmv_weight* sg = p->shared_gate_inp;
            if (sg->fmt != rq::F16 || sg->rows != 1 || sg->cols != D || sg->experts != 1)
                return fail(RQMV_EINVAL, "shared_gate_inp must be a 1 x d_model F16 weight");
        }
    } else if (p->shared_gate_inp) {
        return fail(RQMV_EINVAL, "shared_gate_inp given without a shared expert");
    }
    d->d_model = (int)D;
    d->experts = (int)E;
    d->top = p->top_k;
    d->hidden = (int)H;
    d->hidden_shared = (int)HS;
    d->scoring = p->scoring;
    d->renormalize = p->renormalize ? 1 : 0;
    d->shared_gated = p->shared_gate_inp ? 1 : 0;
    d->scale = p->scale;
    d->activation = p->activation;
    d->shared_gate_act = p->shared_gate_activation;
    d->act_factor = p->activation_factor;
    d->sel_bias = p->selection_bias;
    return RQMV_OK;
}

rq::MoeBank bank_of(const rqmv_weight* w) {
    rq::MoeBank b;
    if (!w) {
        b.P = rq::Planes{nullptr, 0, 0, 0};
        b.rows = 0;
        return b;
    }
    b.P = planes_of(w, 0);
    b.rows = w->rows;
    return b;
}

}  // namespace

extern "C" {

int rqmv_moe_workspace_size(const rqmv_moe_params* params, size_t* bytes) {
    DeviceInfo info;
    if (!bytes) return fail(RQMV_EINVAL, "bytes is NULL");
    rq::MoeDims d;
    int rc = moe_dims(params, &d, info);
    if (rc != RQMV_OK) return rc;
    *bytes = rq::moe_workspace_bytes(d);
    return RQMV_OK;
}

int rqmv_moe_batch(const rqmv_moe_params* params, const void* x_dev, int x_dtype, int m, int64_t ldx, float* y_dev,
                   int64_t ldy, float* route_dev, void* workspace, size_t workspace_bytes, void* stream) {
    DeviceInfo info;
    int rc = check_launch(params ? params->router : nullptr, &info);
    if (rc != RQMV_OK) return rc;
    rq::MoeDims d;
    rc = moe_dims(params, &d, info);
    if (rc != RQMV_OK) return rc;
    if (!x_dev || !y_dev || !workspace) return fail(RQMV_EINVAL, "x, y and workspace are required");
    if (x_dtype != RQMV_DTYPE_F16 && x_dtype != RQMV_DTYPE_F32) return fail(RQMV_EINVAL, "x_dtype must be F16 or F32");
    if (m < 1 || m > 65535) return fail(RQMV_EINVAL, "moe: m must be in 1..65535");
    if (ldx < d.d_model || ldy < d.d_model) return fail(RQMV_EINVAL, "moe: ldx and ldy must be at least d_model");
    const size_t per = rq::moe_workspace_bytes(d);
    if (workspace_bytes / (size_t)m < per) return fail(RQMV_EINVAL, "workspace too small");
    const int xb = x_dtype == RQMV_DTYPE_F16 ? 2 : 4;
    if (reinterpret_cast<uintptr_t>(x_dev) % 16 != 0 || (ldx * xb) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(RQMV_EINVAL, "x rows must be 16-byte and workspace 256-byte aligned");
    for (const rqmv_weight* w : {params->gate_exps, params->up_exps, params->down_exps, params->shared_gate_inp,
                                 params->gate_shexp, params->up_shexp, params->down_shexp})
        if (w && w->device != params->router->device) return fail(RQMV_ESTATE, "moe weights live on different devices");
    hipStream_t s = static_cast<hipStream_t>(stream);
    rq::MoeWorkspace ws = rq::moe_workspace(workspace, d);
    rq::MoeBatch b;
    b.m = m;
    b.x_stride = ldx * xb;
    b.ws_stride = (int64_t)per;
    b.y_stride = ldy;
    b.route_stride = d.experts;
    // router logits and the shared expert's gate logit of every position: one
    // F16 product over both weights (experts + 1 rows), position p's into its
    // own workspace
    rc = matvec_rows(params->router, 0, d.experts, x_dev, x_dtype, m, ldx, ws.logits, (int64_t)(per / sizeof(float)), s,
                     info, nullptr, nullptr, params->shared_gate_inp);
    if (rc != RQMV_OK) return rc;
    const int fmt = params->gate_exps->fmt;
    hipError_t e = rq::launch_moe_glu(fmt, x_dtype, d, bank_of(params->gate_exps), bank_of(params->up_exps),
                                      bank_of(params->gate_shexp), bank_of(params->up_shexp), x_dev, ws, route_dev, b,
                                      info.cus, s);
    if (e != hipSuccess) return hip_fail(e, "moe routing and gate/up launch");
    e = rq::launch_moe_down(fmt, d, bank_of(params->down_exps), bank_of(params->down_shexp), ws, y_dev, b, info.cus, s);
    if (e != hipSuccess) return hip_fail(e, "moe down launch");
    return RQMV_OK;
}

int rqmv_moe_batch_noalloc(const rqmv_moe_params* params, const void* x_dev, int x_dtype, int m, int64_t ldx,
                           float* y_dev, int64_t ldy, float* route_dev, void* stream) {
    DeviceInfo info;
    int rc = check_launch(params ? params->router : nullptr, &info);
    if (rc != RQMV_OK) return rc;
    rq::MoeDims d;
    rc = moe_dims(params, &d, info);
    if (rc != RQMV_OK) return rc;
    if (m < 1 || m > 65535) return fail(RQMV_EINVAL, "moe: m must be in 1..65535");
    const size_t per = rq::moe_workspace_bytes(d);
    if (per * (size_t)m > kMoeScratchBytes)
        return fail(RQMV_EINVAL, "moe_batch_noalloc: " + std::to_string(m) + " position(s) need " +
                                     std::to_string(per * (size_t)m) + " bytes of workspace, beyond its " +
                                     std::to_string(kMoeScratchBytes) + "-byte scratch; use rqmv_moe_batch");
    // every workspace byte is written before it is read (logits, routing, slot
    // activations), so nothing needs clearing between calls
    return rqmv_moe_batch(params, x_dev, x_dtype, m, ldx, y_dev, ldy, route_dev, info.scratch, kMoeScratchBytes,
                          stream);
}

int rqmv_moe(const rqmv_moe_params* params, const void* x_dev, int x_dtype, float* y_dev, float* route_dev,
             void* workspace, size_t workspace_bytes, void* stream) {
    const int64_t d_model = params && params->router ? params->router->cols : 0;
    return rqmv_moe_batch(params, x_dev, x_dtype, 1, d_model, y_dev, d_model, route_dev, workspace, workspace_bytes,
                          stream);
}

int rqmv_add_rmsnorm(float* x, const float* delta, const float* weight, int n, float eps, float* out, void* stream) {
    if (!x || !weight || !out || n <= 0) return fail(RQMV_EINVAL, "add_rmsnorm: bad arguments");
    hipError_t e = rq::launch_add_rmsnorm(x, delta, weight, n, eps, out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "add_rmsnorm launch");
}

int rqmv_rope_kv(float* qkv, const int* pos, int q_heads, int kv_heads, int head_dim, double base, void* k_cache,
                 void* v_cache, int max_ctx, void* stream) {
    if (!qkv || !pos || !k_cache || !v_cache || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 ||
        max_ctx <= 0 || !(base > 1.0))
        return fail(RQMV_EINVAL, "rope_kv: bad arguments");
    hipError_t e = rq::launch_rope_kv(qkv, pos, q_heads, kv_heads, head_dim, base, static_cast<__half*>(k_cache),
                                      static_cast<__half*>(v_cache), max_ctx, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "rope_kv launch");
}

int rqmv_attention_workspace_size(int q_heads, int kv_heads, int head_dim, int max_ctx, size_t* bytes) {
    if (q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || max_ctx <= 0 || !bytes)
        return fail(RQMV_EINVAL, "attention: bad arguments");
    *bytes = rq::attention_workspace_bytes(q_heads, head_dim, max_ctx);
    return RQMV_OK;
}

int rqmv_attention(const float* q, const void* k_cache, const void* v_cache, const int* pos, int q_heads, int kv_heads,
                   int head_dim, int max_ctx, void* workspace, size_t workspace_bytes, float* out, void* stream) {
    if (!q || !k_cache || !v_cache || !pos || !workspace || !out || q_heads <= 0 || kv_heads <= 0 || max_ctx <= 0)
        return fail(RQMV_EINVAL, "attention: bad arguments");
    if (q_heads % kv_heads || q_heads / kv_heads > 8 || (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
        max_ctx > 65536)
        return fail(RQMV_EINVAL,
                    "attention: q_heads must be 1..8 x kv_heads, head_dim 64, 128 or 256, max_ctx at most 65536");
    if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out | (uintptr_t)workspace) & 15)
        return fail(RQMV_EINVAL, "attention: q, caches, workspace and out must be 16-byte aligned");
    if (workspace_bytes < rq::attention_workspace_bytes(q_heads, head_dim, max_ctx))
        return fail(RQMV_EINVAL, "attention: workspace too small");
    hipError_t e = rq::launch_attention(q, static_cast<const __half*>(k_cache), static_cast<const __half*>(v_cache), pos,
                                        q_heads, kv_heads, head_dim, max_ctx, workspace, out,
                                        static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "attention launch");
}

int rqmv_rope_table(float* table, int head_dim, double base, int rows, void* stream) {
    if (!table || head_dim <= 0 || head_dim % 2 || rows <= 0 || !(base > 1.0))
        return fail(RQMV_EINVAL, "rope_table: bad arguments");
    hipError_t e = rq::launch_rope_table(reinterpret_cast<float2*>(table), head_dim, base, rows,
                                         static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "rope_table launch");
}

int rqmv_attention_rope(const float* qkv, const float* rope_table, void* k_cache, void* v_cache, const int* pos,
                        int q_heads, int kv_heads, int head_dim, int max_ctx, void* workspace, size_t workspace_bytes,
                        float* out, void* stream) {
    if (!qkv || !rope_table || !k_cache || !v_cache || !pos || !workspace || !out || q_heads <= 0 || kv_heads <= 0 ||
        max_ctx <= 0)
        return fail(RQMV_EINVAL, "attention_rope: bad arguments");
    if (q_heads % kv_heads || q_heads / kv_heads > 8 || (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
        max_ctx > 65536)
        return fail(RQMV_EINVAL,
                    "attention_rope: q_heads must be 1..8 x kv_heads, head_dim 64, 128 or 256, max_ctx at most 65536");
    if (((uintptr_t)qkv | (uintptr_t)rope_table | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out |
         (uintptr_t)workspace) & 15)
        return fail(RQMV_EINVAL, "attention_rope: pointers must be 16-byte aligned");
    if (workspace_bytes < rq::attention_workspace_bytes(q_heads, head_dim, max_ctx))
        return fail(RQMV_EINVAL, "attention_rope: workspace too small");
    hipError_t e = rq::launch_attention_rope(qkv, reinterpret_cast<const float2*>(rope_table),
                                             static_cast<__half*>(k_cache), static_cast<__half*>(v_cache), pos, q_heads,
                                             kv_heads, head_dim, max_ctx, workspace, out,
                                             static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "attention_rope launch");
}

int rqmv_silu_mul(const float* gate_up, int n, float* out, void* stream) {
    if (!gate_up || !out || n <= 0) return fail(RQMV_EINVAL, "silu_mul: bad arguments");
    hipError_t e = rq::launch_silu_mul(gate_up, n, out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "silu_mul launch");
}

int rqmv_argmax_workspace_size(size_t* bytes) {
    if (!bytes) return fail(RQMV_EINVAL, "argmax: NULL size");
    *bytes = rq::argmax_workspace_bytes();
    return RQMV_OK;
}

int rqmv_matvec_int8(const rqmv_weight* w, const float* x_dev, int m, int64_t ldx, float* y_dev, int64_t ldy,
                     int step, int flags, void* stream) {
    DeviceInfo info;
    int rc = check_launch(w, &info);
    if (rc != RQMV_OK) return rc;
    if (!x_dev || !y_dev) return fail(RQMV_EINVAL, "int8: x or y is NULL");
    if (w->fmt != rq::Q4_K && w->fmt != rq::Q6_K && w->fmt != rq::Q8_0 && w->fmt != rq::Q4_0)
        return fail(RQMV_EINVAL, "int8: a Q4_K, Q6_K, Q8_0 or Q4_0 weight is required");
    if (step != 32 && step != 256) return fail(RQMV_EINVAL, "int8: step must be 32 or 256");
    if (flags & ~RQMV_INT8_TAIL) return fail(RQMV_EINVAL, "int8: unknown flags");
    if (m <= 0 || m > 65535) return fail(RQMV_EINVAL, "int8: m must be in 1..65535");
    const int64_t rows = w->rows * w->experts;
    if (ldx < w->cols || ldy < rows) return fail(RQMV_EINVAL, "int8: ldx < cols or ldy < rows");
    if (reinterpret_cast<uintptr_t>(x_dev) % 16 != 0 || ldx % 4 != 0)
        return fail(RQMV_EINVAL, "int8: x must be 16-byte aligned and ldx a multiple of 4");
    if (rq::int8_lds_bytes(w->cols) > info.lds_limit) return fail(RQMV_EINVAL, "int8: cols too large for the LDS records");
    hipError_t e = rq::launch_matvec_int8(w->fmt, planes_of(w, 0), rows, (int)w->cols, x_dev, m, ldx, y_dev, ldy, step,
                                          (flags & RQMV_INT8_TAIL) ? 1 : 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "int8 launch");
}

int rqmv_q8_records(const float* x_dev, int64_t k, int step, float* d_dev, int8_t* codes_dev, void* stream) {
    if (!x_dev || !d_dev || !codes_dev) return fail(RQMV_EINVAL, "q8_records: NULL argument");
    if (k <= 0 || k % 32 != 0 || k > (1 << 24)) return fail(RQMV_EINVAL, "q8_records: k must be a positive multiple of 32");
    if (reinterpret_cast<uintptr_t>(x_dev) % 16 != 0) return fail(RQMV_EINVAL, "q8_records: x must be 16-byte aligned");
    DeviceInfo info;
    const int dev = current_device(&info);
    if (dev < 0) return dev;
    if (rq::int8_lds_bytes(k) > info.lds_limit) return fail(RQMV_EINVAL, "q8_records: k too large for the LDS records");
    if (step != 32 && step != 256) return fail(RQMV_EINVAL, "q8_records: step must be 32 or 256");
    hipError_t e = rq::launch_q8_records(x_dev, (int)k, step, d_dev, codes_dev, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "q8_records launch");
}

int rqmv_argmax(const float* values, int n, int* out, void* workspace, size_t workspace_bytes, void* stream) {
    if (!values || !out || !workspace || n <= 0) return fail(RQMV_EINVAL, "argmax: bad arguments");
    if (workspace_bytes < rq::argmax_workspace_bytes()) return fail(RQMV_EINVAL, "argmax: workspace too small");
    hipError_t e = rq::launch_argmax(values, n, out, workspace, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "argmax launch");
}

int rqmv_embed_row(const float* table, int rows, int n, const int* token, float* out, void* stream) {
    if (!table || !token || !out || rows <= 0 || n <= 0) return fail(RQMV_EINVAL, "embed_row: bad arguments");
    hipError_t e = rq::launch_embed_row(table, rows, n, token, out, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "embed_row launch");
}

int rqmv_advance(int* pos, void* stream) {
    if (!pos) return fail(RQMV_EINVAL, "advance: NULL position");
    hipError_t e = rq::launch_advance(pos, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RQMV_OK : hip_fail(e, "advance launch");
}

// ------------------------------------------------------------ GGUF files ----

int rqmv_gguf_open(const char* path, rqmv_gguf** out) {
    if (!path || !out) return fail(RQMV_EINVAL, "gguf_open: NULL argument");
    *out = nullptr;
    std::string error;
    std::unique_ptr<rq::GgufFile> f = rq::gguf_open(path, &error);
    if (!f) return fail(RQMV_EINVAL, error);
    rqmv_gguf* g = new rqmv_gguf;
    g->file = std::move(f);
    *out = g;
    return RQMV_OK;
}

int rqmv_gguf_close(rqmv_gguf* g) {
    delete g;
    return RQMV_OK;
}

int rqmv_gguf_tensor_count(const rqmv_gguf* g, int64_t* count) {
    if (!g || !count) return fail(RQMV_EINVAL, "gguf: NULL argument");
    *count = (int64_t)g->file->tensors.size();
    return RQMV_OK;
}

int rqmv_gguf_tensor_info(const rqmv_gguf* g, int64_t index, const char** name, int* ggml_type, int* n_dims,
                          int64_t* dims, size_t* nbytes) {
    if (!g) return fail(RQMV_EINVAL, "gguf: NULL handle");
    if (index < 0 || index >= (int64_t)g->file->tensors.size()) return fail(RQMV_EINVAL, "gguf: tensor index out of range");
    const rq::GgufTensor& t = g->file->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = (int)t.type;
    if (n_dims) *n_dims = (int)t.shape.size();
    if (dims)
        for (size_t d = 0; d < t.shape.size(); ++d) dims[d] = (int64_t)t.shape[d];
    if (nbytes) *nbytes = (size_t)t.bytes;
    return RQMV_OK;
}

int rqmv_gguf_find_tensor(const rqmv_gguf* g, const char* name, int64_t* index) {
    if (!g || !name || !index) return fail(RQMV_EINVAL, "gguf: NULL argument");
    for (size_t k = 0; k < g->file->tensors.size(); ++k)
        if (g->file->tensors[k].name == name) {
            *index = (int64_t)k;
            return RQMV_OK;
        }
    return fail(RQMV_EINVAL, std::string("tensor ") + name + " is absent");
}

int rqmv_gguf_tensor_data(const rqmv_gguf* g, int64_t index, const void** data, size_t* nbytes) {
    if (!g || !data) return fail(RQMV_EINVAL, "gguf: NULL argument");
    if (index < 0 || index >= (int64_t)g->file->tensors.size()) return fail(RQMV_EINVAL, "gguf: tensor index out of range");
    const rq::GgufTensor& t = g->file->tensors[(size_t)index];
    *data = g->file->bytes(t);
    if (nbytes) *nbytes = (size_t)t.bytes;
    return RQMV_OK;
}

int rqmv_gguf_metadata_count(const rqmv_gguf* g, int64_t* count) {
    if (!g || !count) return fail(RQMV_EINVAL, "gguf: NULL argument");
    *count = (int64_t)g->file->metadata.size();
    return RQMV_OK;
}

int rqmv_gguf_metadata_key(const rqmv_gguf* g, int64_t index, const char** key, int* value_type) {
    if (!g || !key) return fail(RQMV_EINVAL, "gguf: NULL argument");
    if (index < 0 || index >= (int64_t)g->file->metadata.size()) return fail(RQMV_EINVAL, "gguf: key index out of range");
    *key = g->file->metadata[(size_t)index].first.c_str();
    if (value_type) *value_type = (int)g->file->metadata[(size_t)index].second.type;
    return RQMV_OK;
}

namespace {
const rq::GgufValue* gguf_value(const rqmv_gguf* g, const char* key, int* rc) {
    if (!g || !key) {
        *rc = fail(RQMV_EINVAL, "gguf: NULL argument");
        return nullptr;
    }
    const rq::GgufValue* v = g->file->value(key);
    if (!v) *rc = fail(RQMV_EINVAL, std::string(key) + " is absent");
    return v;
}
const rq::GgufValue* gguf_element(const rqmv_gguf* g, const char* key, int64_t index, int* rc) {
    const rq::GgufValue* v = gguf_value(g, key, rc);
    if (!v) return nullptr;
    if (v->type != 9) {
        *rc = fail(RQMV_EINVAL, std::string(key) + " is not an array");
        return nullptr;
    }
    if (index < 0 || index >= (int64_t)v->array.size()) {
        *rc = fail(RQMV_EINVAL, std::string(key) + ": index out of range");
        return nullptr;
    }
    return &v->array[(size_t)index];
}
int int_of(const rq::GgufValue* v, const char* key, int64_t* out) {
    uint64_t u;
    if (!v->integer(&u) || u > (uint64_t)INT64_MAX)
        return fail(RQMV_EINVAL, std::string(key) + " is not a nonnegative integer");
    *out = (int64_t)u;
    return RQMV_OK;
}
}  // namespace

int rqmv_gguf_get_int(const rqmv_gguf* g, const char* key, int64_t* out) {
    int rc = RQMV_OK;
    const rq::GgufValue* v = gguf_value(g, key, &rc);
    if (!v) return rc;
    if (!out) return fail(RQMV_EINVAL, "gguf: NULL argument");
    return int_of(v, key, out);
}

int rqmv_gguf_get_float(const rqmv_gguf* g, const char* key, double* out) {
    int rc = RQMV_OK;
    const rq::GgufValue* v = gguf_value(g, key, &rc);
    if (!v) return rc;
    if (!out || !v->real(out)) return fail(RQMV_EINVAL, std::string(key) + " is not a float");
    return RQMV_OK;
}

int rqmv_gguf_get_string(const rqmv_gguf* g, const char* key, const char** out) {
    int rc = RQMV_OK;
    const rq::GgufValue* v = gguf_value(g, key, &rc);
    if (!v) return rc;
    if (!out || v->type != 8) return fail(RQMV_EINVAL, std::string(key) + " is not a string");
    *out = v->s.c_str();
    return RQMV_OK;
}

int rqmv_gguf_get_array(const rqmv_gguf* g, const char* key, int* element_type, int64_t* count) {
    int rc = RQMV_OK;
    const rq::GgufValue* v = gguf_value(g, key, &rc);
    if (!v) return rc;
    if (v->type != 9) return fail(RQMV_EINVAL, std::string(key) + " is not an array");
    if (element_type) *element_type = (int)v->array_type;
    if (count) *count = (int64_t)v->array.size();
    return RQMV_OK;
}

int rqmv_gguf_get_array_int(const rqmv_gguf* g, const char* key, int64_t index, int64_t* out) {
    int rc = RQMV_OK;
    const rq::GgufValue* v = gguf_element(g, key, index, &rc);
    if (!v) return rc;
    if (!out) return fail(RQMV_EINVAL, "gguf: NULL argument");
    return int_of(v, key, out);
}

int rqmv_gguf_get_array_string(const rqmv_gguf* g, const char* key, int64_t index, const char** out) {
    int rc = RQMV_OK;
    const rq::GgufValue* v = gguf_element(g, key, index, &rc);
    if (!v) return rc;
    if (!out || v->type != 8) return fail(RQMV_EINVAL, std::string(key) + ": element is not a string");
    *out = v->s.c_str();
    return RQMV_OK;
}

int rqmv_gguf_weight_create(const rqmv_gguf* g, const char* name, rqmv_weight** out) {
    if (!g || !name || !out) return fail(RQMV_EINVAL, "gguf: NULL argument");
    const rq::GgufTensor* t = g->file->tensor(name);
    if (!t) return fail(RQMV_EINVAL, std::string("tensor ") + name + " is absent");
    if (t->type != rq::F16 && t->type != rq::Q4_0 && t->type != rq::Q8_0 && t->type != rq::Q4_K && t->type != rq::Q6_K)
        return fail(RQMV_EINVAL, "tensor " + t->name + " has GGML type " + std::to_string(t->type) +
                                     "; the library takes F16, Q4_0, Q8_0, Q4_K and Q6_K");
    // GGML order: shape[0] is the row width (cols), shape[1] the rows, shape[2] the experts
    const size_t nd = t->shape.size();
    if (nd < 1 || nd > 3) return fail(RQMV_EINVAL, "tensor " + t->name + " must have 1 to 3 dimensions");
    const int64_t cols = (int64_t)t->shape[0];
    const int64_t rows = nd >= 2 ? (int64_t)t->shape[1] : 1;
    const int64_t experts = nd == 3 ? (int64_t)t->shape[2] : 1;
    return create((int)t->type, experts, rows, cols, g->file->bytes(*t), (size_t)t->bytes, out);
}

int rqmv_layout_bytes(int format, int64_t rows, int64_t cols, size_t* bytes) {
    const int64_t n = rq::layout_bytes(format, rows, cols);
    if (n < 0 || format == rq::F32) return fail(RQMV_EINVAL, "bad format or shape");
    if (bytes) *bytes = (size_t)n;
    return RQMV_OK;
}

int rqmv_repack_host(int format, int64_t rows, int64_t cols, const void* gguf_bytes, void* out) {
    if (!gguf_bytes || !out) return fail(RQMV_EINVAL, "NULL argument");
    if (rq::repack(format, rows, cols, static_cast<const uint8_t*>(gguf_bytes), static_cast<uint8_t*>(out)) != 0)
        return fail(RQMV_EINVAL, "bad format or shape");
    return RQMV_OK;
}

int rqmv_unpack_host(int format, int64_t rows, int64_t cols, const void* in, void* gguf_bytes) {
    if (!gguf_bytes || !in) return fail(RQMV_EINVAL, "NULL argument");
    if (rq::unpack(format, rows, cols, static_cast<const uint8_t*>(in), static_cast<uint8_t*>(gguf_bytes)) != 0)
        return fail(RQMV_EINVAL, "bad format or shape");
    return RQMV_OK;
}

}  // extern "C"
