// rn_api.hip — the C ABI (include/rustyneedle.h): error reporting, device
// plumbing, QuantisedMatrix, Model, Session and the multi-sequence batch.
//
// Device memory layout
//   model  : one arena; per layer the fused QKV [3d][d], out [d][d], gate/up
//            [2f][d] and down [d][f] int8 codes (row-major, rows = outputs),
//            each followed by its [rows][cols/32] fp32 scales; the two norm
//            gain vectors; the tied embedding [vocab][d] and its scales; the
//            final gains; the rotary cos/sin table [max_positions][hd/2].
//   session: one arena; K and V caches [layers][heads][capacity][hd] fp16
//            (each (layer, head) a contiguous run of 128-byte rows), the
//            residual x, the fused QKV output, the attention output, the FFN
//            activation, the hidden state, the logits, a DecodeState and the
//            greedy id buffer.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/rustyneedle.h"
#include "rn_internal.hpp"
#include "rn_matrix.hpp"

using namespace rn;

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return code;
}

#define RN_HIP(call)                                                                                 \
    do {                                                                                             \
        hipError_t e_ = (call);                                                                      \
        if (e_ != hipSuccess)                                                                        \
            return fail(RN_ERR_DEVICE, "%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
    } while (0)

#define RN_REQUIRE(cond, ...)                              \
    do {                                                   \
        if (!(cond)) return fail(RN_ERR_ARGUMENT, __VA_ARGS__); \
    } while (0)

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// Bump allocator over one device allocation.
struct Arena {
    char* base = nullptr;
    size_t used = 0, size = 0;
    void* take(size_t bytes) {
        void* p = base + used;
        used += align_up(bytes);
        return p;
    }
};

struct DevMatrix {
    int8_t* W = nullptr;
    float* sW = nullptr;
};

struct LayerDev {
    DevMatrix qkv, out, gate_up, down;
    float* norm_attn = nullptr;
    float* norm_ffn = nullptr;
};

int check_supported(int columns) {
    return columns == 384 || columns == 512 || columns == 1024 || columns == 1536 || columns == 2048;
}

}  // namespace

namespace rn {
int set_error(int code, const char* message) { return fail(code, "%s", message); }
}  // namespace rn

struct rn_model {
    rn_config cfg{};
    void* arena = nullptr;
    std::vector<LayerDev> layers;
    DevMatrix embedding;
    float* norm_final = nullptr;
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    std::vector<float> rope_cos_host, rope_sin_host;
    float embed_scale = 0.0f;
};

struct rn_session {
    const rn_model* model = nullptr;
    int capacity = 0;
    int length = 0;
    bool has_hidden = false;
    hipStream_t stream = nullptr;
    void* arena = nullptr;
    __half* kc = nullptr;
    __half* vc = nullptr;
    float* x = nullptr;
    float* attn = nullptr;
    float* ffh = nullptr;
    float* hidden = nullptr;
    float* logits = nullptr;
    DecodeState* state = nullptr;
    uint32_t* ids = nullptr;
    unsigned long long* keys = nullptr;  // per-block greedy keys of the logits product
    hipGraphExec_t step_graph = nullptr;
    // prefill scratch, grown on demand
    void* scratch = nullptr;
    int scratch_tokens = 0;
    // constrained choice: the vocabulary mask and the result, allocated on first use
    void* choice_buf = nullptr;
};

struct rn_batch {
    const rn_model* model = nullptr;
    int count = 0, capacity = 0;
    std::vector<int> lengths;
    hipStream_t stream = nullptr;
    void* arena = nullptr;
    __half* kc = nullptr;
    __half* vc = nullptr;
    int32_t* pos = nullptr;
    float *X = nullptr, *QKV = nullptr, *A = nullptr, *F = nullptr, *logits = nullptr;
    int8_t* Xq = nullptr;
    float* sx = nullptr;
    uint32_t* tokens = nullptr;
    int32_t* error = nullptr;
    uint32_t* ids = nullptr;
    int ids_steps = 0;
    bool has_logits = false;
    int32_t* step = nullptr;            // the step of the running decode (its ids slot)
    hipGraphExec_t step_graph = nullptr;  // one step, captured for graph_steps and this ids buffer
    int graph_steps = 0;
};

// ---- the fixed scratch of rn_matrix_multiply_batch_noalloc ------------------------
// The input rows' int8 codes (first kNoAllocCodeBytes bytes) and their scales
// (kNoAllocTokens floats after them). One copy per GPU, at its own address,
// held until the process ends. Host code never passes `scratch` itself to a
// kernel: on the host the name is a stand-in, not a device address. It uses
// the device address that hipGetSymbolAddress returns, looked up once per
// device on the entry point's first call there.
constexpr size_t kNoAllocCodeBytes = size_t(4) << 20;
constexpr int kNoAllocTokens = 4096;
static __device__ __align__(256) unsigned char scratch[kNoAllocCodeBytes + sizeof(float) * kNoAllocTokens];

namespace {
// Per device: the scratch's device address and an event marking the end of
// the last call's kernels there. Calls on one device take g_scratch_mu for
// their whole enqueue, and each call's stream first waits for the previous
// call's event, so calls from several threads and streams run one after
// another on the device instead of racing on the scratch.
struct NoAllocDevice {
    void* ptr = nullptr;
    hipEvent_t last = nullptr;
};
std::mutex g_scratch_mu;
std::vector<NoAllocDevice> g_scratch;  // per device ordinal

// Set-up on a device's first call (caller holds g_scratch_mu): the symbol's
// address and the ordering event (an event is no device-memory allocation).
int scratch_device(NoAllocDevice** out) {
    int device = -1;
    RN_HIP(hipGetDevice(&device));
    if ((size_t)device >= g_scratch.size()) g_scratch.resize(device + 1);
    NoAllocDevice& d = g_scratch[device];
    if (!d.ptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(RN_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
        RN_HIP(hipEventCreateWithFlags(&d.last, hipEventDisableTiming));
        d.ptr = ptr;
    }
    *out = &d;
    return RN_OK;
}
}  // namespace

// ------------------------------------------------------------------------------
extern "C" {

const char* rn_last_error(void) { return g_error; }
int rn_abi_version(void) { return RN_ABI_VERSION; }

int rn_device_count(int* count) {
    RN_REQUIRE(count, "count is null");
    RN_HIP(hipGetDeviceCount(count));
    return RN_OK;
}
int rn_device_set(int device) {
    RN_HIP(hipSetDevice(device));
    return RN_OK;
}
int rn_malloc(void** ptr, size_t bytes) {
    RN_REQUIRE(ptr, "ptr is null");
    if (hipMalloc(ptr, bytes ? bytes : 1) != hipSuccess) return fail(RN_ERR_MEMORY, "hipMalloc(%zu) failed", bytes);
    return RN_OK;
}
int rn_free(void* ptr) {
    if (ptr) RN_HIP(hipFree(ptr));
    return RN_OK;
}
int rn_memcpy_htod(void* dst, const void* src, size_t bytes) {
    RN_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return RN_OK;
}
int rn_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    RN_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return RN_OK;
}
int rn_memcpy_dtod(void* dst, const void* src, size_t bytes) {
    RN_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    RN_HIP(hipStreamSynchronize(nullptr));  // a device-to-device copy may return before it ends
    return RN_OK;
}
int rn_stream_create(void** stream) {
    RN_REQUIRE(stream, "stream is null");
    hipStream_t s;
    RN_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return RN_OK;
}
int rn_stream_destroy(void* stream) {
    if (stream) RN_HIP(hipStreamDestroy((hipStream_t)stream));
    return RN_OK;
}
int rn_stream_synchronize(void* stream) {
    RN_HIP(hipStreamSynchronize((hipStream_t)stream));
    return RN_OK;
}
int rn_event_create(void** event) {
    RN_REQUIRE(event, "event is null");
    hipEvent_t e;
    RN_HIP(hipEventCreate(&e));
    *event = e;
    return RN_OK;
}
int rn_event_destroy(void* event) {
    if (event) RN_HIP(hipEventDestroy((hipEvent_t)event));
    return RN_OK;
}
int rn_event_record(void* event, void* stream) {
    RN_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return RN_OK;
}
int rn_event_elapsed_ms(void* start, void* stop, float* ms) {
    RN_REQUIRE(ms, "ms is null");
    RN_HIP(hipEventSynchronize((hipEvent_t)stop));
    RN_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return RN_OK;
}

// ---- QuantisedMatrix ------------------------------------------------------------

int rn_matrix_create_i8(const int8_t* codes, const float* scales, int rows, int columns, int group, int form,
                        rn_matrix** out) {
    RN_REQUIRE(codes && scales && out, "null argument");
    RN_REQUIRE(rows > 0, "rows must be positive (got %d)", rows);
    RN_REQUIRE(group == kGroup, "group must be 32 (got %d)", group);
    RN_REQUIRE(check_supported(columns), "columns must be 384, 512, 1024, 1536 or 2048 (got %d)", columns);
    RN_REQUIRE(form == RN_FORM_PANEL || form == RN_FORM_PLANE, "unknown form %d", form);
    rn_matrix* m = new (std::nothrow) rn_matrix();
    if (!m) return fail(RN_ERR_MEMORY, "out of host memory");
    const size_t cb = (size_t)rows * columns, sb = (size_t)rows * (columns / group) * sizeof(float);
    if (hipMalloc(&m->W, cb) != hipSuccess || hipMalloc(&m->sW, sb) != hipSuccess) {
        (void)hipFree(m->W);
        delete m;
        return fail(RN_ERR_MEMORY, "device allocation of %zu bytes failed", cb + sb);
    }
    m->rows = rows;
    m->columns = columns;
    m->group = group;
    m->form = form;
    if (hipMemcpy(m->W, codes, cb, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->sW, scales, sb, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(m->W);
        (void)hipFree(m->sW);
        delete m;
        return fail(RN_ERR_DEVICE, "upload of matrix failed");
    }
    *out = m;
    return RN_OK;
}

// QuantisedMatrix::from_parts (matrix.rs:41-59) for a codebook-quantised record.
// The levels follow lookup_table (matrix.rs:499-508, codebook.rs:12-43), the
// integer table IntegerLevels::new (neon.rs:114-124): scale = peak / 127 (1.0
// for a zero peak), entry = level / scale rounded half away from zero.
int rn_matrix_create_codebook(const uint8_t* blob, size_t blob_bytes, int rows, int columns, int group, int bits,
                              const float* codebook, int codebook_len, rn_matrix** out) {
    RN_REQUIRE(blob && codebook && out, "null argument");
    RN_REQUIRE(rows > 0 && columns > 0, "rows and columns must be positive (got %d x %d)", rows, columns);
    RN_REQUIRE(group == 64 || group == 128 || group == 256, "group must be 64, 128 or 256 (got %d)", group);
    RN_REQUIRE(bits >= 1 && bits <= 5, "bits must be 1..4 or 5 (ternary crumbs) (got %d)", bits);
    RN_REQUIRE(codebook_len >= 28, "the codebook holds 28 levels (got %d)", codebook_len);
    const int padded = (columns + group - 1) / group * group;
    const int ib = bits == 5 ? 2 : bits;
    const size_t row_bytes = (size_t)padded * ib / 8;
    const size_t packed = (size_t)rows * row_bytes, norms = (size_t)rows * (padded / group) * 2;
    RN_REQUIRE(padded <= 49152, "padded columns above 49152 are not supported (got %d)", padded);
    RN_REQUIRE(blob_bytes >= packed + norms, "blob of %zu bytes is shorter than indices + norms (%zu)", blob_bytes,
               packed + norms);
    float levels[16] = {0};
    int count = 0;
    if (bits == 1) {  // codebook.rs:34-37
        const float level = sqrtf(2.0f / 3.14159265358979323846f) / sqrtf((float)group);
        levels[0] = -level;
        levels[1] = level;
        count = 2;
    } else if (bits == 2) {
        std::copy(codebook, codebook + 4, levels);
        count = 4;
    } else if (bits == 3) {
        std::copy(codebook + 4, codebook + 12, levels);
        count = 8;
    } else if (bits == 4) {
        std::copy(codebook + 12, codebook + 28, levels);
        count = 16;
    } else {
        const float level = 1.2240064f / sqrtf((float)group);  // codebook.rs:39-42
        levels[1] = level;
        levels[3] = -level;
        count = 4;
    }
    float peak = 0.0f;
    for (int i = 0; i < count; ++i) peak = fmaxf(peak, fabsf(levels[i]));
    const float lscale = peak > 0.0f ? peak / 127.0f : 1.0f;
    uint8_t table[16] = {0};
    for (int i = 0; i < count; ++i) table[i] = (uint8_t)(int8_t)roundf(levels[i] / lscale);

    rn_matrix* m = new (std::nothrow) rn_matrix();
    if (!m) return fail(RN_ERR_MEMORY, "out of host memory");
    const size_t bytes = packed + norms + 16384;  // kernels read norms in 12 KB windows past a block's start
    if (hipMalloc(&m->blob, bytes) != hipSuccess) {
        delete m;
        return fail(RN_ERR_MEMORY, "device allocation of %zu bytes failed", bytes);
    }
    if (hipMemset(m->blob, 0, bytes) != hipSuccess || hipMemcpy(m->blob, blob, packed + norms, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(m->blob);
        delete m;
        return fail(RN_ERR_DEVICE, "upload of matrix failed");
    }
    m->rows = rows;
    m->columns = columns;
    m->group = group;
    m->bits = bits;
    m->form = bits == 2 ? RN_FORM_PANEL : RN_FORM_PLANE;
    CodebookParams& c = m->cb;
    c.packed = m->blob;
    c.norms = reinterpret_cast<const uint16_t*>(m->blob + packed);
    c.rows = rows;
    c.columns = columns;
    c.padded = padded;
    c.group = group;
    c.bits = bits;
    c.row_bytes = (int)row_bytes;
    c.cpr = (int)(row_bytes / 16);
    c.inv_cpr = 1.0f / (float)c.cpr;
    for (int i = 0; i < 4; ++i)
        c.lut[i] = (uint32_t)table[4 * i] | ((uint32_t)table[4 * i + 1] << 8) | ((uint32_t)table[4 * i + 2] << 16) |
                   ((uint32_t)table[4 * i + 3] << 24);
    c.lscale = lscale;
    std::copy(levels, levels + 16, c.levels);
    c.wht_scale = 1.0f / sqrtf((float)group);  // walsh.rs:74
    *out = m;
    return RN_OK;
}

int rn_matrix_free(rn_matrix* m) {
    if (!m) return RN_OK;
    if (m->host_stream) {
        (void)hipStreamSynchronize(m->host_stream);
        (void)hipStreamDestroy(m->host_stream);
    }
    (void)hipFree(m->host_buf);
    (void)hipFree(m->W);
    (void)hipFree(m->sW);
    (void)hipFree(m->blob);
    delete m;
    return RN_OK;
}

int rn_matrix_padded_columns(const rn_matrix* m, int* padded) {
    RN_REQUIRE(m && padded, "null argument");
    *padded = m->bits ? m->cb.padded : m->columns;
    return RN_OK;
}

int rn_matrix_prepare(const rn_matrix* m, const float* x, int count, float* rotated, void* stream) {
    RN_REQUIRE(m && x && rotated, "null argument");
    RN_REQUIRE(m->bits != 0, "int8 matrices take their input unrotated; prepare applies to codebook matrices");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    RN_HIP(launch_codebook_rotate(x, count, m->columns, m->cb.padded, m->group, m->cb.wht_scale, rotated,
                                  (hipStream_t)stream));
    return RN_OK;
}

int rn_matrix_shape(const rn_matrix* m, int* rows, int* columns, int* group) {
    RN_REQUIRE(m, "matrix is null");
    if (rows) *rows = m->rows;
    if (columns) *columns = m->columns;
    if (group) *group = m->group;
    return RN_OK;
}

// 1- and 3-bit matrices have integer levels nowhere in the reference
// (matrix.rs:559-563): every product of theirs is the float path.
static bool float_only(const rn_matrix* m) { return m->bits == 1 || m->bits == 3; }

int rn_matrix_multiply_vector(const rn_matrix* m, const float* x, float* y, int32_t* acc, void* stream) {
    RN_REQUIRE(m && x && y, "null argument");
    if (float_only(m)) {
        RN_REQUIRE(acc == nullptr, "1- and 3-bit matrices have no integer accumulators (the float path)");
        RN_HIP(launch_codebook_float(m->cb, x, 1, y, false, (hipStream_t)stream));
        return RN_OK;
    }
    if (m->bits) {
        RN_HIP(launch_codebook_product(m->cb, x, 1, y, acc, (hipStream_t)stream));
        return RN_OK;
    }
    GemvParams p{};
    const int rpb = gemv_rows_per_block(m->rows, m->columns, kStore);
    const int blocks = (m->rows + rpb - 1) / rpb;
    p.nseg = 1;
    p.seg[0] = Segment{m->W, m->sW, y, acc, m->rows};
    p.x = x;
    RN_HIP(launch_gemv(p, m->columns, kQuant, kStore, m->form, rpb, blocks, (hipStream_t)stream));
    return RN_OK;
}

int rn_matrix_multiply_vector_rows(const rn_matrix* m, const float* x, float* y, int rows_per_block, void* stream) {
    RN_REQUIRE(m && x && y, "null argument");
    RN_REQUIRE(m->bits == 0, "an int8 matrix (codebook matrices have their own kernels)");
    RN_REQUIRE(rows_per_block == 8 || rows_per_block == 16 || rows_per_block == 32, "rows_per_block must be 8, 16 or 32");
    RN_REQUIRE(m->columns == 512 || (m->columns == 384 && rows_per_block >= 8),
               "columns must be 512 or 384 (got %d)", m->columns);
    GemvParams p{};
    const int blocks = (m->rows + rows_per_block - 1) / rows_per_block;
    p.nseg = 1;
    p.seg[0] = Segment{m->W, m->sW, y, nullptr, m->rows};
    p.x = x;
    RN_HIP(launch_gemv(p, m->columns, kQuant, kStore, m->form, rows_per_block, blocks, (hipStream_t)stream));
    return RN_OK;
}

int rn_matrix_multiply_fused(const rn_matrix* const* ms, int count, const float* x, float* const* ys, void* stream) {
    RN_REQUIRE(ms && x && ys, "null argument");
    RN_REQUIRE(count >= 1 && count <= kMaxSegments, "count must be 1..%d (got %d)", kMaxSegments, count);
    const rn_matrix* first = ms[0];
    RN_REQUIRE(first, "matrix 0 is null");
    if (first->bits) {
        // codebook matrices sharing the rotated input: one launch each
        for (int i = 0; i < count; ++i) {
            RN_REQUIRE(ms[i] && ys[i], "matrix or output %d is null", i);
            RN_REQUIRE(ms[i]->bits && ms[i]->cb.padded == first->cb.padded && ms[i]->group == first->group,
                       "fused matrices must share padded columns and group (matrix %d differs)", i);
        }
        for (int i = 0; i < count; ++i) {
            if (float_only(ms[i]))
                RN_HIP(launch_codebook_float(ms[i]->cb, x, 1, ys[i], false, (hipStream_t)stream));
            else
                RN_HIP(launch_codebook_product(ms[i]->cb, x, 1, ys[i], nullptr, (hipStream_t)stream));
        }
        return RN_OK;
    }
    int total_rows = 0;
    for (int i = 0; i < count; ++i) {
        RN_REQUIRE(ms[i] && ys[i], "matrix or output %d is null", i);
        RN_REQUIRE(ms[i]->columns == first->columns && ms[i]->group == first->group && ms[i]->form == first->form,
                   "fused matrices must share columns, group and form (matrix %d differs)", i);
        total_rows += ms[i]->rows;
    }
    const int rpb = gemv_rows_per_block(total_rows, first->columns, kStore);
    GemvParams p{};
    p.nseg = count;
    int blocks = 0;  // per segment (grid row): the widest segment's
    for (int i = 0; i < count; ++i) {
        p.seg[i] = Segment{ms[i]->W, ms[i]->sW, ys[i], nullptr, ms[i]->rows};
        blocks = std::max(blocks, (ms[i]->rows + rpb - 1) / rpb);
    }
    p.x = x;
    RN_HIP(launch_gemv(p, first->columns, kQuant, kStore, first->form, rpb, blocks, (hipStream_t)stream));
    return RN_OK;
}

// The int8 batch product once the input rows have a place for their codes:
// per-row quantisation into xq / sx, then the i8 MFMA product.
static hipError_t batch_product_i8(const rn_matrix* m, const float* x, int count, float* y, int32_t* acc, int8_t* xq,
                                   float* sx, hipStream_t s) {
    hipError_t e = launch_norm_quantise(x, nullptr, count, m->columns, 1e-6f, xq, sx, nullptr, s);
    if (e != hipSuccess) return e;
    GemmParams p{xq, sx, m->W, m->sW, count, m->rows, m->columns, y, m->rows, acc, 0};
    return launch_gemm(p, kGemmStore, m->form, acc != nullptr, s);
}

int rn_matrix_multiply_batch(const rn_matrix* m, const float* x, int count, float* y, int32_t* acc, void* stream) {
    RN_REQUIRE(m && x && y, "null argument");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    hipStream_t s = (hipStream_t)stream;
    if (float_only(m)) {
        RN_REQUIRE(acc == nullptr, "1- and 3-bit matrices have no integer accumulators (the float path)");
        RN_HIP(launch_codebook_float(m->cb, x, count, y, true, s));
        return RN_OK;
    }
    if (m->bits) {
        RN_HIP(launch_codebook_product(m->cb, x, count, y, acc, s));
        return RN_OK;
    }
    void* scratch = nullptr;
    const size_t codes = align_up((size_t)count * m->columns);
    RN_HIP(hipMallocAsync(&scratch, codes + sizeof(float) * (size_t)count, s));
    hipError_t e = batch_product_i8(m, x, count, y, acc, (int8_t*)scratch, (float*)((char*)scratch + codes), s);
    hipError_t f = hipFreeAsync(scratch, s);
    RN_HIP(e);
    RN_HIP(f);
    return RN_OK;
}

int rn_matrix_multiply_batch_noalloc(const rn_matrix* m, const float* x, int count, float* y, int32_t* acc,
                                     void* stream) {
    RN_REQUIRE(m && x && y, "null argument");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    hipStream_t s = (hipStream_t)stream;
    if (float_only(m)) {  // the float path needs no scratch
        RN_REQUIRE(acc == nullptr, "1- and 3-bit matrices have no integer accumulators (the float path)");
        RN_HIP(launch_codebook_float(m->cb, x, count, y, true, s));
        return RN_OK;
    }
    if (m->bits) {  // the codebook product quantises inside its kernel: no scratch
        RN_HIP(launch_codebook_product(m->cb, x, count, y, acc, s));
        return RN_OK;
    }
    const size_t codes = align_up((size_t)count * m->columns);
    RN_REQUIRE(count <= kNoAllocTokens && codes <= kNoAllocCodeBytes,
               "count %d x columns %d exceeds the fixed scratch (at most %d rows and %zu code bytes)", count,
               m->columns, kNoAllocTokens, kNoAllocCodeBytes);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    NoAllocDevice* dev = nullptr;
    int rc = scratch_device(&dev);
    if (rc) return rc;
    // Under stream capture the caller's graph orders its own replays; an event
    // recorded outside the capture cannot be waited on inside it.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    RN_HIP(hipStreamIsCapturing(s, &capture));
    const bool ordered = capture == hipStreamCaptureStatusNone;
    if (ordered) RN_HIP(hipStreamWaitEvent(s, dev->last, 0));
    int8_t* xq = (int8_t*)dev->ptr;
    float* sx = (float*)((char*)dev->ptr + kNoAllocCodeBytes);
    RN_HIP(batch_product_i8(m, x, count, y, acc, xq, sx, s));
    if (ordered) RN_HIP(hipEventRecord(dev->last, s));
    return RN_OK;
}

int rn_matrix_multiply_vector_float(const rn_matrix* m, const float* rotated, float* y, void* stream) {
    RN_REQUIRE(m && rotated && y, "null argument");
    RN_REQUIRE(m->bits != 0, "the float path is a codebook matrix's (int8 matrices have only the integer path)");
    RN_HIP(launch_codebook_float(m->cb, rotated, 1, y, false, (hipStream_t)stream));
    return RN_OK;
}

int rn_matrix_multiply_batch_float(const rn_matrix* m, const float* rotated, int count, float* y, void* stream) {
    RN_REQUIRE(m && (count == 0 || (rotated && y)), "null argument");
    RN_REQUIRE(m->bits != 0, "the float path is a codebook matrix's (int8 matrices have only the integer path)");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    RN_HIP(launch_codebook_float(m->cb, rotated, count, y, true, (hipStream_t)stream));
    return RN_OK;
}

// ---- host-slice products (the reference's &[f32] / &mut [f32] signatures) -------
// The input slice is copied to the matrix's staging buffer, the device entry
// point runs on the matrix's own stream, the output is copied back and the
// stream is synchronised before returning. Caller holds m->host_mu.
static int host_stage(const rn_matrix* m, size_t in_bytes, size_t out_bytes, float** din, float** dout) {
    const size_t need = align_up(in_bytes) + align_up(out_bytes);
    if (!m->host_stream) RN_HIP(hipStreamCreateWithFlags(&m->host_stream, hipStreamNonBlocking));
    if (need > m->host_bytes) {
        RN_HIP(hipStreamSynchronize(m->host_stream));
        if (m->host_buf) RN_HIP(hipFree(m->host_buf));
        m->host_buf = nullptr;
        m->host_bytes = 0;
        if (hipMalloc(&m->host_buf, need) != hipSuccess)
            return fail(RN_ERR_MEMORY, "staging buffer of %zu bytes", need);
        m->host_bytes = need;
    }
    *din = (float*)m->host_buf;
    *dout = (float*)(m->host_buf + align_up(in_bytes));
    return RN_OK;
}

static int matrix_width(const rn_matrix* m) { return m->bits ? m->cb.padded : m->columns; }

int rn_matrix_multiply_vector_host(const rn_matrix* m, const float* x, float* y) {
    RN_REQUIRE(m && x && y, "null argument");
    std::lock_guard<std::mutex> lock(m->host_mu);
    const size_t in = sizeof(float) * matrix_width(m), out = sizeof(float) * m->rows;
    float *dx = nullptr, *dy = nullptr;
    int rc = host_stage(m, in, out, &dx, &dy);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(dx, x, in, hipMemcpyHostToDevice, m->host_stream));
    rc = rn_matrix_multiply_vector(m, dx, dy, nullptr, m->host_stream);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(y, dy, out, hipMemcpyDeviceToHost, m->host_stream));
    RN_HIP(hipStreamSynchronize(m->host_stream));
    return RN_OK;
}

int rn_matrix_multiply_batch_host(const rn_matrix* m, const float* x, int count, float* y) {
    RN_REQUIRE(m && (count == 0 || (x && y)), "null argument");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    std::lock_guard<std::mutex> lock(m->host_mu);
    const size_t in = sizeof(float) * (size_t)count * matrix_width(m), out = sizeof(float) * (size_t)count * m->rows;
    float *dx = nullptr, *dy = nullptr;
    int rc = host_stage(m, in, out, &dx, &dy);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(dx, x, in, hipMemcpyHostToDevice, m->host_stream));
    rc = rn_matrix_multiply_batch(m, dx, count, dy, nullptr, m->host_stream);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(y, dy, out, hipMemcpyDeviceToHost, m->host_stream));
    RN_HIP(hipStreamSynchronize(m->host_stream));
    return RN_OK;
}

int rn_matrix_prepare_host(const rn_matrix* m, const float* x, int count, float* rotated) {
    RN_REQUIRE(m && (count == 0 || (x && rotated)), "null argument");
    RN_REQUIRE(m->bits != 0, "int8 matrices take their input unrotated; prepare applies to codebook matrices");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    std::lock_guard<std::mutex> lock(m->host_mu);
    const size_t in = sizeof(float) * (size_t)count * m->columns, out = sizeof(float) * (size_t)count * m->cb.padded;
    float *dx = nullptr, *dy = nullptr;
    int rc = host_stage(m, in, out, &dx, &dy);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(dx, x, in, hipMemcpyHostToDevice, m->host_stream));
    rc = rn_matrix_prepare(m, dx, count, dy, m->host_stream);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(rotated, dy, out, hipMemcpyDeviceToHost, m->host_stream));
    RN_HIP(hipStreamSynchronize(m->host_stream));
    return RN_OK;
}

int rn_matrix_dequantise_row(const rn_matrix* m, int row, float* out) {
    RN_REQUIRE(m && out, "null argument");
    RN_REQUIRE(row >= 0 && row < m->rows, "row %d out of range [0, %d)", row, m->rows);
    if (m->bits) {
        float* dev = nullptr;
        RN_HIP(hipMalloc(&dev, sizeof(float) * m->cb.padded));
        hipError_t e = launch_codebook_dequantise(m->cb, row, dev, nullptr);
        if (e == hipSuccess) e = hipMemcpy(out, dev, sizeof(float) * m->columns, hipMemcpyDeviceToHost);
        (void)hipFree(dev);
        RN_HIP(e);
        return RN_OK;
    }
    const int G = m->columns / m->group;
    float* dev = nullptr;
    RN_HIP(hipMalloc(&dev, sizeof(float) * m->columns));
    hipError_t e = launch_dequantise_i8(m->W + (size_t)row * m->columns, m->sW + (size_t)row * G, m->columns,
                                        m->group, dev, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dev, sizeof(float) * m->columns, hipMemcpyDeviceToHost);
    (void)hipFree(dev);
    RN_HIP(e);
    return RN_OK;
}

int rn_quantise_int8(const float* x, int count, int columns, int8_t* codes, float* scales, void* stream) {
    RN_REQUIRE(x && codes && scales, "null argument");
    RN_REQUIRE(count >= 0 && columns > 0, "bad shape");
    RN_HIP(launch_quantise_rows(x, count, columns, codes, scales, (hipStream_t)stream));
    return RN_OK;
}

int rn_fast_exp(const float* x, float* y, int n, void* stream) {
    RN_REQUIRE(x && y && n >= 0, "bad argument");
    RN_HIP(launch_fast_exp(x, y, n, 0, (hipStream_t)stream));
    return RN_OK;
}

int rn_silu(const float* x, float* y, int n, void* stream) {
    RN_REQUIRE(x && y && n >= 0, "bad argument");
    RN_HIP(launch_fast_exp(x, y, n, 1, (hipStream_t)stream));
    return RN_OK;
}

int rn_libm_exp(const float* x, float* y, int n, void* stream) {
    RN_REQUIRE(x && y && n >= 0, "bad argument");
    RN_HIP(launch_fast_exp(x, y, n, 2, (hipStream_t)stream));
    return RN_OK;
}

int rn_sigmoid(const float* x, float* y, int n, void* stream) {
    RN_REQUIRE(x && y && n >= 0, "bad argument");
    RN_HIP(launch_fast_exp(x, y, n, 3, (hipStream_t)stream));
    return RN_OK;
}

int rn_libm_log(const float* x, float* y, int n, void* stream) {
    RN_REQUIRE(x && y && n >= 0, "bad argument");
    RN_HIP(launch_fast_exp(x, y, n, 4, (hipStream_t)stream));
    return RN_OK;
}

int rn_reciprocal(const float* x, float* y, int n, void* stream) {
    RN_REQUIRE(x && y && n >= 0, "bad argument");
    RN_HIP(launch_fast_exp(x, y, n, 5, (hipStream_t)stream));
    return RN_OK;
}

int rn_zero_centred_norm(const float* x, const float* gain, int count, int n, float* out, void* stream) {
    RN_REQUIRE(x && gain && out, "null argument");
    RN_REQUIRE(n > 0 && n % 8 == 0 && n <= 4096 && count >= 0, "n must be a multiple of 8 in 8..4096");
    RN_HIP(launch_norm_rows(x, gain, count, n, 1e-6f, out, (hipStream_t)stream));
    return RN_OK;
}

int rn_attend_heads(const float* q, const uint16_t* K, const uint16_t* V, const int32_t* lengths, int count,
                    int stride, int head_dim, float* out, void* stream) {
    RN_REQUIRE(q && K && V && lengths && out, "null argument");
    RN_REQUIRE(head_dim == 64, "head_dim must be 64 (got %d)", head_dim);
    RN_REQUIRE(stride >= 1 && stride <= 16384 && count >= 0, "stride must be 1..16384");
    if (count == 0) return RN_OK;
    hipStream_t s = (hipStream_t)stream;
    int32_t* err = nullptr;
    RN_HIP(hipMallocAsync((void**)&err, sizeof(int32_t), s));
    RN_HIP(hipMemsetAsync(err, 0, sizeof(int32_t), s));
    AttendParams p{};
    p.q = q;
    p.kc = (__half*)K;
    p.vc = (__half*)V;
    p.lengths = lengths;
    p.stride = stride;
    p.out = out;
    p.error = err;
    hipError_t e = launch_attend(p, kAttendRaw, count, 1, stride, s);
    int32_t host_err = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&host_err, err, sizeof(int32_t), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFreeAsync(err, s);
    RN_HIP(e);
    if (host_err) return fail(RN_ERR_ARGUMENT, "a length is outside 1..stride");
    return RN_OK;
}

// ---- Model ----------------------------------------------------------------------

static int validate_config(const rn_config* c) {
    RN_REQUIRE(c, "config is null");
    RN_REQUIRE(c->d_model == 512, "d_model must be 512 (got %d)", c->d_model);
    RN_REQUIRE(c->head_dim == 64, "head_dim must be 64 (got %d)", c->head_dim);
    RN_REQUIRE(c->heads * c->head_dim == c->d_model, "heads * head_dim must equal d_model");
    RN_REQUIRE(c->ffn == 512 || c->ffn == 1024 || c->ffn == 2048, "ffn must be 512, 1024 or 2048 (got %d)", c->ffn);
    RN_REQUIRE(c->group == kGroup, "group must be 32 (got %d)", c->group);
    RN_REQUIRE(c->layers >= 1 && c->layers <= 256, "layers must be 1..256 (got %d)", c->layers);
    RN_REQUIRE(c->vocab >= 1, "vocab must be positive");
    RN_REQUIRE(c->max_positions >= 1 && c->max_positions <= 16384, "max_positions must be 1..16384");
    RN_REQUIRE(c->norm_eps == 1e-6f, "norm_eps must be 1e-6 (the reference's NORM_EPSILON)");
    RN_REQUIRE(c->rope_theta > 0.0f, "rope_theta must be positive");
    return RN_OK;
}

// ops.rs:127-141: frequencies 1/theta^(2i/hd) and the angle position*freq in f32.
static void rotary_table(const rn_config& c, std::vector<float>& cs, std::vector<float>& sn) {
    const int half = c.head_dim / 2;
    std::vector<float> freqs(half);
    for (int i = 0; i < half; ++i) freqs[i] = 1.0f / powf(c.rope_theta, (2.0f * (float)i) / (float)c.head_dim);
    cs.resize((size_t)c.max_positions * half);
    sn.resize(cs.size());
    for (int p = 0; p < c.max_positions; ++p)
        for (int i = 0; i < half; ++i) {
            const float angle = (float)p * freqs[i];
            cs[(size_t)p * half + i] = cosf(angle);
            sn[(size_t)p * half + i] = sinf(angle);
        }
}

int rn_model_create(const rn_config* config, const rn_weights_host* w, rn_model** out) {
    int rc = validate_config(config);
    if (rc) return rc;
    RN_REQUIRE(w && out && w->layers && w->norm_final && w->embedding.codes && w->embedding.scales, "null weights");
    const rn_config& c = *config;
    const size_t d = c.d_model, f = c.ffn, G = d / kGroup, Gf = f / kGroup;
    for (int l = 0; l < c.layers; ++l) {
        const rn_layer_host& L = w->layers[l];
        RN_REQUIRE(L.qkv.codes && L.qkv.scales && L.out.codes && L.out.scales && L.gate_up.codes && L.gate_up.scales &&
                       L.down.codes && L.down.scales && L.norm_attn && L.norm_ffn,
                   "null tensor in layer %d", l);
    }
    rn_model* m = new (std::nothrow) rn_model();
    if (!m) return fail(RN_ERR_MEMORY, "out of host memory");
    m->cfg = c;
    rotary_table(c, m->rope_cos_host, m->rope_sin_host);
    m->embed_scale = sqrtf((float)c.d_model);

    auto qbytes = [](size_t rows, size_t cols) { return align_up(rows * cols) + align_up(rows * (cols / kGroup) * 4); };
    size_t total = 0;
    total += (size_t)c.layers * (qbytes(3 * d, d) + qbytes(d, d) + qbytes(2 * f, d) + qbytes(d, f) + 2 * align_up(4 * d));
    total += qbytes(c.vocab, d) + align_up(4 * d) + 2 * align_up(m->rope_cos_host.size() * 4);
    if (hipMalloc(&m->arena, total) != hipSuccess) {
        delete m;
        return fail(RN_ERR_MEMORY, "device allocation of %zu bytes failed", total);
    }
    Arena a{(char*)m->arena, 0, total};
    std::vector<std::pair<void*, std::pair<const void*, size_t>>> uploads;
    auto place = [&](const void* src, size_t bytes) {
        void* dst = a.take(bytes);
        uploads.push_back({dst, {src, bytes}});
        return dst;
    };
    auto placeq = [&](const rn_qmat_host& q, size_t rows, size_t cols) {
        DevMatrix dm;
        dm.W = (int8_t*)place(q.codes, rows * cols);
        dm.sW = (float*)place(q.scales, rows * (cols / kGroup) * 4);
        return dm;
    };
    m->layers.resize(c.layers);
    for (int l = 0; l < c.layers; ++l) {
        const rn_layer_host& L = w->layers[l];
        LayerDev& D = m->layers[l];
        D.qkv = placeq(L.qkv, 3 * d, d);
        D.out = placeq(L.out, d, d);
        D.gate_up = placeq(L.gate_up, 2 * f, d);
        D.down = placeq(L.down, d, f);
        D.norm_attn = (float*)place(L.norm_attn, 4 * d);
        D.norm_ffn = (float*)place(L.norm_ffn, 4 * d);
    }
    m->embedding = placeq(w->embedding, c.vocab, d);
    m->norm_final = (float*)place(w->norm_final, 4 * d);
    m->rope_cos = (float*)place(m->rope_cos_host.data(), m->rope_cos_host.size() * 4);
    m->rope_sin = (float*)place(m->rope_sin_host.data(), m->rope_sin_host.size() * 4);
    (void)G;
    (void)Gf;
    for (auto& u : uploads) {
        if (hipMemcpy(u.first, u.second.first, u.second.second, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(m->arena);
            delete m;
            return fail(RN_ERR_DEVICE, "weight upload failed");
        }
    }
    *out = m;
    return RN_OK;
}

int rn_model_create_synthetic(const rn_config* config, uint64_t seed, rn_model** out) {
    int rc = validate_config(config);
    if (rc) return rc;
    RN_REQUIRE(out, "out is null");
    const rn_config& c = *config;
    const size_t d = c.d_model, f = c.ffn;
    struct Q {
        std::vector<int8_t> codes;
        std::vector<float> scales;
    };
    auto gen_q = [&](const std::string& name, size_t rows, size_t cols) {
        Q q;
        q.codes.resize(rows * cols);
        q.scales.resize(rows * (cols / kGroup));
        rn_synth_codes(seed, (name + ".codes").c_str(), q.codes.data(), q.codes.size());
        rn_synth_uniform(seed, (name + ".scales").c_str(), 1e-3f, 1e-2f, q.scales.data(), q.scales.size());
        return q;
    };
    auto gen_gain = [&](const std::string& name) {
        std::vector<float> g(d);
        rn_synth_normal(seed, name.c_str(), 0.1f, g.data(), d);
        return g;
    };
    std::vector<Q> qs;
    std::vector<std::vector<float>> gains;
    qs.reserve((size_t)c.layers * 4 + 1);
    gains.reserve((size_t)c.layers * 2 + 1);
    std::vector<rn_layer_host> layers(c.layers);
    for (int l = 0; l < c.layers; ++l) {
        const std::string p = "layers." + std::to_string(l) + ".";
        qs.push_back(gen_q(p + "qkv", 3 * d, d));
        qs.push_back(gen_q(p + "out", d, d));
        qs.push_back(gen_q(p + "gate_up", 2 * f, d));
        qs.push_back(gen_q(p + "down", d, f));
        gains.push_back(gen_gain(p + "norm_attn"));
        gains.push_back(gen_gain(p + "norm_ffn"));
        const size_t qi = qs.size() - 4, gi = gains.size() - 2;
        layers[l].qkv = {qs[qi].codes.data(), qs[qi].scales.data()};
        layers[l].out = {qs[qi + 1].codes.data(), qs[qi + 1].scales.data()};
        layers[l].gate_up = {qs[qi + 2].codes.data(), qs[qi + 2].scales.data()};
        layers[l].down = {qs[qi + 3].codes.data(), qs[qi + 3].scales.data()};
        layers[l].norm_attn = gains[gi].data();
        layers[l].norm_ffn = gains[gi + 1].data();
    }
    qs.push_back(gen_q("embedding", c.vocab, d));
    gains.push_back(gen_gain("norm_final"));
    rn_weights_host w{};
    w.embedding = {qs.back().codes.data(), qs.back().scales.data()};
    w.norm_final = gains.back().data();
    w.layers = layers.data();
    return rn_model_create(config, &w, out);
}

int rn_model_free(rn_model* m) {
    if (!m) return RN_OK;
    (void)hipFree(m->arena);
    delete m;
    return RN_OK;
}

int rn_model_config(const rn_model* m, rn_config* out) {
    RN_REQUIRE(m && out, "null argument");
    *out = m->cfg;
    return RN_OK;
}

int rn_model_rotary_table(const rn_model* m, float* cos_out, float* sin_out) {
    RN_REQUIRE(m && cos_out && sin_out, "null argument");
    memcpy(cos_out, m->rope_cos_host.data(), m->rope_cos_host.size() * 4);
    memcpy(sin_out, m->rope_sin_host.data(), m->rope_sin_host.size() * 4);
    return RN_OK;
}

// ---- Session --------------------------------------------------------------------

static size_t cache_elems(const rn_config& c, int capacity) {
    return (size_t)c.layers * c.heads * capacity * c.head_dim;
}

int rn_session_create(const rn_model* m, int capacity, rn_session** out) {
    RN_REQUIRE(m && out, "null argument");
    const rn_config& c = m->cfg;
    RN_REQUIRE(capacity >= 1 && capacity <= c.max_positions, "capacity must be 1..max_positions (%d)", c.max_positions);
    RN_REQUIRE(capacity <= 16384, "capacity must be at most 16384");
    rn_session* s = new (std::nothrow) rn_session();
    if (!s) return fail(RN_ERR_MEMORY, "out of host memory");
    s->model = m;
    s->capacity = capacity;
    const size_t ce = cache_elems(c, capacity), d = c.d_model;
    const size_t total = 2 * align_up(ce * 2) + align_up(4 * d) * 4 + align_up(4 * (size_t)c.ffn) +
                         align_up(4 * (size_t)c.vocab) + align_up(sizeof(DecodeState)) + align_up(4 * (size_t)capacity) +
                         align_up(8 * (size_t)c.vocab);
    if (hipMalloc(&s->arena, total) != hipSuccess) {
        delete s;
        return fail(RN_ERR_MEMORY, "device allocation of %zu bytes failed", total);
    }
    Arena a{(char*)s->arena, 0, total};
    s->kc = (__half*)a.take(ce * 2);
    s->vc = (__half*)a.take(ce * 2);
    s->x = (float*)a.take(4 * d);
    s->attn = (float*)a.take(4 * d);
    s->ffh = (float*)a.take(4 * (size_t)c.ffn);
    s->hidden = (float*)a.take(4 * d);
    s->logits = (float*)a.take(4 * (size_t)c.vocab);
    s->state = (DecodeState*)a.take(sizeof(DecodeState));
    s->ids = (uint32_t*)a.take(4 * (size_t)capacity);
    s->keys = (unsigned long long*)a.take(8 * (size_t)c.vocab);
    if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess ||
        hipMemsetAsync(s->arena, 0, total, s->stream) != hipSuccess || hipStreamSynchronize(s->stream) != hipSuccess) {
        if (s->stream) (void)hipStreamDestroy(s->stream);
        (void)hipFree(s->arena);
        delete s;
        return fail(RN_ERR_DEVICE, "session initialisation failed");
    }
    *out = s;
    return RN_OK;
}

int rn_session_free(rn_session* s) {
    if (!s) return RN_OK;
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->step_graph) (void)hipGraphExecDestroy(s->step_graph);
    if (s->scratch) (void)hipFree(s->scratch);
    if (s->choice_buf) (void)hipFree(s->choice_buf);
    (void)hipFree(s->arena);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return RN_OK;
}

int rn_session_clone(const rn_session* s, rn_session** out) {
    RN_REQUIRE(s && out, "null argument");
    rn_session* t = nullptr;
    int rc = rn_session_create(s->model, s->capacity, &t);
    if (rc) return rc;
    RN_HIP(hipStreamSynchronize(s->stream));
    // Everything in the arena up to the id buffer is state; copy it wholesale,
    // on the clone's stream (a device-to-device hipMemcpy may return before
    // the copy ends, and the null stream does not order the session streams).
    const size_t bytes = (size_t)((char*)s->ids - (char*)s->arena);
    RN_HIP(hipMemcpyAsync(t->arena, s->arena, bytes, hipMemcpyDeviceToDevice, t->stream));
    RN_HIP(hipStreamSynchronize(t->stream));
    t->length = s->length;
    t->has_hidden = s->has_hidden;
    *out = t;
    return RN_OK;
}

int rn_session_len(const rn_session* s, int* length) {
    RN_REQUIRE(s && length, "null argument");
    *length = s->length;
    return RN_OK;
}

int rn_session_truncate(rn_session* s, int length) {
    RN_REQUIRE(s, "session is null");
    RN_REQUIRE(length >= 0 && length <= s->length, "length %d outside 0..%d", length, s->length);
    s->length = length;
    s->has_hidden = false;
    return RN_OK;
}

int rn_session_stream(const rn_session* s, void** stream) {
    RN_REQUIRE(s && stream, "null argument");
    *stream = s->stream;
    return RN_OK;
}

int rn_session_set_cache(rn_session* s, int length, const uint16_t* keys, const uint16_t* values) {
    RN_REQUIRE(s && (length == 0 || (keys && values)), "null argument");
    RN_REQUIRE(length >= 0 && length <= s->capacity, "length %d outside 0..capacity (%d)", length, s->capacity);
    const rn_config& c = s->model->cfg;
    if (length > 0) {
        const size_t row = (size_t)length * c.head_dim * 2, pitch = (size_t)s->capacity * c.head_dim * 2;
        const size_t heads = (size_t)c.layers * c.heads;
        RN_HIP(hipMemcpy2DAsync(s->kc, pitch, keys, row, row, heads, hipMemcpyHostToDevice, s->stream));
        RN_HIP(hipMemcpy2DAsync(s->vc, pitch, values, row, row, heads, hipMemcpyHostToDevice, s->stream));
        RN_HIP(hipStreamSynchronize(s->stream));
    }
    s->length = length;
    s->has_hidden = false;
    return RN_OK;
}

int rn_session_get_cache(const rn_session* s, int length, uint16_t* keys, uint16_t* values) {
    RN_REQUIRE(s && keys && values, "null argument");
    RN_REQUIRE(length >= 0 && length <= s->capacity, "length %d outside 0..capacity", length);
    if (length == 0) return RN_OK;
    const rn_config& c = s->model->cfg;
    const size_t row = (size_t)length * c.head_dim * 2, pitch = (size_t)s->capacity * c.head_dim * 2;
    const size_t heads = (size_t)c.layers * c.heads;
    RN_HIP(hipStreamSynchronize(s->stream));
    RN_HIP(hipMemcpy2D(keys, row, s->kc, pitch, row, heads, hipMemcpyDeviceToHost));
    RN_HIP(hipMemcpy2D(values, row, s->vc, pitch, row, heads, hipMemcpyDeviceToHost));
    return RN_OK;
}

// The kernels of one decode step (session.rs:76-148): per layer the norm+QKV
// product (layer 0 gathers the embedding of state->token first), attention
// with rotary and the fp16 append, the out product + residual, the
// norm+gate/up product with silu(gate)*up, the down product + residual; then
// the final norm into `hidden`. With `greedy`, the tied-embedding product and
// the on-device argmax follow and feed the next step's embedding.
// Optional per-kernel timing of a decode step: every launch is armed with a
// start/stop event pair that hipExtLaunchKernelGGL records around the kernel
// itself; `kinds` gives each pair's kernel kind (RN_PROFILE_* order).
struct StepProbe {
    std::vector<hipEvent_t> events;  // 2 per launch
    std::vector<int> kinds;
    void arm() {
        const size_t i = kinds.size();
        if (2 * i + 1 < events.size()) {
            launch_events().start = events[2 * i];
            launch_events().stop = events[2 * i + 1];
        }
    }
    void done(int kind) { kinds.push_back(kind); }
};

// The blocks of the logits product of a greedy step: one argmax key each.
static int logits_blocks(const rn_config& c) {
    const int rpb = gemv_rows_per_block(c.vocab, c.d_model, kStore);
    return (c.vocab + rpb - 1) / rpb;
}

// A greedy step is: the head kernel of layer 0 reduces the previous step's
// block keys into the token it embeds (and records it in ids), the layers,
// then the logits product, which leaves its block keys and moves pos and step
// on. The choice of the last step is collected after the run
// (launch_argmax_finalize mode 1); the first step's token is planted as keys
// by launch_greedy_start.
static int enqueue_step(rn_session* s, bool greedy, StepProbe* probe = nullptr) {
    const rn_model* m = s->model;
    const rn_config& c = m->cfg;
    const int d = c.d_model;
    hipStream_t st = s->stream;
#define RN_PROFILED(kind, call) \
    do {                          \
        if (probe) probe->arm();  \
        RN_HIP(call);             \
        if (probe) probe->done(kind); \
    } while (0)
    for (int l = 0; l < c.layers; ++l) {
        const LayerDev& L = m->layers[l];
        {
            QkvAttendParams a{};
            a.W = L.qkv.W;
            a.sW = L.qkv.sW;
            a.x = s->x;
            a.gain = L.norm_attn;
            a.eps = c.norm_eps;
            a.embW = m->embedding.W;
            a.embS = m->embedding.sW;
            a.embed_scale = m->embed_scale;
            a.vocab = c.vocab;
            a.x_out = s->x;
            const size_t layer_base = (size_t)l * c.heads * s->capacity * c.head_dim;
            a.kc = s->kc + layer_base;
            a.vc = s->vc + layer_base;
            a.capacity = s->capacity;
            a.state = s->state;
            a.rope_cos = m->rope_cos;
            a.rope_sin = m->rope_sin;
            a.out = s->attn;
            a.keys = s->keys;
            a.nkeys = logits_blocks(c);
            a.logits = s->logits;
            a.ids = s->ids;
            const int pro = l > 0 ? kNorm : (greedy ? kEmbedArgmax : kEmbedNorm);
            RN_PROFILED(RN_PROFILE_QKV_ATTENTION, launch_qkv_attend(a, d, pro, c.heads, st));
        }
        {
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.out.W, L.out.sW, s->x, nullptr, d};
            p.x = s->attn;
            const int rpb = gemv_rows_per_block(d, d, kResidual);
            RN_PROFILED(RN_PROFILE_OUT, launch_gemv(p, d, kQuant, kResidual, kPanel, rpb, (d + rpb - 1) / rpb, st));
        }
        {
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.gate_up.W, L.gate_up.sW, s->ffh, nullptr, 2 * c.ffn};
            p.half_rows = c.ffn;
            p.x = s->x;
            p.gain = L.norm_ffn;
            p.eps = c.norm_eps;
            const int rpb = gemv_rows_per_block(2 * c.ffn, d, kSilu);
            RN_PROFILED(RN_PROFILE_GATE_UP, launch_gemv(p, d, kNorm, kSilu, kPanel, rpb, (c.ffn + rpb / 2 - 1) / (rpb / 2), st));
        }
        {
            // the 2048-wide input: four waves split the columns (quantise + product + residual)
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.down.W, L.down.sW, s->x, nullptr, d};
            p.x = s->ffh;
            RN_PROFILED(RN_PROFILE_DOWN, launch_gemv_splitk(p, c.ffn, d, st));
        }
    }
    if (!greedy) {
        RN_PROFILED(RN_PROFILE_FINAL, launch_finish_push(s->x, m->norm_final, d, c.norm_eps, s->hidden, s->state, st));
        return RN_OK;
    }
    // Greedy: the logits product takes the final norm as its prologue (block 0
    // also writes the hidden state), each block emits its greedy key, and block
    // 0 moves the position on; the next step's first kernel reduces the keys.
    GemvParams p{};
    p.nseg = 1;
    p.seg[0] = Segment{m->embedding.W, m->embedding.sW, s->logits, nullptr, c.vocab};
    p.x = s->x;
    p.gain = m->norm_final;
    p.eps = c.norm_eps;
    p.hidden_out = s->hidden;
    p.keys = s->keys;
    p.advance = s->state;
    const int rpb = gemv_rows_per_block(c.vocab, d, kStore);
    RN_PROFILED(RN_PROFILE_LOGITS, launch_gemv(p, d, kNorm, kArgmax, kPlane, rpb, logits_blocks(c), st));
    return RN_OK;
#undef RN_PROFILED
}

static int check_state_error(rn_session* s) {
    int32_t err = 0;
    RN_HIP(hipMemcpyAsync(&err, &s->state->error, sizeof err, hipMemcpyDeviceToHost, s->stream));
    RN_HIP(hipStreamSynchronize(s->stream));
    if (err) {
        RN_HIP(hipMemsetAsync(&s->state->error, 0, sizeof(int32_t), s->stream));
        RN_HIP(hipStreamSynchronize(s->stream));
        return fail(RN_ERR_STATE, "device reported error flags 0x%x (1: token >= vocab, 2: position >= capacity)", err);
    }
    return RN_OK;
}

int rn_session_push(rn_session* s, uint32_t token) {
    RN_REQUIRE(s, "session is null");
    RN_REQUIRE(token < (uint32_t)s->model->cfg.vocab, "token %u outside the vocabulary (%d)", token,
               s->model->cfg.vocab);
    if (s->length >= s->capacity) return fail(RN_ERR_CAPACITY, "session is full (%d positions)", s->capacity);
    RN_HIP(launch_set_state(s->state, token, s->length, 0, 0, s->stream));
    int rc = enqueue_step(s, false);
    if (rc) return rc;
    s->length += 1;
    s->has_hidden = true;
    return RN_OK;
}

int rn_session_hidden(const rn_session* s, float* out) {
    RN_REQUIRE(s && out, "null argument");
    if (!s->has_hidden) return fail(RN_ERR_STATE, "no token has been pushed");
    RN_HIP(hipMemcpyAsync(out, s->hidden, 4 * (size_t)s->model->cfg.d_model, hipMemcpyDeviceToHost, s->stream));
    RN_HIP(hipStreamSynchronize(s->stream));
    return RN_OK;
}

int rn_session_logits(rn_session* s, float* out) {
    RN_REQUIRE(s && out, "null argument");
    if (!s->has_hidden) return fail(RN_ERR_STATE, "no token has been pushed");
    const rn_model* m = s->model;
    const rn_config& c = m->cfg;
    GemvParams p{};
    p.nseg = 1;
    p.seg[0] = Segment{m->embedding.W, m->embedding.sW, s->logits, nullptr, c.vocab};
    p.x = s->hidden;
    const int rpb = gemv_rows_per_block(c.vocab, c.d_model, kStore);
    RN_HIP(launch_gemv(p, c.d_model, kQuant, kStore, kPlane, rpb, (c.vocab + rpb - 1) / rpb, s->stream));
    RN_HIP(hipMemcpyAsync(out, s->logits, 4 * (size_t)c.vocab, hipMemcpyDeviceToHost, s->stream));
    return check_state_error(s);
}

// ---- speech front end -------------------------------------------------------------

struct rn_frontend {
    FrontendParams p{};
    float* tables = nullptr;  // window gains, twiddles, mel weights
};

// Frontend::new (frontend.rs:31-40): the Hann window and the twiddles in float
// from cosf / sinf, computed here on the host as the reference does.
int rn_frontend_create(int mels, int fft_size, int window, int hop, const float* mel_weights, rn_frontend** out) {
    RN_REQUIRE(mel_weights && out, "null argument");
    RN_REQUIRE(mels >= 1 && mels <= 256, "mels must be 1..256 (got %d)", mels);
    RN_REQUIRE(fft_size >= 2 && fft_size <= 4096 && (fft_size & (fft_size - 1)) == 0,
               "fft_size must be a power of two in 2..4096 (got %d)", fft_size);
    RN_REQUIRE(window >= 2 && hop >= 1, "window must be at least 2 and hop positive");
    const int bins = fft_size / 2 + 1, half = fft_size / 2;
    std::vector<float> host((size_t)window + 2 * half + (size_t)bins * mels);
    float* win = host.data();
    float* tc = win + window;
    float* ts = tc + half;
    const float pi = 3.14159265358979323846f;
    for (int n = 0; n < window; ++n) win[n] = 0.5f - 0.5f * cosf(((2.0f * pi) * (float)n) / (float)(window - 1));
    for (int k = 0; k < half; ++k) {
        tc[k] = cosf(((2.0f * pi) * (float)k) / (float)fft_size);
        ts[k] = -sinf(((2.0f * pi) * (float)k) / (float)fft_size);
    }
    std::copy(mel_weights, mel_weights + (size_t)bins * mels, ts + half);
    rn_frontend* f = new (std::nothrow) rn_frontend();
    if (!f) return fail(RN_ERR_MEMORY, "out of host memory");
    if (hipMalloc(&f->tables, sizeof(float) * host.size()) != hipSuccess) {
        delete f;
        return fail(RN_ERR_MEMORY, "device allocation failed");
    }
    if (hipMemcpy(f->tables, host.data(), sizeof(float) * host.size(), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(f->tables);
        delete f;
        return fail(RN_ERR_DEVICE, "upload of the front-end tables failed");
    }
    int log2 = 0;
    while ((1 << log2) < fft_size) ++log2;
    f->p = FrontendParams{mels, fft_size, log2, window, hop, f->tables, f->tables + window, f->tables + window + half,
                          f->tables + window + 2 * half};
    *out = f;
    return RN_OK;
}

int rn_frontend_free(rn_frontend* f) {
    if (!f) return RN_OK;
    (void)hipFree(f->tables);
    delete f;
    return RN_OK;
}

int rn_frontend_log_mel(rn_frontend* f, const float* samples, int n, float* features, int* frames, int* valid,
                        float* spread) {
    RN_REQUIRE(f && (samples || n == 0) && features && frames && valid && spread, "null argument");
    RN_REQUIRE(n >= 0, "n must be non-negative");
    const int nf = n / f->p.hop + 1;
    const size_t fb = sizeof(float) * (size_t)nf * f->p.mels;
    char* dev = nullptr;
    RN_HIP(hipMalloc(&dev, align_up(sizeof(float) * (size_t)n + 4) + fb + 4 * (1 + (size_t)f->p.mels)));
    float* ds = (float*)dev;
    float* dd = (float*)(dev + align_up(sizeof(float) * (size_t)n + 4));
    float* dspread = (float*)((char*)dd + fb);
    hipError_t e = n ? hipMemcpy(ds, samples, sizeof(float) * (size_t)n, hipMemcpyHostToDevice) : hipSuccess;
    if (e == hipSuccess) e = launch_log_mel(f->p, ds, n, dd, dspread, nullptr);
    if (e == hipSuccess) e = hipMemcpy(features, dd, fb, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(spread, dspread, sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(dev);
    RN_HIP(e);
    *frames = nf;
    *valid = n / f->p.hop;
    return RN_OK;
}

// ---- the multi-lane hyper-connection (lanes.rs) -------------------------------------

struct rn_lanes {
    int lanes = 0, width = 0, layers = 0;
    const rn_matrix* phi[3] = {nullptr, nullptr, nullptr};
    float* buf = nullptr;  // a_pre, a_post, a_res, b_pre, b_post, b_res, then scratch
    float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res, *normalised, *rotated, *pre;
};

int rn_lanes_create(int lanes, int width, int layers, const float* a_pre, const float* a_post, const float* a_res,
                    const float* b_pre, const float* b_post, const float* b_res, const rn_matrix* phi_pre,
                    const rn_matrix* phi_post, const rn_matrix* phi_res, rn_lanes** out) {
    RN_REQUIRE(a_pre && a_post && a_res && b_pre && b_post && b_res && phi_pre && phi_post && phi_res && out,
               "null argument");
    RN_REQUIRE(lanes >= 1 && lanes <= kMaxLanes, "lanes must be 1..%d (got %d)", kMaxLanes, lanes);
    RN_REQUIRE(width >= 1 && layers >= 1 && (lanes * width) % 8 == 0 && lanes * width <= 49152,
               "lanes * width must be a multiple of 8 up to 49152");
    const rn_matrix* phis[3] = {phi_pre, phi_post, phi_res};
    const int need[3] = {layers * lanes, layers * lanes, layers * lanes * lanes};
    for (int i = 0; i < 3; ++i) {
        RN_REQUIRE(phis[i]->bits != 0, "the routing matrices are codebook matrices");
        RN_REQUIRE(phis[i]->columns == lanes * width, "routing matrix %d has %d columns, the stream %d", i,
                   phis[i]->columns, lanes * width);
        RN_REQUIRE(phis[i]->rows >= need[i], "routing matrix %d has %d rows, %d needed", i, phis[i]->rows, need[i]);
        RN_REQUIRE(phis[i]->cb.padded == phi_pre->cb.padded && phis[i]->group == phi_pre->group,
                   "the routing matrices share padded columns and group (multiply_fused)");
        // a layer's rows start at layer * lanes (layer * lanes^2): for 2-bit
        // matrices the reference takes the integer panel path only from rows on
        // panels of four (matrix.rs:404-409), the only path built here
        RN_REQUIRE(phis[i]->bits != 2 || lanes % 4 == 0,
                   "2-bit routing matrices need lanes a multiple of 4 (got %d): the reference takes the float path", lanes);
    }
    rn_lanes* l = new (std::nothrow) rn_lanes();
    if (!l) return fail(RN_ERR_MEMORY, "out of host memory");
    // every slice starts on a 256-byte boundary (the kernels read the stream and
    // the rotated input as float4)
    auto round64 = [](size_t v) { return (v + 63) / 64 * 64; };
    const size_t nA = round64(layers), nB = round64((size_t)layers * lanes), nR = round64((size_t)layers * lanes * lanes);
    const size_t n = round64((size_t)lanes * width), padded = round64((size_t)phi_pre->cb.padded);
    const size_t total = 3 * nA + 2 * nB + nR + n + padded + lanes;
    if (hipMalloc(&l->buf, sizeof(float) * total) != hipSuccess) {
        delete l;
        return fail(RN_ERR_MEMORY, "device allocation failed");
    }
    float* p = l->buf;
    l->a_pre = p; p += nA;
    l->a_post = p; p += nA;
    l->a_res = p; p += nA;
    l->b_pre = p; p += nB;
    l->b_post = p; p += nB;
    l->b_res = p; p += nR;
    l->normalised = p; p += n;
    l->rotated = p; p += padded;
    l->pre = p;
    const std::pair<float*, const float*> up[6] = {{l->a_pre, a_pre}, {l->a_post, a_post}, {l->a_res, a_res},
                                                   {l->b_pre, b_pre}, {l->b_post, b_post}, {l->b_res, b_res}};
    const size_t sizes[6] = {(size_t)layers, (size_t)layers, (size_t)layers, (size_t)layers * lanes,
                             (size_t)layers * lanes, (size_t)layers * lanes * lanes};
    for (int i = 0; i < 6; ++i)
        if (hipMemcpy(up[i].first, up[i].second, sizeof(float) * sizes[i], hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(l->buf);
            delete l;
            return fail(RN_ERR_DEVICE, "upload of the lane tensors failed");
        }
    l->lanes = lanes;
    l->width = width;
    l->layers = layers;
    l->phi[0] = phi_pre;
    l->phi[1] = phi_post;
    l->phi[2] = phi_res;
    *out = l;
    return RN_OK;
}

int rn_lanes_free(rn_lanes* l) {
    if (!l) return RN_OK;
    (void)hipFree(l->buf);
    delete l;
    return RN_OK;
}

// LaneWeights::route (lanes.rs:48-84): unit_rms + fake_quantise_int8 of the
// stream, prepare with phi_pre, the three products over this layer's rows
// (multiply_fused, matrix.rs:167-193, one launch each), then the gates, the
// post gains and the Sinkhorn-normalised residual mix.
int rn_lanes_route(rn_lanes* l, int layer, int slot, const float* stream, float* input, float* post, float* residual,
                   void* stream_handle) {
    RN_REQUIRE(l && stream && input && post && residual, "null argument");
    RN_REQUIRE(layer >= 0 && layer < l->layers, "layer %d out of range [0, %d)", layer, l->layers);
    RN_REQUIRE(slot >= 0, "slot must be non-negative");
    hipStream_t s = (hipStream_t)stream_handle;
    const int L = l->lanes, n = L * l->width;
    RN_HIP(launch_lanes_prologue(stream, n, l->normalised, s));
    const rn_matrix* pre_m = l->phi[0];
    RN_HIP(launch_codebook_rotate(l->normalised, 1, n, pre_m->cb.padded, pre_m->group, pre_m->cb.wht_scale, l->rotated,
                                  s));
    float* outs[3] = {l->pre, post, residual};
    const int first[3] = {layer * L, layer * L, layer * L * L}, count[3] = {L, L, L * L};
    for (int i = 0; i < 3; ++i) {  // a row range of the matrix: the same blob from its first row
        CodebookParams v = l->phi[i]->cb;
        const int G = v.padded / v.group;
        v.packed += (size_t)first[i] * v.row_bytes;
        v.norms += (size_t)first[i] * G;
        v.rows = count[i];
        RN_HIP(launch_codebook_product(v, l->rotated, 1, outs[i], nullptr, s));
    }
    LanesRouteParams p{L, l->width, layer, slot, l->a_pre, l->a_post, l->a_res, l->b_pre, l->b_post, l->b_res,
                       stream, l->pre, post, residual, input};
    RN_HIP(launch_lanes_route(p, s));
    return RN_OK;
}

int rn_lanes_combine(const rn_lanes* l, const float* post, const float* residual, const float* stream,
                     const float* block_delta, float* next, void* stream_handle) {
    RN_REQUIRE(l && post && residual && stream && block_delta && next, "null argument");
    RN_HIP(launch_lanes_combine(l->lanes, l->width, post, residual, stream, block_delta, next,
                                (hipStream_t)stream_handle));
    return RN_OK;
}

// ---- the depth ladder (ladder.rs) ----------------------------------------------------

// ladder::order (ladder.rs:1-20): the first and last layer, then repeatedly the
// midpoint of the widest gap between chosen layers (the leftmost of equal gaps).
int rn_ladder_order(int layers, int32_t* order) {
    RN_REQUIRE(layers >= 0 && (order || layers == 0), "bad argument");
    if (layers <= 1) {
        for (int i = 0; i < layers; ++i) order[i] = i;
        return RN_OK;
    }
    std::vector<int> selected = {0, layers - 1};
    order[0] = 0;
    order[1] = layers - 1;
    for (int n = 2; n < layers; ++n) {
        std::sort(selected.begin(), selected.end());
        int best_gap = 0, best_left = 0, best_right = 0;
        for (size_t i = 0; i + 1 < selected.size(); ++i) {
            const int gap = selected[i + 1] - selected[i];
            if (gap > 1 && gap > best_gap) {  // ties keep the leftmost (the larger Reverse(left))
                best_gap = gap;
                best_left = selected[i];
                best_right = selected[i + 1];
            }
        }
        const int candidate = (best_left + best_right) / 2;
        selected.push_back(candidate);
        order[n] = candidate;
    }
    return RN_OK;
}

// ladder::select (ladder.rs:22-29): the first `depth` layers of the order, sorted;
// RN_ERR_ARGUMENT where the reference returns None.
int rn_ladder_select(int layers, int depth, int32_t* chosen) {
    RN_REQUIRE(chosen || depth == 0, "null argument");
    RN_REQUIRE(layers >= 0, "layers must be non-negative");
    if (depth < std::min(2, layers) || depth > layers)
        return fail(RN_ERR_ARGUMENT, "depth %d outside [%d, %d]", depth, std::min(2, layers), layers);
    std::vector<int32_t> order(layers);
    const int rc = rn_ladder_order(layers, order.data());
    if (rc != RN_OK) return rc;
    std::copy(order.begin(), order.begin() + depth, chosen);
    std::sort(chosen, chosen + depth);
    return RN_OK;
}

int rn_kronecker_apply(const float* input, const float* left, int left_size, const float* right, int right_size,
                       int count, float* output, void* stream) {
    RN_REQUIRE(input && left && right && output, "null argument");
    RN_REQUIRE(left_size == 32 && right_size == 32, "factors must be 32 x 32 (got %d and %d)", left_size, right_size);
    RN_REQUIRE(count >= 0, "count must be non-negative");
    RN_HIP(launch_kronecker32(input, left, right, count, output, (hipStream_t)stream));
    return RN_OK;
}

static_assert(sizeof(rn_choice) == sizeof(Choice), "rn_choice mirrors rn::Choice");

int rn_choose_allowed(const float* logits, const uint8_t* allowed, int n, int token, rn_choice* out, void* stream) {
    RN_REQUIRE(logits && allowed && out, "null argument");
    RN_REQUIRE(n >= 1, "n must be positive (got %d)", n);
    RN_REQUIRE(token < n, "token %d outside the %d logits", token, n);
    RN_HIP(launch_constrained_choice(logits, allowed, n, token < 0 ? -1 : token, reinterpret_cast<Choice*>(out),
                                     (hipStream_t)stream));
    return RN_OK;
}

int rn_session_choose_allowed(rn_session* s, const uint8_t* allowed, rn_choice* out) {
    RN_REQUIRE(s && allowed && out, "null argument");
    if (!s->has_hidden) return fail(RN_ERR_STATE, "no token has been pushed");
    const rn_model* m = s->model;
    const rn_config& c = m->cfg;
    if (!s->choice_buf) RN_HIP(hipMalloc(&s->choice_buf, align_up((size_t)c.vocab) + sizeof(Choice)));
    uint8_t* mask = (uint8_t*)s->choice_buf;
    Choice* choice = (Choice*)((char*)s->choice_buf + align_up((size_t)c.vocab));
    GemvParams p{};
    p.nseg = 1;
    p.seg[0] = Segment{m->embedding.W, m->embedding.sW, s->logits, nullptr, c.vocab};
    p.x = s->hidden;
    const int rpb = gemv_rows_per_block(c.vocab, c.d_model, kStore);
    RN_HIP(launch_gemv(p, c.d_model, kQuant, kStore, kPlane, rpb, (c.vocab + rpb - 1) / rpb, s->stream));
    RN_HIP(hipMemcpyAsync(mask, allowed, (size_t)c.vocab, hipMemcpyHostToDevice, s->stream));
    RN_HIP(launch_constrained_choice(s->logits, mask, c.vocab, -1, choice, s->stream));
    RN_HIP(hipMemcpyAsync(out, choice, sizeof(Choice), hipMemcpyDeviceToHost, s->stream));
    RN_HIP(hipStreamSynchronize(s->stream));
    return check_state_error(s);
}

int rn_session_decode_greedy(rn_session* s, uint32_t first, int steps, uint32_t* ids) {
    RN_REQUIRE(s && (ids || steps == 0), "null argument");
    RN_REQUIRE(steps >= 0, "steps must be non-negative");
    RN_REQUIRE(first < (uint32_t)s->model->cfg.vocab, "token %u outside the vocabulary", first);
    if (steps == 0) return RN_OK;
    if (s->length + steps > s->capacity)
        return fail(RN_ERR_CAPACITY, "%d + %d positions exceed the capacity %d", s->length, steps, s->capacity);
    // RN_DECODE_GRAPH=0 launches the step's kernels directly instead of replaying
    // the captured graph (same kernels, same results; for kernel-level tracing).
    static const bool use_graph = [] {
        const char* e = getenv("RN_DECODE_GRAPH");
        return !(e && e[0] == '0');
    }();
    const int nkeys = logits_blocks(s->model->cfg);
    if (!use_graph) {
        RN_HIP(launch_greedy_start(s->state, first, s->length, (uint32_t)s->capacity, s->keys, nkeys, s->logits,
                                   s->stream));
        for (int i = 0; i < steps; ++i) {
            const int rc = enqueue_step(s, true);
            if (rc) return rc;
        }
        RN_HIP(launch_argmax_finalize(s->keys, nkeys, s->logits, s->state, s->ids, s->stream, 1));
        RN_HIP(hipMemcpyAsync(ids, s->ids, 4 * (size_t)steps, hipMemcpyDeviceToHost, s->stream));
        s->length += steps;
        s->has_hidden = true;
        return check_state_error(s);
    }
    if (!s->step_graph) {
        hipGraph_t graph = nullptr;
        RN_HIP(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_step(s, true);
        hipError_t e = hipStreamEndCapture(s->stream, &graph);
        if (rc) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        RN_HIP(e);
        e = hipGraphInstantiate(&s->step_graph, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        RN_HIP(e);
    }
    RN_HIP(launch_greedy_start(s->state, first, s->length, (uint32_t)s->capacity, s->keys, nkeys, s->logits,
                               s->stream));
    for (int i = 0; i < steps; ++i) RN_HIP(hipGraphLaunch(s->step_graph, s->stream));
    RN_HIP(launch_argmax_finalize(s->keys, nkeys, s->logits, s->state, s->ids, s->stream, 1));
    RN_HIP(hipMemcpyAsync(ids, s->ids, 4 * (size_t)steps, hipMemcpyDeviceToHost, s->stream));
    s->length += steps;
    s->has_hidden = true;
    return check_state_error(s);
}

int rn_session_profile_step(rn_session* s, uint32_t first, int steps, float* kind_us, int* kind_count) {
    RN_REQUIRE(s && kind_us && kind_count, "null argument");
    RN_REQUIRE(steps >= 1, "steps must be positive");
    RN_REQUIRE(first < (uint32_t)s->model->cfg.vocab, "token %u outside the vocabulary", first);
    if (s->length + steps > s->capacity)
        return fail(RN_ERR_CAPACITY, "%d + %d positions exceed the capacity %d", s->length, steps, s->capacity);
    const size_t launches = ((size_t)s->model->cfg.layers * 5 + 2) * steps;
    StepProbe probe;
    probe.events.resize(2 * launches);
    for (auto& e : probe.events) RN_HIP(hipEventCreate(&e));
    int rc = RN_OK;
    const int nkeys = logits_blocks(s->model->cfg);
    hipError_t e = launch_greedy_start(s->state, first, s->length, (uint32_t)s->capacity, s->keys, nkeys, s->logits,
                                       s->stream);
    for (int i = 0; i < steps && rc == RN_OK && e == hipSuccess; ++i) rc = enqueue_step(s, true, &probe);
    launch_events() = LaunchEvents{};
    if (e == hipSuccess && rc == RN_OK)
        e = launch_argmax_finalize(s->keys, nkeys, s->logits, s->state, s->ids, s->stream, 1);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    double sum[RN_PROFILE_KINDS] = {0};
    int count[RN_PROFILE_KINDS] = {0};
    for (size_t i = 0; i < probe.kinds.size() && e == hipSuccess; ++i) {
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, probe.events[2 * i], probe.events[2 * i + 1]);
        sum[probe.kinds[i]] += ms * 1000.0;
        count[probe.kinds[i]] += 1;
    }
    for (auto& ev : probe.events) (void)hipEventDestroy(ev);
    if (rc) return rc;
    RN_HIP(e);
    for (int k = 0; k < RN_PROFILE_KINDS; ++k) {
        kind_us[k] = count[k] ? (float)(sum[k] / count[k]) : 0.0f;
        kind_count[k] = count[k] / steps;
    }
    s->length += steps;
    s->has_hidden = true;
    return check_state_error(s);
}

static int ensure_scratch(rn_session* s, int count) {
    if (count <= s->scratch_tokens) return RN_OK;
    const rn_config& c = s->model->cfg;
    const size_t d = c.d_model, f = c.ffn;
    const size_t bytes = align_up(4 * count * d) * 3 + align_up(4 * count * 3 * d) + align_up(4 * count * f) +
                         align_up(count * (f > d ? f : d)) + align_up(4 * (size_t)count) + align_up(4 * (size_t)count);
    RN_HIP(hipStreamSynchronize(s->stream));
    if (s->scratch) RN_HIP(hipFree(s->scratch));
    s->scratch = nullptr;
    s->scratch_tokens = 0;
    if (hipMalloc(&s->scratch, bytes) != hipSuccess) return fail(RN_ERR_MEMORY, "prefill scratch of %zu bytes", bytes);
    s->scratch_tokens = count;
    return RN_OK;
}

// Session::feed / prefill (session.rs:56-70, prefill.rs:10-99): all tokens of
// the chunk go through each layer together; the products run on i8 MFMA.
int rn_session_feed(rn_session* s, const uint32_t* tokens, int count) {
    RN_REQUIRE(s && (tokens || count == 0), "null argument");
    RN_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return RN_OK;
    const rn_model* m = s->model;
    const rn_config& c = m->cfg;
    for (int i = 0; i < count; ++i)
        RN_REQUIRE(tokens[i] < (uint32_t)c.vocab, "token %u at %d outside the vocabulary", tokens[i], i);
    if (s->length + count > s->capacity)
        return fail(RN_ERR_CAPACITY, "%d + %d positions exceed the capacity %d", s->length, count, s->capacity);
    int rc = ensure_scratch(s, count);
    if (rc) return rc;
    const int d = c.d_model, f = c.ffn;
    Arena a{(char*)s->scratch, 0, 0};
    float* X = (float*)a.take(4 * (size_t)count * d);
    float* Q = (float*)a.take(4 * (size_t)count * d);
    float* A = (float*)a.take(4 * (size_t)count * d);
    float* QKV = (float*)a.take(4 * (size_t)count * 3 * d);
    float* F = (float*)a.take(4 * (size_t)count * f);
    int8_t* Xq = (int8_t*)a.take((size_t)count * (f > d ? f : d));
    float* sx = (float*)a.take(4 * (size_t)count);
    uint32_t* tok = (uint32_t*)a.take(4 * (size_t)count);
    hipStream_t st = s->stream;
    const int first = s->length;
    RN_HIP(hipMemcpyAsync(tok, tokens, 4 * (size_t)count, hipMemcpyHostToDevice, st));
    RN_HIP(launch_embed_rows(tok, count, m->embedding.W, m->embedding.sW, d, c.vocab, m->embed_scale, X,
                             &s->state->error, st));
    // a product over float rows (quantised by the product, after the norm when
    // `gain` is set); Xq / sx take the codes where a separate quantise runs
    auto rows = [&](const float* in, const float* gain, const DevMatrix& w, int N, int K, float* Y, int ldy, int half) {
        GemmParams g{Xq, sx, w.W, w.sW, count, N, K, Y, ldy, nullptr, half};
        g.Xf = in;
        g.gain = gain;
        g.eps = c.norm_eps;
        return g;
    };
    for (int l = 0; l < c.layers; ++l) {
        const LayerDev& L = m->layers[l];
        GemmParams qkv = rows(X, L.norm_attn, L.qkv, 3 * d, d, QKV, 3 * d, 0);
        if ((d == 384 || d == 512) && c.heads * 64 == d) {
            // the product's epilogue rotates q and k and appends k and v
            qkv.rope = GemmRope{Q, s->kc, s->vc, m->rope_cos, m->rope_sin, l, c.heads, s->capacity, first};
            RN_HIP(launch_gemm(qkv, kGemmRope, kPanel, false, st));
        } else {
            RN_HIP(launch_gemm(qkv, kGemmStore, kPanel, false, st));
            RN_HIP(launch_rope_append(QKV, Q, s->kc, s->vc, l, c.heads, s->capacity, d, first, count, m->rope_cos,
                                      m->rope_sin, st));
        }
        AttendParams ap{};
        ap.q = Q;
        ap.kc = s->kc;
        ap.vc = s->vc;
        ap.layer = l;
        ap.heads = c.heads;
        ap.capacity = s->capacity;
        ap.d_model = d;
        ap.first = first;
        ap.out = A;
        ap.error = &s->state->error;
        RN_HIP(launch_attend_prefill(ap, c.heads, count, st));
        RN_HIP(launch_gemm(rows(A, nullptr, L.out, d, d, X, d, 0), kGemmResidual, kPanel, false, st));
        RN_HIP(launch_gemm(rows(X, L.norm_ffn, L.gate_up, 2 * f, d, F, f, f), kGemmSilu, kPanel, false, st));
        RN_HIP(launch_gemm(rows(F, nullptr, L.down, d, f, X, d, 0), kGemmResidual, kPanel, false, st));
    }
    RN_HIP(hipMemcpyAsync(s->x, X + (size_t)(count - 1) * d, 4 * (size_t)d, hipMemcpyDeviceToDevice, st));
    RN_HIP(launch_norm_rows(s->x, m->norm_final, 1, d, c.norm_eps, s->hidden, st));
    s->length += count;
    s->has_hidden = true;
    return check_state_error(s);
}

// ---- Batch ------------------------------------------------------------------------

int rn_batch_create(const rn_model* m, int count, int capacity, rn_batch** out) {
    RN_REQUIRE(m && out, "null argument");
    const rn_config& c = m->cfg;
    RN_REQUIRE(count >= 1 && count <= 4096, "count must be 1..4096");
    RN_REQUIRE(capacity >= 1 && capacity <= c.max_positions && capacity <= 16384, "capacity must be 1..max_positions");
    rn_batch* b = new (std::nothrow) rn_batch();
    if (!b) return fail(RN_ERR_MEMORY, "out of host memory");
    b->model = m;
    b->count = count;
    b->capacity = capacity;
    b->lengths.assign(count, 0);
    const size_t ce = cache_elems(c, capacity) * count, d = c.d_model, f = c.ffn, n = count;
    const size_t total = 2 * align_up(ce * 2) + align_up(4 * n) + align_up(4 * n * d) * 2 + align_up(4 * n * 3 * d) +
                         align_up(4 * n * f) + align_up(4 * n * c.vocab) + align_up(n * (f > d ? f : d)) +
                         align_up(4 * n) * 3 + align_up(256);
    if (hipMalloc(&b->arena, total) != hipSuccess) {
        delete b;
        return fail(RN_ERR_MEMORY, "device allocation of %zu bytes failed", total);
    }
    Arena a{(char*)b->arena, 0, total};
    b->kc = (__half*)a.take(ce * 2);
    b->vc = (__half*)a.take(ce * 2);
    b->pos = (int32_t*)a.take(4 * n);
    b->X = (float*)a.take(4 * n * d);
    b->A = (float*)a.take(4 * n * d);
    b->QKV = (float*)a.take(4 * n * 3 * d);
    b->F = (float*)a.take(4 * n * f);
    b->logits = (float*)a.take(4 * n * c.vocab);
    b->Xq = (int8_t*)a.take(n * (f > d ? f : d));
    b->sx = (float*)a.take(4 * n);
    b->tokens = (uint32_t*)a.take(4 * n);
    b->error = (int32_t*)a.take(4 * n);
    b->step = (int32_t*)a.take(256);
    if (hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking) != hipSuccess ||
        hipMemsetAsync(b->arena, 0, total, b->stream) != hipSuccess || hipStreamSynchronize(b->stream) != hipSuccess) {
        if (b->stream) (void)hipStreamDestroy(b->stream);
        (void)hipFree(b->arena);
        delete b;
        return fail(RN_ERR_DEVICE, "batch initialisation failed");
    }
    *out = b;
    return RN_OK;
}

int rn_batch_free(rn_batch* b) {
    if (!b) return RN_OK;
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    if (b->step_graph) (void)hipGraphExecDestroy(b->step_graph);
    if (b->ids) (void)hipFree(b->ids);
    (void)hipFree(b->arena);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
    return RN_OK;
}

int rn_batch_truncate(rn_batch* b, const int32_t* lengths) {
    RN_REQUIRE(b && lengths, "null argument");
    for (int i = 0; i < b->count; ++i)
        RN_REQUIRE(lengths[i] >= 0 && lengths[i] <= b->lengths[i], "sequence %d: length %d outside 0..%d", i, lengths[i],
                   b->lengths[i]);
    for (int i = 0; i < b->count; ++i) b->lengths[i] = lengths[i];
    return RN_OK;
}

int rn_batch_stream(const rn_batch* b, void** stream) {
    RN_REQUIRE(b && stream, "null argument");
    *stream = b->stream;
    return RN_OK;
}

int rn_batch_set_cache(rn_batch* b, int sequence, int length, const uint16_t* keys, const uint16_t* values) {
    RN_REQUIRE(b && (length == 0 || (keys && values)), "null argument");
    RN_REQUIRE(sequence >= 0 && sequence < b->count, "sequence %d outside 0..%d", sequence, b->count);
    RN_REQUIRE(length >= 0 && length <= b->capacity, "length %d outside 0..capacity", length);
    const rn_config& c = b->model->cfg;
    const size_t seq = cache_elems(c, b->capacity) * sequence;
    if (length > 0) {
        const size_t row = (size_t)length * c.head_dim * 2, pitch = (size_t)b->capacity * c.head_dim * 2;
        const size_t heads = (size_t)c.layers * c.heads;
        RN_HIP(hipMemcpy2DAsync(b->kc + seq, pitch, keys, row, row, heads, hipMemcpyHostToDevice, b->stream));
        RN_HIP(hipMemcpy2DAsync(b->vc + seq, pitch, values, row, row, heads, hipMemcpyHostToDevice, b->stream));
    }
    b->lengths[sequence] = length;
    RN_HIP(hipMemcpyAsync(b->pos + sequence, &b->lengths[sequence], 4, hipMemcpyHostToDevice, b->stream));
    RN_HIP(hipStreamSynchronize(b->stream));
    return RN_OK;
}

// One step for every sequence: embed the current tokens, the layer stack with
// M=count MFMA products and ragged attention, the final norm, the tied logits
// product and a per-row argmax that becomes the next tokens. The step's ids
// slot and the positions are read from the device (b->step, b->pos), so the
// same launches serve every step: the step is captured once as a hipGraph.
static int enqueue_batch_step(rn_batch* b, int steps) {
    const rn_model* m = b->model;
    const rn_config& c = m->cfg;
    const int n = b->count, d = c.d_model, f = c.ffn;
    hipStream_t st = b->stream;
    RN_HIP(launch_embed_rows(b->tokens, n, m->embedding.W, m->embedding.sW, d, c.vocab, m->embed_scale, b->X, b->error,
                             st));
    // a product over float rows (quantised by the product, after the norm when
    // `gain` is set); Xq / sx take the codes where a separate quantise runs
    auto rows = [&](const float* in, const float* gain, const DevMatrix& w, int N, int K, float* Y, int ldy, int half) {
        GemmParams g{b->Xq, b->sx, w.W, w.sW, n, N, K, Y, ldy, nullptr, half};
        g.Xf = in;
        g.gain = gain;
        g.eps = c.norm_eps;
        return g;
    };
    for (int l = 0; l < c.layers; ++l) {
        const LayerDev& L = m->layers[l];
        RN_HIP(launch_gemm(rows(b->X, L.norm_attn, L.qkv, 3 * d, d, b->QKV, 3 * d, 0), kGemmStore, kPanel, false, st));
        AttendParams ap{};
        ap.qkv = b->QKV;
        ap.kc = b->kc;
        ap.vc = b->vc;
        ap.seq_stride = cache_elems(c, b->capacity);
        ap.layer = l;
        ap.heads = c.heads;
        ap.capacity = b->capacity;
        ap.d_model = d;
        ap.pos = b->pos;
        ap.pos_stride = 1;
        ap.rope_cos = m->rope_cos;
        ap.rope_sin = m->rope_sin;
        ap.out = b->A;
        ap.error = b->error;
        RN_HIP(launch_attend(ap, kAttendDecode, c.heads, n, b->capacity, st));
        RN_HIP(launch_gemm(rows(b->A, nullptr, L.out, d, d, b->X, d, 0), kGemmResidual, kPanel, false, st));
        RN_HIP(launch_gemm(rows(b->X, L.norm_ffn, L.gate_up, 2 * f, d, b->F, f, f), kGemmSilu, kPanel, false, st));
        RN_HIP(launch_gemm(rows(b->F, nullptr, L.down, d, f, b->X, d, 0), kGemmResidual, kPanel, false, st));
    }
    // final norm, then the per-row quantisation of the hidden state (session.rs:140-142, 166-177)
    RN_HIP(launch_norm_quantise(b->X, m->norm_final, n, d, c.norm_eps, b->Xq, b->sx, nullptr, st));
    RN_HIP(launch_gemm(GemmParams{b->Xq, b->sx, m->embedding.W, m->embedding.sW, n, c.vocab, d, b->logits, c.vocab,
                                  nullptr, 0},
                       kGemmStore, kPlane, false, st));
    RN_HIP(launch_argmax_rows(b->logits, n, c.vocab, b->tokens, b->ids, steps, 0, st, b->step));
    RN_HIP(launch_advance_positions(b->pos, n, 1, st, b->step));
    return RN_OK;
}

int rn_batch_decode_greedy(rn_batch* b, const uint32_t* first, int steps, uint32_t* ids) {
    RN_REQUIRE(b && first && (ids || steps == 0), "null argument");
    RN_REQUIRE(steps >= 0, "steps must be non-negative");
    if (steps == 0) return RN_OK;
    const rn_config& c = b->model->cfg;
    for (int i = 0; i < b->count; ++i) {
        RN_REQUIRE(first[i] < (uint32_t)c.vocab, "first token %u of sequence %d outside the vocabulary", first[i], i);
        if (b->lengths[i] + steps > b->capacity)
            return fail(RN_ERR_CAPACITY, "sequence %d: %d + %d positions exceed the capacity %d", i, b->lengths[i], steps,
                        b->capacity);
    }
    if (b->ids_steps < steps) {
        RN_HIP(hipStreamSynchronize(b->stream));
        if (b->ids) RN_HIP(hipFree(b->ids));
        b->ids = nullptr;
        if (hipMalloc(&b->ids, 4 * (size_t)b->count * steps) != hipSuccess) return fail(RN_ERR_MEMORY, "id buffer");
        b->ids_steps = steps;
        if (b->step_graph) RN_HIP(hipGraphExecDestroy(b->step_graph));
        b->step_graph = nullptr;
    }
    RN_HIP(hipMemcpyAsync(b->tokens, first, 4 * (size_t)b->count, hipMemcpyHostToDevice, b->stream));
    RN_HIP(hipMemcpyAsync(b->pos, b->lengths.data(), 4 * (size_t)b->count, hipMemcpyHostToDevice, b->stream));
    RN_HIP(hipMemsetAsync(b->step, 0, sizeof(int32_t), b->stream));
    // RN_DECODE_GRAPH=0 launches the step's kernels directly (same kernels,
    // same arguments; for kernel-level tracing)
    static const bool use_graph = [] {
        const char* e = getenv("RN_DECODE_GRAPH");
        return !(e && e[0] == '0');
    }();
    if (!use_graph) {
        for (int step = 0; step < steps; ++step) {
            int rc = enqueue_batch_step(b, steps);
            if (rc) return rc;
        }
    } else {
        if (b->step_graph && b->graph_steps != steps) {
            RN_HIP(hipGraphExecDestroy(b->step_graph));
            b->step_graph = nullptr;
        }
        if (!b->step_graph) {
            hipGraph_t graph = nullptr;
            RN_HIP(hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue_batch_step(b, steps);
            hipError_t e = hipStreamEndCapture(b->stream, &graph);
            if (rc) {
                if (graph) (void)hipGraphDestroy(graph);
                return rc;
            }
            RN_HIP(e);
            e = hipGraphInstantiate(&b->step_graph, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            RN_HIP(e);
            b->graph_steps = steps;
        }
        for (int step = 0; step < steps; ++step) RN_HIP(hipGraphLaunch(b->step_graph, b->stream));
    }
    RN_HIP(hipMemcpyAsync(ids, b->ids, 4 * (size_t)b->count * steps, hipMemcpyDeviceToHost, b->stream));
    int32_t err = 0;
    RN_HIP(hipMemcpyAsync(&err, b->error, 4, hipMemcpyDeviceToHost, b->stream));
    RN_HIP(hipStreamSynchronize(b->stream));
    for (int i = 0; i < b->count; ++i) b->lengths[i] += steps;
    b->has_logits = true;
    if (err) return fail(RN_ERR_STATE, "device reported error flags 0x%x", err);
    return RN_OK;
}

int rn_batch_logits(const rn_batch* b, float* out) {
    RN_REQUIRE(b && out, "null argument");
    if (!b->has_logits) return fail(RN_ERR_STATE, "no decode step has run on this batch");
    RN_HIP(hipStreamSynchronize(b->stream));
    RN_HIP(hipMemcpy(out, b->logits, sizeof(float) * (size_t)b->count * b->model->cfg.vocab, hipMemcpyDeviceToHost));
    return RN_OK;
}

int rn_batch_get_cache(const rn_batch* b, int sequence, int length, uint16_t* keys, uint16_t* values) {
    RN_REQUIRE(b && keys && values, "null argument");
    RN_REQUIRE(sequence >= 0 && sequence < b->count, "sequence %d outside 0..%d", sequence, b->count);
    RN_REQUIRE(length >= 0 && length <= b->lengths[sequence], "length %d outside 0..%d", length, b->lengths[sequence]);
    if (length == 0) return RN_OK;
    const rn_config& c = b->model->cfg;
    const size_t seq = cache_elems(c, b->capacity) * sequence;
    const size_t row = (size_t)length * c.head_dim * 2, pitch = (size_t)b->capacity * c.head_dim * 2;
    const size_t heads = (size_t)c.layers * c.heads;
    RN_HIP(hipStreamSynchronize(b->stream));
    RN_HIP(hipMemcpy2D(keys, row, b->kc + seq, pitch, row, heads, hipMemcpyDeviceToHost));
    RN_HIP(hipMemcpy2D(values, row, b->vc + seq, pitch, row, heads, hipMemcpyDeviceToHost));
    return RN_OK;
}

// ---- Whistle-style speech path --------------------------------------------------

}  // extern "C"

namespace {

struct WEncLayerDev {
    DevMatrix qkv, out, gate_up, down;
    float *norm_attn = nullptr, *norm_ffn = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct WDecLayerDev {
    DevMatrix qkv, out, cross_q, cross_kv, cross_out, gate_up, down;
    float *norm_attn = nullptr, *norm_cross = nullptr, *post_norm = nullptr, *norm_ffn = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr;
    float cross_gain = 0.0f;
};

// cross.rs:61-72 for frames 0..T-1 (host libm, as the CPU restatement).
void whistle_position(int T, int d, float gate, std::vector<float>& out) {
    const int half = d / 2;
    const float rate = -logf(10000.0f) / ((float)half - 1.0f);
    out.assign((size_t)T * d, 0.0f);
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < half; ++j) {
            const float angle = (float)t * expf(rate * (float)j);
            out[(size_t)t * d + j] = gate * sinf(angle);
            out[(size_t)t * d + half + j] = gate * cosf(angle);
        }
}

float host_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }  // ops.rs:68-71

}  // namespace

struct rn_whistle {
    rn_whistle_config cfg{};
    int T = 0;  // encoder frames
    hipStream_t stream = nullptr;
    void* arena = nullptr;
    float* conv1 = nullptr;
    DevMatrix conv2;  // [d][3 d]
    std::vector<WEncLayerDev> enc;
    float* enc_norm = nullptr;
    float* position = nullptr;
    DevMatrix embedding;
    std::vector<WDecLayerDev> dec;
    float* dec_norm = nullptr;
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    std::vector<float> position_host, gains_host;
    float embed_scale = 0.0f;
    // encoder work
    float *mel = nullptr, *h1 = nullptr, *R = nullptr, *X = nullptr, *Y = nullptr, *F = nullptr, *ctx = nullptr;
    float* encoded = nullptr;
    int8_t* Xq = nullptr;
    float* sx = nullptr;
    int8_t *qc = nullptr, *kc = nullptr, *vc = nullptr;
    float *qs = nullptr, *ks = nullptr, *vs = nullptr;
    // cross memory [dec_layers][T][heads][64] and scales [dec_layers][T][heads]
    int8_t *mem_k = nullptr, *mem_v = nullptr;
    float *mem_ks = nullptr, *mem_vs = nullptr;
    bool encoded_ready = false;
    char* fe_buf = nullptr;  // rn_whistle_encode_samples: samples, features and spread (grown as needed)
    size_t fe_bytes = 0;
    // the decoder session
    __half *kcache = nullptr, *vcache = nullptr;
    int capacity = 0, length = 0;
    bool has_hidden = false;
    float *x = nullptr, *x2 = nullptr, *attn = nullptr, *catt = nullptr;
    float* cpart = nullptr;  // cross-attention value sums per position class [32][d]
    float *ffh = nullptr, *hidden = nullptr, *logits = nullptr;
    DecodeState* state = nullptr;
    uint32_t* ids = nullptr;
    unsigned long long* keys = nullptr;
};

extern "C" {

static int validate_whistle(const rn_whistle_config* c) {
    RN_REQUIRE(c, "config is null");
    RN_REQUIRE(c->d_model == 384 || c->d_model == 512, "d_model must be 384 or 512 (got %d)", c->d_model);
    RN_REQUIRE(c->head_dim == 64 && c->heads * 64 == c->d_model, "heads of 64 must tile d_model");
    RN_REQUIRE(c->ffn == 512 || c->ffn == 1024 || c->ffn == 1536 || c->ffn == 2048, "ffn must be 512, 1024, 1536 or 2048");
    RN_REQUIRE(c->group == kGroup, "group must be 32");
    RN_REQUIRE(c->mels >= 1 && c->mels <= 128, "mels must be 1..128");
    RN_REQUIRE(c->frames >= 2 && c->frames <= 65536, "frames must be 2..65536");
    RN_REQUIRE(c->enc_layers >= 1 && c->enc_layers <= 64 && c->dec_layers >= 1 && c->dec_layers <= 64,
               "layers must be 1..64");
    RN_REQUIRE(c->vocab >= 1 && c->max_positions >= 1 && c->max_positions <= 16384, "vocab / max_positions");
    RN_REQUIRE(c->norm_eps == 1e-6f, "norm_eps must be 1e-6 (the reference's NORM_EPSILON)");
    return RN_OK;
}

// The synthetic weights drawn by name (the same draws as
// rustyneedle_amd.synthetic_whistle_weights), then rn_whistle_create.
int rn_whistle_create_synthetic(const rn_whistle_config* config, uint64_t seed, rn_whistle** out) {
    int rc = validate_whistle(config);
    if (rc) return rc;
    RN_REQUIRE(out, "out is null");
    const rn_whistle_config& c = *config;
    const size_t d = c.d_model, f = c.ffn, M = c.mels, V = c.vocab;
    struct Q {
        std::vector<int8_t> codes;
        std::vector<float> scales;
        rn_qmat_host host() const { return rn_qmat_host{codes.data(), scales.data()}; }
    };
    auto gen_q = [&](const std::string& name, size_t rows, size_t cols) {
        Q q;
        q.codes.resize(rows * cols);
        q.scales.resize(rows * (cols / kGroup));
        rn_synth_codes(seed, (name + ".codes").c_str(), q.codes.data(), q.codes.size());
        rn_synth_uniform(seed, (name + ".scales").c_str(), 1e-3f, 1e-2f, q.scales.data(), q.scales.size());
        return q;
    };
    auto gen_normal = [&](const std::string& name, float sigma, size_t n) {
        std::vector<float> g(n);
        rn_synth_normal(seed, name.c_str(), sigma, g.data(), n);
        return g;
    };
    std::vector<float> conv1 = gen_normal("whistle.conv1", 1.0f / sqrtf((float)(3 * M)), d * 3 * M);
    Q conv2 = gen_q("whistle.conv2", d, 3 * d);
    struct EncHost { Q qkv, out, gate_up, down; std::vector<float> norm_attn, norm_ffn, q_norm, k_norm; };
    struct DecHost {
        Q qkv, out, cross_q, cross_kv, cross_out, gate_up, down;
        std::vector<float> norm_attn, norm_cross, post_norm, norm_ffn, q_norm, k_norm;
        float gate;
    };
    std::vector<EncHost> eh(c.enc_layers);
    std::vector<rn_whistle_enc_host> ew(c.enc_layers);
    for (int l = 0; l < c.enc_layers; ++l) {
        const std::string p = "whistle.enc." + std::to_string(l) + ".";
        eh[l].qkv = gen_q(p + "qkv", 3 * d, d);
        eh[l].out = gen_q(p + "out", d, d);
        eh[l].gate_up = gen_q(p + "gate_up", 2 * f, d);
        eh[l].down = gen_q(p + "down", d, f);
        eh[l].norm_attn = gen_normal(p + "norm_attn", 0.1f, d);
        eh[l].norm_ffn = gen_normal(p + "norm_ffn", 0.1f, d);
        eh[l].q_norm = gen_normal(p + "q_norm", 0.1f, 64);
        eh[l].k_norm = gen_normal(p + "k_norm", 0.1f, 64);
        ew[l] = rn_whistle_enc_host{eh[l].qkv.host(), eh[l].out.host(), eh[l].gate_up.host(), eh[l].down.host(),
                                    eh[l].norm_attn.data(), eh[l].norm_ffn.data(), eh[l].q_norm.data(),
                                    eh[l].k_norm.data()};
    }
    std::vector<float> enc_norm = gen_normal("whistle.enc_norm", 0.1f, d);
    const float position_gate = gen_normal("whistle.position_gate", 1.0f, 1)[0];
    Q embedding = gen_q("whistle.embedding", V, d);
    std::vector<DecHost> dh(c.dec_layers);
    std::vector<rn_whistle_dec_host> dw(c.dec_layers);
    for (int l = 0; l < c.dec_layers; ++l) {
        const std::string p = "whistle.dec." + std::to_string(l) + ".";
        dh[l].qkv = gen_q(p + "qkv", 3 * d, d);
        dh[l].out = gen_q(p + "out", d, d);
        dh[l].cross_q = gen_q(p + "cross_q", d, d);
        dh[l].cross_kv = gen_q(p + "cross_kv", 2 * d, d);
        dh[l].cross_out = gen_q(p + "cross_out", d, d);
        dh[l].gate_up = gen_q(p + "gate_up", 2 * f, d);
        dh[l].down = gen_q(p + "down", d, f);
        dh[l].norm_attn = gen_normal(p + "norm_attn", 0.1f, d);
        dh[l].norm_cross = gen_normal(p + "norm_cross", 0.1f, d);
        dh[l].post_norm = gen_normal(p + "post_norm", 0.1f, d);
        dh[l].norm_ffn = gen_normal(p + "norm_ffn", 0.1f, d);
        dh[l].q_norm = gen_normal(p + "q_norm", 0.1f, 64);
        dh[l].k_norm = gen_normal(p + "k_norm", 0.1f, 64);
        dh[l].gate = gen_normal(p + "gate", 1.0f, 1)[0];
        dw[l] = rn_whistle_dec_host{dh[l].qkv.host(), dh[l].out.host(), dh[l].cross_q.host(), dh[l].cross_kv.host(),
                                    dh[l].cross_out.host(), dh[l].gate_up.host(), dh[l].down.host(),
                                    dh[l].norm_attn.data(), dh[l].norm_cross.data(), dh[l].post_norm.data(),
                                    dh[l].norm_ffn.data(), dh[l].q_norm.data(), dh[l].k_norm.data(), dh[l].gate};
    }
    std::vector<float> dec_norm = gen_normal("whistle.dec_norm", 0.1f, d);
    rn_whistle_weights_host wh{conv1.data(), conv2.host(), ew.data(), enc_norm.data(), position_gate,
                               embedding.host(), dw.data(), dec_norm.data()};
    return rn_whistle_create(config, &wh, out);
}

int rn_whistle_create(const rn_whistle_config* config, const rn_whistle_weights_host* wh, rn_whistle** out) {
    int rc = validate_whistle(config);
    if (rc) return rc;
    RN_REQUIRE(out && wh, "null argument");
    RN_REQUIRE(wh->conv1 && wh->conv2.codes && wh->conv2.scales && wh->enc && wh->enc_norm && wh->embedding.codes &&
                   wh->embedding.scales && wh->dec && wh->dec_norm,
               "null weight pointer");
    const rn_whistle_config& c = *config;
    auto qok = [](const rn_qmat_host& q) { return q.codes != nullptr && q.scales != nullptr; };
    for (int l = 0; l < c.enc_layers; ++l) {
        const rn_whistle_enc_host& e = wh->enc[l];
        RN_REQUIRE(qok(e.qkv) && qok(e.out) && qok(e.gate_up) && qok(e.down) && e.norm_attn && e.norm_ffn && e.q_norm &&
                       e.k_norm,
                   "encoder layer %d has a null weight pointer", l);
    }
    for (int l = 0; l < c.dec_layers; ++l) {
        const rn_whistle_dec_host& e = wh->dec[l];
        RN_REQUIRE(qok(e.qkv) && qok(e.out) && qok(e.cross_q) && qok(e.cross_kv) && qok(e.cross_out) &&
                       qok(e.gate_up) && qok(e.down) && e.norm_attn && e.norm_cross && e.post_norm && e.norm_ffn &&
                       e.q_norm && e.k_norm,
                   "decoder layer %d has a null weight pointer", l);
    }
    const size_t d = c.d_model, f = c.ffn, H = c.heads, M = c.mels, Fr = c.frames, V = c.vocab;
    const size_t T = (size_t)(c.frames - 1) / 2 + 1;
    RN_REQUIRE(T <= 1536, "at most 1536 encoder frames (3072 mel frames): the attention stages a head's values in LDS");
    rn_whistle* w = new (std::nothrow) rn_whistle();
    if (!w) return fail(RN_ERR_MEMORY, "out of host memory");
    w->cfg = c;
    w->T = (int)T;
    w->embed_scale = sqrtf((float)d);
    w->capacity = c.max_positions;
    whistle_position((int)T, (int)d, host_sigmoid(wh->position_gate), w->position_host);
    rn_config rc_rope{};
    rc_rope.head_dim = 64;
    rc_rope.rope_theta = c.rope_theta;
    rc_rope.max_positions = (int)std::max(T, (size_t)c.max_positions);
    std::vector<float> rope_cos, rope_sin;
    rotary_table(rc_rope, rope_cos, rope_sin);

    // one device arena: weights, tables, work buffers, the cross memory, the session
    const size_t Dm = std::max(std::max(d, f), 3 * d), L = c.dec_layers, cap = c.max_positions;
    auto qbytes = [](size_t rows, size_t cols) { return align_up(rows * cols) + align_up(rows * (cols / kGroup) * 4); };
    const size_t conv1_floats = d * 3 * M;
    size_t total = align_up(4 * conv1_floats) + qbytes(d, 3 * d);
    total += (size_t)c.enc_layers * (qbytes(3 * d, d) + qbytes(d, d) + qbytes(2 * f, d) + qbytes(d, f) +
                                     2 * align_up(4 * d) + 2 * align_up(4 * 64));
    total += align_up(4 * d) + align_up(4 * T * d) + qbytes(V, d);
    total += L * (qbytes(3 * d, d) + 3 * qbytes(d, d) + qbytes(2 * d, d) + qbytes(2 * f, d) + qbytes(d, f) +
                  4 * align_up(4 * d) + 2 * align_up(4 * 64));
    total += align_up(4 * d) + 2 * align_up(4 * rope_cos.size());
    total += align_up(4 * Fr * M) + align_up(4 * (Fr + 2) * d) + align_up(4 * T * d) * 4 + align_up(4 * T * 3 * d) +
             align_up(4 * T * Dm) + align_up(T * Dm) + align_up(4 * T) + 3 * align_up(T * d) + 3 * align_up(4 * T * H);
    total += 2 * align_up(L * T * d) + 2 * align_up(4 * L * T * H);
    total += 2 * align_up(2 * L * H * cap * 64) + 5 * align_up(4 * d) + align_up(4 * 32 * d) + align_up(4 * 3 * d) +
             align_up(4 * f) + align_up(4 * V) + align_up(sizeof(DecodeState)) + align_up(4 * cap) + align_up(8 * V);
    if (hipMalloc(&w->arena, total) != hipSuccess) {
        delete w;
        return fail(RN_ERR_MEMORY, "device allocation of %zu bytes failed", total);
    }
    Arena a{(char*)w->arena, 0, total};
    std::vector<std::pair<void*, std::pair<const void*, size_t>>> uploads;
    auto place = [&](const void* src, size_t bytes) {
        void* dst = a.take(bytes);
        uploads.push_back({dst, {src, bytes}});
        return dst;
    };
    auto placeq = [&](const rn_qmat_host& q, size_t rows, size_t cols) {
        DevMatrix dm;
        dm.W = (int8_t*)place(q.codes, rows * cols);
        dm.sW = (float*)place(q.scales, rows * (cols / kGroup) * 4);
        return dm;
    };
    w->conv1 = (float*)place(wh->conv1, 4 * conv1_floats);
    w->conv2 = placeq(wh->conv2, d, 3 * d);
    w->enc.resize(c.enc_layers);
    for (int l = 0; l < c.enc_layers; ++l) {
        const rn_whistle_enc_host& e = wh->enc[l];
        WEncLayerDev& D = w->enc[l];
        D.qkv = placeq(e.qkv, 3 * d, d);
        D.out = placeq(e.out, d, d);
        D.gate_up = placeq(e.gate_up, 2 * f, d);
        D.down = placeq(e.down, d, f);
        D.norm_attn = (float*)place(e.norm_attn, 4 * d);
        D.norm_ffn = (float*)place(e.norm_ffn, 4 * d);
        D.q_norm = (float*)place(e.q_norm, 4 * 64);
        D.k_norm = (float*)place(e.k_norm, 4 * 64);
    }
    w->enc_norm = (float*)place(wh->enc_norm, 4 * d);
    w->position = (float*)place(w->position_host.data(), 4 * T * d);
    w->embedding = placeq(wh->embedding, V, d);
    w->dec.resize(L);
    w->gains_host.resize(L);
    for (size_t l = 0; l < L; ++l) {
        const rn_whistle_dec_host& e = wh->dec[l];
        WDecLayerDev& D = w->dec[l];
        D.qkv = placeq(e.qkv, 3 * d, d);
        D.out = placeq(e.out, d, d);
        D.cross_q = placeq(e.cross_q, d, d);
        D.cross_kv = placeq(e.cross_kv, 2 * d, d);
        D.cross_out = placeq(e.cross_out, d, d);
        D.gate_up = placeq(e.gate_up, 2 * f, d);
        D.down = placeq(e.down, d, f);
        D.norm_attn = (float*)place(e.norm_attn, 4 * d);
        D.norm_cross = (float*)place(e.norm_cross, 4 * d);
        D.post_norm = (float*)place(e.post_norm, 4 * d);
        D.norm_ffn = (float*)place(e.norm_ffn, 4 * d);
        D.q_norm = (float*)place(e.q_norm, 4 * 64);
        D.k_norm = (float*)place(e.k_norm, 4 * 64);
        D.cross_gain = w->gains_host[l] = host_sigmoid(e.gate);
    }
    w->dec_norm = (float*)place(wh->dec_norm, 4 * d);
    w->rope_cos = (float*)place(rope_cos.data(), 4 * rope_cos.size());
    w->rope_sin = (float*)place(rope_sin.data(), 4 * rope_sin.size());
    w->mel = (float*)a.take(4 * Fr * M);
    w->h1 = (float*)a.take(4 * (Fr + 2) * d);  // the first convolution's output, one zero row before and after
    w->R = (float*)a.take(4 * T * d);  // the memory input
    w->X = (float*)a.take(4 * T * d);
    w->ctx = (float*)a.take(4 * T * d);
    w->encoded = (float*)a.take(4 * T * d);
    w->Y = (float*)a.take(4 * T * 3 * d);
    w->F = (float*)a.take(4 * T * Dm);
    w->Xq = (int8_t*)a.take(T * Dm);
    w->sx = (float*)a.take(4 * T);
    w->qc = (int8_t*)a.take(T * d);
    w->kc = (int8_t*)a.take(T * d);
    w->vc = (int8_t*)a.take(T * d);
    w->qs = (float*)a.take(4 * T * H);
    w->ks = (float*)a.take(4 * T * H);
    w->vs = (float*)a.take(4 * T * H);
    w->mem_k = (int8_t*)a.take(L * T * d);
    w->mem_v = (int8_t*)a.take(L * T * d);
    w->mem_ks = (float*)a.take(4 * L * T * H);
    w->mem_vs = (float*)a.take(4 * L * T * H);
    w->kcache = (__half*)a.take(2 * L * H * cap * 64);
    w->vcache = (__half*)a.take(2 * L * H * cap * 64);
    w->x = (float*)a.take(4 * d);
    w->x2 = (float*)a.take(4 * d);
    w->attn = (float*)a.take(4 * d);
    w->cpart = (float*)a.take(4 * 32 * d);
    w->catt = (float*)a.take(4 * d);
    w->hidden = (float*)a.take(4 * d);
    w->ffh = (float*)a.take(4 * f);
    w->logits = (float*)a.take(4 * V);
    w->state = (DecodeState*)a.take(sizeof(DecodeState));
    w->ids = (uint32_t*)a.take(4 * cap);
    w->keys = (unsigned long long*)a.take(8 * V);
    if (a.used > total || hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipFree(w->arena);
        delete w;
        return fail(RN_ERR_MEMORY, "arena layout (%zu of %zu bytes) or stream creation failed", a.used, total);
    }
    for (auto& u : uploads) {
        if (hipMemcpy(u.first, u.second.first, u.second.second, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipStreamDestroy(w->stream);
            (void)hipFree(w->arena);
            delete w;
            return fail(RN_ERR_DEVICE, "weight upload failed");
        }
    }
    // the zero rows around the first convolution's output, and the decoder state
    if (hipMemsetAsync(w->h1, 0, 4 * d, w->stream) != hipSuccess ||
        hipMemsetAsync(w->h1 + (Fr + 1) * d, 0, 4 * d, w->stream) != hipSuccess ||
        hipMemsetAsync(w->state, 0, sizeof(DecodeState), w->stream) != hipSuccess ||
        hipStreamSynchronize(w->stream) != hipSuccess) {
        (void)hipStreamDestroy(w->stream);
        (void)hipFree(w->arena);
        delete w;
        return fail(RN_ERR_DEVICE, "state initialisation failed");
    }
    *out = w;
    return RN_OK;
}

int rn_whistle_free(rn_whistle* w) {
    if (!w) return RN_OK;
    if (w->stream) {
        (void)hipStreamSynchronize(w->stream);
        (void)hipStreamDestroy(w->stream);
    }
    if (w->fe_buf) (void)hipFree(w->fe_buf);
    (void)hipFree(w->arena);
    delete w;
    return RN_OK;
}

int rn_whistle_frames(const rn_whistle* w, int* frames) {
    RN_REQUIRE(w && frames, "null argument");
    *frames = w->T;
    return RN_OK;
}

int rn_whistle_tables(const rn_whistle* w, float* position, float* cross_gains) {
    RN_REQUIRE(w, "whistle is null");
    if (position) memcpy(position, w->position_host.data(), 4 * w->position_host.size());
    if (cross_gains) memcpy(cross_gains, w->gains_host.data(), 4 * w->gains_host.size());
    return RN_OK;
}

int rn_whistle_stream(const rn_whistle* w, void** stream) {
    RN_REQUIRE(w && stream, "null argument");
    *stream = w->stream;
    return RN_OK;
}

// stem.rs:39-115 as two conv1d layers: the first convolution + silu into rows
// 1..F of h1 (rows 0 and F + 1 stay zero), then the second (kernel 3, stride 2)
// as the int8 product of conv2 with the im2col rows: row t is h1 rows 2t..2t+2
// (frames 2t-1..2t+1), contiguous, so the rows are read in place with a
// stride of two frames and quantised per row; silu, into w->X.
// The stem over host features (copied to the device first) or, with
// `on_device`, over features already on the device ([frames][mels], the first
// c.frames rows read).
static int whistle_stem(rn_whistle* w, const float* mel, bool on_device = false) {
    const rn_whistle_config& c = w->cfg;
    const int d = c.d_model, T = w->T;
    hipStream_t st = w->stream;
    const float* src = mel;
    if (!on_device) {
        RN_HIP(hipMemcpyAsync(w->mel, mel, 4 * (size_t)c.frames * c.mels, hipMemcpyHostToDevice, st));
        src = w->mel;
    }
    RN_HIP(launch_stem(src, w->conv1, c.frames, c.mels, d, w->h1 + d, st));
    RN_HIP(launch_quantise_strided(w->h1, 2 * (size_t)d, T, 3 * d, w->Xq, w->sx, st));
    RN_HIP(launch_gemm(GemmParams{w->Xq, w->sx, w->conv2.W, w->conv2.sW, T, d, 3 * d, w->X, d, nullptr, 0},
                       kGemmStoreSilu, kPanel, false, st));
    return RN_OK;
}

int rn_whistle_stem(rn_whistle* w, const float* mel, float* out) {
    RN_REQUIRE(w && mel && out, "null argument");
    int rc = whistle_stem(w, mel);
    if (rc) return rc;
    RN_HIP(hipMemcpyAsync(out, w->X, 4 * (size_t)w->T * w->cfg.d_model, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipStreamSynchronize(w->stream));
    return RN_OK;
}

// encoder.rs:145-297 for one synthetic layer over w->X.
static int whistle_encoder_layer(rn_whistle* w, int l) {
    const rn_whistle_config& c = w->cfg;
    const int d = c.d_model, T = w->T, H = c.heads, f = c.ffn;
    const WEncLayerDev& L = w->enc[l];
    hipStream_t st = w->stream;
    RN_HIP(launch_norm_quantise(w->X, L.norm_attn, T, d, c.norm_eps, w->Xq, w->sx, nullptr, st));
    RN_HIP(launch_gemm(GemmParams{w->Xq, w->sx, L.qkv.W, L.qkv.sW, T, 3 * d, d, w->Y, 3 * d, nullptr, 0}, kGemmStore,
                       kPanel, false, st));
    HeadCodesParams hp{};
    hp.src = w->Y;
    hp.src_stride = 3 * d;
    hp.frames = T;
    hp.heads = H;
    hp.nsec = 3;
    hp.sec[0] = HeadSection{0, L.q_norm, 1, 1.0f / sqrtf(64.0f), w->qc, w->qs};
    hp.sec[1] = HeadSection{d, L.k_norm, 1, 1.0f, w->kc, w->ks};
    hp.sec[2] = HeadSection{2 * d, nullptr, 0, 1.0f, w->vc, w->vs};
    hp.rope_cos = w->rope_cos;
    hp.rope_sin = w->rope_sin;
    hp.pos0 = 0;
    hp.eps = c.norm_eps;
    RN_HIP(launch_head_codes(hp, st));
    Int8AttendParams ap{w->qc, w->qs, w->kc, w->ks, w->vc, w->vs, T, H, w->ctx, d};
    RN_HIP(launch_int8_attend(ap, T, st));
    RN_HIP(launch_norm_quantise(w->ctx, nullptr, T, d, c.norm_eps, w->Xq, w->sx, nullptr, st));
    RN_HIP(launch_gemm(GemmParams{w->Xq, w->sx, L.out.W, L.out.sW, T, d, d, w->X, d, nullptr, 0}, kGemmResidual, kPanel,
                       false, st));
    RN_HIP(launch_norm_quantise(w->X, L.norm_ffn, T, d, c.norm_eps, w->Xq, w->sx, nullptr, st));
    RN_HIP(launch_gemm(GemmParams{w->Xq, w->sx, L.gate_up.W, L.gate_up.sW, T, 2 * f, d, w->F, f, nullptr, f},
                       kGemmSilu, kPanel, false, st));
    RN_HIP(launch_norm_quantise(w->F, nullptr, T, f, c.norm_eps, w->Xq, w->sx, nullptr, st));
    RN_HIP(launch_gemm(GemmParams{w->Xq, w->sx, L.down.W, L.down.sW, T, d, f, w->X, d, nullptr, 0}, kGemmResidual,
                       kPanel, false, st));
    return RN_OK;
}

// cross.rs:58-99: position term added, rows quantised, then per decoder layer
// the key/value product and their per-head codes (keys after k_norm).
static int whistle_memory(rn_whistle* w) {
    const rn_whistle_config& c = w->cfg;
    const int d = c.d_model, T = w->T, H = c.heads;
    hipStream_t st = w->stream;
    RN_HIP(launch_add(w->encoded, w->position, (size_t)T * d, w->R, st));
    RN_HIP(launch_norm_quantise(w->R, nullptr, T, d, c.norm_eps, w->Xq, w->sx, nullptr, st));
    for (int l = 0; l < c.dec_layers; ++l) {
        const WDecLayerDev& L = w->dec[l];
        RN_HIP(launch_gemm(GemmParams{w->Xq, w->sx, L.cross_kv.W, L.cross_kv.sW, T, 2 * d, d, w->Y, 2 * d, nullptr, 0},
                           kGemmStore, kPanel, false, st));
        HeadCodesParams hp{};
        hp.src = w->Y;
        hp.src_stride = 2 * d;
        hp.frames = T;
        hp.heads = H;
        hp.nsec = 2;
        const size_t off = (size_t)l * T * d, soff = (size_t)l * T * H;
        hp.sec[0] = HeadSection{0, L.k_norm, 0, 1.0f, w->mem_k + off, w->mem_ks + soff};
        hp.sec[1] = HeadSection{d, nullptr, 0, 1.0f, w->mem_v + off, w->mem_vs + soff};
        hp.eps = c.norm_eps;
        RN_HIP(launch_head_codes(hp, st));
    }
    return RN_OK;
}

static int whistle_encode(rn_whistle* w, const float* mel, bool on_device, float* encoded) {
    const rn_whistle_config& c = w->cfg;
    int rc = whistle_stem(w, mel, on_device);
    if (rc) return rc;
    for (int l = 0; l < c.enc_layers; ++l) {
        rc = whistle_encoder_layer(w, l);
        if (rc) return rc;
    }
    RN_HIP(launch_norm_rows(w->X, w->enc_norm, w->T, c.d_model, c.norm_eps, w->encoded, w->stream));
    rc = whistle_memory(w);
    if (rc) return rc;
    if (encoded)
        RN_HIP(hipMemcpyAsync(encoded, w->encoded, 4 * (size_t)w->T * c.d_model, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipStreamSynchronize(w->stream));
    w->encoded_ready = true;
    w->length = 0;
    w->has_hidden = false;
    return RN_OK;
}

int rn_whistle_encode(rn_whistle* w, const float* mel, float* encoded) {
    RN_REQUIRE(w && mel, "null argument");
    return whistle_encode(w, mel, false, encoded);
}

// Whistle::encode from samples (lib.rs:155-161): Frontend::log_mel on the
// device into a buffer the stem then reads in place, so the features make no
// round trip through the host. The front end must give the model's frames
// (valid = n / hop == frames) of its mels; the frame past the valid ones is
// zero after the normalisation, as the stem's zero padding is.
int rn_whistle_encode_samples(rn_whistle* w, const rn_frontend* f, const float* samples, int n, float* encoded,
                              float* spread) {
    RN_REQUIRE(w && f && (samples || n == 0), "null argument");
    RN_REQUIRE(n >= 0, "n must be non-negative");
    const rn_whistle_config& c = w->cfg;
    RN_REQUIRE(f->p.mels == c.mels, "the front end has %d mels, the model %d", f->p.mels, c.mels);
    RN_REQUIRE(n / f->p.hop == c.frames, "%d samples give %d valid frames, the model takes %d", n, n / f->p.hop,
               c.frames);
    const int nf = n / f->p.hop + 1;
    const size_t sb = align_up(sizeof(float) * (size_t)n + 4), fb = align_up(sizeof(float) * (size_t)nf * c.mels);
    const size_t need = sb + fb + align_up(4 * (1 + (size_t)c.mels));
    if (w->fe_bytes < need) {
        RN_HIP(hipStreamSynchronize(w->stream));
        if (w->fe_buf) RN_HIP(hipFree(w->fe_buf));
        w->fe_buf = nullptr;
        w->fe_bytes = 0;
        if (hipMalloc(&w->fe_buf, need) != hipSuccess) return fail(RN_ERR_MEMORY, "front-end buffer of %zu bytes", need);
        w->fe_bytes = need;
    }
    float* ds = (float*)w->fe_buf;
    float* dd = (float*)(w->fe_buf + sb);
    float* dspread = (float*)(w->fe_buf + sb + fb);
    if (n) RN_HIP(hipMemcpyAsync(ds, samples, sizeof(float) * (size_t)n, hipMemcpyHostToDevice, w->stream));
    RN_HIP(launch_log_mel(f->p, ds, n, dd, dspread, w->stream));
    if (spread) RN_HIP(hipMemcpyAsync(spread, dspread, sizeof(float), hipMemcpyDeviceToHost, w->stream));
    return whistle_encode(w, dd, true, encoded);
}

int rn_whistle_memory(const rn_whistle* w, int8_t* keys, float* key_scales, int8_t* values, float* value_scales) {
    RN_REQUIRE(w && keys && key_scales && values && value_scales, "null argument");
    RN_REQUIRE(w->encoded_ready, "no audio has been encoded");
    const size_t n = (size_t)w->cfg.dec_layers * w->T * w->cfg.d_model;
    const size_t ns = (size_t)w->cfg.dec_layers * w->T * w->cfg.heads;
    RN_HIP(hipMemcpyAsync(keys, w->mem_k, n, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipMemcpyAsync(values, w->mem_v, n, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipMemcpyAsync(key_scales, w->mem_ks, 4 * ns, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipMemcpyAsync(value_scales, w->mem_vs, 4 * ns, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipStreamSynchronize(w->stream));
    return RN_OK;
}

int rn_whistle_reset(rn_whistle* w) {
    RN_REQUIRE(w, "whistle is null");
    w->length = 0;
    w->has_hidden = false;
    return RN_OK;
}

// One decoder step (session.rs:76-148 with the cross hook of cross.rs:126-182):
// per layer the self-attention block, the cross-attention block and the gated
// FFN; then either the final norm (push) or the logits product with the
// on-device greedy argmax (decode).
static int enqueue_whistle_step(rn_whistle* w, bool greedy) {
    const rn_whistle_config& c = w->cfg;
    const int d = c.d_model, H = c.heads, f = c.ffn, T = w->T;
    hipStream_t st = w->stream;
    for (int l = 0; l < c.dec_layers; ++l) {
        const WDecLayerDev& L = w->dec[l];
        {
            QkvAttendParams a{};
            a.W = L.qkv.W;
            a.sW = L.qkv.sW;
            a.x = w->x;
            a.gain = L.norm_attn;
            a.eps = c.norm_eps;
            a.embW = w->embedding.W;
            a.embS = w->embedding.sW;
            a.embed_scale = w->embed_scale;
            a.vocab = c.vocab;
            a.x_out = w->x;
            const size_t layer_base = (size_t)l * H * w->capacity * 64;
            a.kc = w->kcache + layer_base;
            a.vc = w->vcache + layer_base;
            a.capacity = w->capacity;
            a.state = w->state;
            a.rope_cos = w->rope_cos;
            a.rope_sin = w->rope_sin;
            a.out = w->attn;
            RN_HIP(launch_qkv_attend(a, d, l == 0 ? kEmbedNorm : kNorm, H, st));
        }
        {
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.out.W, L.out.sW, w->x, nullptr, d};
            p.x = w->attn;
            const int rpb = gemv_rows_per_block(d, d, kResidual);
            RN_HIP(launch_gemv(p, d, kQuant, kResidual, kPanel, rpb, (d + rpb - 1) / rpb, st));
        }
        {
            // norm, q product, q codes and attention in one launch; it leaves
            // the value sums per position class, which the out product adds
            const size_t off = (size_t)l * T * d, soff = (size_t)l * T * H;
            CrossAttendParams ap{L.cross_q.W, L.cross_q.sW, w->x, L.norm_cross, L.q_norm, c.norm_eps,
                                 w->mem_k + off, w->mem_ks + soff, w->mem_v + off, w->mem_vs + soff,
                                 T, H, w->cpart};
            RN_HIP(launch_cross_attend(ap, d, st));
        }
        {
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.cross_out.W, L.cross_out.sW, w->catt, nullptr, d};
            p.x = w->cpart;
            const int rpb = gemv_rows_per_block(d, d, kStore);
            RN_HIP(launch_gemv(p, d, kClassSum, kStore, kPanel, rpb, (d + rpb - 1) / rpb, st));
        }
        {
            // the cross residual in every block's prologue (block 0 keeps the sum
            // in x2, read by the down product as its residual: x itself is read
            // by the other blocks of this launch), then the FFN norm
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.gate_up.W, L.gate_up.sW, w->ffh, nullptr, 2 * f};
            p.half_rows = f;
            p.x = w->x;
            p.attended = w->catt;
            p.post_gain = L.post_norm;
            p.cross_gain = L.cross_gain;
            p.x_out = w->x2;
            p.gain = L.norm_ffn;
            p.eps = c.norm_eps;
            const int rpb = gemv_rows_per_block(2 * f, d, kSilu);
            RN_HIP(launch_gemv(p, d, kCrossNorm, kSilu, kPanel, rpb, (f + rpb / 2 - 1) / (rpb / 2), st));
        }
        {
            GemvParams p{};
            p.nseg = 1;
            p.seg[0] = Segment{L.down.W, L.down.sW, w->x, nullptr, d};
            p.res = w->x2;
            p.x = w->ffh;
            const int rpb = gemv_rows_per_block(d, f, kResidual);
            RN_HIP(launch_gemv(p, f, kQuant, kResidual, kPanel, rpb, (d + rpb - 1) / rpb, st));
        }
    }
    if (!greedy) {
        RN_HIP(launch_finish_push(w->x, w->dec_norm, d, c.norm_eps, w->hidden, w->state, st));
        return RN_OK;
    }
    GemvParams p{};
    p.nseg = 1;
    p.seg[0] = Segment{w->embedding.W, w->embedding.sW, w->logits, nullptr, c.vocab};
    p.x = w->x;
    p.gain = w->dec_norm;
    p.eps = c.norm_eps;
    p.hidden_out = w->hidden;
    p.keys = w->keys;
    const int rpb = gemv_rows_per_block(c.vocab, d, kStore);
    const int blocks = (c.vocab + rpb - 1) / rpb;
    RN_HIP(launch_gemv(p, d, kNorm, kArgmax, kPlane, rpb, blocks, st));
    RN_HIP(launch_argmax_finalize(w->keys, blocks, w->logits, w->state, w->ids, st));
    return RN_OK;
}

static int whistle_state_error(rn_whistle* w) {
    int32_t err = 0;
    RN_HIP(hipMemcpyAsync(&err, &w->state->error, sizeof err, hipMemcpyDeviceToHost, w->stream));
    RN_HIP(hipStreamSynchronize(w->stream));
    if (err) {
        RN_HIP(hipMemsetAsync(&w->state->error, 0, sizeof(int32_t), w->stream));
        RN_HIP(hipStreamSynchronize(w->stream));
        return fail(RN_ERR_STATE, "device reported error flags 0x%x (1: token >= vocab, 2: position >= capacity)", err);
    }
    return RN_OK;
}

int rn_whistle_push(rn_whistle* w, uint32_t token) {
    RN_REQUIRE(w, "whistle is null");
    RN_REQUIRE(w->encoded_ready, "no audio has been encoded");
    RN_REQUIRE(token < (uint32_t)w->cfg.vocab, "token %u outside the vocabulary (%d)", token, w->cfg.vocab);
    if (w->length >= w->capacity) return fail(RN_ERR_CAPACITY, "decoder is full (%d positions)", w->capacity);
    RN_HIP(launch_set_state(w->state, token, w->length, 0, 0, w->stream));
    int rc = enqueue_whistle_step(w, false);
    if (rc) return rc;
    w->length += 1;
    w->has_hidden = true;
    return whistle_state_error(w);
}

int rn_whistle_logits(rn_whistle* w, float* out) {
    RN_REQUIRE(w && out, "null argument");
    if (!w->has_hidden) return fail(RN_ERR_STATE, "no token has been pushed");
    const rn_whistle_config& c = w->cfg;
    GemvParams p{};
    p.nseg = 1;
    p.seg[0] = Segment{w->embedding.W, w->embedding.sW, w->logits, nullptr, c.vocab};
    p.x = w->hidden;
    const int rpb = gemv_rows_per_block(c.vocab, c.d_model, kStore);
    RN_HIP(launch_gemv(p, c.d_model, kQuant, kStore, kPlane, rpb, (c.vocab + rpb - 1) / rpb, w->stream));
    RN_HIP(hipMemcpyAsync(out, w->logits, 4 * (size_t)c.vocab, hipMemcpyDeviceToHost, w->stream));
    return whistle_state_error(w);
}

int rn_whistle_decode_greedy(rn_whistle* w, uint32_t first, int steps, uint32_t* ids) {
    RN_REQUIRE(w && (ids || steps == 0), "null argument");
    RN_REQUIRE(w->encoded_ready, "no audio has been encoded");
    RN_REQUIRE(steps >= 0, "steps must be non-negative");
    RN_REQUIRE(first < (uint32_t)w->cfg.vocab, "token %u outside the vocabulary", first);
    if (steps == 0) return RN_OK;
    if (w->length + steps > w->capacity)
        return fail(RN_ERR_CAPACITY, "%d + %d positions exceed the capacity %d", w->length, steps, w->capacity);
    RN_HIP(launch_set_state(w->state, first, w->length, 0, (uint32_t)w->capacity, w->stream));
    for (int i = 0; i < steps; ++i) {
        const int rc = enqueue_whistle_step(w, true);
        if (rc) return rc;
    }
    RN_HIP(hipMemcpyAsync(ids, w->ids, 4 * (size_t)steps, hipMemcpyDeviceToHost, w->stream));
    w->length += steps;
    w->has_hidden = true;
    return whistle_state_error(w);
}

}  // extern "C"
