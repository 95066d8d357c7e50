// rn_archive.cpp — the .cact archive reader (host code).
//
// Replaces crates/cact (archive.rs, geometry.rs, record.rs, cursor.rs) for
// what the product path needs: the 196-byte header (geometry.rs:39-114), the
// codebook section (archive.rs:45-50), the directory of 44-byte records
// (record.rs:38-51) with the bounds and alignment checks of archive.rs:56-70,
// and the bytes of a tensor (archive.rs:88-96). The file is memory-mapped and
// never copied; rn_matrix_from_archive (QuantisedMatrix::from_archive,
// matrix.rs:35-40) uploads one codebook-quantised record to the device.
// The archive is little-endian (docs/format.md), as is every host here.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <vector>

#include "../../include/rustyneedle.h"
#include "rn_internal.hpp"

namespace {

constexpr uint32_t kFormatTag = 0x05E12A84u;  // geometry.rs:4
constexpr size_t kHeaderBytes = 196;          // geometry.rs:5
constexpr size_t kRecordBytes = 44;           // record.rs:4

// Little-endian reads that fail past the end (cursor.rs:19-44).
struct Cursor {
    const uint8_t* bytes;
    size_t size, pos;
    bool ok = true;
    template <typename T>
    T take() {
        T v{};
        if (!ok || pos + sizeof(T) > size) {
            ok = false;
            return v;
        }
        memcpy(&v, bytes + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
};

}  // namespace

struct rn_archive {
    const uint8_t* data = nullptr;
    size_t size = 0;
    bool mapped = false;
    std::vector<uint8_t> owned;  // rn_archive_from_memory keeps a copy
    rn_geometry geometry{};
    std::vector<float> codebook;
    std::vector<rn_tensor_record> records;
};

namespace {

int archive_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return rn::set_error(code, buf);
}

// Archive::from_map (archive.rs:43-70) over bytes that stay valid while `a` lives.
int parse(rn_archive* a) {
    Cursor c{a->data, a->size, 0};
    const uint32_t tag = c.take<uint32_t>();
    if (!c.ok) return archive_fail(RN_ERR_ARGUMENT, "archive is truncated inside the header");
    if (tag != kFormatTag) return archive_fail(RN_ERR_ARGUMENT, "not a Needle 3 archive (format tag 0x%08x)", tag);
    rn_geometry& g = a->geometry;
    uint32_t* fields[] = {&g.tensor_count, &g.codebook_len, &g.kv_window, &g.kv_bits, &g.vocab, &g.out_vocab,
                          &g.d_model, &g.num_heads, &g.num_kv_heads, &g.num_layers, &g.qk_head_dim, &g.v_head_dim,
                          &g.max_seq_len, &g.hada_n, &g.mhc_lanes, &g.sliding_window};
    for (uint32_t* f : fields) *f = c.take<uint32_t>();
    const uint64_t low = c.take<uint32_t>(), high = c.take<uint32_t>();
    g.global_layers = low | (high << 32);
    uint32_t* more[] = {&g.qkv_conv_taps, &g.engram_slots, &g.engram_sub_dim, &g.engram_tables, &g.engram_conv_taps,
                        &g.engram_conv_dilation, &g.engram_seed_heads, &g.engram_order_count};
    for (uint32_t* f : more) *f = c.take<uint32_t>();
    for (uint32_t& o : g.engram_orders) o = c.take<uint32_t>();
    g.engram_site_count = c.take<uint32_t>();
    for (uint32_t& s : g.engram_sites) s = c.take<uint32_t>();
    g.rope_theta = c.take<float>();
    if (!c.ok) return archive_fail(RN_ERR_ARGUMENT, "archive is truncated inside the header");
    if (c.pos != kHeaderBytes) return archive_fail(RN_ERR_STATE, "header parse consumed %zu bytes", c.pos);
    if (g.engram_order_count > 4 || g.engram_site_count > 16)
        return archive_fail(RN_ERR_ARGUMENT,
                            "unexpected tensor layout: engram order or site count exceeds the header capacity");
    a->codebook.resize(g.codebook_len);
    for (float& v : a->codebook) v = c.take<float>();
    if (!c.ok) return archive_fail(RN_ERR_ARGUMENT, "archive is truncated inside the codebook");
    a->records.resize(g.tensor_count);
    for (rn_tensor_record& r : a->records) {  // record.rs:38-51
        const uint8_t kind = c.take<uint8_t>();
        const uint8_t rank = c.take<uint8_t>();
        (void)c.take<uint16_t>();
        for (uint32_t& d : r.shape) d = c.take<uint32_t>();
        r.offset = c.take<uint64_t>();
        r.nbytes = c.take<uint64_t>();
        r.group_size = c.take<uint32_t>();
        r.bits = c.take<uint32_t>();
        if (!c.ok) return archive_fail(RN_ERR_ARGUMENT, "archive is truncated inside the tensor directory");
        if (kind < RN_KIND_HALF || kind > RN_KIND_RAW)
            return archive_fail(RN_ERR_ARGUMENT, "unknown tensor element kind %u", kind);
        r.kind = kind;
        r.rank = rank < 4 ? rank : 4;
        for (int i = r.rank; i < 4; ++i) r.shape[i] = 0;  // shape is dims[..rank]
    }
    if (c.pos != kHeaderBytes + 4 * (size_t)g.codebook_len + kRecordBytes * (size_t)g.tensor_count)
        return archive_fail(RN_ERR_STATE, "directory parse ended at byte %zu", c.pos);  // archive.rs:69
    for (size_t i = 0; i < a->records.size(); ++i) {  // archive.rs:56-70
        const rn_tensor_record& r = a->records[i];
        if (r.offset > a->size || r.nbytes > a->size - r.offset)
            return archive_fail(RN_ERR_ARGUMENT, "tensor %zu lies outside the archive", i);
        const uint64_t width = r.kind == RN_KIND_HALF ? 2 : (r.kind == RN_KIND_SINGLE ? 4 : 1);
        if (r.offset % width != 0 || r.nbytes % width != 0)
            return archive_fail(RN_ERR_ARGUMENT,
                                "unexpected tensor layout: tensor %zu is not aligned to its element width", i);
    }
    return RN_OK;
}

}  // namespace

extern "C" {

int rn_archive_open(const char* path, rn_archive** out) {
    if (!path || !out) return archive_fail(RN_ERR_ARGUMENT, "null argument");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return archive_fail(RN_ERR_ARGUMENT, "%s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return archive_fail(RN_ERR_ARGUMENT, "%s: %s", path, strerror(e));
    }
    rn_archive* a = new (std::nothrow) rn_archive();
    if (!a) {
        close(fd);
        return archive_fail(RN_ERR_MEMORY, "out of host memory");
    }
    a->size = (size_t)st.st_size;
    if (a->size > 0) {
        void* m = mmap(nullptr, a->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int e = errno;
            close(fd);
            delete a;
            return archive_fail(RN_ERR_ARGUMENT, "%s: mmap: %s", path, strerror(e));
        }
        a->data = (const uint8_t*)m;
        a->mapped = true;
    }
    close(fd);
    const int rc = parse(a);
    if (rc != RN_OK) {
        rn_archive_close(a);
        return rc;
    }
    *out = a;
    return RN_OK;
}

int rn_archive_from_memory(const uint8_t* bytes, size_t nbytes, rn_archive** out) {
    if ((!bytes && nbytes) || !out) return archive_fail(RN_ERR_ARGUMENT, "null argument");
    rn_archive* a = new (std::nothrow) rn_archive();
    if (!a) return archive_fail(RN_ERR_MEMORY, "out of host memory");
    a->owned.assign(bytes, bytes + nbytes);
    a->data = a->owned.data();
    a->size = nbytes;
    const int rc = parse(a);
    if (rc != RN_OK) {
        delete a;
        return rc;
    }
    *out = a;
    return RN_OK;
}

int rn_archive_close(rn_archive* a) {
    if (!a) return RN_OK;
    if (a->mapped) munmap((void*)a->data, a->size);
    delete a;
    return RN_OK;
}

int rn_archive_geometry(const rn_archive* a, rn_geometry* out) {
    if (!a || !out) return archive_fail(RN_ERR_ARGUMENT, "null argument");
    *out = a->geometry;
    return RN_OK;
}

int rn_archive_codebook(const rn_archive* a, const float** values, int* count) {
    if (!a || !values || !count) return archive_fail(RN_ERR_ARGUMENT, "null argument");
    *values = a->codebook.data();
    *count = (int)a->codebook.size();
    return RN_OK;
}

int rn_archive_record(const rn_archive* a, int index, rn_tensor_record* out) {
    if (!a || !out) return archive_fail(RN_ERR_ARGUMENT, "null argument");
    if (index < 0 || (size_t)index >= a->records.size())
        return archive_fail(RN_ERR_ARGUMENT, "tensor %d out of range [0, %zu)", index, a->records.size());
    *out = a->records[index];
    return RN_OK;
}

int rn_archive_tensor_bytes(const rn_archive* a, int index, const uint8_t** data, size_t* nbytes) {
    if (!a || !data || !nbytes) return archive_fail(RN_ERR_ARGUMENT, "null argument");
    if (index < 0 || (size_t)index >= a->records.size())
        return archive_fail(RN_ERR_ARGUMENT, "tensor %d out of range [0, %zu)", index, a->records.size());
    const rn_tensor_record& r = a->records[index];
    *data = a->data + r.offset;
    *nbytes = (size_t)r.nbytes;
    return RN_OK;
}

// QuantisedMatrix::from_archive (matrix.rs:35-40): rows = shape[0], columns =
// shape[1] (1 for a rank-1 record, record.rs:53-59).
int rn_matrix_from_archive(const rn_archive* a, int index, rn_matrix** out) {
    rn_tensor_record r;
    int rc = rn_archive_record(a, index, &r);
    if (rc != RN_OK) return rc;
    if (r.kind != RN_KIND_CODEBOOK)
        return archive_fail(RN_ERR_ARGUMENT, "tensor %d is not codebook-quantised (kind %d)", index, r.kind);
    const int rows = r.rank >= 1 ? (int)r.shape[0] : 0;
    const int columns = r.rank >= 2 ? (int)r.shape[1] : 1;
    return rn_matrix_create_codebook(a->data + r.offset, (size_t)r.nbytes, rows, columns, (int)r.group_size,
                                     (int)r.bits, a->codebook.data(), (int)a->codebook.size(), out);
}

}  // extern "C"
