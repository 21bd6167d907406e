// The .llmpk expert pack (crates/llmpager-core/src/pack.rs): the on-disk
// layout the pager fills expert slots from.  Little-endian, every section
// 4096-byte aligned:
//   [0, 4096)  magic "LLMPK1\0\0", u32 version 1, u32 json_len, the metadata
//              JSON, zero padding;
//   [4096, .)  one {u64 offset, u64 nbytes} entry per (layer, expert),
//              row-major by layer, zero-padded to 4096;
//   then the blobs, each starting on a 4096 boundary.
// The writer streams blobs in (layer, expert) order and back-fills header
// and index (pack.rs:67-150); the reader keeps the index in memory and reads
// a blob's whole aligned span with pread, optionally through O_DIRECT
// (pack.rs:152-260).  Compressed packs (zstd frames) are refused.
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/llmpager_hip.h"
#include "lp_internal.h"

namespace {

constexpr char kMagic[8] = {'L', 'L', 'M', 'P', 'K', '1', '\0', '\0'};
constexpr uint32_t kVersion = 1;
constexpr uint64_t kAlign = 4096;

uint64_t align_up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int fail(int code, const std::string& m) { return lpi::set_error(code, m); }

// pread of exactly n bytes (retrying short reads)
bool pread_full(int fd, void* buf, size_t n, uint64_t off) {
    uint8_t* p = static_cast<uint8_t*>(buf);
    while (n > 0) {
        const ssize_t r = pread(fd, p, n, (off_t)off);
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

bool write_full(int fd, const void* buf, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(buf);
    while (n > 0) {
        const ssize_t r = write(fd, p, n);
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
    }
    return true;
}

// The value after "key": in a compact JSON object (the metadata the
// reference's serde writer emits: no nesting of these keys).
bool json_field(const std::string& js, const char* key, std::string* out) {
    const std::string k = std::string("\"") + key + "\"";
    size_t at = js.find(k);
    if (at == std::string::npos) return false;
    at = js.find(':', at + k.size());
    if (at == std::string::npos) return false;
    ++at;
    while (at < js.size() && (js[at] == ' ' || js[at] == '\t')) ++at;
    if (at < js.size() && js[at] == '"') {
        const size_t end = js.find('"', at + 1);
        if (end == std::string::npos) return false;
        *out = js.substr(at + 1, end - at - 1);
        return true;
    }
    size_t end = at;
    while (end < js.size() && js[end] != ',' && js[end] != '}') ++end;
    *out = js.substr(at, end - at);
    while (!out->empty() && (out->back() == ' ' || out->back() == '\n')) out->pop_back();
    return true;
}

// A JSON unsigned integer: digits only (no sign, no fraction, no exponent),
// at most 20 of them, parsed without exceptions or wrap-around.
bool parse_count(const std::string& v, uint64_t* out) {
    if (v.empty() || v.size() > 20) return false;
    for (char ch : v)
        if (ch < '0' || ch > '9') return false;
    errno = 0;
    char* end = nullptr;
    const unsigned long long x = strtoull(v.c_str(), &end, 10);
    if (errno != 0 || !end || *end != '\0') return false;
    *out = (uint64_t)x;
    return true;
}

std::string json_escape(const char* s) {
    std::string o;
    for (const char* c = s ? s : ""; *c; ++c) {
        if (*c == '"' || *c == '\\') o += '\\';
        o += *c;
    }
    return o;
}

}  // namespace

struct lp_pack_writer {
    int fd = -1;
    uint32_t layers = 0, experts = 0;
    std::string json;
    std::vector<uint64_t> index;  // offset, nbytes pairs
    uint64_t index_end = 0, cursor = 0;
};

struct lp_pack {
    int fd = -1;
    bool direct = false;
    uint32_t layers = 0, experts = 0;
    std::string dtype, model;
    std::vector<uint64_t> index;  // offset, nbytes pairs
    uint64_t max_blob = 0;
};

extern "C" {

int lp_pack_create(const char* path, const char* model, const char* dtype, uint32_t layers, uint32_t experts,
                   lp_pack_writer** out) {
    if (!out) return fail(LP_E_INVALID, "lp_pack_create: null out");
    *out = nullptr;
    if (!path || layers == 0 || experts == 0 || layers > 65535 || experts > 65535)
        return fail(LP_E_INVALID, "lp_pack_create: bad arguments");
    const int fd = open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) return fail(LP_E_INVALID, std::string("lp_pack_create: cannot create ") + path);
    lp_pack_writer* w = new lp_pack_writer();
    w->fd = fd;
    w->layers = layers;
    w->experts = experts;
    // PackMeta (pack.rs:29-48), in the field order serde writes it
    w->json = std::string("{\"model\":\"") + json_escape(model) + "\",\"num_layers\":" + std::to_string(layers) +
              ",\"experts_per_layer\":" + std::to_string(experts) + ",\"dtype\":\"" + json_escape(dtype) + "\"}";
    if (w->json.size() > kAlign - 16) {
        close(fd);
        delete w;
        return fail(LP_E_INVALID, "lp_pack_create: metadata JSON too large for the header block");
    }
    const uint64_t total = (uint64_t)layers * experts;
    w->index_end = align_up(kAlign + total * 16);
    w->cursor = w->index_end;
    *out = w;
    return LP_OK;
}

int lp_pack_add_blob(lp_pack_writer* w, const void* blob, uint64_t nbytes) {
    if (!w || (!blob && nbytes)) return fail(LP_E_INVALID, "lp_pack_add_blob: bad arguments");
    const uint64_t total = (uint64_t)w->layers * w->experts;
    if (w->index.size() / 2 == total) return fail(LP_E_INVALID, "lp_pack_add_blob: pack already has every blob");
    w->index.push_back(w->cursor);
    w->index.push_back(nbytes);
    if (lseek(w->fd, (off_t)w->cursor, SEEK_SET) < 0 || !write_full(w->fd, blob, nbytes))
        return fail(LP_E_INVALID, "lp_pack_add_blob: write failed");
    const uint64_t padded = align_up(nbytes);
    if (padded > nbytes) {
        std::vector<uint8_t> zero(padded - nbytes, 0);
        if (!write_full(w->fd, zero.data(), zero.size())) return fail(LP_E_INVALID, "lp_pack_add_blob: write failed");
    }
    w->cursor += padded;
    return LP_OK;
}

int lp_pack_finish(lp_pack_writer* w) {
    if (!w) return fail(LP_E_INVALID, "lp_pack_finish: null writer");
    const uint64_t total = (uint64_t)w->layers * w->experts;
    int rc = LP_OK;
    if (w->index.size() / 2 != total) {
        rc = fail(LP_E_INVALID, "lp_pack_finish: pack incomplete");
    } else {
        std::vector<uint8_t> head(w->index_end, 0);
        memcpy(head.data(), kMagic, 8);
        const uint32_t ver = kVersion, jl = (uint32_t)w->json.size();
        memcpy(head.data() + 8, &ver, 4);
        memcpy(head.data() + 12, &jl, 4);
        memcpy(head.data() + 16, w->json.data(), jl);
        memcpy(head.data() + kAlign, w->index.data(), w->index.size() * 8);
        if (lseek(w->fd, 0, SEEK_SET) < 0 || !write_full(w->fd, head.data(), head.size()))
            rc = fail(LP_E_INVALID, "lp_pack_finish: write failed");
    }
    if (close(w->fd) != 0 && rc == LP_OK) rc = fail(LP_E_INVALID, "lp_pack_finish: close failed");
    delete w;
    return rc;
}

int lp_pack_open(const char* path, int direct, lp_pack** out) {
    if (!out) return fail(LP_E_INVALID, "lp_pack_open: null out");
    *out = nullptr;
    if (!path) return fail(LP_E_INVALID, "lp_pack_open: null path");
    const int fd = open(path, O_RDONLY | (direct ? O_DIRECT : 0));
    if (fd < 0) return fail(LP_E_INVALID, std::string("lp_pack_open: cannot open ") + path);
    lp_pack* p = new lp_pack();
    p->fd = fd;
    p->direct = direct != 0;
    auto bad = [&](const std::string& m) {
        close(fd);
        delete p;
        return fail(LP_E_INVALID, std::string(path) + ": " + m);
    };
    void* hb = nullptr;
    if (posix_memalign(&hb, kAlign, kAlign) != 0) return bad("out of memory");
    std::vector<uint8_t> head(kAlign);
    const bool ok = pread_full(fd, hb, kAlign, 0);
    memcpy(head.data(), hb, kAlign);
    free(hb);
    if (!ok) return bad("cannot read the header");
    if (memcmp(head.data(), kMagic, 8) != 0) return bad("not an llmpk file");
    uint32_t ver = 0, jl = 0;
    memcpy(&ver, head.data() + 8, 4);
    memcpy(&jl, head.data() + 12, 4);
    if (ver != kVersion) return bad("unsupported pack version " + std::to_string(ver));
    if (jl > kAlign - 16) return bad("metadata JSON overruns the header");
    const std::string js(reinterpret_cast<const char*>(head.data() + 16), jl);
    // PackMeta (pack.rs:29-48) holds num_layers and experts_per_layer as
    // u16: anything else is not a pack this format can describe
    std::string v;
    uint64_t nl = 0, ne = 0;
    if (!json_field(js, "num_layers", &v)) return bad("metadata has no num_layers");
    if (!parse_count(v, &nl) || nl > 65535) return bad("num_layers is not an integer in 0..65535");
    if (!json_field(js, "experts_per_layer", &v)) return bad("metadata has no experts_per_layer");
    if (!parse_count(v, &ne) || ne > 65535) return bad("experts_per_layer is not an integer in 0..65535");
    p->layers = (uint32_t)nl;
    p->experts = (uint32_t)ne;
    if (json_field(js, "dtype", &v)) p->dtype = v;
    if (json_field(js, "model", &v)) p->model = v;
    if (json_field(js, "compression", &v) && v != "null") return bad("compressed packs are not supported");
    if (p->layers == 0 || p->experts == 0) return bad("empty pack");
    // at most 65535^2 entries of 16 bytes: no overflow in 64 bits
    const uint64_t total = (uint64_t)p->layers * p->experts;
    const uint64_t span = align_up(total * 16);
    struct stat st;
    if (fstat(fd, &st) != 0) return bad("cannot stat the file");
    const uint64_t fsize = (uint64_t)st.st_size;
    if (fsize < kAlign + span) return bad("the file is shorter than its index");
    void* ib = nullptr;
    if (posix_memalign(&ib, kAlign, span) != 0) return bad("out of memory");
    const bool iok = pread_full(fd, ib, span, kAlign);
    if (iok) p->index.assign(static_cast<const uint64_t*>(ib), static_cast<const uint64_t*>(ib) + 2 * total);
    free(ib);
    if (!iok) return bad("cannot read the index");
    // every blob starts on a 4096 boundary past the index and its aligned
    // span lies inside the file (the reads take whole spans)
    for (uint64_t i = 0; i < total; ++i) {
        const uint64_t off = p->index[2 * i], n = p->index[2 * i + 1];
        if (off % kAlign || off < kAlign + span || n > fsize || align_up(n) > fsize || off > fsize - align_up(n))
            return bad("index entry " + std::to_string(i) + " lies outside the file or is not 4096-aligned");
        p->max_blob = std::max(p->max_blob, n);
    }
    *out = p;
    return LP_OK;
}

void lp_pack_close(lp_pack* p) {
    if (!p) return;
    close(p->fd);
    delete p;
}

int lp_pack_info(const lp_pack* p, uint32_t* layers, uint32_t* experts, uint64_t* max_blob_bytes) {
    if (!p) return fail(LP_E_INVALID, "lp_pack_info: null pack");
    if (layers) *layers = p->layers;
    if (experts) *experts = p->experts;
    if (max_blob_bytes) *max_blob_bytes = p->max_blob;
    return LP_OK;
}

int lp_pack_entry(const lp_pack* p, uint32_t layer, uint32_t expert, uint64_t* offset, uint64_t* nbytes) {
    if (!p || layer >= p->layers || expert >= p->experts) return fail(LP_E_INVALID, "lp_pack_entry: out of range");
    const uint64_t i = (uint64_t)layer * p->experts + expert;
    if (offset) *offset = p->index[2 * i];
    if (nbytes) *nbytes = p->index[2 * i + 1];
    return LP_OK;
}

// pread of [offset, offset + n) of the pack into buf (the pager's staging
// pieces; under O_DIRECT offset, n and buf must be 4096-aligned).
int lp_pack_read_range(lp_pack* p, uint64_t offset, void* buf, uint64_t n) {
    if (!p || !buf) return LP_E_INVALID;
    if (p->direct && ((offset | n | reinterpret_cast<uintptr_t>(buf)) % kAlign)) return LP_E_INVALID;
    return pread_full(p->fd, buf, n, offset) ? LP_OK : LP_E_INVALID;
}

int64_t lp_pack_read_blob(lp_pack* p, uint32_t layer, uint32_t expert, void* buf, uint64_t buf_len) {
    if (!p || !buf || layer >= p->layers || expert >= p->experts)
        return fail(LP_E_INVALID, "lp_pack_read_blob: bad arguments");
    const uint64_t i = (uint64_t)layer * p->experts + expert;
    const uint64_t off = p->index[2 * i], n = p->index[2 * i + 1];
    const uint64_t span = align_up(n);
    if (buf_len < span) return fail(LP_E_INVALID, "lp_pack_read_blob: buffer smaller than the blob's aligned span");
    if (p->direct && (reinterpret_cast<uintptr_t>(buf) % kAlign) != 0)
        return fail(LP_E_INVALID, "lp_pack_read_blob: O_DIRECT reads need a 4096-aligned buffer");
    if (!pread_full(p->fd, buf, span, off)) return fail(LP_E_INVALID, "lp_pack_read_blob: read failed");
    return (int64_t)n;
}

}  // extern "C"
