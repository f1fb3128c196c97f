// model_files.hip -- the on-disk sources of expert pages, read into HBM.
//
//  * GGUF model files (the format ggml/src/gguf.cpp reads and writes,
//    versions 2 and 3): the tensor table, and the stacked expert tensors
//    (blk.L.ffn_{gate_up,down}_exps.{weight,scale}) as the page groups the
//    memmgr registers from them (moe_dual_init.cpp:230-263: expert axis =
//    the highest dimension equal to n_expert, bytes per expert = its stride).
//  * The expert store v0 (experts.index + experts.pack, moert/store.h,
//    moert/memmgr/store_format.h): probe, verify, writer and per-page reader
//    under the reference's names, the byte layout unchanged.
//  * Uploads into device memory: pages are read with pread into two pinned
//    staging buffers in turn, each copied with hipMemcpyAsync while the next
//    read runs; a buffer is reused only after its copy's event.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <ctime>
#include <string>
#include <vector>

#include "../../include/llapis_moe.h"
#include "../../include/moert_store.h"

namespace {

thread_local char g_ferr[512];
int32_t ffail(const std::string & msg) {
    snprintf(g_ferr, sizeof g_ferr, "%s", msg.c_str());
    return -1;
}

// ggml type traits needed to size a tensor: {block bytes, values per block}
// (ggml.c type_traits; unknown types size to 0)
struct TypeSize {
    int bytes, blck;
};
TypeSize type_size(int t) {
    switch (t) {
        case 0: return {4, 1};      // F32
        case 1: return {2, 1};      // F16
        case 2: return {18, 32};    // Q4_0
        case 3: return {20, 32};    // Q4_1
        case 6: return {22, 32};    // Q5_0
        case 7: return {24, 32};    // Q5_1
        case 8: return {34, 32};    // Q8_0
        case 9: return {36, 32};    // Q8_1
        case 10: return {84, 256};  // Q2_K
        case 11: return {110, 256}; // Q3_K
        case 12: return {144, 256}; // Q4_K
        case 13: return {176, 256}; // Q5_K
        case 14: return {210, 256}; // Q6_K
        case 15: return {292, 256}; // Q8_K
        case 16: return {66, 256};  // IQ2_XXS
        case 17: return {74, 256};  // IQ2_XS
        case 18: return {98, 256};  // IQ3_XXS
        case 19: return {50, 256};  // IQ1_S
        case 20: return {18, 32};   // IQ4_NL
        case 21: return {110, 256}; // IQ3_S
        case 22: return {82, 256};  // IQ2_S
        case 23: return {136, 256}; // IQ4_XS
        case 24: return {1, 1};     // I8
        case 25: return {2, 1};     // I16
        case 26: return {4, 1};     // I32
        case 27: return {8, 1};     // I64
        case 28: return {8, 1};     // F64
        case 29: return {56, 256};  // IQ1_M
        case 30: return {2, 1};     // BF16
        case 34: return {54, 256};  // TQ1_0
        case 35: return {66, 256};  // TQ2_0
        case 39: return {17, 32};   // MXFP4
    }
    return {0, 1};
}

// ------------------------------------------------------------ reading a file

struct Reader {
    FILE * f = nullptr;
    bool ok = true;
    template <typename T> T get() {
        T v{};
        if (ok && fread(&v, sizeof(T), 1, f) != 1) ok = false;
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1ull << 24)) {
            ok = false;
            return {};
        }
        std::string s(n, '\0');
        if (n && fread(&s[0], 1, n, f) != n) ok = false;
        return s;
    }
    void skip(uint64_t n) {
        if (ok && fseeko(f, (off_t)n, SEEK_CUR) != 0) ok = false;
    }
};

// GGUF value types (gguf.h gguf_type) and their sizes; 0 = string / array
int gguf_scalar_bytes(int t) {
    switch (t) {
        case 0: case 1: case 7: return 1;      // u8 i8 bool
        case 2: case 3: return 2;              // u16 i16
        case 4: case 5: case 6: return 4;      // u32 i32 f32
        case 10: case 11: case 12: return 8;   // u64 i64 f64
    }
    return 0;
}

int read_fully(int fd, void * dst, uint64_t n, uint64_t off) {
    uint8_t * p = (uint8_t *)dst;
    while (n) {
        const ssize_t r = pread(fd, p, n > (1ull << 30) ? (1ull << 30) : n, (off_t)off);
        if (r <= 0) return -1;
        p += r;
        n -= (uint64_t)r;
        off += (uint64_t)r;
    }
    return 0;
}

// Two pinned staging buffers: file ranges read into one while the other's
// copy to the device runs.
struct Staging {
    static constexpr size_t CAP = 16u << 20;
    char * buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    int next = 0;
    bool init() {
        for (int i = 0; i < 2; ++i) {
            if (hipHostMalloc((void **)&buf[i], CAP, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                return false;
            }
        }
        return true;
    }
    ~Staging() {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) {
                (void)hipEventSynchronize(ev[i]);
                (void)hipEventDestroy(ev[i]);
            }
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
    // a free buffer (waits for its previous copy)
    char * take(int * which) {
        const int i = next;
        next ^= 1;
        if (used[i] && hipEventSynchronize(ev[i]) != hipSuccess) return nullptr;
        *which = i;
        return buf[i];
    }
    bool copy(int i, void * dst, size_t n, hipStream_t s) {
        if (hipMemcpyAsync(dst, buf[i], n, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipEventRecord(ev[i], s) != hipSuccess)
            return false;
        used[i] = true;
        return true;
    }
};

// Copies n bytes at file offset off into dst through the staging buffers.
int32_t upload_range(Staging & st, int fd, uint64_t off, uint64_t n, uint8_t * dst, hipStream_t s,
                     uint64_t * hash, const char * what) {
    while (n) {
        int i;
        char * b = st.take(&i);
        if (!b) return ffail(std::string(what) + ": staging wait failed");
        const uint64_t c = std::min<uint64_t>(n, Staging::CAP);
        if (read_fully(fd, b, c, off) != 0) return ffail(std::string(what) + ": read failed");
        if (hash)
            for (uint64_t k = 0; k < c; ++k) {
                *hash ^= (uint8_t)b[k];
                *hash *= 1099511628211ull;
            }
        if (!st.copy(i, dst, c, s)) {
            (void)hipGetLastError();
            return ffail(std::string(what) + ": copy to the device failed");
        }
        off += c;
        dst += c;
        n -= c;
    }
    return 0;
}

}  // namespace

// ------------------------------------------------------------------- GGUF

struct llapis_gguf {
    std::string path;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<llapis_gguf_tensor_info> tensors;
    std::vector<std::pair<std::string, uint32_t>> u32_kv;   // the u32 keys (alignment, counts)
};

extern "C" {

const char * llapis_files_last_error(void) { return g_ferr; }

llapis_gguf * llapis_gguf_open(const char * path) {
    if (!path) {
        ffail("llapis_gguf_open: null path");
        return nullptr;
    }
    Reader r;
    r.f = fopen(path, "rb");
    if (!r.f) {
        ffail(std::string("llapis_gguf_open: cannot open ") + path);
        return nullptr;
    }
    llapis_gguf * g = new llapis_gguf();
    g->path = path;
    auto bail = [&](const char * why) -> llapis_gguf * {
        ffail(std::string("llapis_gguf_open: ") + path + ": " + why);
        fclose(r.f);
        delete g;
        return nullptr;
    };
    char magic[4];
    if (fread(magic, 1, 4, r.f) != 4 || memcmp(magic, "GGUF", 4) != 0) return bail("not a GGUF file");
    g->version = r.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return bail("unsupported GGUF version");
    const int64_t n_tensors = r.get<int64_t>(), n_kv = r.get<int64_t>();
    if (!r.ok || n_tensors < 0 || n_kv < 0 || n_tensors > (1 << 24) || n_kv > (1 << 24)) return bail("bad counts");
    for (int64_t i = 0; i < n_kv && r.ok; ++i) {
        const std::string key = r.str();
        const int32_t t = r.get<int32_t>();
        if (t == 8) {
            r.str();
        } else if (t == 9) {
            const int32_t et = r.get<int32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (et == 8) {
                for (uint64_t k = 0; k < n && r.ok; ++k) r.str();
            } else if (gguf_scalar_bytes(et)) {
                r.skip(n * (uint64_t)gguf_scalar_bytes(et));
            } else {
                return bail("unsupported array element type");
            }
        } else if (gguf_scalar_bytes(t)) {
            if (t == 4) {
                const uint32_t v = r.get<uint32_t>();
                g->u32_kv.push_back({key, v});
                if (key == "general.alignment") g->alignment = v;
            } else {
                r.skip((uint64_t)gguf_scalar_bytes(t));
            }
        } else {
            return bail("unknown value type");
        }
    }
    if (!r.ok) return bail("truncated key/value section");
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1))) return bail("alignment is not a power of two");
    for (int64_t i = 0; i < n_tensors && r.ok; ++i) {
        llapis_gguf_tensor_info t = {};
        const std::string name = r.str();
        if (name.size() >= sizeof(t.name)) return bail("tensor name too long");
        memcpy(t.name, name.c_str(), name.size() + 1);
        const uint32_t nd = r.get<uint32_t>();
        if (nd < 1 || nd > 4) return bail("tensor rank out of range");
        t.n_dims = (int32_t)nd;
        for (int d = 0; d < 4; ++d) t.ne[d] = d < (int)nd ? r.get<int64_t>() : 1;
        t.type = r.get<int32_t>();
        t.offset = r.get<uint64_t>();
        const TypeSize ts = type_size(t.type);
        if (ts.bytes && t.ne[0] % ts.blck == 0) {
            t.nb[0] = (uint64_t)ts.bytes;
            t.nb[1] = t.nb[0] * (uint64_t)(t.ne[0] / ts.blck);
            for (int d = 2; d < 4; ++d) t.nb[d] = t.nb[d - 1] * (uint64_t)t.ne[d - 1];
            t.nbytes = t.nb[3] * (uint64_t)t.ne[3];
        }
        g->tensors.push_back(t);
    }
    if (!r.ok) return bail("truncated tensor table");
    const uint64_t pos = (uint64_t)ftello(r.f);
    g->data_offset = (pos + g->alignment - 1) & ~(g->alignment - 1);
    fclose(r.f);
    for (auto & t : g->tensors) t.offset += g->data_offset;   // absolute file offsets
    return g;
}

void llapis_gguf_close(llapis_gguf * g) { delete g; }

int64_t llapis_gguf_n_tensors(const llapis_gguf * g) { return g ? (int64_t)g->tensors.size() : -1; }
uint64_t llapis_gguf_data_offset(const llapis_gguf * g) { return g ? g->data_offset : 0; }
uint64_t llapis_gguf_alignment(const llapis_gguf * g) { return g ? g->alignment : 0; }

int32_t llapis_gguf_tensor(const llapis_gguf * g, int64_t i, llapis_gguf_tensor_info * out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return ffail("llapis_gguf_tensor: bad index");
    *out = g->tensors[(size_t)i];
    return 0;
}

int64_t llapis_gguf_find(const llapis_gguf * g, const char * name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); ++i)
        if (strcmp(g->tensors[i].name, name) == 0) return (int64_t)i;
    return -1;
}

int32_t llapis_gguf_expert_group(const llapis_gguf * g, int32_t layer, int32_t kind, int32_t is_scale,
                                 int32_t n_expert, llapis_page_group * out) {
    if (!g || !out || layer < 0 || (kind != 0 && kind != 1) || n_expert <= 0)
        return ffail("llapis_gguf_expert_group: bad arguments");
    const std::string want = "blk." + std::to_string(layer) + (kind == 0 ? ".ffn_gate_up_exps" : ".ffn_down_exps") +
                             (is_scale ? ".scale" : ".weight");
    const int64_t i = llapis_gguf_find(g, want.c_str());
    if (i < 0) return ffail("llapis_gguf_expert_group: no tensor " + want);
    const llapis_gguf_tensor_info & t = g->tensors[(size_t)i];
    int axis = -1;
    for (int d = 3; d >= 0; --d)
        if (t.ne[d] == n_expert) {
            axis = d;
            break;
        }
    if (axis < 0) return ffail("llapis_gguf_expert_group: " + want + " has no expert axis");
    if (!t.nbytes) return ffail("llapis_gguf_expert_group: " + want + " has a type this build cannot size");
    // the experts must be whole contiguous slabs (axis outermost of the non-unit dims)
    for (int d = axis + 1; d < 4; ++d)
        if (t.ne[d] != 1) return ffail("llapis_gguf_expert_group: " + want + ": experts are not contiguous slabs");
    memset(out, 0, sizeof(*out));
    out->type = t.type;
    out->offset = t.offset;
    out->bytes_per_expert = t.nb[axis];
    out->n_expert = n_expert;
    out->expert_axis = axis;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    return 0;
}

int32_t llapis_gguf_upload(const llapis_gguf * g, const llapis_page_group * grp, int32_t e0, int32_t n, void * dst,
                           void * stream) {
    if (!g || !grp || !dst || e0 < 0 || n <= 0 || e0 + n > grp->n_expert)
        return ffail("llapis_gguf_upload: bad arguments");
    const int fd = open(g->path.c_str(), O_RDONLY);
    if (fd < 0) return ffail("llapis_gguf_upload: cannot open " + g->path);
    Staging st;
    int32_t rc = st.init() ? 0 : ffail("llapis_gguf_upload: pinned staging allocation failed");
    if (rc == 0)
        rc = upload_range(st, fd, grp->offset + (uint64_t)e0 * grp->bytes_per_expert,
                          (uint64_t)n * grp->bytes_per_expert, (uint8_t *)dst, (hipStream_t)stream, nullptr,
                          "llapis_gguf_upload");
    if (rc == 0 && hipStreamSynchronize((hipStream_t)stream) != hipSuccess) {
        (void)hipGetLastError();
        rc = ffail("llapis_gguf_upload: stream failed");
    }
    close(fd);
    return rc;
}

}  // extern "C"

// ------------------------------------------------------------ expert store

namespace {

constexpr char INDEX_MAGIC[8] = {'E', 'X', 'I', 'D', 'X', '1', '\0', '\0'};
constexpr char PACK_MAGIC[8] = {'E', 'X', 'P', 'A', 'C', 'K', '1', '\0'};
constexpr uint32_t VERSION = 1, FNV_ALGO = 1;
constexpr uint64_t PAGE_ALIGN = 256;
constexpr int MAX_KIND = 4;

#pragma pack(push, 1)
struct IdxHeader {            // 96 bytes on disk
    char magic[8];
    uint32_t version, header_bytes;
    uint64_t source_uuid;
    char arch[16];
    uint32_t n_layers, n_expert;
    uint64_t n_embd, n_ff_exp, pack_uuid, record_count;
    uint32_t record_stride, checksum_algo;
    uint64_t reserved;
};
struct IdxRecord {            // 72 bytes on disk
    uint16_t layer, expert;
    uint8_t kind, reserved8;
    uint16_t quant_type;
    uint64_t offset, nbytes;
    int64_t shape[4];
    uint64_t checksum;
    uint16_t source_quant, reserved16;
    uint32_t flags;
};
struct PkHeader {             // 32 bytes on disk
    char magic[8];
    uint32_t version, reserved32;
    uint64_t pack_uuid, reserved64;
};
#pragma pack(pop)
static_assert(sizeof(IdxHeader) == 96 && sizeof(IdxRecord) == 72 && sizeof(PkHeader) == 32, "store layout");

bool header_ok(const IdxHeader & h) {
    return memcmp(h.magic, INDEX_MAGIC, 8) == 0 && h.version == VERSION && h.record_stride >= sizeof(IdxRecord) &&
           h.header_bytes >= sizeof(IdxHeader) && h.checksum_algo == FNV_ALGO;
}

std::string pack_path_of(const std::string & index) {
    const std::string suf = MOERT_STORE_INDEX_SUFFIX;
    if (index.size() > suf.size() && index.compare(index.size() - suf.size(), suf.size(), suf) == 0)
        return index.substr(0, index.size() - suf.size()) + MOERT_STORE_PACK_SUFFIX;
    return index + ".pack";
}

// the index's header and records, and the pack opened (uuid checked)
bool load_store(const char * index_path, IdxHeader & h, std::vector<IdxRecord> & recs, int * pack_fd) {
    FILE * f = fopen(index_path, "rb");
    if (!f) {
        ffail(std::string("moert-store: cannot open index ") + index_path);
        return false;
    }
    // the index's own size bounds the record count, and the page table the
    // reader builds (n_layers x n_expert x 8 entries) stays below 64 MB
    off_t idx_size = -1;
    if (fseeko(f, 0, SEEK_END) == 0) idx_size = ftello(f);
    bool ok = idx_size > 0 && fseeko(f, 0, SEEK_SET) == 0 && fread(&h, sizeof h, 1, f) == 1 && header_ok(h) &&
              h.header_bytes <= (uint64_t)idx_size &&
              h.record_count <= ((uint64_t)idx_size - h.header_bytes) / h.record_stride &&
              h.n_layers >= 1 && h.n_expert >= 1 && (uint64_t)h.n_layers * h.n_expert <= (1ull << 20) &&
              fseeko(f, (off_t)h.header_bytes, SEEK_SET) == 0;
    if (ok) {
        recs.resize(h.record_count);
        for (uint64_t i = 0; i < h.record_count && ok; ++i) {
            ok = fread(&recs[i], sizeof(IdxRecord), 1, f) == 1;
            if (ok && h.record_stride > sizeof(IdxRecord))
                ok = fseeko(f, (off_t)(h.record_stride - sizeof(IdxRecord)), SEEK_CUR) == 0;
        }
    }
    fclose(f);
    if (!ok) {
        ffail(std::string("moert-store: ") + index_path + ": bad or truncated index");
        return false;
    }
    const std::string pp = pack_path_of(index_path);
    const int fd = open(pp.c_str(), O_RDONLY);
    PkHeader ph;
    if (fd < 0 || read_fully(fd, &ph, sizeof ph, 0) != 0 || memcmp(ph.magic, PACK_MAGIC, 8) != 0 ||
        ph.version != VERSION || ph.pack_uuid != h.pack_uuid) {
        if (fd >= 0) close(fd);
        ffail("moert-store: " + pp + ": missing pack, bad pack header or index/pack uuid mismatch");
        return false;
    }
    // every record inside the pack
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        ffail("moert-store: " + pp + ": cannot stat the pack");
        return false;
    }
    const uint64_t pack_size = (uint64_t)st.st_size;
    for (const IdxRecord & r : recs) {
        if (r.offset > pack_size || r.nbytes > pack_size - r.offset) {
            close(fd);
            ffail("moert-store: " + std::string(index_path) + ": a record lies outside the pack");
            return false;
        }
    }
    *pack_fd = fd;
    return true;
}

}  // namespace

struct moert_store_reader {
    int fd = -1;
    IdxHeader h{};
    std::vector<IdxRecord> recs;
    std::vector<int64_t> slot;   // (layer, kind, is_scale, expert) -> record | -1
    int64_t key(int layer, int kind, int is_scale, int e) const {
        if (layer < 0 || layer >= (int)h.n_layers || kind < 0 || kind >= MAX_KIND || is_scale < 0 || is_scale > 1 ||
            e < 0 || e >= (int)h.n_expert)
            return -1;
        return ((int64_t)layer * MAX_KIND * 2 + kind * 2 + is_scale) * h.n_expert + e;
    }
    const IdxRecord * rec(int layer, int kind, int is_scale, int e) const {
        const int64_t k = key(layer, kind, is_scale, e);
        return k < 0 || slot[(size_t)k] < 0 ? nullptr : &recs[(size_t)slot[(size_t)k]];
    }
};

struct moert_store_writer {
    FILE * pack = nullptr;
    std::string index_path;
    IdxHeader h{};
    std::vector<IdxRecord> recs;
    uint64_t pos = 0;
    bool failed = false;
};

extern "C" {

uint64_t moert_store_fnv1a64(const void * data, uint64_t nbytes, uint64_t seed) {
    const uint8_t * p = (const uint8_t *)data;
    uint64_t h = seed;
    for (uint64_t i = 0; i < nbytes; ++i) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

int32_t moert_store_probe(const char * index_path, moert_store_info * out) {
    if (!index_path || !out) return 0;
    FILE * f = fopen(index_path, "rb");
    if (!f) return 0;
    IdxHeader h;
    const bool ok = fread(&h, sizeof h, 1, f) == 1 && header_ok(h);
    fclose(f);
    if (!ok) return 0;
    out->format_version = h.version;
    out->source_uuid = h.source_uuid;
    memcpy(out->arch, h.arch, sizeof out->arch);
    out->arch[sizeof out->arch - 1] = '\0';
    out->n_layers = (int32_t)h.n_layers;
    out->n_expert = (int32_t)h.n_expert;
    out->n_embd = h.n_embd;
    out->n_ff_exp = h.n_ff_exp;
    out->pack_uuid = h.pack_uuid;
    out->record_count = h.record_count;
    return 1;
}

int64_t moert_store_verify(const char * index_path) {
    IdxHeader h;
    std::vector<IdxRecord> recs;
    int fd;
    if (!index_path || !load_store(index_path, h, recs, &fd)) return -1;
    // each page hashed through a fixed buffer (FNV-1a continues from the
    // running value)
    std::vector<uint8_t> buf(1 << 20);
    int64_t bad = 0;
    for (const IdxRecord & r : recs) {
        uint64_t hsh = MOERT_STORE_FNV_SEED, done = 0;
        bool ok = true;
        while (ok && done < r.nbytes) {
            const uint64_t n = std::min<uint64_t>(buf.size(), r.nbytes - done);
            ok = read_fully(fd, buf.data(), n, r.offset + done) == 0;
            if (ok) hsh = moert_store_fnv1a64(buf.data(), n, hsh);
            done += n;
        }
        if (!ok || hsh != r.checksum) ++bad;
    }
    close(fd);
    return bad;
}

moert_store_writer * moert_store_writer_open(const char * index_path, const char * pack_path,
                                             const moert_store_info * info) {
    if (!index_path || !pack_path || !info || info->n_layers <= 0 || info->n_expert <= 0) return nullptr;
    moert_store_writer * w = new moert_store_writer();
    w->index_path = index_path;
    w->pack = fopen(pack_path, "wb");
    if (!w->pack) {
        delete w;
        return nullptr;
    }
    memcpy(w->h.magic, INDEX_MAGIC, 8);
    w->h.version = VERSION;
    w->h.header_bytes = sizeof(IdxHeader);
    w->h.source_uuid = info->source_uuid;
    strncpy(w->h.arch, info->arch, sizeof w->h.arch - 1);
    w->h.n_layers = (uint32_t)info->n_layers;
    w->h.n_expert = (uint32_t)info->n_expert;
    w->h.n_embd = info->n_embd;
    w->h.n_ff_exp = info->n_ff_exp;
    w->h.pack_uuid = info->pack_uuid ? info->pack_uuid
                                     : moert_store_fnv1a64(index_path, strlen(index_path),
                                                           MOERT_STORE_FNV_SEED ^ (uint64_t)time(nullptr));
    w->h.record_stride = sizeof(IdxRecord);
    w->h.checksum_algo = FNV_ALGO;
    PkHeader ph = {};
    memcpy(ph.magic, PACK_MAGIC, 8);
    ph.version = VERSION;
    ph.pack_uuid = w->h.pack_uuid;
    if (fwrite(&ph, sizeof ph, 1, w->pack) != 1) w->failed = true;
    w->pos = sizeof ph;
    return w;
}

int32_t moert_store_writer_add_page(moert_store_writer * w, int32_t layer, int32_t expert_id, int32_t kind,
                                    int32_t is_scale, int32_t quant_type, int32_t source_quant, uint32_t extra_flags,
                                    const int64_t * shape, int32_t ndim, const void * bytes, uint64_t nbytes) {
    if (!w || w->failed || !bytes || ndim < 0 || ndim > 4 || layer < 0 || expert_id < 0) return 0;
    const uint64_t at = (w->pos + PAGE_ALIGN - 1) & ~(PAGE_ALIGN - 1);
    static const uint8_t zeros[PAGE_ALIGN] = {};
    if ((at > w->pos && fwrite(zeros, 1, at - w->pos, w->pack) != at - w->pos) ||
        fwrite(bytes, 1, nbytes, w->pack) != nbytes) {
        w->failed = true;
        return 0;
    }
    w->pos = at + nbytes;
    IdxRecord r = {};
    r.layer = (uint16_t)layer;
    r.expert = (uint16_t)expert_id;
    r.kind = (uint8_t)kind;
    r.quant_type = (uint16_t)quant_type;
    r.offset = at;
    r.nbytes = nbytes;
    for (int i = 0; i < 4; ++i) r.shape[i] = i < ndim && shape ? shape[i] : 1;
    r.checksum = moert_store_fnv1a64(bytes, nbytes, MOERT_STORE_FNV_SEED);
    r.source_quant = (uint16_t)source_quant;
    r.flags = extra_flags | (is_scale ? (uint32_t)MOERT_PAGE_SCALE : 0u);
    w->recs.push_back(r);
    return 1;
}

int32_t moert_store_writer_close(moert_store_writer * w) {
    if (!w) return 0;
    bool ok = !w->failed && fflush(w->pack) == 0 && fsync(fileno(w->pack)) == 0;
    ok = fclose(w->pack) == 0 && ok;
    if (ok) {
        w->h.record_count = w->recs.size();
        FILE * f = fopen(w->index_path.c_str(), "wb");
        ok = f && fwrite(&w->h, sizeof w->h, 1, f) == 1 &&
             (w->recs.empty() || fwrite(w->recs.data(), sizeof(IdxRecord), w->recs.size(), f) == w->recs.size()) &&
             fflush(f) == 0 && fsync(fileno(f)) == 0;
        if (f) ok = fclose(f) == 0 && ok;
    }
    delete w;
    return ok ? 1 : 0;
}

moert_store_reader * moert_store_reader_open(const char * index_path, uint64_t expect_source_uuid) {
    if (!index_path) return nullptr;
    moert_store_reader * r = new moert_store_reader();
    if (!load_store(index_path, r->h, r->recs, &r->fd)) {
        delete r;
        return nullptr;
    }
    if (expect_source_uuid && r->h.source_uuid != expect_source_uuid) {
        ffail(std::string("moert-store: ") + index_path + ": source_uuid does not match");
        close(r->fd);
        delete r;
        return nullptr;
    }
    r->slot.assign((size_t)r->h.n_layers * MAX_KIND * 2 * r->h.n_expert, -1);
    for (size_t i = 0; i < r->recs.size(); ++i) {
        const IdxRecord & rec = r->recs[i];
        const int64_t k = r->key(rec.layer, rec.kind, (rec.flags & MOERT_PAGE_SCALE) ? 1 : 0, rec.expert);
        if (k >= 0) r->slot[(size_t)k] = (int64_t)i;
    }
    return r;
}

void moert_store_reader_free(moert_store_reader * r) {
    if (!r) return;
    if (r->fd >= 0) close(r->fd);
    delete r;
}

int32_t moert_store_reader_geometry(const moert_store_reader * r, int32_t * n_layers, int32_t * n_expert) {
    if (!r) return 0;
    if (n_layers) *n_layers = (int32_t)r->h.n_layers;
    if (n_expert) *n_expert = (int32_t)r->h.n_expert;
    return 1;
}

uint64_t moert_store_reader_page_nbytes(const moert_store_reader * r, int32_t layer, int32_t kind, int32_t is_scale,
                                        int32_t expert) {
    const IdxRecord * rec = r ? r->rec(layer, kind, is_scale, expert) : nullptr;
    return rec ? rec->nbytes : 0;
}

int32_t moert_store_reader_page_info(const moert_store_reader * r, int32_t layer, int32_t kind, int32_t is_scale,
                                     int32_t expert, int32_t * quant_type, uint64_t * nbytes, int64_t shape[4]) {
    const IdxRecord * rec = r ? r->rec(layer, kind, is_scale, expert) : nullptr;
    if (!rec) return 0;
    if (quant_type) *quant_type = rec->quant_type;
    if (nbytes) *nbytes = rec->nbytes;
    if (shape)
        for (int i = 0; i < 4; ++i) shape[i] = rec->shape[i];
    return 1;
}

uint64_t moert_store_reader_read(moert_store_reader * r, int32_t layer, int32_t kind, int32_t is_scale, int32_t expert,
                                 void * dst, uint64_t dst_cap, int32_t verify) {
    const IdxRecord * rec = r && dst ? r->rec(layer, kind, is_scale, expert) : nullptr;
    if (!rec || rec->nbytes > dst_cap) return 0;
    if (read_fully(r->fd, dst, rec->nbytes, rec->offset) != 0) return 0;
    if (verify && moert_store_fnv1a64(dst, rec->nbytes, MOERT_STORE_FNV_SEED) != rec->checksum) {
        ffail("moert-store: reader: checksum mismatch");
        return 0;
    }
    return rec->nbytes;
}

int32_t llapis_store_upload(moert_store_reader * r, int32_t layer, int32_t kind, int32_t is_scale,
                            const int32_t * experts, int32_t n, void * dst, uint64_t dst_stride, int32_t verify,
                            void * stream) {
    if (!r || !experts || n <= 0 || !dst) return ffail("llapis_store_upload: bad arguments");
    for (int32_t i = 0; i < n; ++i) {
        const IdxRecord * rec = r->rec(layer, kind, is_scale, experts[i]);
        if (!rec) return ffail("llapis_store_upload: page absent");
        if (rec->nbytes > dst_stride) return ffail("llapis_store_upload: page larger than the destination stride");
    }
    Staging st;
    if (!st.init()) return ffail("llapis_store_upload: pinned staging allocation failed");
    for (int32_t i = 0; i < n; ++i) {
        const IdxRecord * rec = r->rec(layer, kind, is_scale, experts[i]);
        uint64_t h = MOERT_STORE_FNV_SEED;
        if (upload_range(st, r->fd, rec->offset, rec->nbytes, (uint8_t *)dst + (uint64_t)i * dst_stride,
                         (hipStream_t)stream, verify ? &h : nullptr, "llapis_store_upload") != 0)
            return -1;
        if (verify && h != rec->checksum) return ffail("llapis_store_upload: checksum mismatch");
    }
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) {
        (void)hipGetLastError();
        return ffail("llapis_store_upload: stream failed");
    }
    return 0;
}

}  // extern "C"
