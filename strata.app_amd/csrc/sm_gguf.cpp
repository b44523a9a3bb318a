// GGUF expert tensors -> device storage and the [layer][E][3] expert address table.
//
// The reference keeps every layer's routed experts as three GGUF tensors,
// blk.<l>.ffn_{gate,up,down}_exps.weight with ne = [d, I, E] (gate, up) and [I, d, E] (down)
// (docs/mac/03-model-reference.md:292-297), and resolves each expert slab to a GPU address in
// a row-major [layer * n_expert + expert][gate, up, down] u64 table
// (src/metal/engine/window.cpp:128-270, include/strata/metal/window.hpp:34-44), which the
// expert encoders then validate against declared storage
// (prefill_moe_expert_dispatch.mm:377-448). Here the tensors are read from the file into one
// caller-registered device allocation (HBM holds a whole model's experts), in pinned chunks
// on the caller's stream, and the table is filled with device addresses. GGUF is parsed from
// its published layout (v2/v3, little-endian): header, metadata key/values (only
// general.alignment is used), tensor directory, aligned data section.
#include <hip/hip_runtime_api.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <string>
#include <vector>

#include "../../include/strata_moe.h"
#include "sm_internal.h"

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint64_t kMaxString = 1ull << 24;   // longest key / string value accepted
constexpr uint64_t kPlaceAlign = 256;         // device placement of each expert tensor

// ggml type ids of the formats the expert kernels decode, and the dense ones the directory
// may hold beside them.
enum GgmlType : uint32_t { kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ2_K = 10, kQ4_K = 12, kBF16 = 30 };

// (values per block, bytes per block) of the ggml types with a published block layout.
bool block_geometry(uint32_t t, uint64_t& vals, uint64_t& bytes) {
    switch (t) {
        case 0: vals = 1; bytes = 4; return true;     // F32
        case 1: vals = 1; bytes = 2; return true;     // F16
        case 30: vals = 1; bytes = 2; return true;    // BF16
        case 2: vals = 32; bytes = 18; return true;   // Q4_0
        case 3: vals = 32; bytes = 20; return true;   // Q4_1
        case 6: vals = 32; bytes = 22; return true;   // Q5_0
        case 7: vals = 32; bytes = 24; return true;   // Q5_1
        case 8: vals = 32; bytes = 34; return true;   // Q8_0
        case 9: vals = 32; bytes = 36; return true;   // Q8_1
        case 10: vals = 256; bytes = 84; return true; // Q2_K
        case 11: vals = 256; bytes = 110; return true; // Q3_K
        case 12: vals = 256; bytes = 144; return true; // Q4_K
        case 13: vals = 256; bytes = 176; return true; // Q5_K
        case 14: vals = 256; bytes = 210; return true; // Q6_K
        case 15: vals = 256; bytes = 292; return true; // Q8_K
        default: return false;
    }
}

int format_of(uint32_t t) {
    switch (t) {
        case kQ8_0: return SM_FMT_Q8_0;
        case kQ4_K: return SM_FMT_Q4_K;
        case kQ2_K: return SM_FMT_Q2_K;
        default: return 0;
    }
}

bool add_ok(uint64_t a, uint64_t b, uint64_t& out) {
    if (a > std::numeric_limits<uint64_t>::max() - b) return false;
    out = a + b;
    return true;
}
bool mul_ok2(uint64_t a, uint64_t b, uint64_t& out) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
    out = a * b;
    return true;
}

// Sequential little-endian reader over a file descriptor (pread in 1 MiB buffered pieces).
struct Reader {
    int fd = -1;
    uint64_t size = 0, pos = 0;
    std::vector<uint8_t> buf;
    uint64_t buf_pos = 0, buf_len = 0;
    bool ok = true;

    bool fill(uint64_t at) {
        buf.resize(1u << 20);
        const ssize_t n = ::pread(fd, buf.data(), buf.size(), off_t(at));
        if (n <= 0) return false;
        buf_pos = at;
        buf_len = uint64_t(n);
        return true;
    }
    bool read(void* dst, uint64_t n) {
        uint8_t* d = static_cast<uint8_t*>(dst);
        while (n > 0) {
            if (pos >= size) return ok = false;
            if (pos < buf_pos || pos >= buf_pos + buf_len)
                if (!fill(pos)) return ok = false;
            const uint64_t take = std::min(n, buf_pos + buf_len - pos);
            std::memcpy(d, buf.data() + (pos - buf_pos), take);
            d += take;
            pos += take;
            n -= take;
        }
        return true;
    }
    bool skip(uint64_t n) {
        uint64_t e;
        if (!add_ok(pos, n, e) || e > size) return ok = false;
        pos = e;
        return true;
    }
    template <class T>
    bool get(T& v) { return read(&v, sizeof v); }
    bool string(std::string& s) {
        uint64_t n = 0;
        if (!get(n) || n > kMaxString) return ok = false;
        s.resize(n);
        return n == 0 || read(&s[0], n);
    }
};

// Skips (or, for general.alignment, reads) one metadata value of GGUF type `t`.
bool skip_value(Reader& r, uint32_t t, int depth) {
    switch (t) {
        case 0: case 1: case 7: return r.skip(1);           // u8, i8, bool
        case 2: case 3: return r.skip(2);                   // u16, i16
        case 4: case 5: case 6: return r.skip(4);           // u32, i32, f32
        case 10: case 11: case 12: return r.skip(8);        // u64, i64, f64
        case 8: {                                           // string
            uint64_t n = 0;
            return r.get(n) && r.skip(n);
        }
        case 9: {                                           // array
            uint32_t et = 0;
            uint64_t n = 0;
            if (depth > 4 || !r.get(et) || !r.get(n)) return false;
            uint64_t width = 0;
            switch (et) {
                case 0: case 1: case 7: width = 1; break;
                case 2: case 3: width = 2; break;
                case 4: case 5: case 6: width = 4; break;
                case 10: case 11: case 12: width = 8; break;
                default: break;
            }
            if (width != 0) {
                uint64_t b;
                return mul_ok2(n, width, b) && r.skip(b);
            }
            for (uint64_t i = 0; i < n; ++i)
                if (!skip_value(r, et, depth + 1)) return false;
            return true;
        }
        default: return false;
    }
}

std::string layer_name(uint32_t l, const char* role) {
    return "blk." + std::to_string(l) + ".ffn_" + role + "_exps.weight";
}

}  // namespace

struct sm_gguf {
    int fd = -1;
    uint64_t file_size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    struct Tensor {
        std::string name;
        uint32_t type = 0, n_dims = 0;
        uint64_t ne[4] = {1, 1, 1, 1};
        uint64_t offset = 0;  // absolute file offset of the data
        uint64_t bytes = 0;   // 0 when the type has no known block layout
    };
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> index;
};

namespace {
sm_status fail(char* err, size_t cap, sm_status st, const std::string& msg) {
    if (err && cap) std::snprintf(err, cap, "%s", msg.c_str());
    return st;
}
}  // namespace

extern "C" {

sm_status sm_gguf_open(const char* path, sm_gguf** out, char* err, size_t cap) {
    if (!path || !out) return fail(err, cap, SM_E_ARGUMENT, "GGUF path or output is null");
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(err, cap, SM_E_FILE, std::string("GGUF file cannot be opened: ") + path);
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        return fail(err, cap, SM_E_FILE, "GGUF file cannot be read");
    }
    auto* g = new (std::nothrow) sm_gguf();
    if (!g) {
        ::close(fd);
        return fail(err, cap, SM_E_DEVICE, "out of host memory");
    }
    g->fd = fd;
    g->file_size = uint64_t(st.st_size);
    Reader r;
    r.fd = fd;
    r.size = g->file_size;
    auto bad = [&](const std::string& msg) {
        sm_gguf_close(g);
        return fail(err, cap, SM_E_FILE, "GGUF " + msg);
    };
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.get(magic) || magic != kGgufMagic) return bad("magic is missing");
    if (!r.get(g->version) || (g->version != 2 && g->version != 3)) return bad("version is not 2 or 3");
    if (!r.get(n_tensors) || !r.get(n_kv)) return bad("header is truncated");
    if (n_tensors > (1u << 24) || n_kv > (1u << 24)) return bad("header counts are implausible");
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t t = 0;
        if (!r.string(key) || !r.get(t)) return bad("metadata is truncated");
        if (key == "general.alignment") {
            uint32_t a = 0;
            if (t != 4 || !r.get(a) || a == 0 || (a & (a - 1)) != 0) return bad("general.alignment is not a power of two");
            g->alignment = a;
        } else if (!skip_value(r, t, 0)) {
            return bad("metadata value of key " + key + " is malformed");
        }
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        sm_gguf::Tensor t;
        if (!r.string(t.name) || t.name.empty() || !r.get(t.n_dims) || t.n_dims == 0 || t.n_dims > 4)
            return bad("tensor directory entry " + std::to_string(i) + " is malformed");
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (!r.get(t.ne[d])) return bad("tensor directory is truncated");
        uint64_t rel = 0;
        if (!r.get(t.type) || !r.get(rel)) return bad("tensor directory is truncated");
        if (g->index.count(t.name)) return bad("tensor " + t.name + " appears twice");
        t.offset = rel;  // relative until the data section is known
        uint64_t vals = 0, bb = 0;
        if (block_geometry(t.type, vals, bb)) {
            uint64_t n = t.ne[0], rows = 1, b = 0;
            for (uint32_t d = 1; d < 4; ++d)
                if (!mul_ok2(rows, t.ne[d], rows)) return bad("tensor " + t.name + " is too large");
            if (n % vals != 0) return bad("tensor " + t.name + " rows are not whole blocks");
            if (!mul_ok2(n / vals, bb, b) || !mul_ok2(b, rows, t.bytes)) return bad("tensor " + t.name + " is too large");
        }
        g->index[t.name] = g->tensors.size();
        g->tensors.push_back(t);
    }
    uint64_t data = 0;
    if (!add_ok(r.pos, g->alignment - 1, data)) return bad("data section offset overflows");
    data &= ~(g->alignment - 1);
    g->data_offset = data;
    for (auto& t : g->tensors) {
        uint64_t abs = 0, end = 0;
        if (t.offset % g->alignment != 0 || !add_ok(data, t.offset, abs) || !add_ok(abs, t.bytes, end) ||
            end > g->file_size)
            return bad("tensor " + t.name + " data lies outside the file or is misaligned");
        t.offset = abs;
    }
    *out = g;
    if (err && cap) err[0] = 0;
    return SM_OK;
}

void sm_gguf_close(sm_gguf* g) {
    if (!g) return;
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

uint64_t sm_gguf_tensor_count(const sm_gguf* g) { return g ? g->tensors.size() : 0; }

sm_status sm_internal_gguf_read(const sm_gguf* g, uint64_t offset, uint64_t bytes, void* dst) {
    if (!g || !dst) return SM_E_ARGUMENT;
    uint64_t got = 0;
    while (got < bytes) {
        const ssize_t rd = ::pread(g->fd, static_cast<uint8_t*>(dst) + got, bytes - got, off_t(offset + got));
        if (rd <= 0) return SM_E_FILE;
        got += uint64_t(rd);
    }
    return SM_OK;
}

sm_status sm_gguf_find(const sm_gguf* g, const char* name, sm_gguf_tensor* out) {
    if (!g || !name || !out) return SM_E_ARGUMENT;
    auto it = g->index.find(name);
    if (it == g->index.end()) return SM_E_ARGUMENT;
    const auto& t = g->tensors[it->second];
    out->ggml_type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->bytes = t.bytes;
    return SM_OK;
}

sm_status sm_gguf_expert_layout(const sm_gguf* g, uint32_t n_layers, sm_expert_layout* out, char* err, size_t cap) {
    if (!g || !out) return fail(err, cap, SM_E_ARGUMENT, "GGUF handle or output is null");
    if (n_layers == 0 || n_layers > SM_GGUF_MAX_LAYERS)
        return fail(err, cap, SM_E_SHAPE, "expert layout needs 1..SM_GGUF_MAX_LAYERS layers");
    sm_expert_layout L{};
    L.n_layers = n_layers;
    uint64_t place = 0;
    const char* roles[3] = {"gate", "up", "down"};
    for (uint32_t l = 0; l < n_layers; ++l) {
        const sm_gguf::Tensor* t3[3];
        for (int r = 0; r < 3; ++r) {
            const std::string name = layer_name(l, roles[r]);
            auto it = g->index.find(name);
            if (it == g->index.end()) return fail(err, cap, SM_E_SHAPE, "GGUF has no tensor " + name);
            t3[r] = &g->tensors[it->second];
            const auto& t = *t3[r];
            if (t.n_dims != 3) return fail(err, cap, SM_E_SHAPE, name + " is not a 3-D [k, rows, experts] tensor");
            if (format_of(t.type) == 0)
                return fail(err, cap, SM_E_FORMAT, name + " is not Q8_0, Q4_K or Q2_K");
        }
        const auto &tg = *t3[0], &tu = *t3[1], &td = *t3[2];
        if (tg.type != tu.type) return fail(err, cap, SM_E_FORMAT, "gate and up experts of layer " + std::to_string(l) + " differ in type");
        if (tg.ne[0] != tu.ne[0] || tg.ne[1] != tu.ne[1] || tg.ne[2] != tu.ne[2] || td.ne[0] != tg.ne[1] ||
            td.ne[1] != tg.ne[0] || td.ne[2] != tg.ne[2])
            return fail(err, cap, SM_E_SHAPE, "expert tensors of layer " + std::to_string(l) + " disagree in shape");
        if (tg.ne[0] > UINT32_MAX || tg.ne[1] > UINT32_MAX || tg.ne[2] == 0 || tg.ne[2] > SM_MAX_EXPERTS)
            return fail(err, cap, SM_E_SHAPE, "expert tensors of layer " + std::to_string(l) + " are out of range");
        if (l == 0) {
            L.hidden = uint32_t(tg.ne[0]);
            L.expert_ff = uint32_t(tg.ne[1]);
            L.n_experts = uint32_t(tg.ne[2]);
            L.gate_up = sm_format(format_of(tg.type));
            L.down = sm_format(format_of(td.type));
        } else if (L.hidden != tg.ne[0] || L.expert_ff != tg.ne[1] || L.n_experts != tg.ne[2] ||
                   L.gate_up != format_of(tg.type) || L.down != format_of(td.type)) {
            return fail(err, cap, SM_E_SHAPE, "layer " + std::to_string(l) + " differs from layer 0 in shape or type");
        }
        for (int r = 0; r < 3; ++r) {
            // Each expert slab must start where the kernels can read it: 16 bytes for the
            // K-quants, 4 for Q8_0 (tensor bases are placed 256-aligned).
            const uint64_t slab = t3[r]->bytes / t3[r]->ne[2];
            const uint64_t need = format_of(t3[r]->type) == SM_FMT_Q8_0 ? 4 : 16;
            if (slab % need != 0)
                return fail(err, cap, SM_E_ADDRESS, layer_name(l, roles[r]) + " expert slabs are not " + std::to_string(need) + "-byte aligned");
            L.offsets[l][r] = place;
            uint64_t end = 0;
            if (!add_ok(place, t3[r]->bytes, end) || !add_ok(end, kPlaceAlign - 1, end))
                return fail(err, cap, SM_E_SHAPE, "expert storage size overflows");
            place = end & ~(kPlaceAlign - 1);
        }
    }
    L.total_bytes = place;
    *out = L;
    if (err && cap) err[0] = 0;
    return SM_OK;
}

sm_status sm_gguf_load_experts(sm_gguf* g, sm_context* ctx, void* stream, const sm_expert_layout* L, sm_view storage,
                               uint64_t* addresses, uint64_t n_addresses, char* err, size_t cap) {
    if (!g || !ctx || !L || !addresses) return fail(err, cap, SM_E_ARGUMENT, "GGUF load arguments are null");
    // The caller's layout is a plain struct: it must be the one this file gives for its layer
    // count (an edited layout, or one made from another file, could place a tensor past the
    // storage or name a tensor the file lacks). Everything below uses the recomputed one.
    if (L->n_layers == 0 || L->n_layers > SM_GGUF_MAX_LAYERS)
        return fail(err, cap, SM_E_ARGUMENT, "expert layout needs 1..SM_GGUF_MAX_LAYERS layers");
    sm_expert_layout mine{};
    char why[256] = {0};
    if (sm_gguf_expert_layout(g, L->n_layers, &mine, why, sizeof why) != SM_OK)
        return fail(err, cap, SM_E_ARGUMENT, std::string("expert layout does not fit this GGUF file: ") + why);
    bool same = L->n_experts == mine.n_experts && L->hidden == mine.hidden && L->expert_ff == mine.expert_ff &&
                L->gate_up == mine.gate_up && L->down == mine.down && L->total_bytes == mine.total_bytes;
    for (uint32_t l = 0; l < mine.n_layers && same; ++l)
        for (int r = 0; r < 3; ++r) same = same && L->offsets[l][r] == mine.offsets[l][r];
    if (!same) return fail(err, cap, SM_E_ARGUMENT, "expert layout does not match this GGUF file");
    L = &mine;
    const uint64_t E = L->n_experts;
    uint64_t need_words = 0;
    if (!mul_ok2(uint64_t(L->n_layers) * E, 3, need_words) || n_addresses < need_words)
        return fail(err, cap, SM_E_ARGUMENT, "address table is shorter than n_layers * n_experts * 3");
    uintptr_t base = 0;
    const sm_status vs = sm_internal_resolve_view(ctx, storage, L->total_bytes, kPlaceAlign, &base);
    if (vs != SM_OK)
        return fail(err, cap, vs, vs == SM_E_OWNERSHIP ? "expert storage view is not owned by this context"
                                                       : "expert storage view is undersized or misaligned");
    if (sm_internal_make_current(ctx) != SM_OK) return fail(err, cap, SM_E_DEVICE, "the context's device cannot be made current");
    const char* roles[3] = {"gate", "up", "down"};
    // Pinned staging: two chunks, each copied while the other is read from the file.
    constexpr uint64_t kChunk = 16ull << 20;
    uint8_t* pinned = nullptr;
    hipEvent_t done[2] = {nullptr, nullptr};
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (hipHostMalloc(reinterpret_cast<void**>(&pinned), 2 * kChunk, hipHostMallocDefault) != hipSuccess)
        return fail(err, cap, SM_E_DEVICE, "pinned staging buffer cannot be allocated");
    sm_status st = SM_OK;
    std::string msg;
    for (int i = 0; i < 2 && st == SM_OK; ++i)
        if (hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) st = SM_E_DEVICE;
    bool pending[2] = {false, false};
    uint64_t k = 0;  // chunk counter
    for (uint32_t l = 0; l < L->n_layers && st == SM_OK; ++l) {
        for (int r = 0; r < 3 && st == SM_OK; ++r) {
            const auto it = g->index.find(layer_name(l, roles[r]));  // present: the layout found it
            const auto& t = g->tensors[it->second];
            const uint64_t dst = base + L->offsets[l][r];
            for (uint64_t off = 0; off < t.bytes && st == SM_OK; off += kChunk, ++k) {
                const int b = int(k & 1);
                if (pending[b] && hipEventSynchronize(done[b]) != hipSuccess) { st = SM_E_DEVICE; break; }
                const uint64_t n = std::min(kChunk, t.bytes - off);
                uint64_t got = 0;
                while (got < n) {
                    const ssize_t rd = ::pread(g->fd, pinned + b * kChunk + got, n - got, off_t(t.offset + off + got));
                    if (rd <= 0) break;
                    got += uint64_t(rd);
                }
                if (got != n) { st = SM_E_FILE; msg = "GGUF tensor " + t.name + " cannot be read"; break; }
                if (hipMemcpyAsync(reinterpret_cast<void*>(dst + off), pinned + b * kChunk, n, hipMemcpyHostToDevice,
                                   s) != hipSuccess ||
                    hipEventRecord(done[b], s) != hipSuccess) {
                    st = SM_E_DEVICE;
                    break;
                }
                pending[b] = true;
            }
            const uint64_t slab = t.bytes / E;
            for (uint64_t e = 0; e < E; ++e)
                addresses[(uint64_t(l) * E + e) * 3 + uint64_t(r)] = dst + e * slab;
        }
    }
    if (hipStreamSynchronize(s) != hipSuccess && st == SM_OK) st = SM_E_DEVICE;
    for (auto& e : done)
        if (e) (void)hipEventDestroy(e);  // teardown of the loader's own events
    (void)hipHostFree(pinned);
    if (st != SM_OK) return fail(err, cap, st, msg.empty() ? "expert upload failed" : msg);
    if (err && cap) err[0] = 0;
    return SM_OK;
}

}  // extern "C"
