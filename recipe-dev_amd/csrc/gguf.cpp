// GGUF v3 reader (see gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace rq {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
constexpr int kMaxDepth = 64;

struct Fail {
    std::string msg;
};

struct Reader {
    const uint8_t* p;
    size_t n, at = 0;
    int depth = 0;
    const uint8_t* take(size_t count) {
        if (count > n - at) throw Fail{"GGUF header is truncated"};
        const uint8_t* s = p + at;
        at += count;
        return s;
    }
    template <typename T>
    T get() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));  // the file is little-endian, as the host
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (len > n - at) throw Fail{"GGUF header is truncated"};
        const uint8_t* s = take((size_t)len);
        return std::string(reinterpret_cast<const char*>(s), (size_t)len);
    }
    GgufValue value(uint32_t type) {
        GgufValue v;
        v.type = type;
        switch (type) {
            case 0: v.u = get<uint8_t>(); break;
            case 1: v.i = get<int8_t>(); break;
            case 2: v.u = get<uint16_t>(); break;
            case 3: v.i = get<int16_t>(); break;
            case 4: v.u = get<uint32_t>(); break;
            case 5: v.i = get<int32_t>(); break;
            case 6: v.f = get<float>(); break;
            case 7: v.u = get<uint8_t>() != 0; break;
            case 8: v.s = str(); break;
            case 9: {
                v.array_type = get<uint32_t>();
                const uint64_t count = get<uint64_t>();
                if (++depth > kMaxDepth) throw Fail{"GGUF arrays nest deeper than 64 levels"};
                if (count > n - at) throw Fail{"GGUF header is truncated"};  // every element takes a byte or more
                v.array.reserve((size_t)count);
                for (uint64_t k = 0; k < count; ++k) v.array.push_back(value(v.array_type));
                --depth;
                break;
            }
            case 10: v.u = get<uint64_t>(); break;
            case 11: v.i = get<int64_t>(); break;
            case 12: v.f = get<double>(); break;
            default: throw Fail{"GGUF value type " + std::to_string(type) + " is unsupported"};
        }
        return v;
    }
};

bool map_file(const std::string& path, GgufMapping* m, std::string* error) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        *error = "cannot open " + path + ": " + std::strerror(errno);
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        *error = "cannot inspect " + path + ": " + std::strerror(errno);
        ::close(fd);
        return false;
    }
    if (st.st_size == 0) {
        *error = path + " is empty";
        ::close(fd);
        return false;
    }
    void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) {
        *error = "cannot map " + path + ": " + std::strerror(errno);
        return false;
    }
    m->data = static_cast<const uint8_t*>(p);
    m->length = (size_t)st.st_size;
    return true;
}

struct Shard {
    std::unique_ptr<GgufMapping> map;
    uint64_t data = 0;
    std::vector<std::pair<std::string, GgufValue>> metadata;
    std::vector<GgufTensor> tensors;
};

const GgufValue* find_value(const std::vector<std::pair<std::string, GgufValue>>& md, const char* key) {
    for (const auto& kv : md)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

// One shard's header (recipe.rs:10095-10131).
bool read_shard(const std::string& path, uint64_t index, Shard* s, std::string* error) {
    s->map.reset(new GgufMapping);
    if (!map_file(path, s->map.get(), error)) return false;
    try {
        Reader r{s->map->data, s->map->length};
        if (r.get<uint32_t>() != kMagic) throw Fail{path + " is not a GGUF file"};
        const uint32_t version = r.get<uint32_t>();
        if (version != kVersion)
            throw Fail{path + " is GGUF version " + std::to_string(version) + "; version 3 is supported"};
        const uint64_t tensor_count = r.get<uint64_t>(), pair_count = r.get<uint64_t>();
        for (uint64_t k = 0; k < pair_count; ++k) {
            std::string key = r.str();
            const uint32_t type = r.get<uint32_t>();
            s->metadata.emplace_back(std::move(key), r.value(type));
        }
        uint64_t alignment = kDefaultAlignment;
        if (const GgufValue* a = find_value(s->metadata, "general.alignment")) {
            uint64_t v;
            if (a->integer(&v)) alignment = v;
        }
        if (alignment == 0 || (alignment & (alignment - 1)))
            throw Fail{path + " declares alignment " + std::to_string(alignment)};
        if (const GgufValue* no = find_value(s->metadata, "split.no")) {
            uint64_t v;
            if (no->integer(&v) && v != index)
                throw Fail{path + " is shard " + std::to_string(v) + ", expected shard " + std::to_string(index)};
        }
        for (uint64_t k = 0; k < tensor_count; ++k) {
            GgufTensor t;
            t.name = r.str();
            const uint32_t dims = r.get<uint32_t>();
            if (dims > 8) throw Fail{"tensor " + t.name + " has " + std::to_string(dims) + " dimensions"};
            for (uint32_t d = 0; d < dims; ++d) t.shape.push_back(r.get<uint64_t>());
            t.type = r.get<uint32_t>();
            t.offset = r.get<uint64_t>();
            uint64_t be, bb;
            if (!ggml_block(t.type, &be, &bb))
                throw Fail{"GGUF tensor type " + std::to_string(t.type) + " is unsupported"};
            unsigned __int128 elements = 1;
            for (uint64_t d : t.shape) {
                elements *= d;
                if (elements >> 64) throw Fail{"tensor " + t.name + " shape overflows"};
            }
            if ((uint64_t)elements % be)
                throw Fail{"tensor " + t.name + " holds " + std::to_string((uint64_t)elements) +
                           " elements, not a multiple of its " + std::to_string(be) + "-element block"};
            // the byte count in 128 bits: a shape whose bytes do not fit in 63 bits is refused
            // before any size derived from it can wrap
            const unsigned __int128 nbytes = elements / be * bb;
            if (nbytes >> 63) throw Fail{"tensor " + t.name + " shape overflows"};
            t.bytes = (uint64_t)nbytes;
            t.shard = (int)index;
            s->tensors.push_back(std::move(t));
        }
        s->data = (r.at + alignment - 1) / alignment * alignment;
        for (const GgufTensor& t : s->tensors) {
            const uint64_t len = s->map->length;
            if (s->data > len || t.offset > len - s->data || t.bytes > len - s->data - t.offset)
                throw Fail{"tensor " + t.name + " runs past the end of " + path};
        }
    } catch (const Fail& f) {
        *error = f.msg;
        return false;
    }
    return true;
}

// The path of shard `index` of a split named <prefix>-<n>-of-<count>.gguf (recipe.rs:10319-10325).
bool sibling(const std::string& path, uint64_t index, uint64_t count, std::string* out, std::string* error) {
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? "" : path.substr(0, slash + 1);
    const std::string name = slash == std::string::npos ? path : path.substr(slash + 1);
    const std::string suffix = ".gguf";
    bool ok = name.size() > suffix.size() && name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0;
    std::string prefix;
    if (ok) {
        const std::string stem = name.substr(0, name.size() - suffix.size());
        const size_t of = stem.rfind("-of-");
        ok = of != std::string::npos;
        if (ok) {
            const std::string head = stem.substr(0, of);
            const size_t dash = head.rfind('-');
            ok = dash != std::string::npos;
            if (ok) prefix = head.substr(0, dash);
        }
    }
    if (!ok) {
        *error = name + " declares a split but is not named <prefix>-<number>-of-<count>.gguf";
        return false;
    }
    char buf[64];
    snprintf(buf, sizeof buf, "-%05llu-of-%05llu.gguf", (unsigned long long)(index + 1), (unsigned long long)count);
    *out = dir + prefix + buf;
    return true;
}

}  // namespace

GgufMapping::~GgufMapping() {
    if (data) munmap(const_cast<uint8_t*>(data), length);
}

bool GgufValue::integer(uint64_t* out) const {
    switch (type) {
        case 0: case 2: case 4: case 10: *out = u; return true;
        case 1: case 3: case 5: case 11:
            if (i < 0) return false;
            *out = (uint64_t)i;
            return true;
        default: return false;
    }
}

bool GgufValue::real(double* out) const {
    if (type != 6 && type != 12) return false;
    *out = f;
    return true;
}

const GgufValue* GgufFile::value(const std::string& key) const {
    for (const auto& kv : metadata)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
    for (const GgufTensor& t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

const uint8_t* GgufFile::bytes(const GgufTensor& t) const {
    return shards[t.shard]->data + data_start[t.shard] + t.offset;
}

// recipe.rs:9927-9961 (element and byte counts of the GGML block layouts).
bool ggml_block(uint32_t type, uint64_t* elements, uint64_t* bytes) {
    struct B {
        uint32_t id, e, b;
    };
    static const B table[] = {
        {0, 1, 4},     {1, 1, 2},     {24, 1, 1},    {25, 1, 2},    {26, 1, 4},    {27, 1, 8},   {28, 1, 8},
        {30, 1, 2},    {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},   {8, 32, 34},  {9, 32, 36},
        {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292},
        {16, 256, 66}, {17, 256, 74},  {18, 256, 98},  {19, 256, 50},  {20, 32, 18},  {21, 256, 110},
        {22, 256, 82}, {23, 256, 136}, {29, 256, 56},
    };
    for (const B& b : table)
        if (b.id == type) {
            *elements = b.e;
            *bytes = b.b;
            return true;
        }
    return false;
}

std::unique_ptr<GgufFile> gguf_open(const std::string& path, std::string* error) {
    std::vector<Shard> shards(1);
    if (!read_shard(path, 0, &shards[0], error)) return nullptr;
    uint64_t count = 1;
    if (const GgufValue* c = find_value(shards[0].metadata, "split.count")) {
        uint64_t v;
        if (c->integer(&v)) count = v;
    }
    for (uint64_t k = 1; k < count; ++k) {
        std::string next;
        if (!sibling(path, k, count, &next, error)) return nullptr;
        shards.emplace_back();
        if (!read_shard(next, k, &shards.back(), error)) return nullptr;
    }
    std::unique_ptr<GgufFile> f(new GgufFile);
    f->metadata = shards[0].metadata;
    for (Shard& s : shards) {
        for (GgufTensor& t : s.tensors) f->tensors.push_back(std::move(t));
        f->data_start.push_back(s.data);
        f->shards.push_back(std::move(s.map));
    }
    if (const GgufValue* d = f->value("split.tensors.count")) {
        uint64_t v;
        if (d->integer(&v) && v != f->tensors.size()) {
            *error = "GGUF split declares " + std::to_string(v) + " tensors and holds " +
                     std::to_string(f->tensors.size());
            return nullptr;
        }
    }
    return f;
}

}  // namespace rq
