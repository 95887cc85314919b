// GGUF header and tensor-directory reader: the checks, limits and messages
// of ggufindex.Open (ggufindex/index.go:60-234), readFile (:236-414),
// readString / metadataWidth / skipValue (:416-533), tensorSize (:535-574)
// and sameMetadata (ggufindex/metadata.go:139-180).  Only headers are read;
// tensor bytes stay in their files until uploaded.
#include "spt_gguf_index.h"

#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <set>

namespace spt {
namespace gguf {
namespace {

// Go's %q for the names and keys the messages quote.
std::string quote(const std::string &s) {
    std::string q = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            q += '\\';
            q += (char)c;
        } else if (c < 0x20 || c == 0x7f) {
            char b[8];
            snprintf(b, sizeof b, "\\x%02x", c);
            q += b;
        } else {
            q += (char)c;
        }
    }
    return q + "\"";
}

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
    char b[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(b, sizeof b, f, ap);
    va_end(ap);
    return b;
}

// A file read front to back with the io errors of encoding/binary and
// io.ReadFull: "EOF" when no byte of a value is left, "unexpected EOF" when
// only part of it is.
struct Reader {
    FILE *f = nullptr;
    uint64_t size = 0, pos = 0;
    std::string err;

    ~Reader() {
        if (f) fclose(f);
    }
    bool read(void *dst, uint64_t n) {
        const size_t got = n ? fread(dst, 1, (size_t)n, f) : 0;
        pos += got;
        if (got == n) return true;
        err = got == 0 ? "EOF" : "unexpected EOF";
        return false;
    }
    bool u32(uint32_t *v) {
        uint8_t b[4];
        if (!read(b, 4)) return false;
        *v = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
        return true;
    }
    bool u64(uint64_t *v) {
        uint8_t b[8];
        if (!read(b, 8)) return false;
        *v = 0;
        for (int i = 7; i >= 0; i--) *v = *v << 8 | b[i];
        return true;
    }
    bool skip(uint64_t n) {  // a seek forward (bounds checked by the caller)
        if (fseeko(f, (off_t)n, SEEK_CUR) != 0) {
            err = "seek failed";
            return false;
        }
        pos += n;
        return true;
    }
    bool string(std::string *s) {
        uint64_t len;
        if (!u64(&len)) return false;
        if (len > (1u << 20)) {
            err = fmt("GGUF string is too long: %llu", (unsigned long long)len);
            return false;
        }
        s->assign((size_t)len, '\0');
        return read(&(*s)[0], len);
    }
};

int metadata_width(uint32_t typ) {
    switch (typ) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

// skipValue (index.go:445-533): *numeric for the unsigned integer types
// 0, 2, 4, 10 (*number then holds the value).
bool skip_value(Reader &r, uint32_t typ, int depth, uint64_t *number, bool *numeric) {
    *number = 0;
    *numeric = false;
    if (depth > 8) {
        r.err = "metadata nesting is too deep";
        return false;
    }
    if (typ == 9) {
        uint32_t elem;
        uint64_t count;
        if (!r.u32(&elem) || !r.u64(&count)) return false;
        if (count > 100000000ull) {
            r.err = "array is too large";
            return false;
        }
        const int width = metadata_width(elem);
        if (width == 0 && elem != 8 && elem != 9) {
            r.err = fmt("unknown metadata type %u", elem);
            return false;
        }
        if (width != 0) {
            if (count == 0) return true;
            if (depth == 8) {
                r.err = "metadata nesting is too deep";
                return false;
            }
            if (count > (uint64_t)INT64_MAX / (uint64_t)width) {
                r.err = "array byte size overflows";
                return false;
            }
            const uint64_t length = count * (uint64_t)width;
            if (r.pos > r.size || length > r.size - r.pos) {
                r.err = "unexpected EOF";
                return false;
            }
            return r.skip(length);
        }
        for (uint64_t i = 0; i < count; i++) {
            uint64_t n;
            bool num;
            if (!skip_value(r, elem, depth + 1, &n, &num)) return false;
        }
        return true;
    }
    if (typ == 8) {
        std::string s;
        return r.string(&s);
    }
    const int width = metadata_width(typ);
    if (width == 0) {
        r.err = fmt("unknown metadata type %u", typ);
        return false;
    }
    uint8_t b[8] = {0};
    if (!r.read(b, (uint64_t)width)) return false;
    uint64_t v = 0;
    for (int i = width - 1; i >= 0; i--) v = v << 8 | b[i];
    if (typ == 0 || typ == 2 || typ == 4 || typ == 10) {
        *number = v;
        *numeric = true;
    }
    return true;
}

struct FileIndex {
    std::vector<Tensor> tensors;
    std::map<std::string, uint64_t> numbers;
    std::map<std::string, MetaValue> entries;
    uint64_t alignment = 0;
};

struct Info {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t type = 0;
    uint64_t offset = 0;
};

// readFile (index.go:236-414).
bool read_file(const std::string &path, int file, FileIndex *out, std::string *err) {
    Reader r;
    r.f = fopen(path.c_str(), "rb");
    if (!r.f) {
        *err = fmt("open %s: %s", path.c_str(), strerror(errno));
        return false;
    }
    if (fseeko(r.f, 0, SEEK_END) != 0) {
        *err = "cannot stat the file";
        return false;
    }
    r.size = (uint64_t)ftello(r.f);
    rewind(r.f);
    if (r.size < 24) {
        *err = "file is too small";
        return false;
    }
    char magic[4];
    if (!r.read(magic, 4)) return *err = r.err, false;
    if (memcmp(magic, "GGUF", 4) != 0) {
        *err = "not a GGUF file";
        return false;
    }
    uint32_t version;
    if (!r.u32(&version)) return *err = r.err, false;
    if (version != 2 && version != 3) {
        *err = fmt("unsupported GGUF version %u", version);
        return false;
    }
    uint64_t tensor_count, metadata_count;
    if (!r.u64(&tensor_count) || !r.u64(&metadata_count)) return *err = r.err, false;
    if (tensor_count > 10000000ull || metadata_count > 1000000ull) {
        *err = "implausible header count";
        return false;
    }
    for (uint64_t i = 0; i < metadata_count; i++) {
        std::string key;
        if (!r.string(&key)) return *err = r.err, false;
        if (out->entries.count(key)) {
            *err = "duplicate metadata key " + quote(key);
            return false;
        }
        uint32_t typ;
        if (!r.u32(&typ)) return *err = r.err, false;
        const uint64_t start = r.pos;
        uint64_t number;
        bool numeric;
        if (!skip_value(r, typ, 0, &number, &numeric)) {
            *err = "metadata " + quote(key) + ": " + r.err;
            return false;
        }
        MetaValue mv;
        mv.type = typ;
        mv.range = Range{file, start, r.pos};
        out->entries[key] = mv;
        if (numeric) out->numbers[key] = number;
    }
    std::vector<Info> infos;
    infos.reserve((size_t)std::min<uint64_t>(tensor_count, 1u << 16));
    for (uint64_t i = 0; i < tensor_count; i++) {
        Info info;
        if (!r.string(&info.name)) return *err = r.err, false;
        uint32_t dims;
        if (!r.u32(&dims)) return *err = r.err, false;
        if (dims == 0 || dims > 8) {
            *err = "tensor " + quote(info.name) + ": invalid dimension count";
            return false;
        }
        info.shape.resize(dims);
        for (uint32_t j = 0; j < dims; j++)
            if (!r.u64(&info.shape[j])) return *err = r.err, false;
        if (!r.u32(&info.type) || !r.u64(&info.offset)) return *err = r.err, false;
        infos.push_back(std::move(info));
    }
    uint64_t alignment = out->numbers.count("general.alignment") ? out->numbers["general.alignment"] : 0;
    if (alignment == 0) alignment = 32;
    if (alignment > (1u << 20) || (alignment & (alignment - 1)) != 0) {
        *err = fmt("invalid alignment %llu", (unsigned long long)alignment);
        return false;
    }
    const uint64_t base = (r.pos + alignment - 1) & ~(alignment - 1);
    if (base > r.size) {
        *err = "tensor data starts beyond the end of the file";
        return false;
    }
    for (const Info &info : infos) {
        uint64_t bytes;
        std::string e;
        if (!tensor_size(info.type, info.shape, &bytes, &e)) {
            *err = "tensor " + quote(info.name) + ": " + e;
            return false;
        }
        if (info.offset > r.size - base || bytes > r.size - base - info.offset) {
            *err = "tensor " + quote(info.name) + ": byte range extends beyond the file";
            return false;
        }
        Tensor t;
        t.name = info.name;
        t.type = info.type;
        t.shape = info.shape;
        t.range = Range{file, base + info.offset, base + info.offset + bytes};
        out->tensors.push_back(std::move(t));
    }
    out->alignment = alignment;
    return true;
}

// sameMetadata (metadata.go:139-180): same type and identical encoded bytes.
bool same_metadata(const std::vector<std::string> &paths, const MetaValue &a, const MetaValue &b, bool *equal,
                   std::string *err) {
    *equal = false;
    if (a.type != b.type) return true;
    const uint64_t la = a.range.end - a.range.start, lb = b.range.end - b.range.start;
    if (la != lb) return true;
    FILE *fa = fopen(paths[a.range.file].c_str(), "rb");
    FILE *fb = fopen(paths[b.range.file].c_str(), "rb");
    bool ok = fa && fb && fseeko(fa, (off_t)a.range.start, SEEK_SET) == 0 &&
              fseeko(fb, (off_t)b.range.start, SEEK_SET) == 0;
    bool eq = true;
    std::vector<char> ba(32 * 1024), bb(32 * 1024);
    for (uint64_t left = la; ok && eq && left;) {
        const size_t n = (size_t)std::min<uint64_t>(left, ba.size());
        ok = fread(ba.data(), 1, n, fa) == n && fread(bb.data(), 1, n, fb) == n;
        eq = ok && memcmp(ba.data(), bb.data(), n) == 0;
        left -= n;
    }
    if (fa) fclose(fa);
    if (fb) fclose(fb);
    if (!ok) {
        *err = "unexpected EOF";
        return false;
    }
    *equal = eq;
    return true;
}

// `^blk\.([0-9]+)\.`: the layer number (strconv.Atoi range: int64), or
// -1 for names outside the layers; false when the digits overflow.
bool layer_of(const std::string &name, int64_t *layer) {
    *layer = -1;
    if (name.compare(0, 4, "blk.") != 0) return true;
    size_t i = 4;
    while (i < name.size() && name[i] >= '0' && name[i] <= '9') i++;
    if (i == 4 || i >= name.size() || name[i] != '.') return true;
    int64_t v = 0;
    for (size_t k = 4; k < i; k++) {
        const int d = name[k] - '0';
        if (v > (INT64_MAX - d) / 10) return false;
        v = v * 10 + d;
    }
    *layer = v;
    return true;
}

}  // namespace

bool tensor_size(uint32_t type, const std::vector<uint64_t> &shape, uint64_t *bytes, std::string *err) {
    uint64_t elems_per, bytes_per;
    switch (type) {
    case 0: elems_per = 1; bytes_per = 4; break;
    case 1: elems_per = 1; bytes_per = 2; break;
    case 2: elems_per = 32; bytes_per = 18; break;
    case 3: elems_per = 32; bytes_per = 20; break;
    case 6: elems_per = 32; bytes_per = 22; break;
    case 7: elems_per = 32; bytes_per = 24; break;
    case 8: elems_per = 32; bytes_per = 34; break;
    case 9: elems_per = 32; bytes_per = 40; break;
    case 28: elems_per = 1; bytes_per = 2; break;
    case 39: elems_per = 32; bytes_per = 17; break;
    default:
        *err = fmt("unsupported GGML tensor type %u", type);
        return false;
    }
    uint64_t elements = 1;
    for (uint64_t d : shape) {
        if (d == 0 || elements > UINT64_MAX / d) {
            *err = "invalid tensor shape";
            return false;
        }
        elements *= d;
    }
    if (elements % elems_per != 0 || elements / elems_per > UINT64_MAX / bytes_per) {
        *err = "invalid block size or tensor is too large";
        return false;
    }
    *bytes = elements / elems_per * bytes_per;
    return true;
}

bool open(const std::vector<std::string> &paths, Model *model, std::string *err) {
    *model = Model{};
    if (paths.empty()) {
        *err = "no GGUF files provided";
        return false;
    }
    model->paths = paths;
    std::set<std::string> seen_paths, seen_tensors;
    std::map<int64_t, std::vector<Tensor>> layers;
    std::set<uint64_t> split_numbers;
    int64_t declared = -1;
    uint64_t split_count = 0;
    bool has_split_count = false;
    for (size_t fi = 0; fi < paths.size(); fi++) {
        const std::string &path = paths[fi];
        if (seen_paths.count(path)) {
            *err = "duplicate file: " + path;
            return false;
        }
        seen_paths.insert(path);
        FileIndex fx;
        std::string e;
        if (!read_file(path, (int)fi, &fx, &e)) {
            *err = path + ": " + e;
            return false;
        }
        if (model->alignment == 0) {
            model->alignment = fx.alignment;
        } else if (model->alignment != fx.alignment) {
            *err = path + ": inconsistent tensor alignment";
            return false;
        }
        for (const auto &kv : fx.entries) {
            auto it = model->metadata.find(kv.first);
            if (it == model->metadata.end()) {
                model->metadata[kv.first] = kv.second;
                continue;
            }
            if (kv.first == "split.no") continue;
            bool equal;
            if (!same_metadata(paths, it->second, kv.second, &equal, &e)) {
                *err = path + ": compare metadata " + quote(kv.first) + ": " + e;
                return false;
            }
            if (!equal) {
                *err = path + ": inconsistent metadata " + quote(kv.first);
                return false;
            }
        }
        auto num = [&](const char *k, uint64_t *v) {
            auto it = fx.numbers.find(k);
            if (it == fx.numbers.end()) return false;
            *v = it->second;
            return true;
        };
        uint64_t v;
        if (num("gpt_oss.block_count", &v)) {
            if (v > (uint64_t)INT64_MAX) {
                *err = path + ": layer count is too large";
                return false;
            }
            if (declared >= 0 && (uint64_t)declared != v) {
                *err = path + ": inconsistent layer count";
                return false;
            }
            declared = (int64_t)v;
        }
        if (num("split.count", &v)) {
            if (has_split_count && split_count != v) {
                *err = path + ": inconsistent split count";
                return false;
            }
            split_count = v;
            has_split_count = true;
        }
        if (num("split.no", &v)) {
            if (split_numbers.count(v)) {
                *err = fmt("%s: duplicate split %llu", path.c_str(), (unsigned long long)v);
                return false;
            }
            split_numbers.insert(v);
        }
        for (Tensor &t : fx.tensors) {
            if (seen_tensors.count(t.name)) {
                *err = path + ": duplicate tensor " + quote(t.name);
                return false;
            }
            seen_tensors.insert(t.name);
            int64_t layer;
            if (!layer_of(t.name, &layer)) {
                *err = path + ": invalid layer number in " + quote(t.name);
                return false;
            }
            t.layer = layer;
            if (layer < 0)
                model->shared.push_back(std::move(t));
            else
                layers[layer].push_back(std::move(t));
        }
    }
    if (has_split_count && (uint64_t)paths.size() != split_count) {
        *err = fmt("incomplete model: %zu of %llu splits provided", paths.size(), (unsigned long long)split_count);
        return false;
    }
    if (!split_numbers.empty()) {
        if (split_numbers.size() != paths.size()) {
            *err = "a file is missing its split number";
            return false;
        }
        for (uint64_t n = 0; n < paths.size(); n++)
            if (!split_numbers.count(n)) {
                *err = fmt("split %llu is missing", (unsigned long long)n);
                return false;
            }
    }
    if (declared < 0) declared = (int64_t)layers.size();
    model->layer_count = declared;
    if ((int64_t)layers.size() != declared) {
        *err = fmt("expected %lld layers, found %zu", (long long)declared, layers.size());
        return false;
    }
    auto by_name = [](const Tensor &a, const Tensor &b) { return a.name < b.name; };
    for (int64_t n = 0; n < declared; n++) {
        auto it = layers.find(n);
        if (it == layers.end()) {
            *err = fmt("layer %lld is missing", (long long)n);
            return false;
        }
        std::vector<Tensor> &ts = it->second;
        std::sort(ts.begin(), ts.end(), by_name);
        std::map<std::string, Range> by_file;
        for (const Tensor &t : ts) {
            const std::string &p = paths[t.range.file];
            auto s = by_file.find(p);
            if (s == by_file.end()) {
                by_file[p] = t.range;
            } else {
                s->second.start = std::min(s->second.start, t.range.start);
                s->second.end = std::max(s->second.end, t.range.end);
            }
        }
        std::vector<Range> spans;
        for (const auto &kv : by_file) spans.push_back(kv.second);  // map order: sorted by path
        model->layers.push_back(std::move(ts));
        model->spans.push_back(std::move(spans));
    }
    std::sort(model->shared.begin(), model->shared.end(), by_name);
    return true;
}

const Tensor *find(const Model &m, const std::string &name) {
    for (const Tensor &t : m.shared)
        if (t.name == name) return &t;
    for (const auto &layer : m.layers)
        for (const Tensor &t : layer)
            if (t.name == name) return &t;
    return nullptr;
}

}  // namespace gguf
}  // namespace spt
