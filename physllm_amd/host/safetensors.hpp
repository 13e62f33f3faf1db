// Read-only safetensors access without copying: each file is memory-mapped and
// its header parsed once; a tensor is a (dtype, shape, pointer, byte count) view
// into the mapping. Replaces the whole-file reads of the reference loader
// (crates/llm-core/src/gpt_oss_loader.rs:81-94, which calls safetensors 0.4.5's
// SafeTensors::deserialize on a Vec<u8> of every shard).
//
// Format (the safetensors specification): an 8-byte little-endian header length
// N, N bytes of UTF-8 JSON mapping each tensor name to {"dtype", "shape",
// "data_offsets": [begin, end]} (offsets relative to the byte after the header),
// an optional "__metadata__" object of strings, then the data. Checks: the header
// fits the file, the JSON is well formed, every dtype is known, end - begin equals
// the element count times the dtype size, and every range lies inside the data.
//
// No HIP dependency: the parser runs and is tested on the CPU.
#pragma once

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace safetensors {

struct Error : std::runtime_error {
    explicit Error(const std::string& m) : std::runtime_error(m) {}
};

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----------

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0;
    bool is_int = false;  // the literal was an integer that fits int64
    int64_t i = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;  // in file order

    const Json* find(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
  public:
    JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}

    Json parse_document() {
        Json v = value(0);
        ws();
        if (p_ != end_) fail("trailing characters after the JSON value");
        return v;
    }

  private:
    const char* p_;
    const char* end_;

    [[noreturn]] void fail(const char* what) { throw Error(std::string("safetensors header JSON: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    char peek() {
        ws();
        if (p_ >= end_) fail("unexpected end");
        return *p_;
    }
    void expect(char c) {
        if (peek() != c) fail("unexpected character");
        ++p_;
    }
    Json value(int depth) {
        if (depth > 64) fail("nesting too deep");
        const char c = peek();
        if (c == '{') return object(depth);
        if (c == '[') return array(depth);
        if (c == '"') {
            Json v;
            v.kind = Json::String;
            v.str = string();
            return v;
        }
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        return literal();
    }
    Json object(int depth) {
        Json v;
        v.kind = Json::Object;
        expect('{');
        if (peek() == '}') {
            ++p_;
            return v;
        }
        for (;;) {
            if (peek() != '"') fail("object key must be a string");
            std::string k = string();
            expect(':');
            for (const auto& kv : v.obj)
                if (kv.first == k) fail("duplicate key");
            v.obj.emplace_back(std::move(k), value(depth + 1));
            const char c = peek();
            ++p_;
            if (c == '}') return v;
            if (c != ',') fail("expected ',' or '}'");
        }
    }
    Json array(int depth) {
        Json v;
        v.kind = Json::Array;
        expect('[');
        if (peek() == ']') {
            ++p_;
            return v;
        }
        for (;;) {
            v.arr.push_back(value(depth + 1));
            const char c = peek();
            ++p_;
            if (c == ']') return v;
            if (c != ',') fail("expected ',' or ']'");
        }
    }
    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string s;
        for (;;) {
            if (p_ >= end_) fail("unterminated string");
            const char c = *p_++;
            if (c == '"') return s;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) fail("unterminated escape");
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') fail("lone surrogate");
                        p_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        fail("lone surrogate");
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
    }
    Json number() {
        const char* s = p_;
        if (*p_ == '-') ++p_;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad number");
        if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9') fail("leading zero");
        bool integral = true;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < end_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        const std::string lit(s, p_);
        Json v;
        v.kind = Json::Number;
        v.num = std::strtod(lit.c_str(), nullptr);
        if (integral) {
            errno = 0;
            char* e = nullptr;
            const long long ll = std::strtoll(lit.c_str(), &e, 10);
            if (errno == 0 && e && *e == 0) {
                v.is_int = true;
                v.i = ll;
            }
        }
        return v;
    }
    Json literal() {
        auto word = [&](const char* w) {
            const size_t n = std::strlen(w);
            if ((size_t)(end_ - p_) >= n && std::memcmp(p_, w, n) == 0) {
                p_ += n;
                return true;
            }
            return false;
        };
        Json v;
        if (word("true")) {
            v.kind = Json::Bool;
            v.b = true;
        } else if (word("false")) {
            v.kind = Json::Bool;
        } else if (!word("null")) {
            fail("unexpected token");
        }
        return v;
    }
};

inline Json parse_json(const std::string& text) { return JsonParser(text.data(), text.size()).parse_document(); }

// ---- tensors ---------------------------------------------------------------------

// Element size in bytes of a safetensors dtype string; 0 if unknown.
inline size_t dtype_size(const std::string& d) {
    static const std::pair<const char*, size_t> table[] = {
        {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E4M3", 1}, {"F8_E5M2", 1}, {"I16", 2}, {"U16", 2}, {"F16", 2},
        {"BF16", 2}, {"I32", 4}, {"U32", 4}, {"F32", 4},     {"I64", 8},     {"U64", 8}, {"F64", 8}};
    for (const auto& e : table)
        if (d == e.first) return e.second;
    return 0;
}

struct TensorView {
    std::string name;
    std::string dtype;
    std::vector<int64_t> shape;
    const uint8_t* data = nullptr;  // inside the file mapping
    size_t nbytes = 0;
    size_t offset = 0;  // from the start of the data section

    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

class File {
  public:
    explicit File(const std::string& path) : path_(path) {
        fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd_ < 0) throw Error("cannot open " + path + ": " + std::strerror(errno));
        struct stat st;
        if (::fstat(fd_, &st) != 0) {
            ::close(fd_);
            throw Error("cannot stat " + path);
        }
        size_ = (size_t)st.st_size;
        if (size_ < 8) {
            ::close(fd_);
            throw Error(path + ": shorter than the 8-byte header length");
        }
        void* m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (m == MAP_FAILED) {
            ::close(fd_);
            throw Error("cannot map " + path + ": " + std::strerror(errno));
        }
        map_ = (const uint8_t*)m;
        try {
            parse();
        } catch (...) {
            unmap();
            throw;
        }
    }
    File(const File&) = delete;
    File& operator=(const File&) = delete;
    ~File() { unmap(); }

    const std::string& path() const { return path_; }
    const std::vector<TensorView>& tensors() const { return tensors_; }
    const std::vector<std::pair<std::string, std::string>>& metadata() const { return metadata_; }
    const TensorView* find(const std::string& name) const {
        auto it = index_.find(name);
        return it == index_.end() ? nullptr : &tensors_[it->second];
    }

  private:
    std::string path_;
    int fd_ = -1;
    size_t size_ = 0;
    const uint8_t* map_ = nullptr;
    std::vector<TensorView> tensors_;
    std::map<std::string, size_t> index_;
    std::vector<std::pair<std::string, std::string>> metadata_;

    void unmap() {
        if (map_) ::munmap((void*)map_, size_);
        map_ = nullptr;
        if (fd_ >= 0) ::close(fd_);
        fd_ = -1;
    }
    [[noreturn]] void fail(const std::string& m) const { throw Error(path_ + ": " + m); }

    void parse() {
        uint64_t n = 0;
        for (int k = 7; k >= 0; --k) n = (n << 8) | map_[k];
        if (n > size_ - 8) fail("header length " + std::to_string(n) + " exceeds the file");
        const std::string text((const char*)map_ + 8, (size_t)n);
        Json root;
        try {
            root = parse_json(text);
        } catch (const Error& e) {
            fail(e.what());
        }
        if (root.kind != Json::Object) fail("header is not a JSON object");
        const uint8_t* data = map_ + 8 + n;
        const size_t data_bytes = size_ - 8 - (size_t)n;
        for (const auto& kv : root.obj) {
            if (kv.first == "__metadata__") {
                if (kv.second.kind != Json::Object) fail("__metadata__ is not an object");
                for (const auto& m : kv.second.obj) {
                    if (m.second.kind != Json::String) fail("__metadata__ values must be strings");
                    metadata_.emplace_back(m.first, m.second.str);
                }
                continue;
            }
            const Json& t = kv.second;
            if (t.kind != Json::Object) fail("entry '" + kv.first + "' is not an object");
            const Json* dt = t.find("dtype");
            const Json* sh = t.find("shape");
            const Json* off = t.find("data_offsets");
            if (!dt || dt->kind != Json::String) fail("'" + kv.first + "': missing dtype");
            if (!sh || sh->kind != Json::Array) fail("'" + kv.first + "': missing shape");
            if (!off || off->kind != Json::Array || off->arr.size() != 2) fail("'" + kv.first + "': bad data_offsets");
            TensorView v;
            v.name = kv.first;
            v.dtype = dt->str;
            const size_t es = dtype_size(v.dtype);
            if (!es) fail("'" + kv.first + "': unknown dtype " + v.dtype);
            uint64_t numel = 1;
            for (const Json& d : sh->arr) {
                if (d.kind != Json::Number || !d.is_int || d.i < 0) fail("'" + kv.first + "': bad dimension");
                v.shape.push_back(d.i);
                if (d.i != 0 && numel > (UINT64_MAX / 16) / (uint64_t)d.i) fail("'" + kv.first + "': shape overflows");
                numel *= (uint64_t)d.i;
            }
            const Json& b = off->arr[0];
            const Json& e = off->arr[1];
            if (b.kind != Json::Number || e.kind != Json::Number || !b.is_int || !e.is_int || b.i < 0 || e.i < b.i)
                fail("'" + kv.first + "': bad data_offsets");
            if ((uint64_t)e.i > data_bytes) fail("'" + kv.first + "': data_offsets past the end of the file");
            if ((uint64_t)(e.i - b.i) != numel * es)
                fail("'" + kv.first + "': " + std::to_string(e.i - b.i) + " bytes for " + std::to_string(numel) +
                     " elements of " + v.dtype);
            v.offset = (size_t)b.i;
            v.nbytes = (size_t)(e.i - b.i);
            v.data = data + v.offset;
            index_[v.name] = tensors_.size();
            tensors_.push_back(std::move(v));
        }
        // ranges must not overlap (the specification also requires them to be dense)
        std::vector<std::pair<size_t, size_t>> r;
        for (const auto& t : tensors_)
            if (t.nbytes) r.emplace_back(t.offset, t.offset + t.nbytes);
        std::sort(r.begin(), r.end());
        for (size_t k = 1; k < r.size(); ++k)
            if (r[k].first < r[k - 1].second) fail("tensor data ranges overlap");
    }
};

// Every *.safetensors file of a directory, sorted by name (the shard discovery of
// gpt_oss_loader.rs:64-79), or one file. A tensor name must be unique across shards.
class Checkpoint {
  public:
    explicit Checkpoint(const std::string& path) {
        struct stat st;
        if (::stat(path.c_str(), &st) != 0) throw Error("cannot stat " + path);
        std::vector<std::string> files;
        if (S_ISDIR(st.st_mode)) {
            dir_ = path;
            files = list_dir(path);
            if (files.empty()) throw Error("no .safetensors files found in " + path);
        } else {
            const size_t slash = path.rfind('/');
            dir_ = slash == std::string::npos ? "." : path.substr(0, slash);
            files.push_back(path);
        }
        for (const auto& f : files) {
            shards_.push_back(std::make_unique<File>(f));
            const File& sf = *shards_.back();
            for (const auto& t : sf.tensors()) {
                if (where_.count(t.name)) throw Error("tensor '" + t.name + "' appears in more than one shard");
                where_[t.name] = &t;
            }
        }
    }

    const std::string& dir() const { return dir_; }
    size_t num_shards() const { return shards_.size(); }
    bool has(const std::string& name) const { return where_.count(name) != 0; }
    const TensorView& get(const std::string& name) const {
        auto it = where_.find(name);
        if (it == where_.end()) throw Error("tensor '" + name + "' not found in any shard of " + dir_);
        return *it->second;
    }
    // (key, value) pairs of every shard's __metadata__, in shard order
    std::vector<std::pair<std::string, std::string>> metadata() const {
        std::vector<std::pair<std::string, std::string>> m;
        for (const auto& f : shards_) m.insert(m.end(), f->metadata().begin(), f->metadata().end());
        return m;
    }
    std::vector<std::string> names() const {
        std::vector<std::string> v;
        for (const auto& kv : where_) v.push_back(kv.first);
        return v;
    }

  private:
    std::string dir_;
    std::vector<std::unique_ptr<File>> shards_;
    std::map<std::string, const TensorView*> where_;

    static std::vector<std::string> list_dir(const std::string& d) {
        std::vector<std::string> out;
        DIR* dp = ::opendir(d.c_str());
        if (!dp) throw Error("cannot read directory " + d);
        const std::string suf = ".safetensors";
        while (struct dirent* e = ::readdir(dp)) {
            const std::string n = e->d_name;
            if (n.size() > suf.size() && n.compare(n.size() - suf.size(), suf.size(), suf) == 0)
                out.push_back(d + "/" + n);
        }
        ::closedir(dp);
        std::sort(out.begin(), out.end());
        return out;
    }
};

}  // namespace safetensors
