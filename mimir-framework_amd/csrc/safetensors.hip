// safetensors.hip -- SafeTensors checkpoints read straight into HBM.
//
// The reference reads a checkpoint (Mimir::Serialization::load_checkpoint,
// Serialization.hpp:114 -> SafeTensorsReader, SafeTensorsReader.cpp) into
// host weight blocks with one std::ifstream seek + read per tensor.  Here the
// header is parsed once (same format and checks: 8-byte little-endian header
// length, 0 < length <= 100 MiB, a JSON object of {dtype, shape,
// data_offsets} entries plus "__metadata__", (end - begin) == prod(shape) *
// dtype size), and a tensor's bytes go from the file to device memory through
// four pinned staging buffers: two threads read a pair of chunks from the file
// while the previous pair's DMAs run on the context's stream.  Measured on
// the MI355X box: one reader reaches ~22 GB/s from the page cache into a cold
// buffer, pinned 8 MiB DMAs ~54 GB/s; one reader into two staging buffers
// ingested ~40 GB/s, two readers leave the DMA as the bound.
//
// The JSON reader below follows the library the reference parses headers
// with (nlohmann::json 3.11.2, vendored as src/include/json.hpp) wherever a
// header's outcome depends on it: RFC 8259 syntax with no comments, leading
// zeros or trailing commas; strings must be well-formed UTF-8 with paired
// surrogate escapes; a leading byte order mark is skipped; a NUL byte between
// tokens ends the input (json.hpp:8885);
// objects keep the last of duplicate keys and are visited in byte order of
// their keys (std::map).  Nesting is limited to 512 levels (the library has
// no limit).
#include "internal.hpp"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <condition_variable>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// Minimal JSON reader
// ---------------------------------------------------------------------------

struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    bool is_int = false;   // the literal had no fraction / exponent
    uint64_t u = 0;        // its value when is_int and non-negative
    bool neg = false;
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;  // in file order
};

class JParser {
public:
    JParser(const char* p, size_t n) : p_(p), end_(p + n) {}

    bool parse(JVal& out, std::string& err) {
        if (end_ - p_ >= 3 && static_cast<unsigned char>(p_[0]) == 0xEF && static_cast<unsigned char>(p_[1]) == 0xBB &&
            static_cast<unsigned char>(p_[2]) == 0xBF)
            p_ += 3;  // a leading UTF-8 byte order mark is skipped (json.hpp, lexer::skip_bom)
        if (!value(out, 0)) {
            err = err_;
            return false;
        }
        ws();
        if (p_ != end_ && *p_ != '\0') {  // a NUL ends the input, as in json.hpp:8885-8888
            err = "trailing characters after the JSON value";
            return false;
        }
        return true;
    }

private:
    // After lead byte c (>= 0x80, already consumed): check the continuation
    // bytes of a well-formed sequence (RFC 3629, section 4) and set seq_end_.
    bool utf8_tail(unsigned char c) {
        int n;
        unsigned char lo = 0x80, hi = 0xBF;  // range of the first continuation byte
        if (c >= 0xC2 && c <= 0xDF) n = 1;
        else if (c == 0xE0) n = 2, lo = 0xA0;
        else if ((c >= 0xE1 && c <= 0xEC) || c == 0xEE || c == 0xEF) n = 2;
        else if (c == 0xED) n = 2, hi = 0x9F;
        else if (c == 0xF0) n = 3, lo = 0x90;
        else if (c >= 0xF1 && c <= 0xF3) n = 3;
        else if (c == 0xF4) n = 3, hi = 0x8F;
        else return false;
        if (end_ - p_ < n) return false;
        for (int i = 0; i < n; ++i) {
            const unsigned char b = static_cast<unsigned char>(p_[i]);
            if (b < (i ? 0x80 : lo) || b > (i ? 0xBF : hi)) return false;
        }
        seq_end_ = p_ + n;
        return true;
    }
    bool fail(const char* m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = std::strlen(w);
        if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return fail("invalid literal");
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += static_cast<char>(cp);
        } else if (cp < 0x800) {
            s += static_cast<char>(0xC0 | (cp >> 6));
            s += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += static_cast<char>(0xE0 | (cp >> 12));
            s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            s += static_cast<char>(0xF0 | (cp >> 18));
            s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (end_ - p_ < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string& out) {
        if (p_ >= end_ || *p_ != '"') return fail("expected a string");
        ++p_;
        out.clear();
        while (p_ < end_ && *p_ != '"') {
            const unsigned char c = static_cast<unsigned char>(*p_++);
            if (c < 0x20) return fail("control character in a string");
            if (c >= 0x80) {  // a UTF-8 sequence, RFC 3629 well-formed
                if (!utf8_tail(c)) return fail("ill-formed UTF-8 byte");
                out.append(p_ - 1, seq_end_);
                p_ = seq_end_;
                continue;
            }
            if (c != '\\') {
                out += static_cast<char>(c);
                continue;
            }
            if (p_ >= end_) return fail("truncated escape");
            const char e = *p_++;
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo > 0xDFFF) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                        return fail("lone low surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p_ >= end_) return fail("unterminated string");
        ++p_;
        return true;
    }
    bool number(JVal& v) {
        const char* s = p_;
        v.kind = JVal::Num;
        v.neg = false;
        if (p_ < end_ && *p_ == '-') {
            v.neg = true;
            ++p_;
        }
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
        if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9') return fail("leading zero in a number");
        uint64_t u = 0;
        bool overflow = false;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = static_cast<uint64_t>(*p_ - '0');
            if (u > (UINT64_MAX - d) / 10) overflow = true;
            u = u * 10 + d;
            ++p_;
        }
        v.is_int = !overflow;
        if (p_ < end_ && *p_ == '.') {
            v.is_int = false;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            v.is_int = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.u = u;
        v.num = std::strtod(std::string(s, p_).c_str(), nullptr);
        return true;
    }
    bool value(JVal& v, int depth) {
        if (depth > 512) return fail("JSON nested too deeply");
        ws();
        if (p_ >= end_) return fail("unexpected end of JSON");
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = JVal::Obj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!str(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
                ++p_;
                JVal item;
                if (!value(item, depth + 1)) return false;
                v.obj.emplace_back(std::move(key), std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = JVal::Arr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                JVal item;
                if (!value(item, depth + 1)) return false;
                v.arr.push_back(std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = JVal::Str;
            return str(v.s);
        }
        if (c == 't') {
            v.kind = JVal::Bool;
            v.b = true;
            return lit("true");
        }
        if (c == 'f') {
            v.kind = JVal::Bool;
            return lit("false");
        }
        if (c == 'n') {
            v.kind = JVal::Null;
            return lit("null");
        }
        return number(v);
    }

    const char* p_;
    const char* end_;
    const char* seq_end_ = nullptr;
    std::string err_;
};

// Serialization.cpp:124-144 (string_to_dtype, dtype_size).
bool dtype_of(const std::string& s, int* code, size_t* size) {
    struct D {
        const char* a;
        const char* b;
        int code;
        size_t size;
    };
    static const D table[] = {{"F32", "float32", MIMIR_ST_F32, 4}, {"F16", "float16", MIMIR_ST_F16, 2},
                              {"I32", "int32", MIMIR_ST_I32, 4},   {"I16", "int16", MIMIR_ST_I16, 2},
                              {"U16", "uint16", MIMIR_ST_U16, 2},  {"U8", "uint8", MIMIR_ST_U8, 1}};
    for (const D& d : table) {
        if (s == d.a || s == d.b) {
            *code = d.code;
            *size = d.size;
            return true;
        }
    }
    return false;
}

const char* kind_name(const JVal& v) {
    switch (v.kind) {
        case JVal::Null: return "null";
        case JVal::Bool: return "boolean";
        case JVal::Num: return "number";
        case JVal::Str: return "string";
        case JVal::Arr: return "array";
        default: return "object";
    }
}

// A header number read as a size, as the reference's json get<size_t>()
// reads it (size_t is the library's unsigned number type, so
// get_arithmetic_value, json.hpp:4607-4637 and :4683): unsigned integers as
// they are, floats truncated toward zero.  NotNumber: any other kind,
// booleans included (the reference throws a type error).  Wraps: a negative
// integer, or a float outside (-1, 2^64): the reference's conversion wraps
// modulo 2^64 (or is undefined for such floats); refused here.
enum class SizeOf { Ok, NotNumber, Wraps };

SizeOf as_size(const JVal& v, uint64_t* out) {
    if (v.kind != JVal::Num) return SizeOf::NotNumber;
    if (v.is_int) {
        if (v.neg && v.u != 0) return SizeOf::Wraps;
        *out = v.u;
        return SizeOf::Ok;
    }
    if (!(v.num > -1.0 && v.num < 18446744073709551616.0)) return SizeOf::Wraps;
    *out = v.num < 1.0 ? 0 : static_cast<uint64_t>(v.num);
    return SizeOf::Ok;
}

struct Entry {
    std::string name;
    int dtype;
    std::vector<int64_t> shape;
    uint64_t begin;
    uint64_t end;
};

constexpr size_t kStageBytes = size_t(8) << 20;  // per staging buffer
constexpr int kStages = 4;                       // two pairs: one being read, one in DMA

// The message of this thread's last failed open (there is no handle then).
thread_local std::string g_open_error;

}  // namespace

struct mimir_safetensors {
    mimir_ctx* ctx = nullptr;
    int fd = -1;
    uint64_t file_size = 0;
    uint64_t data_offset = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> index;
    void* stage[kStages] = {};  // pinned host memory, allocated on first read
    hipEvent_t done[kStages] = {};
    std::string error;  // when there is no context to hold it
};

namespace {

int st_fail(mimir_safetensors* f, mimir_ctx* ctx, int code, const std::string& msg) {
    if (f) f->error = msg;
    return mimir::fail(ctx, code, "%s", msg.c_str());
}

// SafeTensorsReader::parse_header (SafeTensorsReader.cpp:52-166).
int parse_header(mimir_safetensors* f, const char* path) {
    mimir_ctx* ctx = f->ctx;
    uint8_t len8[8];
    if (pread(f->fd, len8, 8, 0) != 8) return st_fail(f, ctx, MIMIR_EINVAL, "Invalid header length");
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= static_cast<uint64_t>(len8[i]) << (8 * i);  // :200-208
    if (hlen == 0 || hlen > (uint64_t(100) << 20))  // :68-74
        return st_fail(f, ctx, MIMIR_EINVAL, "Invalid header length");
    if (8 + hlen > f->file_size) return st_fail(f, ctx, MIMIR_EINVAL, "Failed to read header");  // :77-85
    std::vector<char> text(hlen);
    if (pread(f->fd, text.data(), hlen, 8) != static_cast<ssize_t>(hlen))
        return st_fail(f, ctx, MIMIR_EINVAL, "Failed to read header");
    JVal root;
    std::string err;
    if (!JParser(text.data(), text.size()).parse(root, err))
        return st_fail(f, ctx, MIMIR_EINVAL, std::string("Header parse error: ") + err + " in " + path);
    f->data_offset = 8 + hlen;  // :93
    // The reference iterates the parsed value with it.key() (:96): null and
    // an empty array hold no entries; any other non-object throws.
    const bool empty = root.kind == JVal::Null || (root.kind == JVal::Arr && root.arr.empty());
    if (root.kind != JVal::Obj && !empty)
        return st_fail(f, ctx, MIMIR_EINVAL, "Header parse error: cannot use key() for non-object iterators");
    // Entries in key order, the last of duplicate keys (a std::map object).
    std::map<std::string, const JVal*> by_name;
    for (auto& kv : root.obj) by_name[kv.first] = &kv.second;
    auto not_number = [&](const JVal& v) {
        return st_fail(f, ctx, MIMIR_EINVAL, std::string("Header parse error: type must be number, but is ") +
                                                 kind_name(v));
    };
    for (auto& kv : by_name) {
        if (kv.first == "__metadata__") continue;  // :97-99
        const std::string& name = kv.first;
        const JVal& e = *kv.second;
        const JVal* dt = nullptr;
        const JVal* shape = nullptr;
        const JVal* offs = nullptr;
        for (auto& m : e.obj) {  // empty unless e is an object; the last of duplicate fields
            if (m.first == "dtype") dt = &m.second;
            else if (m.first == "shape") shape = &m.second;
            else if (m.first == "data_offsets") offs = &m.second;
        }
        Entry t;
        t.name = name;
        size_t esize = 0;
        if (!dt) return st_fail(f, ctx, MIMIR_EINVAL, "Missing dtype for tensor: " + name);  // :108-113
        if (dt->kind != JVal::Str)
            return st_fail(f, ctx, MIMIR_EINVAL,
                           std::string("Header parse error: type must be string, but is ") + kind_name(*dt));
        if (!dtype_of(dt->s, &t.dtype, &esize))
            return st_fail(f, ctx, MIMIR_EINVAL, "Header parse error: Unknown dtype string: " + dt->s);
        if (!shape) return st_fail(f, ctx, MIMIR_EINVAL, "Missing shape for tensor: " + name);  // :117-122
        if (shape->kind != JVal::Arr)
            return st_fail(f, ctx, MIMIR_EINVAL,
                           std::string("Header parse error: type must be array, but is ") + kind_name(*shape));
        uint64_t count = 1;
        bool overflow = false;
        for (const JVal& d : shape->arr) {
            uint64_t dim = 0;
            const SizeOf k = as_size(d, &dim);
            if (k == SizeOf::NotNumber) return not_number(d);
            if (k == SizeOf::Wraps)
                return st_fail(f, ctx, MIMIR_EINVAL, "Header parse error: negative or out-of-range dimension for " + name);
            if (dim && count > UINT64_MAX / dim) overflow = true;
            count *= dim;
            t.shape.push_back(static_cast<int64_t>(dim));
        }
        if (!offs) return st_fail(f, ctx, MIMIR_EINVAL, "Missing data_offsets for tensor: " + name);  // :126-131
        if (offs->kind != JVal::Arr || offs->arr.size() != 2)  // :132-137
            return st_fail(f, ctx, MIMIR_EINVAL, "Invalid data_offsets for tensor: " + name);
        uint64_t* ends[2] = {&t.begin, &t.end};
        for (int i = 0; i < 2; ++i) {
            const SizeOf k = as_size(offs->arr[i], ends[i]);
            if (k == SizeOf::NotNumber) return not_number(offs->arr[i]);
            if (k == SizeOf::Wraps)
                return st_fail(f, ctx, MIMIR_EINVAL, "Header parse error: negative or out-of-range offset for " + name);
        }
        // :142-153, without the wrap-around of the reference's size_t
        // arithmetic (a product past 2^64 or end < begin is a mismatch); also
        // refuse ranges that run past the end of the file, which the
        // reference only finds when the read comes up short.
        if (overflow || t.end < t.begin || count > UINT64_MAX / esize || t.end - t.begin != count * esize)
            return st_fail(f, ctx, MIMIR_EINVAL, "Size mismatch for tensor: " + name);
        if (t.end > f->file_size - f->data_offset)
            return st_fail(f, ctx, MIMIR_EINVAL, "Tensor data past the end of the file: " + name);
        f->index[name] = f->entries.size();
        f->entries.push_back(std::move(t));
    }
    return MIMIR_OK;
}

// pread until n bytes are in dst (false on an error or end of file).
bool read_full(int fd, char* dst, size_t n, off_t pos) {
    size_t got = 0;
    while (got < n) {
        const ssize_t r = pread(fd, dst + got, n - got, pos + static_cast<off_t>(got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        got += static_cast<size_t>(r);
    }
    return true;
}

// A second reader: reads one chunk per job handed over by read_to_device.
// Joined by its destructor on every path out of read_to_device.
class Reader {
  public:
    explicit Reader(int fd) : fd_(fd), th_([this] { loop(); }) {}
    ~Reader() {
        {
            std::lock_guard<std::mutex> l(m_);
            quit_ = true;
        }
        cv_.notify_all();
        th_.join();
    }
    void start(char* dst, size_t n, off_t pos) {
        {
            std::lock_guard<std::mutex> l(m_);
            dst_ = dst;
            n_ = n;
            pos_ = pos;
            pending_ = true;
        }
        cv_.notify_all();
    }
    bool wait() {  // the job's result
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [this] { return !pending_; });
        return ok_;
    }

  private:
    void loop() {
        std::unique_lock<std::mutex> l(m_);
        for (;;) {
            cv_.wait(l, [this] { return pending_ || quit_; });
            if (pending_) {
                char* dst = dst_;
                const size_t n = n_;
                const off_t pos = pos_;
                l.unlock();
                const bool ok = read_full(fd_, dst, n, pos);
                l.lock();
                ok_ = ok;
                pending_ = false;
                cv_.notify_all();
            } else {
                return;  // quit, nothing pending
            }
        }
    }
    int fd_;
    std::mutex m_;
    std::condition_variable cv_;
    char* dst_ = nullptr;
    size_t n_ = 0;
    off_t pos_ = 0;
    bool pending_ = false, ok_ = true, quit_ = false;
    std::thread th_;  // last: started once the members above exist
};

// SafeTensorsReader::load_tensor_data (:168-216), into device memory.
int read_to_device(mimir_safetensors* f, const Entry& t, void* dst, size_t dst_bytes) {
    mimir_ctx* ctx = f->ctx;
    const uint64_t bytes = t.end - t.begin;
    if (bytes > dst_bytes) return st_fail(f, ctx, MIMIR_EINVAL, "Buffer too small for tensor: " + t.name);  // :192-198
    if (bytes == 0) return MIMIR_OK;
    MIMIR_ENTER(ctx);
    for (int i = 0; i < kStages; ++i) {
        if (!f->stage[i]) {
            hipError_t e = hipHostMalloc(&f->stage[i], kStageBytes, hipHostMallocDefault);
            if (e != hipSuccess) {
                f->stage[i] = nullptr;
                return mimir::hip_fail(ctx, e, "hipHostMalloc (staging)");
            }
        }
        if (!f->done[i]) {
            hipError_t e = hipEventCreateWithFlags(&f->done[i], hipEventDisableTiming);
            if (e != hipSuccess) {
                f->done[i] = nullptr;
                return mimir::hip_fail(ctx, e, "hipEventCreate");
            }
        }
    }
    // Pair p is chunks 2p and 2p+1, read into stage[2p % 4] and
    // stage[(2p+1) % 4] (this thread and the second reader) once the DMAs of
    // pair p-2 out of those buffers have finished; its DMAs then run while
    // pair p+1 is read.  A tensor of one or two chunks needs no second reader.
    const uint64_t nchunks = (bytes + kStageBytes - 1) / kStageBytes;
    std::unique_ptr<Reader> helper;
    if (nchunks > 2) helper.reset(new Reader(f->fd));
    bool used[kStages] = {};
    auto wait_buffer = [&](int b) -> int {
        if (!used[b]) return MIMIR_OK;
        hipError_t e = hipEventSynchronize(f->done[b]);
        return e == hipSuccess ? MIMIR_OK : mimir::hip_fail(ctx, e, "hipEventSynchronize");
    };
    // Every exit waits for the DMAs already queued: they read the staging
    // buffers, which the next read of this file refills (its `used` flags
    // start clear).
    auto drain = [&](int st) {
        (void)hipStreamSynchronize(ctx->stream);
        return st;
    };
    auto fail_read = [&]() {
        return drain(st_fail(f, ctx, MIMIR_EINVAL, "Failed to read tensor data: " + t.name));  // :201-206
    };
    const off_t base = static_cast<off_t>(f->data_offset + t.begin);
    for (uint64_t c = 0; c < nchunks; c += 2) {
        const int b0 = static_cast<int>(c % kStages), b1 = static_cast<int>((c + 1) % kStages);
        const uint64_t off0 = c * kStageBytes, off1 = off0 + kStageBytes;
        const size_t n0 = static_cast<size_t>(bytes - off0 < kStageBytes ? bytes - off0 : kStageBytes);
        const size_t n1 = off1 < bytes ? static_cast<size_t>(bytes - off1 < kStageBytes ? bytes - off1 : kStageBytes) : 0;
        if (int st = wait_buffer(b0)) return drain(st);
        if (n1 > 0)
            if (int st = wait_buffer(b1)) return drain(st);
        char* s0 = static_cast<char*>(f->stage[b0]);
        char* s1 = static_cast<char*>(f->stage[b1]);
        if (n1 > 0 && helper) helper->start(s1, n1, base + static_cast<off_t>(off1));
        bool ok = read_full(f->fd, s0, n0, base + static_cast<off_t>(off0));
        if (n1 > 0) ok = (helper ? helper->wait() : read_full(f->fd, s1, n1, base + static_cast<off_t>(off1))) && ok;
        if (!ok) return fail_read();
        for (int k = 0; k < (n1 > 0 ? 2 : 1); ++k) {
            const int bk = k ? b1 : b0;
            hipError_t e = hipMemcpyAsync(static_cast<char*>(dst) + (k ? off1 : off0), k ? s1 : s0, k ? n1 : n0,
                                          hipMemcpyHostToDevice, ctx->stream);
            if (e != hipSuccess) return drain(mimir::hip_fail(ctx, e, "hipMemcpyAsync"));
            e = hipEventRecord(f->done[bk], ctx->stream);
            if (e != hipSuccess) return drain(mimir::hip_fail(ctx, e, "hipEventRecord"));
            used[bk] = true;
        }
    }
    // The staging buffers are reused by the next read: wait for the last DMAs.
    for (int i = 0; i < kStages; ++i)
        if (int st = wait_buffer(i)) return drain(st);
    return MIMIR_OK;
}

}  // namespace

extern "C" {

int mimir_safetensors_open(mimir_ctx* ctx, const char* path, mimir_safetensors** out) {
    if (!path || !out) return mimir::fail(ctx, MIMIR_EINVAL, "mimir_safetensors_open: invalid argument");
    *out = nullptr;
    mimir_safetensors* f = new (std::nothrow) mimir_safetensors();
    if (!f) return MIMIR_ENOMEM;
    f->ctx = ctx;
    f->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    struct stat sb;
    if (f->fd < 0 || fstat(f->fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
        g_open_error = std::string("File not found: ") + path;  // SafeTensorsReader.cpp:22-27
        const int st = mimir::fail(ctx, MIMIR_EINVAL, "%s", g_open_error.c_str());
        if (f->fd >= 0) ::close(f->fd);
        delete f;
        return st;
    }
    f->file_size = static_cast<uint64_t>(sb.st_size);
    if (int st = parse_header(f, path)) {
        g_open_error = f->error;
        ::close(f->fd);
        delete f;
        return st;
    }
    *out = f;
    return MIMIR_OK;
}

int mimir_safetensors_close(mimir_safetensors* f) {
    if (!f) return MIMIR_EINVAL;
    for (int i = 0; i < kStages; ++i) {
        if (f->done[i]) (void)hipEventDestroy(f->done[i]);
        if (f->stage[i]) (void)hipHostFree(f->stage[i]);
    }
    if (f->fd >= 0) ::close(f->fd);
    delete f;
    return MIMIR_OK;
}

int64_t mimir_safetensors_count(const mimir_safetensors* f) {
    return f ? static_cast<int64_t>(f->entries.size()) : -1;
}

int mimir_safetensors_entry(const mimir_safetensors* f, int64_t i, const char** name, int32_t* dtype,
                            int64_t* shape, int32_t max_dims, int32_t* ndims, int64_t* nbytes) {
    if (!f || i < 0 || i >= static_cast<int64_t>(f->entries.size())) return MIMIR_EINVAL;
    const Entry& t = f->entries[static_cast<size_t>(i)];
    if (name) *name = t.name.c_str();
    if (dtype) *dtype = t.dtype;
    if (ndims) *ndims = static_cast<int32_t>(t.shape.size());
    if (shape)
        for (size_t d = 0; d < t.shape.size() && static_cast<int32_t>(d) < max_dims; ++d) shape[d] = t.shape[d];
    if (nbytes) *nbytes = static_cast<int64_t>(t.end - t.begin);
    return MIMIR_OK;
}

int64_t mimir_safetensors_find(const mimir_safetensors* f, const char* name) {
    if (!f || !name) return -1;
    auto it = f->index.find(name);
    return it == f->index.end() ? -1 : static_cast<int64_t>(it->second);
}

const char* mimir_safetensors_error(const mimir_safetensors* f) {
    return f ? f->error.c_str() : g_open_error.c_str();
}

int mimir_safetensors_read(mimir_safetensors* f, const char* name, void* dst_device, size_t dst_bytes) {
    if (!f) return MIMIR_EINVAL;
    MIMIR_REQUIRE(f->ctx, f->ctx, "mimir_safetensors_read: opened without a device context");
    MIMIR_REQUIRE(f->ctx, name && (dst_device || dst_bytes == 0), "mimir_safetensors_read: invalid argument");
    auto it = f->index.find(name);
    if (it == f->index.end()) return st_fail(f, f->ctx, MIMIR_EINVAL, std::string("No tensor named ") + name);
    return read_to_device(f, f->entries[it->second], dst_device, dst_bytes);
}

int mimir_safetensors_load_layers(mimir_safetensors* f, const mimir_layer* layers, int32_t n_layers, int strict) {
    if (!f) return MIMIR_EINVAL;
    MIMIR_REQUIRE(f->ctx, f->ctx, "mimir_safetensors_load_layers: opened without a device context");
    MIMIR_REQUIRE(f->ctx, n_layers >= 0 && (n_layers == 0 || layers), "mimir_safetensors_load_layers: invalid argument");
    // SafeTensorsReader::apply_tensors_to_model, the weight-block loop (:263-317).
    for (int32_t i = 0; i < n_layers; ++i) {
        const mimir_layer& L = layers[i];
        if (!L.weights || L.weights_len <= 0) continue;  // no weight block
        const std::string tname = std::string(L.name ? L.name : "") + "/weights";
        auto it = f->index.find(tname);
        if (it == f->index.end()) {
            if (strict) return st_fail(f, f->ctx, MIMIR_EINVAL, "Missing tensor in strict mode: " + tname);
            continue;
        }
        const Entry& t = f->entries[it->second];
        int64_t count = 1;
        for (int64_t d : t.shape) count *= d;
        if (count != L.weights_len)
            return st_fail(f, f->ctx, MIMIR_EINVAL,
                           "Size mismatch for " + tname + ": expected " + std::to_string(count) + " got " +
                               std::to_string(L.weights_len));
        // The bytes are copied as stored, as the reference reads them into the
        // float block whatever the recorded dtype (:307-313).
        if (int st = read_to_device(f, t, const_cast<float*>(L.weights), static_cast<size_t>(L.weights_len) * 4))
            return st;
    }
    return MIMIR_OK;
}

}  // extern "C"
