// weight_io.cpp -- safetensors header parsing and host views into a mapping.
// Same contract as the reference's reader (xstar_cpp/include/weight_io.h:25-56)
// with the quantized dtypes of FP8 / FP4 checkpoints added.
#include "weight_io.h"

#include <cstdint>
#include <cstring>
#include <stdexcept>

namespace {

// A cursor over the JSON header.  The header is machine-written: strings hold
// no escapes and no non-ASCII bytes (both rejected), numbers are non-negative
// integers where this reader needs them; any other value (the __metadata__
// object) is skipped structurally.
class Scanner
{
public:
    Scanner(const char *p, const char *end) : p_(p), end_(end) {}

    void ws()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool at_end()
    {
        ws();
        return p_ >= end_;
    }
    char peek()
    {
        ws();
        if (p_ >= end_) throw std::runtime_error("closing '}' not found before end");
        return *p_;
    }
    void expect(char c, const char *what)
    {
        if (peek() != c) throw std::runtime_error(what);
        ++p_;
    }
    // ',' -> true (another member follows), '}' or ']' (== close) -> false
    bool next_member(char close, const char *what)
    {
        const char c = peek();
        ++p_;
        if (c == ',') {
            if (peek() == close) {   // a trailing comma is tolerated
                ++p_;
                return false;
            }
            return true;
        }
        if (c == close) return false;
        throw std::runtime_error(what);
    }
    std::string str()
    {
        if (peek() != '"') throw std::runtime_error("JSON syntax error (expected a string)");
        ++p_;
        const char *s = p_;
        while (p_ < end_ && *p_ != '"') {
            const unsigned char c = static_cast<unsigned char>(*p_);
            if (c == '\\' || c >= 0x80)
                throw std::runtime_error("backslash or non-ASCII byte in a string is not supported");
            ++p_;
        }
        if (p_ >= end_) throw std::runtime_error("unterminated string in header");
        std::string out(s, p_);
        ++p_;
        return out;
    }
    std::uint64_t uint()
    {
        ws();
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') throw std::runtime_error("JSON syntax error (expected an integer)");
        std::uint64_t v = 0;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const std::uint64_t d = static_cast<std::uint64_t>(*p_ - '0');
            if (v > (UINT64_MAX - d) / 10) throw std::runtime_error("integer overflow in header");
            v = v * 10 + d;
            ++p_;
        }
        return v;
    }
    std::vector<std::uint64_t> uint_array()
    {
        expect('[', "JSON syntax error (expected '[')");
        std::vector<std::uint64_t> out;
        if (peek() == ']') {
            ++p_;
            return out;
        }
        do out.push_back(uint());
        while (next_member(']', "JSON syntax error (expected ',' or ']' in an array)"));
        return out;
    }
    // Skips one JSON value of any kind.
    void skip_value(int depth = 0)
    {
        if (depth > 64) throw std::runtime_error("header nesting too deep");
        const char c = peek();
        if (c == '"') {
            str();
        } else if (c == '{') {
            ++p_;
            if (peek() == '}') { ++p_; return; }
            do {
                str();
                expect(':', "expected ':' after key");
                skip_value(depth + 1);
            } while (next_member('}', "JSON syntax error (expected ',' or '}' in an object)"));
        } else if (c == '[') {
            ++p_;
            if (peek() == ']') { ++p_; return; }
            do skip_value(depth + 1);
            while (next_member(']', "JSON syntax error (expected ',' or ']' in an array)"));
        } else {
            const char *s = p_;
            while (p_ < end_ && (std::strchr("+-.eE", *p_) || (*p_ >= '0' && *p_ <= '9') || (*p_ >= 'a' && *p_ <= 'z')))
                ++p_;
            if (p_ == s) throw std::runtime_error("JSON syntax error (unexpected character during scan)");
        }
    }

private:
    const char *p_, *end_;
};

DType dtype_of(const std::string &d)
{
    if (d == "F32") return DType::Float32;
    if (d == "BF16") return DType::BFloat16;
    if (d == "F8_E4M3") return DType::Float8E4M3;
    if (d == "F8_E8M0") return DType::Float8E8M0;
    if (d == "U8") return DType::UInt8;
    if (d == "I32") return DType::Int32;
    throw std::runtime_error("dtype not supported: \"" + d + "\" (F32, BF16, F8_E4M3, F8_E8M0, U8, I32)");
}

}  // namespace

Tensor make_weight_view(MMapFile &mf, std::size_t offset, std::vector<std::int64_t> shape, DType dtype)
{
    const std::size_t es = dtype_size(dtype);
    if (offset % es != 0) throw std::runtime_error("offset not aligned to dtype size");
    std::size_t numel = 1;
    for (auto d : shape) {
        if (d < 0) throw std::runtime_error("negative dimension");
        if (d != 0 && numel > SIZE_MAX / static_cast<std::size_t>(d))
            throw std::runtime_error("element count overflows");
        numel *= static_cast<std::size_t>(d);
    }
    if (numel > SIZE_MAX / es) throw std::runtime_error("element count overflows");
    const std::size_t nbytes = numel * es;
    if (offset > mf.size() || nbytes > mf.size() - offset) throw std::runtime_error("weight view exceeds mmap region");
    return Tensor(static_cast<const char *>(mf.addr()) + offset, std::move(shape), dtype, Device::CPU);
}

std::unordered_map<std::string, TensorMeta> parse_safetensors_header(const MMapFile &mf)
{
    if (mf.size() < 8) throw std::runtime_error("file smaller than 8 bytes (cannot read header_len)");
    const char *base = static_cast<const char *>(mf.addr());
    std::uint64_t hlen = 0;
    std::memcpy(&hlen, base, 8);   // little-endian on every target this library builds for
    if (hlen > mf.size() - 8) throw std::runtime_error("header_len exceeds remaining file bytes (truncated header)");
    const std::size_t data_start = 8 + static_cast<std::size_t>(hlen);
    const std::size_t data_bytes = mf.size() - data_start;

    Scanner sc(base + 8, base + data_start);
    if (sc.at_end()) throw std::runtime_error("empty header");
    sc.expect('{', "top-level is not a JSON object");
    std::unordered_map<std::string, TensorMeta> out;
    if (sc.peek() == '}') return out;
    do {
        const std::string key = sc.str();
        sc.expect(':', "expected ':' after key");
        if (key == "__metadata__") {
            sc.skip_value();
            continue;
        }
        sc.expect('{', "tensor descriptor is not a JSON object");
        bool has_dtype = false, has_shape = false, has_off = false;
        DType dtype = DType::Float32;
        std::vector<std::int64_t> shape;
        std::uint64_t b0 = 0, b1 = 0;
        if (sc.peek() != '}') {
            do {
                const std::string field = sc.str();
                sc.expect(':', "expected ':' after field");
                if (field == "dtype") {
                    dtype = dtype_of(sc.str());
                    has_dtype = true;
                } else if (field == "shape") {
                    for (auto d : sc.uint_array()) {
                        if (d > static_cast<std::uint64_t>(INT64_MAX)) throw std::runtime_error("dimension too large");
                        shape.push_back(static_cast<std::int64_t>(d));
                    }
                    has_shape = true;
                } else if (field == "data_offsets") {
                    auto a = sc.uint_array();
                    if (a.size() != 2) throw std::runtime_error("data_offsets must have exactly 2 elements");
                    b0 = a[0];
                    b1 = a[1];
                    has_off = true;
                } else {
                    throw std::runtime_error("unsupported field encountered: " + field);
                }
            } while (sc.next_member('}', "expected ',' or '}' between tensor descriptor fields"));
        } else {
            sc.expect('}', "tensor descriptor is not a JSON object");
        }
        if (!has_dtype || !has_shape || !has_off)
            throw std::runtime_error("tensor descriptor missing required field (dtype/shape/data_offsets)");
        std::uint64_t numel = 1;
        for (auto d : shape) {
            if (d != 0 && numel > UINT64_MAX / static_cast<std::uint64_t>(d))
                throw std::runtime_error("header inconsistent: element count overflows");
            numel *= static_cast<std::uint64_t>(d);
        }
        if (numel > UINT64_MAX / dtype_size(dtype))
            throw std::runtime_error("header inconsistent: element count overflows");
        const std::uint64_t nbytes = numel * dtype_size(dtype);
        if (b1 < b0 || b1 - b0 != nbytes)
            throw std::runtime_error("header inconsistent: data_offsets span " + std::to_string(b1 - b0) +
                                     " bytes but shape*dtype expects " + std::to_string(nbytes));
        if (b1 > data_bytes) throw std::runtime_error("header inconsistent: tensor " + key + " ends past the file");
        out[key] = TensorMeta{data_start + static_cast<std::size_t>(b0), std::move(shape), dtype};
    } while (sc.next_member('}', "JSON syntax error (unexpected character during scan)"));
    return out;
}
