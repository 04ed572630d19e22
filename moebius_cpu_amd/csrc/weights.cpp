// Safetensors weights of the converter's moebius-cpu/1 format (src/weights.rs,
// src/unet/load.rs, src/vae/mod.rs:88-93): mapping, header parsing and the
// shape-checked tensor sets of the two models.
#include "weights.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <sstream>

#include "common.hpp"

namespace mh {

namespace {

// ---- a JSON reader for the safetensors header: objects, arrays, strings,
// integers (the only value kinds the format uses; anything else is an error).
struct Json {
    enum Kind { Null, Str, Num, Arr, Obj } kind = Null;
    std::string s;
    int64_t n = 0;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;
    const Json *get(const std::string &k) const {
        for (const auto &kv : o)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
  public:
    JsonReader(const char *p, size_t n) : p_(p), end_(p + n) {}
    Json parse() {
        Json v = value(0);
        ws();
        if (p_ != end_) bad("trailing bytes after the header object");
        return v;
    }

  private:
    const char *p_, *end_;
    [[noreturn]] void bad(const char *what) { fail(kWeights, std::string("safetensors header: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    char peek() {
        ws();
        if (p_ >= end_) bad("unexpected end");
        return *p_;
    }
    void expect(char c) {
        if (peek() != c) bad("unexpected character");
        ++p_;
    }
    std::string str() {
        expect('"');
        std::string out;
        while (true) {
            if (p_ >= end_) bad("unterminated string");
            const char c = *p_++;
            if (c == '"') return out;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= end_) bad("unterminated escape");
            const char e = *p_++;
            switch (e) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (end_ - p_ < 4) bad("short \\u escape");
                    unsigned cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = *p_++;
                        cp <<= 4;
                        if (h >= '0' && h <= '9') cp |= unsigned(h - '0');
                        else if (h >= 'a' && h <= 'f') cp |= unsigned(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') cp |= unsigned(h - 'A' + 10);
                        else bad("bad \\u escape");
                    }
                    // UTF-8 of a basic-plane code point (tensor names are ASCII in practice)
                    if (cp < 0x80) {
                        out.push_back(char(cp));
                    } else if (cp < 0x800) {
                        out.push_back(char(0xC0 | (cp >> 6)));
                        out.push_back(char(0x80 | (cp & 0x3F)));
                    } else {
                        out.push_back(char(0xE0 | (cp >> 12)));
                        out.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back(char(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: bad("bad escape");
            }
        }
    }
    Json value(int depth) {
        if (depth > 16) bad("nesting too deep");
        Json v;
        const char c = peek();
        if (c == '{') {
            v.kind = Json::Obj;
            ++p_;
            if (peek() == '}') {
                ++p_;
                return v;
            }
            while (true) {
                std::string k = str();
                expect(':');
                v.o.emplace_back(std::move(k), value(depth + 1));
                const char d = peek();
                ++p_;
                if (d == '}') return v;
                if (d != ',') bad("expected , or }");
            }
        }
        if (c == '[') {
            v.kind = Json::Arr;
            ++p_;
            if (peek() == ']') {
                ++p_;
                return v;
            }
            while (true) {
                v.a.push_back(value(depth + 1));
                const char d = peek();
                ++p_;
                if (d == ']') return v;
                if (d != ',') bad("expected , or ]");
            }
        }
        if (c == '"') {
            v.kind = Json::Str;
            v.s = str();
            return v;
        }
        if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Json::Num;
            bool neg = false;
            if (*p_ == '-') neg = true, ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') bad("bad number");
            uint64_t x = 0;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
                if (x > (uint64_t(1) << 62) / 10) bad("number out of range");
                x = x * 10 + uint64_t(*p_++ - '0');
            }
            if (p_ < end_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) bad("non-integer number");
            v.n = neg ? -int64_t(x) : int64_t(x);
            return v;
        }
        bad("unsupported value");
    }
};

}  // namespace

WeightsFile::WeightsFile(const std::string &path, const std::string &expected_format) : path_(path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) fail(kIo, path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        fail(kIo, path + ": " + std::strerror(e));
    }
    size_ = size_t(st.st_size);
    if (size_ < 8) {
        ::close(fd);
        fail(kWeights, path + ": file too small for a safetensors header");
    }
    map_ = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        fail(kIo, path + ": mmap: " + std::strerror(errno));
    }
    try {
        const unsigned char *base = static_cast<const unsigned char *>(map_);
        uint64_t hlen = 0;
        for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | base[i];
        if (hlen > size_ - 8) fail(kWeights, path + ": header length past the end of the file");
        const Json root = JsonReader(reinterpret_cast<const char *>(base + 8), size_t(hlen)).parse();
        if (root.kind != Json::Obj) fail(kWeights, path + ": header is not an object");
        const size_t data_start = size_t(8 + hlen);
        const size_t data_len = size_ - data_start;
        for (const auto &kv : root.o) {
            if (kv.first == "__metadata__") {
                if (kv.second.kind != Json::Obj) fail(kWeights, path + ": __metadata__ is not an object");
                for (const auto &m : kv.second.o) {
                    if (m.second.kind != Json::Str) fail(kWeights, path + ": metadata values must be strings");
                    meta_[m.first] = m.second.s;
                }
                continue;
            }
            const Json &t = kv.second;
            const Json *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
            if (t.kind != Json::Obj || !dt || !sh || !off || dt->kind != Json::Str || sh->kind != Json::Arr ||
                off->kind != Json::Arr || off->a.size() != 2)
                fail(kWeights, path + ": tensor " + kv.first + ": malformed entry");
            FileTensor ft;
            int64_t esize = 0;
            if (dt->s == "F32") ft.dtype = kF32, esize = 4;
            else if (dt->s == "F16") ft.dtype = kF16, esize = 2;
            else fail(kWeights, kv.first + ": unsupported dtype " + dt->s);
            ft.numel = 1;
            for (const Json &d : sh->a) {
                if (d.kind != Json::Num || d.n < 0) fail(kWeights, kv.first + ": bad shape");
                ft.shape.push_back(d.n);
                if (d.n && ft.numel > (int64_t(1) << 40) / d.n) fail(kWeights, kv.first + ": shape too large");
                ft.numel *= d.n;
            }
            const int64_t b0 = off->a[0].n, b1 = off->a[1].n;
            if (off->a[0].kind != Json::Num || off->a[1].kind != Json::Num || b0 < 0 || b1 < b0 ||
                uint64_t(b1) > data_len)
                fail(kWeights, kv.first + ": data offsets outside the file");
            if (b1 - b0 != ft.numel * esize)
                fail(kWeights, kv.first + ": byte range does not match its shape and dtype");
            if ((data_start + size_t(b0)) % size_t(esize) != 0) fail(kWeights, kv.first + ": misaligned data");
            ft.data = base + data_start + size_t(b0);
            tensors_[kv.first] = std::move(ft);
        }
        const std::string *found = metadata("format");
        if (!found || *found != expected_format) {
            fail(kWeights, path + ": format " + (found ? "\"" + *found + "\"" : std::string("None")) +
                               ", expected \"" + expected_format + "\" (re-run tools/convert_weights.py)");
        }
    } catch (...) {
        ::munmap(map_, size_);
        map_ = nullptr;
        throw;
    }
}

WeightsFile::~WeightsFile() {
    if (map_) ::munmap(map_, size_);
}

const std::string *WeightsFile::metadata(const std::string &key) const {
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

const FileTensor *WeightsFile::find(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

// ---- the models' converted tensor sets

namespace {

using Shapes = std::map<std::string, std::vector<int64_t>>;

void lin(Shapes &s, const std::string &p, int64_t ci, int64_t co, bool bias = true) {
    s[p + ".weight"] = {co, ci};
    if (bias) s[p + ".bias"] = {co};
}
void norm(Shapes &s, const std::string &p, int64_t c) {
    s[p + ".weight"] = {c};
    s[p + ".bias"] = {c};
}
void conv3(Shapes &s, const std::string &p, int64_t ci, int64_t co) {
    s[p + ".weight"] = {co, 3, 3, ci};
    s[p + ".bias"] = {co};
}

// src/unet/blocks.rs:31-113, transformer.rs:65-87, lambda.rs:86-104 and 205-249,
// embed.rs:40-83, mod.rs:86-140 (src/config.rs: 320/640/1280 channels, 2 layers
// down and 3 up, 8 heads, hidden 2.5 C, 10 tokens of 768).
void unet_shapes(Shapes &s) {
    const int64_t CH[3] = {320, 640, 1280}, HEADS = 8, TEMB = 1280, XDIM = 768;
    auto dwconv = [&](const std::string &p, int64_t ci, int64_t co) {
        s[p + ".conv_dw.weight"] = {3, 3, ci};
        s[p + ".conv_dw.bias"] = {ci};
        lin(s, p + ".conv_pw", ci, co);
    };
    auto resnet = [&](const std::string &p, int64_t ci, int64_t co) {
        norm(s, p + ".norm1", ci);
        dwconv(p + ".conv1", ci, co);
        lin(s, p + ".time_emb_proj", TEMB, co);
        norm(s, p + ".norm2", co);
        dwconv(p + ".conv2", co, co);
        if (ci != co) lin(s, p + ".conv_shortcut", ci, co);
    };
    auto transformer = [&](const std::string &p, int64_t c) {
        const int64_t k = c / HEADS, hidden = c * 5 / 2, side = 64 * 320 / c;
        const std::string b = p + ".transformer_blocks.0";
        norm(s, p + ".norm", c);
        lin(s, p + ".proj_in", c, c);
        norm(s, b + ".norm1", c);
        lin(s, b + ".attn1.to_q", c, c);
        lin(s, b + ".attn1.to_k", c, k, false);
        lin(s, b + ".attn1.to_v", c, k);
        s[b + ".attn1.pos_conv.weight"] = {k, 225};
        s[b + ".attn1.pos_conv.bias"] = {k};
        norm(s, b + ".norm2", c);
        s[b + ".attn2.rel_pos_emb"] = {side * side, 10, k};
        lin(s, b + ".attn2.to_q", c, c);
        s[b + ".attn2.to_k.weight"] = {k, XDIM};
        s[b + ".attn2.to_v.weight"] = {k, XDIM};
        s[b + ".attn2.to_v.bias"] = {k};
        norm(s, b + ".norm3", c);
        lin(s, b + ".ff.inverted_conv.conv", c, 2 * hidden);
        s[b + ".ff.depth_conv.conv.weight"] = {3, 3, 2 * hidden};
        s[b + ".ff.depth_conv.conv.bias"] = {2 * hidden};
        lin(s, b + ".ff.point_conv.conv", hidden, c, false);
        lin(s, p + ".proj_out", c, c);
    };
    s["embedding_layer.weight"] = {20, 3072};
    const std::string d = "diff_model";
    lin(s, d + ".encoder_hid_proj", 3072, XDIM);
    lin(s, d + ".time_embedding.linear_1", 320, TEMB);
    lin(s, d + ".time_embedding.linear_2", TEMB, TEMB);
    dwconv(d + ".conv_in", 9, CH[0]);
    int64_t c_prev = CH[0];
    std::vector<int64_t> skips = {CH[0]};
    for (int i = 0; i < 3; ++i) {
        const std::string l = d + ".down_blocks." + std::to_string(i);
        for (int j = 0; j < 2; ++j) {
            resnet(l + ".resnets." + std::to_string(j), j == 0 ? c_prev : CH[i], CH[i]);
            transformer(l + ".attentions." + std::to_string(j), CH[i]);
            skips.push_back(CH[i]);
        }
        if (i < 2) {
            conv3(s, l + ".downsamplers.0.conv", CH[i], CH[i]);
            skips.push_back(CH[i]);
        }
        c_prev = CH[i];
    }
    int64_t h_c = CH[2];
    for (int i = 0; i < 3; ++i) {
        const int64_t c = CH[2 - i];
        const std::string l = d + ".up_blocks." + std::to_string(i);
        for (int j = 0; j < 3; ++j) {
            const int64_t skip = skips.back();
            skips.pop_back();
            resnet(l + ".resnets." + std::to_string(j), h_c + skip, c);
            transformer(l + ".attentions." + std::to_string(j), c);
            h_c = c;
        }
        if (i < 2) conv3(s, l + ".upsamplers.0.conv", c, c);
    }
    norm(s, d + ".conv_norm_out", CH[0]);
    dwconv(d + ".conv_out", CH[0], 4);
}

// src/vae/encoder.rs:47-73, decoder.rs:44-70, mod.rs:174-189, 227-236, 297-312
// (src/config.rs: 128/256/512/512 channels, 2 layers down and 3 up).
void vae_shapes(Shapes &s) {
    const int64_t CH[4] = {128, 256, 512, 512};
    auto resnet = [&](const std::string &p, int64_t ci, int64_t co) {
        norm(s, p + ".norm1", ci);
        conv3(s, p + ".conv1", ci, co);
        norm(s, p + ".norm2", co);
        conv3(s, p + ".conv2", co, co);
        if (ci != co) lin(s, p + ".conv_shortcut", ci, co);
    };
    auto mid = [&](const std::string &p, int64_t c) {
        const std::string a = p + ".attentions.0";
        norm(s, a + ".group_norm", c);
        for (const char *t : {"to_q", "to_k", "to_v", "to_out.0"}) lin(s, a + "." + t, c, c);
        resnet(p + ".resnets.0", c, c);
        resnet(p + ".resnets.1", c, c);
    };
    conv3(s, "encoder.conv_in", 3, CH[0]);
    int64_t c_prev = CH[0];
    for (int i = 0; i < 4; ++i) {
        const std::string l = "encoder.down_blocks." + std::to_string(i);
        for (int j = 0; j < 2; ++j) resnet(l + ".resnets." + std::to_string(j), j == 0 ? c_prev : CH[i], CH[i]);
        if (i < 3) conv3(s, l + ".downsamplers.0.conv", CH[i], CH[i]);
        c_prev = CH[i];
    }
    mid("encoder.mid_block", CH[3]);
    norm(s, "encoder.conv_norm_out", CH[3]);
    conv3(s, "encoder.conv_out", CH[3], 8);
    lin(s, "quant_conv", 8, 8);
    lin(s, "post_quant_conv", 4, 4);
    conv3(s, "decoder.conv_in", 4, CH[3]);
    mid("decoder.mid_block", CH[3]);
    c_prev = CH[3];
    for (int i = 0; i < 4; ++i) {
        const int64_t c = CH[3 - i];
        const std::string l = "decoder.up_blocks." + std::to_string(i);
        for (int j = 0; j < 3; ++j) resnet(l + ".resnets." + std::to_string(j), j == 0 ? c_prev : c, c);
        if (i < 3) conv3(s, l + ".upsamplers.0.conv", c, c);
        c_prev = c;
    }
    norm(s, "decoder.conv_norm_out", CH[0]);
    conv3(s, "decoder.conv_out", CH[0], 3);
}

std::string shape_text(const std::vector<int64_t> &v) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
    os << "]";
    return os.str();
}

}  // namespace

std::map<std::string, std::vector<int64_t>> expected_tensors(ModelKind kind) {
    Shapes s;
    if (kind == ModelKind::UNet) unet_shapes(s);
    else vae_shapes(s);
    return s;
}

std::vector<NamedTensor> model_tensors(const WeightsFile &f, ModelKind kind) {
    if (kind == ModelKind::Vae) {
        // src/vae/mod.rs:88-93: the file must come from the 0.13025-scaled VAE
        const std::string *sf = f.metadata("scaling_factor");
        char *end = nullptr;
        const float v = sf ? std::strtof(sf->c_str(), &end) : 0.0f;
        if (!sf || end == sf->c_str() || *end || v != 0.13025f)
            fail(kWeights, "vae scaling_factor metadata " + (sf ? "\"" + *sf + "\"" : std::string("None")) +
                               ", expected \"0.13025\"");
    }
    std::vector<NamedTensor> out;
    for (const auto &kv : expected_tensors(kind)) {
        const FileTensor *t = f.find(kv.first);
        if (!t) fail(kWeights, "missing tensor " + kv.first);
        if (t->shape != kv.second)
            fail(kWeights, kv.first + ": shape " + shape_text(t->shape) + ", expected " + shape_text(kv.second));
        NamedTensor n;
        n.name = f.tensors().find(kv.first)->first.c_str();  // the expected map is a temporary
        n.data = t->data;
        n.dtype = t->dtype;
        n.numel = uint64_t(t->numel);
        out.push_back(n);
    }
    return out;
}

}  // namespace mh
