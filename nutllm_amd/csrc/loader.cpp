// loader.cpp — a llama2.c checkpoint straight into HBM:
// load_llama2c_quantized_model (src/llama2.cpp:339-412) for the device model.
//
// The header and size checks are the reference's (parse_layout,
// src/llama2.cpp:199-296), with its messages, and all run before the device
// is touched. The file is read with pread, one projection at a time (the
// reference reads the same way, src/llama2.cpp:100-125); each layer's seven
// projections are quantised by the product quantiser (bit-identical to
// QuantizedMatrix::quantize) on a worker thread while the previous layer is
// uploaded, so reading, quantising and the host-to-device copies overlap.
// Projections are [out x in] as stored: query dim x dim, key / value
// kv_dim x dim, output dim x dim, gate (w1) and up (w3) ffn x dim, down
// (w2) dim x ffn; eos is 1 (src/llama2.cpp:222-223).
#include "model.hpp"

#include <cerrno>
#include <chrono>
#include <climits>
#include <cstring>
#include <fcntl.h>
#include <future>
#include <limits>
#include <string>
#include <sys/stat.h>
#include <unistd.h>
#include <vector>

namespace nut {

void quantize(const float *source, size_t rows, size_t cols, int type, size_t block_size,
              uint8_t *data, uint16_t *scales);

namespace {

class File {
public:
    explicit File(const std::string &path)
    {
        fd_ = open(path.c_str(), O_RDONLY);
        if (fd_ < 0)
            fail(NUT_ERUNTIME, "llama2 checkpoint: cannot open " + path + ": " +
                                   std::strerror(errno));
        struct stat st {};
        if (fstat(fd_, &st) != 0 || st.st_size < 0) {
            close(fd_);
            fd_ = -1;
            fail(NUT_ERUNTIME, "llama2 checkpoint: cannot stat " + path);
        }
        size_ = size_t(st.st_size);
        if (size_ == 0) {
            close(fd_);
            fd_ = -1;
            fail(NUT_ERUNTIME, "llama2 checkpoint: empty file");
        }
    }
    ~File()
    {
        if (fd_ >= 0)
            close(fd_);
    }
    File(const File &) = delete;
    File &operator=(const File &) = delete;
    size_t size() const { return size_; }
    // count floats from byte offset `at`
    void read_floats(float *dst, size_t at, size_t count) const
    {
        require(count <= SIZE_MAX / sizeof(float), NUT_ELENGTH, "llama2 checkpoint: read overflows");
        const size_t bytes = count * sizeof(float);
        if (at > size_ || bytes > size_ - at)
            fail(NUT_ERUNTIME, "llama2 checkpoint: read outside file");
        size_t done = 0;
        while (done < bytes) {
            const ssize_t r = pread(fd_, reinterpret_cast<char *>(dst) + done, bytes - done,
                                    off_t(at + done));
            if (r < 0 && errno == EINTR)
                continue;
            if (r <= 0)
                fail(NUT_ERUNTIME, "llama2 checkpoint: read failed");
            done += size_t(r);
        }
    }

private:
    int fd_ = -1;
    size_t size_ = 0;
};

size_t product(size_t a, size_t b, const char *label)
{
    if (a != 0 && b > std::numeric_limits<size_t>::max() / a)
        fail(NUT_ELENGTH, std::string("llama2 checkpoint: ") + label + " overflows");
    return a * b;
}

void add(size_t &total, size_t v)
{
    if (v > std::numeric_limits<size_t>::max() - total)
        fail(NUT_ELENGTH, "llama2 checkpoint: size overflows");
    total += v;
}

size_t positive(int32_t v, const char *name)
{
    if (v <= 0)
        fail(NUT_ERUNTIME, std::string("llama2 checkpoint: invalid ") + name);
    return size_t(v);
}

// Byte offsets of every tensor in the file (llama2.c order).
struct Layout {
    nut_config config{};
    bool shared = false;
    size_t embeddings, attention_norms, queries, keys, values, outputs, ffn_norms, gates, downs,
        ups, final_norm, classifier;
    size_t attention_matrix, kv_matrix, ffn_matrix;
};

Layout parse(const File &file)
{
    if (file.size() < 7 * sizeof(int32_t))
        fail(NUT_ERUNTIME, "llama2 checkpoint: truncated header");
    int32_t h[7];
    file.read_floats(reinterpret_cast<float *>(h), 0, 7);
    Layout l;
    nut_config &c = l.config;
    c.dim = positive(h[0], "dimension");
    c.ffn_dim = positive(h[1], "ffn dimension");
    c.layers = positive(h[2], "layer count");
    c.heads = positive(h[3], "head count");
    c.kv_heads = positive(h[4], "kv head count");
    if (h[5] == 0 || h[5] == INT32_MIN)
        fail(NUT_ERUNTIME, "llama2 checkpoint: invalid vocabulary");
    l.shared = h[5] > 0;
    c.vocab_size = size_t(h[5] > 0 ? h[5] : -h[5]);
    c.max_seq = positive(h[6], "context length");
    if (c.dim % c.heads != 0)
        fail(NUT_ERUNTIME, "llama2 checkpoint: heads do not divide dimension");
    c.head_dim = c.dim / c.heads;
    c.eos_token = 1;
    require(config_valid(c), NUT_EINVAL, "model config: invalid dimensions");
    const size_t kvd = c.kv_heads * c.head_dim;
    const size_t emb = product(c.vocab_size, c.dim, "embeddings");
    const size_t norms = product(c.layers, c.dim, "norms");
    l.attention_matrix = product(c.dim, c.dim, "attention matrix");
    const size_t attention = product(c.layers, l.attention_matrix, "attention weights");
    l.kv_matrix = product(c.dim, kvd, "kv matrix");
    const size_t kv = product(c.layers, l.kv_matrix, "kv weights");
    l.ffn_matrix = product(c.dim, c.ffn_dim, "ffn matrix");
    const size_t ffn = product(c.layers, l.ffn_matrix, "ffn weights");
    const size_t freq = product(c.max_seq, c.head_dim, "rope frequencies");
    size_t total = 0;
    for (size_t v : {emb, norms, attention, kv, kv, attention, norms, ffn, ffn, ffn, c.dim, freq})
        add(total, v);
    if (!l.shared)
        add(total, emb);
    if (total > (std::numeric_limits<size_t>::max() - 7 * sizeof(int32_t)) / sizeof(float))
        fail(NUT_ELENGTH, "llama2 checkpoint: file size overflows");
    if (file.size() != 7 * sizeof(int32_t) + total * sizeof(float))
        fail(NUT_ERUNTIME, "llama2 checkpoint: size does not match configuration");
    size_t at = 7 * sizeof(int32_t);
    auto take = [&](size_t count) {
        const size_t r = at;
        at += count * sizeof(float);
        return r;
    };
    l.embeddings = take(emb);
    l.attention_norms = take(norms);
    l.queries = take(attention);
    l.keys = take(kv);
    l.values = take(kv);
    l.outputs = take(attention);
    l.ffn_norms = take(norms);
    l.gates = take(ffn);
    l.downs = take(ffn);
    l.ups = take(ffn);
    l.final_norm = take(c.dim);
    (void)take(freq);
    l.classifier = l.shared ? l.embeddings : take(emb);
    return l;
}

// One layer read and quantised on the host.
struct HostLayer {
    std::vector<uint8_t> data[7];
    std::vector<uint16_t> scales[7];
    size_t rows[7], cols[7];
    std::vector<float> attention_norm, ffn_norm;
};

HostLayer quantize_layer(const File &file, const Layout &l, int type, size_t layer)
{
    const nut_config &c = l.config;
    const size_t kvd = c.kv_heads * c.head_dim;
    // query, key, value, output, gate, up, down: offset, rows, cols
    const size_t src[7][3] = {
        {l.queries + layer * l.attention_matrix * 4, c.dim, c.dim},
        {l.keys + layer * l.kv_matrix * 4, kvd, c.dim},
        {l.values + layer * l.kv_matrix * 4, kvd, c.dim},
        {l.outputs + layer * l.attention_matrix * 4, c.dim, c.dim},
        {l.gates + layer * l.ffn_matrix * 4, c.ffn_dim, c.dim},
        {l.ups + layer * l.ffn_matrix * 4, c.ffn_dim, c.dim},
        {l.downs + layer * l.ffn_matrix * 4, c.dim, c.ffn_dim}};
    HostLayer h;
    std::vector<float> buffer;
    for (int i = 0; i < 7; i++) {
        const size_t rows = src[i][1], cols = src[i][2], n = rows * cols;
        buffer.resize(n);
        file.read_floats(buffer.data(), src[i][0], n);
        h.rows[i] = rows;
        h.cols[i] = cols;
        h.data[i].resize(type == NUT_INT4 ? (n + 1) / 2 : n);
        h.scales[i].resize((n + 31) / 32);
        quantize(buffer.data(), rows, cols, type, 32, h.data[i].data(), h.scales[i].data());
    }
    h.attention_norm.resize(c.dim);
    h.ffn_norm.resize(c.dim);
    file.read_floats(h.attention_norm.data(), l.attention_norms + layer * c.dim * 4, c.dim);
    file.read_floats(h.ffn_norm.data(), l.ffn_norms + layer * c.dim * 4, c.dim);
    return h;
}

} // namespace

nut_model *load_llama2c(const char *path, int type, double *seconds)
{
    const auto t0 = std::chrono::steady_clock::now();
    require(path != nullptr, NUT_EINVAL, "llama2 checkpoint: null path");
    require(type == NUT_INT8 || type == NUT_INT4, NUT_EINVAL,
            "quantized model: unknown quant type");
    File file(path);
    const Layout l = parse(file);
    const nut_config &c = l.config;
    std::unique_ptr<nut_model> m(create_model(c, type, l.shared));
    // layer 0 is quantised while the globals are read and uploaded
    std::future<HostLayer> next =
        std::async(std::launch::async, quantize_layer, std::cref(file), std::cref(l), type, 0);
    {
        std::vector<float> emb(c.vocab_size * c.dim), norm(c.dim), head;
        file.read_floats(emb.data(), l.embeddings, emb.size());
        file.read_floats(norm.data(), l.final_norm, c.dim);
        if (!l.shared) {
            head.resize(emb.size());
            file.read_floats(head.data(), l.classifier, head.size());
        }
        set_globals(*m, emb.data(), norm.data(), l.shared ? nullptr : head.data());
    }
    for (size_t layer = 0; layer < c.layers; layer++) {
        HostLayer h = next.get();
        if (layer + 1 < c.layers)
            next = std::async(std::launch::async, quantize_layer, std::cref(file), std::cref(l),
                              type, layer + 1);
        nut_qmatrix q[7];
        const nut_qmatrix *mats[7];
        for (int i = 0; i < 7; i++) {
            q[i] = nut_qmatrix{h.data[i].data(), h.scales[i].data(), h.rows[i], h.cols[i], 32,
                               type};
            mats[i] = &q[i];
        }
        set_layer(*m, layer, mats, h.attention_norm.data(), h.ffn_norm.data());
    }
    if (seconds != nullptr)
        *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return m.release();
}

} // namespace nut
