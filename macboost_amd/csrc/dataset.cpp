// dataset.cpp — the preprocessed training set (BinnedDataset,
// Dataset.swift:11-86): makeDataset (Booster.swift:392-436) with edges and
// bins computed on the device, and the little-endian .mbds file.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>

#include "core.hpp"
#include "json.hpp"

namespace mb {

namespace {

constexpr uint32_t MBDS_MAGIC = 0x4D424453u;   // "MBDS" (bytes "SDBM" on disk)
constexpr uint32_t MBDS_VERSION = 1;
constexpr uint32_t MBDS_TILE = 8;

// Feature names as Foundation's JSONEncoder writes a [String]: compact, with
// '/' escaped.
std::string names_json(const std::vector<std::string> &names) {
    std::string o = "[";
    for (size_t i = 0; i < names.size(); ++i) {
        if (i) o.push_back(',');
        o.push_back('"');
        for (unsigned char c : names[i]) {
            switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '/': o += "\\/"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            case '\b': o += "\\b"; break;
            case '\f': o += "\\f"; break;
            default:
                if (c < 0x20) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\u%04x", c);
                    o += b;
                } else {
                    o.push_back((char)c);
                }
            }
        }
        o.push_back('"');
    }
    o.push_back(']');
    return o;
}

template <typename T>
void put(std::string &d, T v) {                  // little-endian host
    char b[sizeof(T)];
    std::memcpy(b, &v, sizeof(T));
    d.append(b, sizeof(T));
}

struct Reader {
    const std::string &d;
    size_t pos = 0;
    const char *take(size_t n) {
        if (n > d.size() || pos > d.size() - n) invalid("truncated .mbds file");
        const char *p = d.data() + pos;
        pos += n;
        return p;
    }
    uint32_t u32() { uint32_t v; std::memcpy(&v, take(4), 4); return v; }
    uint64_t u64() { uint64_t v; std::memcpy(&v, take(8), 8); return v; }
};

}  // namespace

BinnedDataset *dataset_make(const Params &p, const float *x, int64_t rows, int64_t cols,
                            bool row_major, const float *y,
                            const std::vector<std::string> *feature_names) {
    validate_params(p);
    if (!(rows > 0 && cols > 0) || !x || !y)
        invalid("dataset shapes inconsistent (rows=" + std::to_string(rows) +
                ", cols=" + std::to_string(cols) + ")");
    if (rows > 0xFFFFFFF0LL) invalid("more than 2^32 rows are not supported");
    for (int64_t i = 0; i < rows; ++i)
        if (!std::isfinite(y[i]))
            invalid("label at row " + std::to_string(i) + " is " + swift_float(y[i]) +
                    "; labels must be finite");
    const int64_t rs = row_major ? cols : 1, cs = row_major ? 1 : rows;
    validate_categoricals(p, x, rows, cols, rs, cs);
    if (feature_names && (int64_t)feature_names->size() != cols)
        invalid("featureNames has " + std::to_string(feature_names->size()) +
                " entries, X has " + std::to_string(cols) + " features");

    auto ds = std::make_unique<BinnedDataset>();
    ds->rows = rows;
    ds->cols = cols;
    ds->num_bins = p.num_bins;
    ds->categorical.assign(p.categorical.begin(), p.categorical.end());
    if (feature_names) {
        ds->has_feature_names = true;
        ds->feature_names = *feature_names;
    }
    ds->labels.assign(y, y + rows);

    Device dev(0);
    hipStream_t s = dev.stream;
    std::vector<uint8_t> is_cat((size_t)cols, 0);
    for (int f : p.categorical) is_cat[(size_t)f] = 1;
    const size_t ne = (size_t)p.num_bins - 2;
    const int64_t groups = (cols + 7) / 8;
    DevBuf<float> xd((size_t)rows * (size_t)cols);
    DevBuf<float> ed(std::max<size_t>(1, (size_t)cols * ne));
    DevBuf<uint8_t> cat((size_t)cols), fm((size_t)rows * (size_t)cols);
    DevBuf<uint8_t> tiled((size_t)rows * 8);     // one 8-wide tile: the kernel's other output
    DevBuf<uint64_t> out((size_t)groups * (size_t)rows);
    MB_HIP(hipMemcpyAsync(cat.ptr, is_cat.data(), (size_t)cols, hipMemcpyHostToDevice, s));
    upload(xd.ptr, x, xd.bytes(), s);
    {
        const size_t cap = mbk::edge_sample_cap(rows);
        DevBuf<uint32_t> ka((size_t)cols * cap), kb((size_t)cols * cap), cnt((size_t)cols);
        MB_HIP(mbk::launch_edges(s, xd.ptr, rows, (int)cols, rs, cs, p.num_bins, cat.ptr, ka.ptr,
                                 kb.ptr, cnt.ptr, ed.ptr));
        MB_HIP(hipStreamSynchronize(s));
    }
    // bin_data into the feature-major layout (the first tile of the gather
    // layout is written too and dropped), then regroup into tile-8 words
    for (int64_t f0 = 0; f0 < cols; f0 += 8) {
        const int n = (int)std::min<int64_t>(8, cols - f0);
        MB_HIP(mbk::launch_bin_data(s, xd.ptr + f0 * cs, rows, n, rs, cs, ed.ptr + f0 * (int64_t)ne,
                                    cat.ptr + f0, p.num_bins, 8, 1, tiled.ptr,
                                    fm.ptr + f0 * rows));
    }
    MB_HIP(mbk::launch_fm_to_tile8(s, fm.ptr, rows, (int)cols, out.ptr));
    ds->edges.resize((size_t)cols * ne);
    ds->bins.resize((size_t)groups * (size_t)rows * 8);
    if (!ds->edges.empty())
        MB_HIP(hipMemcpyAsync(ds->edges.data(), ed.ptr, ds->edges.size() * 4,
                              hipMemcpyDeviceToHost, s));
    MB_HIP(hipMemcpyAsync(ds->bins.data(), out.ptr, ds->bins.size(), hipMemcpyDeviceToHost, s));
    MB_HIP(hipStreamSynchronize(s));
    return ds.release();
}

// BinnedDataset.save (Dataset.swift:26-41).
void dataset_save(const BinnedDataset &ds, const std::string &path) {
    std::string d;
    d.reserve(64 + ds.edges.size() * 4 + ds.labels.size() * 4 + ds.bins.size());
    put<uint32_t>(d, MBDS_MAGIC);
    put<uint32_t>(d, MBDS_VERSION);
    put<uint32_t>(d, MBDS_TILE);
    put<uint64_t>(d, (uint64_t)ds.rows);
    put<uint32_t>(d, (uint32_t)ds.cols);
    put<uint32_t>(d, (uint32_t)ds.num_bins);
    put<uint32_t>(d, (uint32_t)ds.categorical.size());
    for (int32_t c : ds.categorical) put<uint32_t>(d, (uint32_t)c);
    const std::string names = ds.has_feature_names ? names_json(ds.feature_names) : std::string();
    put<uint32_t>(d, (uint32_t)names.size());
    d += names;
    put<uint64_t>(d, (uint64_t)ds.edges.size());
    d.append(reinterpret_cast<const char *>(ds.edges.data()), ds.edges.size() * 4);
    put<uint64_t>(d, (uint64_t)ds.labels.size());
    d.append(reinterpret_cast<const char *>(ds.labels.data()), ds.labels.size() * 4);
    put<uint64_t>(d, (uint64_t)ds.bins.size());
    d.append(reinterpret_cast<const char *>(ds.bins.data()), ds.bins.size());
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw Error("cannot write " + path);
    f.write(d.data(), (std::streamsize)d.size());
    if (!f) throw Error("cannot write " + path);
}

// BinnedDataset.load (Dataset.swift:43-86).
BinnedDataset *dataset_load(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error("cannot read " + path);
    std::string d((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    Reader r{d};
    if (r.u32() != MBDS_MAGIC) invalid("not a MacBoost dataset (.mbds) file");
    if (r.u32() != MBDS_VERSION) invalid("unsupported .mbds version");
    if (r.u32() != MBDS_TILE) invalid(".mbds tile width mismatch");
    auto ds = std::make_unique<BinnedDataset>();
    const uint64_t rows = r.u64();
    ds->cols = r.u32();
    ds->num_bins = (int32_t)r.u32();
    const uint32_t ncat = r.u32();
    std::vector<int32_t> cats;
    for (uint32_t i = 0; i < ncat; ++i) cats.push_back((int32_t)r.u32());
    std::sort(cats.begin(), cats.end());
    cats.erase(std::unique(cats.begin(), cats.end()), cats.end());
    for (int32_t c : cats)
        if (c < 0 || (int64_t)c >= ds->cols) invalid(".mbds categorical feature index out of range");
    ds->categorical = cats;
    const uint32_t names_len = r.u32();
    if (names_len > 0) {
        const std::string text(r.take(names_len), names_len);
        mbjson::Value v;
        try {
            v = mbjson::Parser(text).parse();
        } catch (const std::exception &) {
            invalid(".mbds feature names are not a JSON string array");
        }
        if (v.kind != mbjson::Value::Array) invalid(".mbds feature names are not a JSON string array");
        for (const auto &e : v.arr) {
            if (e.kind != mbjson::Value::String)
                invalid(".mbds feature names are not a JSON string array");
            ds->feature_names.push_back(e.str);
        }
        ds->has_feature_names = true;
    }
    const uint64_t edge_count = r.u64();
    if (edge_count > d.size() / 4) invalid("truncated .mbds file");
    const char *ep = r.take((size_t)edge_count * 4);
    ds->edges.resize((size_t)edge_count);
    std::memcpy(ds->edges.data(), ep, (size_t)edge_count * 4);
    const uint64_t label_count = r.u64();
    if (label_count > d.size() / 4) invalid("truncated .mbds file");
    const char *lp = r.take((size_t)label_count * 4);
    ds->labels.resize((size_t)label_count);
    std::memcpy(ds->labels.data(), lp, (size_t)label_count * 4);
    const uint64_t bin_count = r.u64();
    const char *bp = r.take((size_t)bin_count);
    ds->bins.assign(reinterpret_cast<const uint8_t *>(bp),
                    reinterpret_cast<const uint8_t *>(bp) + bin_count);
    const uint64_t tiles = ((uint64_t)ds->cols + 7) / 8;
    if (label_count != rows || bin_count != rows * tiles * 8 ||
        edge_count != (uint64_t)ds->cols * (uint64_t)(ds->num_bins - 2))
        invalid(".mbds sizes are inconsistent");
    ds->rows = (int64_t)rows;
    return ds.release();
}

}  // namespace mb
