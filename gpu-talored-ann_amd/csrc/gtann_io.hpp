// gtann_io.hpp -- readers and writers of the pipeline's on-disk files.
//
// Layouts (byte-identical with the reference's files):
//   dataset   .fbin/.bin  int32 N, int32 D, N*D float32     (src/load.hpp:67-84)
//             .u8bin      int32 N, int32 D, N*D uint8       (src/load.hpp:94-117)
//             .i8bin      int32 N, int32 D, N*D int8, signed (src/load.hpp:86-92)
//   vector_knn.bin        int64 N, int32 M, int32[N*M], -1 = padding
//                         (src/graph_io.hpp:26-30, 286-329)
//   vector_dists.bin      int64 N, int32 M, float32[N*M] (src/bucket.cu:5563-5573)
//   graph / final_graph   int64 N, int32 K, uint32[N*K]  (src/graph_io.hpp:8-11, 50-96)
//   inverse_perm.bin      uint32[N], no header           (src/graph_io.hpp:369-377)
//   *.npy                 NumPy format 1.0, C order, little endian (src/load.hpp:535-590)
//
// Errors throw std::runtime_error naming the file.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace gtann_io {

enum class Elem { F32, U8, I8 };

inline size_t elem_size(Elem e) { return e == Elem::F32 ? 4 : 1; }

inline bool ends_with(const std::string& s, const char* suf)
{
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// element type a dataset path stands for, by extension
inline Elem dataset_elem(const std::string& path)
{
    if (ends_with(path, ".fbin") || ends_with(path, ".bin")) return Elem::F32;
    if (ends_with(path, ".u8bin")) return Elem::U8;
    if (ends_with(path, ".i8bin")) return Elem::I8;
    throw std::runtime_error("unsupported dataset extension (.fbin/.bin/.u8bin/.i8bin): " + path);
}

class File {
public:
    File(const std::string& path, const char* mode) : path_(path), f_(std::fopen(path.c_str(), mode))
    {
        if (!f_) throw std::runtime_error("cannot open " + path);
    }
    ~File() { if (f_) std::fclose(f_); }
    File(const File&) = delete;
    File& operator=(const File&) = delete;
    void read(void* p, size_t bytes, const char* what)
    {
        if (bytes && std::fread(p, 1, bytes, f_) != bytes)
            throw std::runtime_error(std::string("short read of ") + what + ": " + path_);
    }
    void write(const void* p, size_t bytes)
    {
        if (bytes && std::fwrite(p, 1, bytes, f_) != bytes) throw std::runtime_error("write failed: " + path_);
    }
    void close()
    {
        if (f_ && std::fclose(f_) != 0) { f_ = nullptr; throw std::runtime_error("close failed: " + path_); }
        f_ = nullptr;
    }
    int64_t size()
    {
        const long cur = std::ftell(f_);
        std::fseek(f_, 0, SEEK_END);
        const long end = std::ftell(f_);
        std::fseek(f_, cur, SEEK_SET);
        return end;
    }

private:
    std::string path_;
    std::FILE* f_;
};

struct Dataset {
    int32_t N = 0, D = 0;
    Elem elem = Elem::F32;
    std::vector<uint8_t> bytes;   // N*D elements as stored in the file
    const void* data() const { return bytes.data(); }
};

inline Dataset read_dataset(const std::string& path)
{
    Dataset ds;
    ds.elem = dataset_elem(path);
    File f(path, "rb");
    int32_t hdr[2];
    f.read(hdr, sizeof(hdr), "header");
    if (hdr[0] <= 0 || hdr[1] <= 0) throw std::runtime_error("bad header (N, D) in " + path);
    ds.N = hdr[0];
    ds.D = hdr[1];
    ds.bytes.resize(static_cast<size_t>(ds.N) * ds.D * elem_size(ds.elem));
    f.read(ds.bytes.data(), ds.bytes.size(), "payload");
    return ds;
}

inline void write_dataset(const std::string& path, const void* data, int32_t N, int32_t D, Elem elem)
{
    File f(path, "wb");
    const int32_t hdr[2] = {N, D};
    f.write(hdr, sizeof(hdr));
    f.write(data, static_cast<size_t>(N) * D * elem_size(elem));
    f.close();
}

// int64 N, int32 W, T[N*W]: vector_knn.bin (int32), vector_dists.bin (float),
// graphs (uint32)
template <typename T>
struct Table {
    int64_t N = 0;
    int32_t W = 0;
    std::vector<T> v;
};

template <typename T>
inline Table<T> read_table(const std::string& path)
{
    Table<T> t;
    File f(path, "rb");
    f.read(&t.N, sizeof(t.N), "header");
    f.read(&t.W, sizeof(t.W), "header");
    if (t.N <= 0 || t.W <= 0) throw std::runtime_error("bad header (N, width) in " + path);
    t.v.resize(static_cast<size_t>(t.N) * t.W);
    f.read(t.v.data(), t.v.size() * sizeof(T), "payload");
    return t;
}

template <typename T>
inline void write_table(const std::string& path, const T* v, int64_t N, int32_t W)
{
    File f(path, "wb");
    f.write(&N, sizeof(N));
    f.write(&W, sizeof(W));
    f.write(v, static_cast<size_t>(N) * W * sizeof(T));
    f.close();
}

inline std::vector<uint32_t> read_inverse_perm(const std::string& path)
{
    File f(path, "rb");
    const int64_t bytes = f.size();
    if (bytes <= 0 || bytes % 4) throw std::runtime_error("inverse permutation size is not a multiple of 4: " + path);
    std::vector<uint32_t> p(static_cast<size_t>(bytes / 4));
    f.read(p.data(), static_cast<size_t>(bytes), "payload");
    return p;
}

inline void write_inverse_perm(const std::string& path, const uint32_t* p, int64_t N)
{
    File f(path, "wb");
    f.write(p, static_cast<size_t>(N) * 4);
    f.close();
}

template <typename T> inline const char* npy_descr();
template <> inline const char* npy_descr<int64_t>() { return "<i8"; }
template <> inline const char* npy_descr<int32_t>() { return "<i4"; }
template <> inline const char* npy_descr<uint32_t>() { return "<u4"; }
template <> inline const char* npy_descr<float>() { return "<f4"; }

// NumPy format 1.0: magic, version, uint16 header length, a dict padded with
// spaces and a newline so that the data starts at a multiple of 64 bytes
template <typename T>
inline void write_npy(const std::string& path, const T* v, int64_t rows, int64_t cols)
{
    std::string dict = std::string("{'descr': '") + npy_descr<T>() + "', 'fortran_order': False, 'shape': (" +
                       std::to_string(rows) + ", " + std::to_string(cols) + "), }";
    const size_t pre = 10;
    size_t total = pre + dict.size() + 1;
    const size_t pad = (64 - total % 64) % 64;
    dict.append(pad, ' ');
    dict.push_back('\n');
    const uint16_t hlen = static_cast<uint16_t>(dict.size());
    File f(path, "wb");
    const char magic[8] = {'\x93', 'N', 'U', 'M', 'P', 'Y', 1, 0};
    f.write(magic, 8);
    f.write(&hlen, 2);
    f.write(dict.data(), dict.size());
    f.write(v, static_cast<size_t>(rows * cols) * sizeof(T));
    f.close();
}

// bucket_offsets.bin: int32 n_buckets, uint32[n_buckets + 1], indexed by
// processing position (src/graph_io.hpp:13-17, 178-205)
inline void write_bucket_offsets(const std::string& path, const uint32_t* off, int32_t n_buckets)
{
    File f(path, "wb");
    f.write(&n_buckets, sizeof(n_buckets));
    f.write(off, (static_cast<size_t>(n_buckets) + 1) * sizeof(uint32_t));
    f.close();
}

inline std::vector<uint32_t> read_bucket_offsets(const std::string& path)
{
    File f(path, "rb");
    int32_t n = 0;
    f.read(&n, sizeof(n), "header");
    if (n <= 0) throw std::runtime_error("bad bucket-offsets header: " + path);
    std::vector<uint32_t> v(static_cast<size_t>(n) + 1);
    f.read(v.data(), v.size() * sizeof(uint32_t), "payload");
    return v;
}

// bucket_process_order.bin: int32 n, int32[n] = bucket id at each
// processing position (src/graph_io.hpp:207-244)
inline void write_bucket_process_order(const std::string& path, const int32_t* order, int32_t n)
{
    File f(path, "wb");
    f.write(&n, sizeof(n));
    f.write(order, static_cast<size_t>(n) * sizeof(int32_t));
    f.close();
}

// Step 5 of bucket2 (src/bucket.cu:3434-3510): bucket_data.bin holds the
// point ids of bucket 0, 1, ... as int32 (each bucket's ids ascending);
// bucket_index.bin is int64 n_buckets, int64 N, then per bucket int64 byte
// offset into bucket_data.bin and int32 count, packed (12 bytes a record).
// bucket[i] is point i's bucket; ids outside [0, n_buckets) are left out.
inline void write_bucket_files(const std::string& index_path, const std::string& data_path, const int32_t* bucket,
                               int64_t N, int64_t n_buckets)
{
    std::vector<int64_t> count(static_cast<size_t>(n_buckets) + 1, 0);
    for (int64_t i = 0; i < N; ++i)
        if (bucket[i] >= 0 && bucket[i] < n_buckets) ++count[static_cast<size_t>(bucket[i]) + 1];
    for (int64_t c = 0; c < n_buckets; ++c) count[static_cast<size_t>(c) + 1] += count[static_cast<size_t>(c)];
    std::vector<int32_t> ids(static_cast<size_t>(count[static_cast<size_t>(n_buckets)]));
    std::vector<int64_t> cur(count.begin(), count.end() - 1);
    for (int64_t i = 0; i < N; ++i)
        if (bucket[i] >= 0 && bucket[i] < n_buckets) ids[static_cast<size_t>(cur[static_cast<size_t>(bucket[i])]++)] =
            static_cast<int32_t>(i);
    File d(data_path, "wb");
    d.write(ids.data(), ids.size() * sizeof(int32_t));
    d.close();
    std::vector<unsigned char> idx(16 + static_cast<size_t>(n_buckets) * 12);
    std::memcpy(idx.data(), &n_buckets, 8);
    std::memcpy(idx.data() + 8, &N, 8);
    for (int64_t c = 0; c < n_buckets; ++c) {
        const int64_t off = count[static_cast<size_t>(c)] * 4;
        const int32_t cnt = static_cast<int32_t>(count[static_cast<size_t>(c) + 1] - count[static_cast<size_t>(c)]);
        std::memcpy(idx.data() + 16 + c * 12, &off, 8);
        std::memcpy(idx.data() + 16 + c * 12 + 8, &cnt, 4);
    }
    File f(index_path, "wb");
    f.write(idx.data(), idx.size());
    f.close();
}

// centroid_global_indices.bin: int64 n, int64[n] (src/bucket.cu:9561-9568)
inline void write_centroid_indices(const std::string& path, const int64_t* ids, int64_t n)
{
    File f(path, "wb");
    f.write(&n, sizeof(n));
    f.write(ids, static_cast<size_t>(n) * sizeof(int64_t));
    f.close();
}

inline std::vector<int32_t> read_bucket_process_order(const std::string& path)
{
    File f(path, "rb");
    int32_t n = 0;
    f.read(&n, sizeof(n), "header");
    if (n <= 0) throw std::runtime_error("bad bucket-process-order header: " + path);
    std::vector<int32_t> v(static_cast<size_t>(n));
    f.read(v.data(), v.size() * sizeof(int32_t), "payload");
    return v;
}

// 2-D .npy of int64, int32 or uint32 (format 1.x/2.x, C order, little
// endian), widened to int64: neighbors.npy and exact-kNN indices, the files
// bd/load.hpp:103 (read_npy_int64_2d) reads.
inline std::vector<int64_t> read_npy_2d(const std::string& path, int64_t& rows, int64_t& cols)
{
    File f(path, "rb");
    char magic[8];
    f.read(magic, 8, "npy magic");
    if (static_cast<unsigned char>(magic[0]) != 0x93 || std::string(magic + 1, 5) != "NUMPY")
        throw std::runtime_error("not a .npy file: " + path);
    uint32_t hlen = 0;
    if (magic[6] == 1) {
        uint16_t h16;
        f.read(&h16, 2, "npy header length");
        hlen = h16;
    } else if (magic[6] == 2 || magic[6] == 3) {
        f.read(&hlen, 4, "npy header length");
    } else {
        throw std::runtime_error("unsupported .npy version in " + path);
    }
    std::string h(hlen, '\0');
    f.read(&h[0], hlen, "npy header");
    auto field = [&](const char* key) -> std::string {
        const size_t k = h.find(key);
        if (k == std::string::npos) throw std::runtime_error(std::string("no ") + key + " in .npy header: " + path);
        return h.substr(k + std::strlen(key));
    };
    const std::string descr = field("'descr':");
    const std::string order = field("'fortran_order':");
    if (order.find("True") < order.find(',')) throw std::runtime_error("Fortran-order .npy not supported: " + path);
    size_t esz = 0;
    int kind = 0;   // 0 i8, 1 i4, 2 u4
    if (descr.find("'<i8'") < descr.find(',')) { esz = 8; kind = 0; }
    else if (descr.find("'<i4'") < descr.find(',')) { esz = 4; kind = 1; }
    else if (descr.find("'<u4'") < descr.find(',')) { esz = 4; kind = 2; }
    else throw std::runtime_error("unsupported .npy dtype (int64, int32, uint32): " + path);
    const std::string shape = field("'shape':");
    const size_t o = shape.find('('), c = shape.find(')');
    if (o == std::string::npos || c == std::string::npos) throw std::runtime_error("bad .npy shape: " + path);
    const std::string dims = shape.substr(o + 1, c - o - 1);
    const size_t comma = dims.find(',');
    if (comma == std::string::npos) throw std::runtime_error(".npy array is not 2-D: " + path);
    rows = std::stoll(dims.substr(0, comma));
    const std::string rest = dims.substr(comma + 1);
    if (rest.find_first_of("0123456789") == std::string::npos) throw std::runtime_error(".npy array is not 2-D: " + path);
    cols = std::stoll(rest);
    if (rows <= 0 || cols <= 0) throw std::runtime_error("empty .npy array: " + path);
    const size_t n = static_cast<size_t>(rows) * static_cast<size_t>(cols);
    std::vector<int64_t> out(n);
    if (kind == 0) {
        f.read(out.data(), n * 8, "npy payload");
    } else {
        std::vector<uint32_t> tmp(n);
        f.read(tmp.data(), n * esz, "npy payload");
        for (size_t i = 0; i < n; ++i)
            out[i] = kind == 1 ? static_cast<int64_t>(static_cast<int32_t>(tmp[i])) : static_cast<int64_t>(tmp[i]);
    }
    return out;
}

// ground truth .ibin: int32 N, int32 K, int32[N*K] (bd/load.py:43-58)
inline std::vector<int32_t> read_ibin(const std::string& path, int32_t& N, int32_t& K)
{
    File f(path, "rb");
    int32_t hdr[2];
    f.read(hdr, sizeof(hdr), "header");
    if (hdr[0] <= 0 || hdr[1] <= 0) throw std::runtime_error("bad header (N, K) in " + path);
    N = hdr[0];
    K = hdr[1];
    std::vector<int32_t> v(static_cast<size_t>(N) * K);
    f.read(v.data(), v.size() * 4, "payload");
    return v;
}

}  // namespace gtann_io
