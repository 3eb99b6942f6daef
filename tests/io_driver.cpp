// Test driver for gpu-talored-ann_amd/csrc/gtann_io.hpp (CPU only): writes
// every file type from deterministic contents, or reads a dataset back.
//   io_driver write <dir>      files named as the tests expect
//   io_driver read <dataset>   prints "N D sum" of the elements as stored
#include "gtann_io.hpp"

#include <cstdio>
#include <string>
#include <vector>

using namespace gtann_io;

int main(int argc, char** argv)
{
    if (argc < 3) return 2;
    const std::string mode = argv[1], arg = argv[2];
    try {
        if (mode == "write") {
            const int64_t N = 37;
            const int32_t W = 5, D = 7;
            std::vector<int32_t> knn(N * W);
            std::vector<float> dist(N * W), x(N * D);
            std::vector<uint32_t> g(N * W), perm(N);
            std::vector<uint8_t> u8(N * D);
            std::vector<int8_t> i8(N * D);
            std::vector<int64_t> i64(N * W);
            for (int64_t i = 0; i < N * W; ++i) {
                knn[i] = (i % 11 == 0) ? -1 : static_cast<int32_t>((i * 7) % N);
                dist[i] = 0.25f * static_cast<float>(i);
                g[i] = static_cast<uint32_t>((i * 13) % N);
                i64[i] = knn[i];
            }
            for (int64_t i = 0; i < N * D; ++i) {
                x[i] = 0.5f * static_cast<float>(i) - 3.0f;
                u8[i] = static_cast<uint8_t>(i * 5);
                i8[i] = static_cast<int8_t>(static_cast<int>(i * 5) - 128);
            }
            for (int64_t i = 0; i < N; ++i) perm[i] = static_cast<uint32_t>((i * 5) % N);
            write_table<int32_t>(arg + "/vector_knn.bin", knn.data(), N, W);
            write_table<float>(arg + "/vector_dists.bin", dist.data(), N, W);
            write_table<uint32_t>(arg + "/graph.bin", g.data(), N, W);
            write_inverse_perm(arg + "/inverse_perm.bin", perm.data(), N);
            write_dataset(arg + "/x.fbin", x.data(), static_cast<int32_t>(N), D, Elem::F32);
            write_dataset(arg + "/x.u8bin", u8.data(), static_cast<int32_t>(N), D, Elem::U8);
            write_dataset(arg + "/x.i8bin", i8.data(), static_cast<int32_t>(N), D, Elem::I8);
            write_npy<int64_t>(arg + "/ids.npy", i64.data(), N, W);
            write_npy<float>(arg + "/dist.npy", dist.data(), N, W);
            std::vector<uint32_t> boff(12);
            std::vector<int32_t> bord(11);
            for (int b = 0; b < 11; ++b) {
                boff[b + 1] = boff[b] + static_cast<uint32_t>((b * 3) % 5);
                bord[b] = (b * 7) % 11;
            }
            write_bucket_offsets(arg + "/bucket_offsets.bin", boff.data(), 11);
            write_bucket_process_order(arg + "/bucket_process_order.bin", bord.data(), 11);
            return 0;
        }
        if (mode == "read") {
            Dataset ds = read_dataset(arg);
            double s = 0;
            const size_t n = static_cast<size_t>(ds.N) * ds.D;
            for (size_t i = 0; i < n; ++i) {
                if (ds.elem == Elem::F32) s += reinterpret_cast<const float*>(ds.bytes.data())[i];
                else if (ds.elem == Elem::U8) s += ds.bytes[i];
                else s += static_cast<int8_t>(ds.bytes[i]);
            }
            std::printf("%d %d %.6f\n", ds.N, ds.D, s);
            return 0;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FATAL: %s\n", e.what());
        return 1;
    }
    return 2;
}
