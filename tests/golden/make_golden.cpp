// make_golden.cpp — writes the known-answer fixtures of the reference's own
// tests (tests/*.cpp of Ligo04/lc_parallel_primitive), regenerated with the
// same standard-library calls the reference tests make (std::mt19937 seeded
// 114521, std::shuffle, std::uniform_real_distribution<float>), with the
// expected outputs computed by the same std:: algorithms the reference
// tests check against (std::accumulate, std::min/max_element, std::sort).
// Built with g++/libstdc++ by make_golden.py; the outputs are raw
// little-endian arrays described by golden.json.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <functional>
#include <numeric>
#include <random>
#include <string>
#include <vector>

static std::string g_dir;

template <class T>
static void dump(const char *name, const std::vector<T> &v)
{
    std::string path = g_dir + "/" + name;
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) { std::perror(path.c_str()); std::exit(1); }
    std::fwrite(v.data(), sizeof(T), v.size(), f);
    std::fclose(f);
}

int main(int argc, char **argv)
{
    g_dir = argc > 1 ? argv[1] : ".";

    // device_reduce_test.cpp:53-62, 120-166: 0..4095 shuffled with mt19937(114521)
    {
        std::vector<int32_t> a(1 << 12);
        std::iota(a.begin(), a.end(), 0);
        std::mt19937 rng(114521);
        std::shuffle(a.begin(), a.end(), rng);
        dump("reduce_shuffled_4096_i32.bin", a);
        std::vector<int32_t> expect = {*std::min_element(a.begin(), a.end()),
                                       *std::max_element(a.begin(), a.end()),
                                       std::accumulate(a.begin(), a.end(), 0)};
        dump("reduce_shuffled_4096_expect_min_max_sum_i32.bin", expect);
    }
    // device_segment_reduce.cpp:62-125: 0..1023 shuffled, segments of 100
    {
        const int n = 1024, per = 100;
        std::vector<int32_t> a(n);
        std::iota(a.begin(), a.end(), 0);
        std::mt19937 rng(114521);
        std::shuffle(a.begin(), a.end(), rng);
        const int segs = n / per + 1;
        std::vector<uint32_t> b(segs), e(segs);
        std::vector<int32_t> sums(segs);
        for (int i = 0; i < n; ++i)
            if (i % per == 0) {
                b[i / per] = i;
                e[i / per] = std::min(i + per, n);
                sums[i / per] = std::accumulate(a.begin() + i, a.begin() + i + std::min(n - i, per), 0);
            }
        dump("segment_shuffled_1024_i32.bin", a);
        dump("segment_shuffled_1024_begin_u32.bin", b);
        dump("segment_shuffled_1024_end_u32.bin", e);
        dump("segment_shuffled_1024_expect_i32.bin", sums);
    }
    // device_radix_sort_one_sweep.cpp:61-118: float keys, ascending and
    // descending, keys drawn alternately from one mt19937(114521) stream
    for (int lg : {5, 8, 12}) {
        const int n = 1 << lg;
        std::vector<float> asc(n), desc(n);
        std::mt19937 rng(114521);
        std::uniform_real_distribution<float> dist(0.0f, 1.0f);
        for (int i = 0; i < n; ++i) {
            asc[i] = dist(rng);
            desc[i] = dist(rng);
        }
        dump(("sort_float_" + std::to_string(n) + "_asc_in_f32.bin").c_str(), asc);
        dump(("sort_float_" + std::to_string(n) + "_desc_in_f32.bin").c_str(), desc);
        std::sort(asc.begin(), asc.end());
        std::sort(desc.begin(), desc.end(), std::greater<float>());
        dump(("sort_float_" + std::to_string(n) + "_asc_expect_f32.bin").c_str(), asc);
        dump(("sort_float_" + std::to_string(n) + "_desc_expect_f32.bin").c_str(), desc);
    }
    // device_radix_sort_one_sweep.cpp:153-279: pairs (uint key, float value);
    // keys are a shuffled iota, values U[0,1).  The reference uses 524288
    // items; the fixture uses the same procedure at 16384 items to stay small.
    {
        const int n = 1 << 14;
        std::vector<uint32_t> key(n), dkey(n);
        std::vector<float> val(n), dval(n);
        std::mt19937 rng(114521);
        std::uniform_real_distribution<float> dist(0.0f, 1.0f);
        for (int i = 0; i < n; ++i) key[i] = dkey[i] = (uint32_t)i;
        std::shuffle(key.begin(), key.end(), rng);
        std::shuffle(dkey.begin(), dkey.end(), rng);
        for (int i = 0; i < n; ++i) {
            val[i] = dist(rng);
            dval[i] = dist(rng);
        }
        std::vector<std::pair<uint32_t, float>> kv(n);
        for (int i = 0; i < n; ++i) kv[i] = {key[i], val[i]};
        std::sort(kv.begin(), kv.end(), [](auto &a, auto &b) { return a.first < b.first; });
        std::vector<uint32_t> ek(n);
        std::vector<float> ev(n);
        for (int i = 0; i < n; ++i) {
            ek[i] = kv[i].first;
            ev[i] = kv[i].second;
        }
        dump("sort_pairs_16384_keys_in_u32.bin", key);
        dump("sort_pairs_16384_vals_in_f32.bin", val);
        dump("sort_pairs_16384_keys_expect_u32.bin", ek);
        dump("sort_pairs_16384_vals_expect_f32.bin", ev);
        // SortPairsDescending on the second stream (:220-231, 244-248)
        std::vector<std::pair<uint32_t, float>> dkv(n);
        for (int i = 0; i < n; ++i) dkv[i] = {dkey[i], dval[i]};
        std::sort(dkv.begin(), dkv.end(), [](auto &a, auto &b) { return a.first > b.first; });
        for (int i = 0; i < n; ++i) {
            ek[i] = dkv[i].first;
            ev[i] = dkv[i].second;
        }
        dump("sort_pairs_desc_16384_keys_in_u32.bin", dkey);
        dump("sort_pairs_desc_16384_vals_in_f32.bin", dval);
        dump("sort_pairs_desc_16384_keys_expect_u32.bin", ek);
        dump("sort_pairs_desc_16384_vals_expect_f32.bin", ev);
    }
    return 0;
}
