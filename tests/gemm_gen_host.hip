// Host harness for tests/test_gemm_gen_formats.py.
//   gemm_gen_host DTYPE N K IN_GGUF_BYTES OUT_F16
// runs gemm_gen.hip's per-format load + dequant policies on the host, over
// a weight relaid out exactly as the library uploads it, and writes the
// binary16 weights the GEMM would put in its LDS tile (row-major [n][k]).
//   gemm_gen_host sched NCHUNKS
// runs the kernel's chunk pipeline (gen_pipeline, with the kernel's DEPTH
// and CPB) and prints its operations, one per line: "S" (barrier),
// "L slot chunk", "M chunk buf", "T slot chunk buf" (store).
#include "../rce_amd/csrc/gemm_gen.hip"

#include <cstdio>
#include <cstring>
#include <vector>

using namespace rce_qmm;

template <class F>
static void run(const DevWeight &w, uint16_t *out) {
    const int nch = (int)(w.n_cols / 64);
    for (size_t r = 0; r < w.n_rows; r++)
        for (int c = 0; c < nch; c++)
            for (int o = 0; o < 8; o++) {
                typename F::Raw raw;
                F::load(raw, w, r, c, o);
                const half8 h = F::dequant(raw, c, o);
                std::memcpy(out + r * w.n_cols + 64 * c + 8 * o, &h, 16);
            }
}

static int sched(int nchunks) {
    gen_pipeline<DEPTH, CPB>(
        nchunks, [] { std::printf("S\n"); }, [](int slot, int ch) { std::printf("L %d %d\n", slot, ch); },
        [](int ch, int buf) { std::printf("M %d %d\n", ch, buf); },
        [](int slot, int ch, int buf) { std::printf("T %d %d %d\n", slot, ch, buf); });
    std::printf("E %d %d\n", DEPTH, CPB);
    return 0;
}

int main(int argc, char **argv) {
    if (argc == 3 && std::strcmp(argv[1], "sched") == 0) return sched(atoi(argv[2]));
    if (argc != 6) return 2;
    const uint32_t dt = (uint32_t)atoi(argv[1]);
    const size_t n = (size_t)atol(argv[2]), k = (size_t)atol(argv[3]);
    FILE *f = fopen(argv[4], "rb");
    if (!f) return 3;
    std::vector<uint8_t> src;
    uint8_t buf[65536];
    size_t got;
    while ((got = fread(buf, 1, sizeof buf, f)) > 0) src.insert(src.end(), buf, buf + got);
    fclose(f);
    DevWeight w{};
    w.dtype = dt;
    w.n_rows = n;
    w.n_cols = k;
    const size_t bytes = plan_layout(w);
    if (bytes == 0) return 4;
    std::vector<uint8_t> dev(bytes + layout_pad_bytes(w), 0);
    relayout_host(src.data(), w, dev.data());
    w.base = dev.data();
    std::vector<uint16_t> out(n * k);
    switch (dt) {
    case T_Q8_0: run<FQ8_0>(w, out.data()); break;
    case T_Q5_0: run<FQ32<1>>(w, out.data()); break;
    case T_Q4_1: run<FQ32<2>>(w, out.data()); break;
    case T_Q4_0: run<FQ32<0>>(w, out.data()); break;
    case T_F16: run<FF16>(w, out.data()); break;
    case T_Q5_K: run<FQK<true>>(w, out.data()); break;
    case T_Q4_K: run<FQK<false>>(w, out.data()); break;
    case T_Q6_K: run<FQ6_K>(w, out.data()); break;
    default: return 5;
    }
    f = fopen(argv[5], "wb");
    if (!f) return 6;
    fwrite(out.data(), 2, n * k, f);
    fclose(f);
    return 0;
}
