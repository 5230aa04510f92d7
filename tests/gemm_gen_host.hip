// Host harness for tests/test_gemm_gen_formats.py.
//   gemm_gen_host DTYPE N K IN_GGUF_BYTES OUT_F16
// runs gemm_gen.hip's per-format load + dequant policies on the host, over
// a weight relaid out exactly as the library uploads it, and writes the
// binary16 weights the GEMM would put in its LDS tile (row-major [n][k]).
//   gemm_gen_host sched NCHUNKS
// runs the kernel's chunk pipeline (gen_pipeline, with the kernel's DEPTH
// and CPB) and prints its operations, one per line: "S" (barrier),
// "L slot chunk", "M chunk buf", "T slot chunk buf" (store).
//   gemm_gen_host pairs DTYPE N K IN_GGUF_BYTES OUT
// writes the binary16 {scale, bias} pairs the upload forms for the nibble
// GEMM (Q4_K / Q5_K: 8 per super-block, Q6_K: 16), [row][super-block][pair],
// 4 bytes each, read from the relaid-out weight.
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
    const bool pairs = argc == 7 && std::strcmp(argv[1], "pairs") == 0;
    if (pairs) {
        argv++;
        argc--;
    }
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
    if (pairs) {
        const size_t nsb = k / 256, np = dt == T_Q6_K ? 16 : 8;
        std::vector<uint8_t> pr(n * nsb * np * 4);
        for (size_t r = 0; r < n; r++)
            for (size_t sb = 0; sb < nsb; sb++)
                for (size_t j = 0; j < np; j++) {
                    const uint8_t *src_p =
                        dt == T_Q6_K ? dev.data() + (r >> 6) * w.group_stride + sb * IL64_Q6K_SB + IL64_Q6K_P +
                                           (j * 64 + (r & 63)) * 4
                                     : dev.data() + r * w.row_stride + w.plane4 + 32 * sb + 4 * j;
                    std::memcpy(pr.data() + ((r * nsb + sb) * np + j) * 4, src_p, 4);
                }
        f = fopen(argv[5], "wb");
        if (!f) return 6;
        fwrite(pr.data(), 1, pr.size(), f);
        fclose(f);
        return 0;
    }
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
