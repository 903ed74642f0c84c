// san_readers.cpp -- runs the host code that reads untrusted files (model
// GGUFs and .oikv state files) over a list of files, for a build under
// AddressSanitizer and UndefinedBehaviorSanitizer (Makefile beside this file).
//
//   san_readers gguf FILE...
//       per file: the product's GGUF reader (GgufFile::open; every accepted
//       tensor's first and last byte read, and each matrix repacked into the
//       device layout on the host, as the upload does), the product's model loader
//       oi_engine_load (it parses and checks everything before it looks for a
//       device, so on a machine without one an accepted model ends in
//       OI_E_DEVICE), and the oracle's ref_engine_load followed by one
//       forward step when it accepts the file.
//   san_readers oikv MODEL GOOD FILE...
//       GOOD is a valid state file of MODEL; its header stands for the
//       engine's own.  Per file: the product's oikv_open_checked, and the
//       oracle's ref_engine_load_kv on MODEL.
//
// Prints one line per file, "<rc product> <rc oracle> <file>"; the exit
// status is 0 unless a sanitizer stops the process (it aborts on the first
// report: -fno-sanitize-recover=all).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>

#include "engine_internal.h"
#include "gguf.h"
#include "oi.h"
#include "oikv.h"

extern "C" {
void *ref_engine_load(const char *path, int max_ctx, int num_threads, int kv_f16);
void ref_engine_destroy(void *h);
const float *ref_engine_forward(void *h, int token, int pos);
int ref_engine_load_kv(void *h, const char *path);
}

// Reads every accepted tensor's first and last byte, and repacks each matrix
// of a device type into the device layout as the weight upload does.
static unsigned touch_tensors(const oi::GgufFile &g) {
    unsigned acc = 0;
    std::vector<uint8_t> stage;
    for (const auto &t : g.tensors()) {
        if (!t.nbytes) continue;
        const volatile uint8_t *p = t.data;
        acc += p[0] + p[t.nbytes - 1];
        const uint32_t k = t.kind;
        if (k == 0 || k == 1 || k == 2 || k == 3 || k == 6 || k == 7 || k == 8 || k == 12 || k == 14) {
            const int64_t cols = (int64_t)t.dims[0], rows = (int64_t)(t.nelems() / t.dims[0]);
            if (oi::repack_matrix_host(k, t.data, rows, cols, stage) == OI_OK && !stage.empty()) acc += stage[0];
        }
    }
    return acc;
}

static int run_gguf(int n, char **files) {
    for (int i = 0; i < n; i++) {
        const char *path = files[i];
        oi::GgufFile g;
        std::string err;
        int rc = g.open(path, err);
        if (rc == 0) (void)touch_tensors(g);
        oi_opts o;
        memset(&o, 0, sizeof o);
        o.max_ctx = 64;
        o.num_threads = 1;
        o.use_hip = 1;
        oi_engine *e = nullptr;
        int prc = oi_engine_load(path, &o, &e);
        if (e) oi_engine_destroy(e);
        void *h = ref_engine_load(path, 64, 1, 1);
        int orc = h ? 0 : -1;
        if (h) {
            orc = ref_engine_forward(h, 0, 0) ? 0 : -2;
            ref_engine_destroy(h);
        }
        printf("%d %d %d %s\n", rc == 0 ? prc : rc, orc, rc, path);
    }
    return 0;
}

static int run_oikv(const char *model, const char *good, int n, char **files) {
    FILE *gf = fopen(good, "rb");
    if (!gf) {
        fprintf(stderr, "cannot open %s\n", good);
        return 2;
    }
    uint8_t hb[oi::OIKV_HEADER_BYTES];
    if (fread(hb, 1, sizeof hb, gf) != sizeof hb) {
        fprintf(stderr, "short %s\n", good);
        fclose(gf);
        return 2;
    }
    fclose(gf);
    const oi::OikvHeader mine = oi::oikv_decode(hb);
    void *h = ref_engine_load(model, (int)mine.seq_len, 1, 0);
    if (!h) {
        fprintf(stderr, "oracle cannot load %s\n", model);
        return 2;
    }
    for (int i = 0; i < n; i++) {
        FILE *f = fopen(files[i], "rb");
        int prc = OI_E_IO;
        if (f) {
            oi::OikvHeader fh;
            std::string msg;
            prc = oi::oikv_open_checked(f, mine, fh, msg);
            fclose(f);
        }
        int orc = ref_engine_load_kv(h, files[i]);
        printf("%d %d %s\n", prc, orc, files[i]);
    }
    ref_engine_destroy(h);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && !strcmp(argv[1], "gguf")) return run_gguf(argc - 2, argv + 2);
    if (argc >= 4 && !strcmp(argv[1], "oikv")) return run_oikv(argv[2], argv[3], argc - 4, argv + 4);
    fprintf(stderr, "usage: san_readers gguf FILE... | san_readers oikv MODEL GOOD FILE...\n");
    return 2;
}
