// MFMA f32_32x32x16_f16 rounding probe: test t gives a[16], b[16] (fp16) and
// c (fp32); every row of A is a, every column of B is b and every C element
// c, so each output is c + sum_k a_k b_k as the matrix core computes it.
// One wave per test; lane 0 writes D[0]; flag[t] = 1 if the 16 outputs of
// lane 0 and of lane 63 disagree (they should all be equal).
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__global__ void probe(const _Float16* a, const _Float16* b, const float* c, float* d, int* flag, int n)
{
    const int t = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (t >= n) return;
    const int lane = threadIdx.x % 64;
    half8 av, bv;
    for (int j = 0; j < 8; ++j) {
        av[j] = a[t * 16 + 8 * (lane / 32) + j];
        bv[j] = b[t * 16 + 8 * (lane / 32) + j];
    }
    floatx16 cv;
    for (int j = 0; j < 16; ++j) cv[j] = c[t];
    floatx16 dv = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, cv, 0, 0, 0);
    int bad = 0;
    for (int j = 1; j < 16; ++j) bad |= __float_as_uint(dv[j]) != __float_as_uint(dv[0]);
    if (lane == 0) d[t] = dv[0];
    if (lane == 63 && bad) flag[t] = 1;
    if (lane == 0 && bad) flag[t] = 1;
}

int main(int argc, char** argv)
{
    if (argc != 3) { fprintf(stderr, "usage: probe in.bin out.bin\n"); return 2; }
    FILE* f = fopen(argv[1], "rb");
    if (!f) { perror(argv[1]); return 2; }
    int n = 0;
    if (fread(&n, 4, 1, f) != 1 || n <= 0 || n > (1 << 24)) { fprintf(stderr, "bad n\n"); return 2; }
    std::vector<_Float16> a(16 * (size_t)n), b(16 * (size_t)n);
    std::vector<float> c(n), d(n);
    std::vector<int> flag(n, 0);
    if (fread(a.data(), 2, a.size(), f) != a.size() || fread(b.data(), 2, b.size(), f) != b.size() ||
        fread(c.data(), 4, c.size(), f) != c.size()) { fprintf(stderr, "short file\n"); return 2; }
    fclose(f);
    _Float16 *da, *db; float *dc, *dd; int* df;
    if (hipMalloc(&da, a.size() * 2) || hipMalloc(&db, b.size() * 2) || hipMalloc(&dc, n * 4) ||
        hipMalloc(&dd, n * 4) || hipMalloc(&df, n * 4)) { fprintf(stderr, "malloc\n"); return 1; }
    hipMemcpy(da, a.data(), a.size() * 2, hipMemcpyHostToDevice);
    hipMemcpy(db, b.data(), b.size() * 2, hipMemcpyHostToDevice);
    hipMemcpy(dc, c.data(), n * 4, hipMemcpyHostToDevice);
    hipMemcpy(df, flag.data(), n * 4, hipMemcpyHostToDevice);
    const int waves = 4;
    probe<<<(n + waves - 1) / waves, 64 * waves>>>(da, db, dc, dd, df, n);
    if (hipDeviceSynchronize() != hipSuccess) { fprintf(stderr, "kernel failed\n"); return 1; }
    hipMemcpy(d.data(), dd, n * 4, hipMemcpyDeviceToHost);
    hipMemcpy(flag.data(), df, n * 4, hipMemcpyDeviceToHost);
    int nbad = 0;
    for (int i = 0; i < n; ++i) nbad += flag[i];
    FILE* o = fopen(argv[2], "wb");
    fwrite(d.data(), 4, n, o);
    fclose(o);
    printf("probe: %d tests, %d with unequal outputs\n", n, nbad);
    return 0;
}
