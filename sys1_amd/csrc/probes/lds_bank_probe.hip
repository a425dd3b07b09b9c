// Measurement probe, not part of libsys1hip: LDS bank conflicts of 16-byte
// per-lane operand-read patterns on gfx950.  The reads go through a volatile
// generic pointer, which compiles to flat_load_dwordx4 on LDS addresses (not
// ds_read_b128); the patterns that the production and probe GEMMs use were
// also counted with ds_read_b128 in those kernels, with the same verdicts.
// Each dispatch makes every
// lane of 256 workgroups read 16 bytes at a per-lane LDS byte offset (a table
// computed on the host, one table per dispatch) 256 times; rocprofv3 counts
// SQ_LDS_BANK_CONFLICT and SQ_INSTS_LDS per dispatch, and their ratio is the
// conflict cycles per read instruction.  Dispatch i prints its pattern's name
// as line "i name".
//
//   hipcc --offload-arch=gfx950 -O3 sys1_amd/csrc/probes/lds_bank_probe.hip -o /tmp/lds_bank_probe
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS --output-format csv -d <dir> -o p -- /tmp/lds_bank_probe
//
// Patterns: the contiguous 1 KB read; 128-byte rows (64 k values) with chunk
// c of row r at position c ^ ((r ^ r / 8) & 7) read as 32 x 32 x 16 operands
// (lanes 0-31: rows 0-31 of chunk 0, lanes 32-63: chunk 1) and as 16 x 16 x 32
// operands (lane l: row l % 16, chunk l / 16, or the chunk order 0, 2, 1, 3);
// 64-byte rows (32 k values) read as 16 x 16 x 32 operands under the swizzles
// ((r >> a) ^ (r >> b)) & 3 (a = b: (r >> a) & 3), with either chunk order.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <vector>
#include <string>
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
// Each lane reads 16 B at LDS byte offset tab[lane], 256 times.
__global__ __launch_bounds__(256) void probe(const int* tab, int* out) {
  __shared__ __attribute__((aligned(1024))) i32x4 lds[2048];
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 2048; i += 256) lds[i] = i32x4{i, i, i, i};
  __syncthreads();
  const int off = tab[lane];
  i32x4 acc = {0, 0, 0, 0};
  const char* p = reinterpret_cast<const char*>(lds) + off;
  for (int it = 0; it < 256; ++it) {
    i32x4 v = *(volatile const i32x4*)p;
    acc[0] ^= v[0]; acc[1] += v[1]; acc[2] ^= v[2]; acc[3] += v[3];
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}
#define CK(x)                                                               \
  do {                                                                      \
    hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                 \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(1);                                                              \
    }                                                                       \
  } while (0)
int main() {
  std::vector<std::vector<int>> tabs; std::vector<std::string> names;
  auto add = [&](std::string n, std::vector<int> t) { names.push_back(n); tabs.push_back(t); };
  std::vector<int> t(64);
  // 128 B rows, f(r) = (r ^ r>>3) & 7
  auto f8 = [](int r) { return (r ^ (r >> 3)) & 7; };
  for (int l = 0; l < 64; ++l) t[l] = l * 16; add("P0 contiguous", t);
  for (int l = 0; l < 64; ++l) { int r = l & 31, c = l >> 5; t[l] = r * 128 + ((c ^ f8(r)) << 4); } add("R128 32x32", t);
  for (int l = 0; l < 64; ++l) { int r = l & 15, q = l >> 4; t[l] = r * 128 + ((q ^ f8(r)) << 4); } add("R128 16x16 q", t);
  for (int l = 0; l < 64; ++l) { int r = l & 15, q = l >> 4; int c = ((q & 1) << 1) | (q >> 1); t[l] = r * 128 + ((c ^ f8(r)) << 4); } add("R128 16x16 perm", t);
  // 64 B rows with f(r) = ((r >> a) ^ (r >> b)) & 3 (a < b) or (r >> a) & 3
  for (int a = 0; a < 4; ++a)
    for (int b = a; b < 6; ++b)
      for (int perm = 0; perm < 2; ++perm) {
        auto f4 = [&](int r) { return b == a ? (r >> a) & 3 : ((r >> a) ^ (r >> b)) & 3; };
        for (int l = 0; l < 64; ++l) {
          int r = l & 15, q = l >> 4;
          int c = perm ? (((q & 1) << 1) | (q >> 1)) : q;
          t[l] = r * 64 + ((c ^ f4(r)) << 4);
        }
        add("R64 16x16 a" + std::to_string(a) + " b" + std::to_string(b) + " perm" + std::to_string(perm), t);
      }
  // 64 B rows, 16x16, rows 16..31 (second block) with (r ^ r>>2)
  for (int l = 0; l < 64; ++l) { int r = 16 + (l & 15), q = l >> 4; t[l] = r * 64 + ((q ^ ((r ^ (r >> 2)) & 3)) << 4); } add("R64 16x16 rows16-31 a0b2", t);
  int* dt; CK(hipMalloc(&dt, 64 * 4)); int* o; CK(hipMalloc(&o, 256 * 256 * 4));
  for (size_t i = 0; i < tabs.size(); ++i) {
    CK(hipMemcpy(dt, tabs[i].data(), 256, hipMemcpyHostToDevice));
    probe<<<256, 256>>>(dt, o);
    CK(hipDeviceSynchronize());
    printf("%zu %s\n", i, names[i].c_str());
  }
}
