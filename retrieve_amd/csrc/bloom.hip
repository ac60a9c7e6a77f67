// Bloom index over bit-sliced 2048-doc bundles: build, and the plan search that turns a batch of
// AND/OR/NOT term expressions into the scans' packed mask.
//
// Layout (bloom_indexer.cpp:79-110): bundle beta = d / 2048 is w_beta = off[beta+1] - off[beta]
// bits per doc; bit position p of doc d is word (off[beta] + p) * 32 + (d % 2048) / 64, bit
// 63 - d % 64. So word (off[beta] + p) * 32 + j holds position p of the 64 docs of global column
// 32 beta + j, in the bit order of the scans' mask words.
//
// Terms: a token (feature id f, value v) hashes to murmur(f, v, seed) = h1 ^ h2 of
// MurmurHash3_x64_128 (Austin Appleby's published algorithm, public domain) over the 16-byte
// key f || v (little-endian words), seeds 0, 1, ... (bloom_index_util.cuh:60-107). Build: the
// first k distinct hash % w_beta over seeds 0, 1, ... (:185-208). Search: the first k distinct
// hash % w_beta among the hash_k stored hashes (bloom_index_search_cuda.cu:305-349); a term
// holds for a doc iff all its positions are set.
//
// Build: one wave per 64-doc column (lane <-> doc). Each lane gathers its doc's positions into
// a bit mask; position p of the column is then one ballot, bit-reversed, written once by lane
// 0 -- every word of the index is written exactly once, with no atomics and no clearing pass.
//
// Plans (the parser's encoding, retrieve_amd/bloom.py): per plan 8 byte offsets [ops, offsets,
// parameters, hashes] x [begin, end) into the data, each segment 8-aligned; ops are uint8
// AND=1 OR=2 NOT=3 TERM=4 EMPTY=5 in post-order (bloom_index_util.h:49-56), offsets int32 [ops
// + 1] (parameter ranges: AND/OR take offsets[j+1] - offsets[j] children), hashes uint64
// [terms * hash_k] in the order the terms appear. Search: lane <-> column, a workgroup loops over
// its plans (wave-uniform instruction stream), the evaluation stack lives in LDS. When every
// bundle has the same width a resolve pass first turns each term's stored hashes into its k
// positions once, so the column pass does no 64-bit division.
#include "bloom_prog.h"
#include "rt_common.h"

namespace rt {

constexpr int kBloomDocsPerBundle = 2048;
constexpr int kBloomWordsPerBundle = 32;
constexpr int kBloomMaxK = 10;            // positions per term (MAX_K_V2)
constexpr int kBloomMaxBuildWidth = 256;  // bits per doc the build keeps in registers
constexpr int kBloomMaxStack = 64;
constexpr int kBloomThreads = 256;
constexpr int kBloomMaxSeeds = 4096;  // build: bound on the seeds tried for k distinct positions
static_assert(kColPosBytes == kBloomWordsPerBundle * sizeof(uint64_t), "a position's column words");

enum BloomOp : uint8_t { kOpAnd = 1, kOpOr = 2, kOpNot = 3, kOpTerm = 4, kOpEmpty = 5 };

__host__ __device__ inline uint64_t rotl64(uint64_t x, int r) {
  return (x << r) | (x >> (64 - r));
}

__host__ __device__ inline uint64_t fmix64(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

// MurmurHash3_x64_128 of the one 16-byte block x || y, folded h1 ^ h2.
__host__ __device__ inline uint64_t murmur_2x64(uint64_t x, uint64_t y, uint64_t seed) {
  const uint64_t c1 = 0x87c37b91114253d5ull;
  const uint64_t c2 = 0x4cf5ad432745937full;
  uint64_t h1 = seed;
  uint64_t h2 = seed;
  uint64_t k1 = x * c1;
  k1 = rotl64(k1, 31);
  k1 *= c2;
  h1 ^= k1;
  h1 = rotl64(h1, 27);
  h1 += h2;
  h1 = h1 * 5 + 0x52dce729;
  uint64_t k2 = y * c2;
  k2 = rotl64(k2, 33);
  k2 *= c1;
  h2 ^= k2;
  h2 = rotl64(h2, 31);
  h2 += h1;
  h2 = h2 * 5 + 0x38495ab5;
  h1 ^= 16;
  h2 ^= 16;
  h1 += h2;
  h2 += h1;
  h1 = fmix64(h1);
  h2 = fmix64(h2);
  h1 += h2;
  h2 += h1;
  return h1 ^ h2;
}

// ---- build --------------------------------------------------------------------------------

// max over the bundle's docs of the doc's value count (all features). One workgroup per bundle.
__global__ void __launch_bounds__(kBloomThreads) bloom_terms_kernel(const int64_t* fo, int64_t N,
                                                                    int C, int64_t* max_terms) {
  __shared__ int64_t red[kBloomThreads / kWave];
  const int64_t beta = blockIdx.x;
  int64_t m = 0;
  for (int i = threadIdx.x; i < kBloomDocsPerBundle; i += kBloomThreads) {
    const int64_t d = beta * kBloomDocsPerBundle + i;
    if (d < N) {
      const int64_t t = fo[(d + 1) * C] - fo[d * C];
      m = t > m ? t : m;
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int64_t o = __shfl_xor(m, off);
    m = o > m ? o : m;
  }
  if (lane_id() == 0) red[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBloomThreads / kWave; ++w) m = red[w] > m ? red[w] : m;
    max_terms[beta] = m;
  }
}

struct BloomBuildArgs {
  const int32_t* feature_ids;  // [C]
  int C;
  const int64_t* fo;  // [N * C + 1] value ranges per (doc, feature)
  const int64_t* values;
  int64_t N;
  const int64_t* bundle_off;  // [nb + 1]
  int k;
  uint64_t* words;
};

// grid covers every doc slot of every bundle (nb * 2048), so the words of columns past the last
// doc are written too (as zeros)
__global__ void __launch_bounds__(kBloomThreads) bloom_build_kernel(BloomBuildArgs a) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kBloomThreads + threadIdx.x;
  const int lane = lane_id();
  const int64_t beta = d / kBloomDocsPerBundle;
  const int j = static_cast<int>((d % kBloomDocsPerBundle) / 64);
  const int64_t off = a.bundle_off[beta];
  const int64_t w = a.bundle_off[beta + 1] - off;  // the same for the whole wave
  uint64_t pm[kBloomMaxBuildWidth / 64] = {0ull, 0ull, 0ull, 0ull};
  if (d < a.N && w > 0) {
    const uint64_t uw = static_cast<uint64_t>(w);
    for (int c = 0; c < a.C; ++c) {
      const uint64_t f = static_cast<uint64_t>(static_cast<int64_t>(a.feature_ids[c]));
      const int64_t i1 = a.fo[d * a.C + c + 1];
      for (int64_t i = a.fo[d * a.C + c]; i < i1; ++i) {
        const uint64_t v = static_cast<uint64_t>(a.values[i]);
        int got = 0;
        uint32_t pos[kBloomMaxK];
        for (int seed = 0; got < a.k && seed < kBloomMaxSeeds; ++seed) {
          const uint32_t p = static_cast<uint32_t>(murmur_2x64(f, v, seed) % uw);
          bool dup = false;
          for (int q = 0; q < got; ++q) dup |= pos[q] == p;
          if (!dup) {
            pos[got++] = p;
            const uint64_t bit = 1ull << (p & 63);
            // (a select per slot keeps pm in registers)
#pragma unroll
            for (int s = 0; s < kBloomMaxBuildWidth / 64; ++s) pm[s] |= (p >> 6) == s ? bit : 0ull;
          }
        }
      }
    }
  }
  for (int64_t p = 0; p < w; ++p) {
    const uint64_t m = pm[p >> 6];
    const uint64_t word = __builtin_bitreverse64(__ballot((m >> (p & 63)) & 1ull));
    if (lane == 0) a.words[(off + p) * kBloomWordsPerBundle + j] = word;
  }
}

// ---- search -------------------------------------------------------------------------------

struct BloomSearchArgs {
  const uint64_t* words;
  const int64_t* bundle_off;  // [nb + 1]
  int64_t nb;
  const int64_t* plan_offsets;  // [plan_count, 8] byte offsets into data
  const int8_t* data;
  int64_t data_bytes;
  int64_t plan_count;
  int64_t plans_per_wg;
  int max_stack;
  int k;
  int hash_k;
  bool words_aligned16;
  const int32_t* hdr;    // [plan_count, 4] from the prep pass: PlanStatus, ops, hash word 0
  const uint32_t* prog;   // [plan_count, kProgMaxOps, 2] program words
  // clause mode (see "Clauses" below): the batch's distinct clauses and the plans over them
  const uint32_t* clause_ptr;    // [n_clauses + 1]: clause c's terms are entries [ptr[c], ptr[c+1])
  const uint32_t* clause_terms;  // [*, 4]: a term's program word pair, its hashes' index lo / hi
  const uint32_t* plan_desc;     // [plan_count]: bit 31 a clause plan, bits 12-30 its first
                                 // ref, bits 0-11 its ref count; 0: the plan runs its program
  const uint32_t* plan_refs;     // bits 0-14 a clause, bit 15 NOT
  int n_clauses;                 // 0: every plan runs its program
  bool all_clauses;              // every plan is a clause plan (none runs a program)
  int64_t* out_mask;      // [plan_count, nb * 32] or null
  uint8_t* out_bool;      // [plan_count, nb * 32 * 64] or null
  uint64_t* out_mask_t;   // [nb * 32, out_t_stride]: the words transposed, or null
  int64_t out_t_stride;
};

// The first k distinct hash % w among a term's stored hashes (fewer if they do not hold k).
__device__ inline int resolve_positions(const uint64_t* h, int hash_k, int k, uint64_t w,
                                        uint32_t (&pos)[kBloomMaxK]) {
  int got = 0;
  for (int s = 0; s < hash_k && got < k; ++s) {
    const uint32_t p = static_cast<uint32_t>(h[s] % w);
    bool dup = false;
    for (int q = 0; q < got; ++q) dup |= pos[q] == p;
    if (!dup) pos[got++] = p;
  }
  return got;
}

// A plan's offsets are inside the data, ordered, and aligned for their element types.
__device__ inline bool plan_ok(const int64_t* o, int64_t data_bytes) {
  bool ok = true;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    ok &= o[2 * s] >= 0 && o[2 * s] <= o[2 * s + 1] && o[2 * s + 1] <= data_bytes;
  }
  return ok && (o[2] % 4) == 0 && (o[4] % 4) == 0 && (o[6] % 8) == 0;
}

// One plan's result word for this lane's column, in the mask layout and/or as 64 bytes.
__device__ inline void write_column(const BloomSearchArgs& a, int64_t b, int64_t ncol,
                                    int64_t col, uint64_t res) {
  // through global-address-space views: counted in vmcnt only (flat stores also hold lgkmcnt,
  // which the evaluation's LDS waits would then wait on)
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(1))) int64_t gi64;
  typedef __attribute__((address_space(1))) u32x4 gu4;
  if (a.out_mask != nullptr) {
    gi64* om = (gi64*)(a.out_mask);
    om[b * ncol + col] = static_cast<int64_t>(res);
  }
  if (a.out_mask_t != nullptr) {
    // (a workgroup takes a run of consecutive plans over its columns: their words of a column
    // share lines, which fill in L2 before they are written back)
    gi64* ot = (gi64*)(a.out_mask_t);
    ot[col * a.out_t_stride + b] = static_cast<int64_t>(res);
  }
  if (a.out_bool != nullptr) {
    // 64 bytes per column, doc 64 col + q at byte q (bit 63 - q of the word)
    gu4* ob = (gu4*)(a.out_bool + (b * ncol + col) * 64);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u32x4 x;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        uint32_t y = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int q = 16 * v + 4 * u + t;
          y |= static_cast<uint32_t>((res >> (63 - q)) & 1ull) << (8 * t);
        }
        x[u] = y;
      }
      ob[v] = x;
    }
  }
}

// ---- plan prep: a program for the column kernel ----------------------------------------
//
// The program format is bloom_prog.h's.
//
// Clauses: a batch's plans are mostly ANDs of value-set clauses (an OR of terms, a term, or the
// NOT of either), and plans repeat clauses (a popular value set). A host pass over the compiled
// programs (retrieve_amd/st.py) finds the plans of that form and the batch's distinct clauses
// (the same set of stored hash lists: the same word in every column, whatever the bundle's
// width). The column kernel's CLAUSES form evaluates each distinct clause once per column into
// LDS, and such a plan is the AND of a few LDS words; the other plans run their programs.
constexpr int kMaxClauses = 128;  // LDS: 128 clauses x 64 columns x 8 bytes beside the staging
// rt_bloom_search_compiled's plan_flags
constexpr int64_t kPlansAllClauses = 1;  // every plan is a clause plan
constexpr int64_t kPlansNoStack = 2;     // no plan takes the stack evaluation
constexpr int kPrepThreads = 256;

// A plan's header: its status, op count and first hash word, one 16-byte load for the column
// kernel (whose program slot sits at a fixed place, so nothing waits on the plan's offsets).
__device__ inline void write_header(int32_t* hdr, int64_t b, int32_t status, int32_t n_ops,
                                    int64_t h0) {
  int32_t* h = hdr + 4 * b;
  h[0] = status;
  h[1] = n_ops;
  h[2] = static_cast<int32_t>(h0);
  h[3] = static_cast<int32_t>(h0 >> 32);
}

// Block-wide exclusive prefix sum of one value per thread (every thread calls it); total gets
// the sum over the block. tmp: kPrepThreads / kWave ints of LDS.
__device__ inline int prep_scan_excl(int v, int* tmp, int& total) {
  const int lane = lane_id();
  const int w = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off);
    x += lane >= off ? y : 0;
  }
  if (lane == kWave - 1) tmp[w] = x;
  __syncthreads();
  int base = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < kPrepThreads / kWave; ++i) {
    base += i < w ? tmp[i] : 0;
    total += tmp[i];
  }
  __syncthreads();
  return base + x - v;
}

// Block-wide maximum (every thread calls it).
__device__ inline int prep_max(int v, int* tmp) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int y = __shfl_xor(v, off);
    v = y > v ? y : v;
  }
  if (lane_id() == 0) tmp[threadIdx.x / kWave] = v;
  __syncthreads();
  int m = tmp[0];
#pragma unroll
  for (int i = 1; i < kPrepThreads / kWave; ++i) m = tmp[i] > m ? tmp[i] : m;
  __syncthreads();
  return m;
}

// One workgroup per plan. The stack check (the stack evaluation's, recording each node's parent
// and first child) is a single pass of one thread over LDS copies of the ops and child counts;
// the flattening, the places, the term numbering and the folded depth are computed by the whole
// workgroup (a walk up the parent links per op, block prefix sums).
__global__ void __launch_bounds__(kPrepThreads) bloom_prep_kernel(BloomSearchArgs a,
                                                                  int32_t* hdr,
                                                                  uint32_t* prog) {
  __shared__ uint8_t ops[kProgMaxOps];
  __shared__ uint8_t place[kProgMaxOps];
  __shared__ uint8_t flat[kProgMaxOps];        // an AND / OR under a parent of the same operator
  __shared__ int16_t parent[kProgMaxOps];      // -1 for the root
  __shared__ int16_t first_child[kProgMaxOps];
  __shared__ int32_t nchild[kProgMaxOps];      // an AND / OR's child count (offs[i+1] - offs[i])
  __shared__ uint32_t term_pos[kProgMaxOps][2];  // the positions part of each term's words
  __shared__ int32_t stk[kBloomMaxStack];
  __shared__ int32_t red[kPrepThreads / kWave];
  __shared__ int32_t verdict;
  const int64_t b = blockIdx.x;
  const int64_t* o = a.plan_offsets + 8 * b;
  const int tid = threadIdx.x;
  if (!plan_ok(o, a.data_bytes)) {
    if (tid == 0) write_header(hdr, b, kPlanNone, 0, 0);
    return;
  }
  const int64_t n_ops = o[1] - o[0];
  const int64_t nh = (o[7] - o[6]) / 8;
  const int64_t n_terms = nh / a.hash_k;
  const int64_t w0 = a.bundle_off[1] - a.bundle_off[0];
  const int kk = a.k < a.hash_k ? a.k : a.hash_k;
  if (n_ops > kProgMaxOps || w0 < 1 || w0 > kColMaxWidth || kk > kProgMaxPos) {
    if (tid == 0) write_header(hdr, b, kPlanStack, 0, 0);
    return;
  }
  const uint8_t* src = reinterpret_cast<const uint8_t*>(a.data + o[0]);
  const int32_t* offs = reinterpret_cast<const int32_t*>(a.data + o[2]);
  const int64_t n_offs = (o[3] - o[2]) / 4;
  for (int64_t i = tid; i < n_ops; i += kPrepThreads) {
    ops[i] = src[i];
    parent[i] = -1;
    first_child[i] = -1;
    nchild[i] = i + 1 < n_offs ? offs[i + 1] - offs[i] : -1;  // -1: no count (a bad AND / OR)
  }
  const uint64_t* hashes = reinterpret_cast<const uint64_t*>(a.data) + o[6] / 8;
  // a valid plan uses at most n_ops terms (each is an op)
  const int64_t used_terms = n_terms < n_ops ? n_terms : n_ops;
  for (int64_t t = tid; t < used_terms; t += kPrepThreads) {
    uint32_t pos[kBloomMaxK];
    const int got = resolve_positions(hashes + t * a.hash_k, a.hash_k, a.k,
                                      static_cast<uint64_t>(w0), pos);
    uint32_t off[kProgMaxPos];
    for (int q = 0; q < kProgMaxPos; ++q) off[q] = pos[q < got ? q : 0] * kColPosBytes;
    term_pos[t][0] = (off[0] << 4) | (off[1] << 18);
    term_pos[t][1] = off[2] | (off[3] << 16);
  }
  __syncthreads();

  if (tid == 0) {
    // the stack evaluation's checks, recording each node's parent and first child
    bool bad = false;
    int sp = 0;
    int64_t term = 0;
    for (int64_t i = 0; i < n_ops && !bad; ++i) {
      const uint8_t op = ops[i];
      if (op == kOpTerm) {
        if ((term + 1) * a.hash_k > nh) {
          bad = true;
          break;
        }
        ++term;
      } else if (op == kOpAnd || op == kOpOr) {
        const int n = nchild[i];
        if (n < 1 || n > sp) {
          bad = true;
          break;
        }
        for (int q = sp - n; q < sp; ++q) parent[stk[q]] = static_cast<int16_t>(i);
        first_child[i] = static_cast<int16_t>(stk[sp - n]);
        sp -= n;
      } else if (op == kOpNot) {
        if (sp < 1) {
          bad = true;
          break;
        }
        parent[stk[sp - 1]] = static_cast<int16_t>(i);
        first_child[i] = static_cast<int16_t>(stk[sp - 1]);
        sp -= 1;
      } else if (op != kOpEmpty) {
        bad = true;
        break;
      }
      if (sp >= a.max_stack) {
        bad = true;
        break;
      }
      stk[sp++] = static_cast<int32_t>(i);
    }
    verdict = bad || sp != 1 ? 1 : 0;
    if (verdict) write_header(hdr, b, kPlanNone, 0, 0);
  }
  __syncthreads();
  if (verdict) return;

  // An AND / OR under a parent of the same operator is flattened into it (associativity): its
  // first child takes its place and it becomes a no-op, so nested fan-out-limited ORs of a long
  // value set fold at one level.
  for (int64_t i = tid; i < n_ops; i += kPrepThreads) {
    const int p = parent[i];
    const uint8_t op = ops[i];
    flat[i] = p >= 0 && (op == kOpAnd || op == kOpOr) && ops[p] == op ? 1 : 0;
  }
  __syncthreads();
  // Places: a first child pushes (or, under a flattened parent, takes the parent's place: walk
  // up); the others fold with their parent's operator.
  for (int64_t i = tid; i < n_ops; i += kPrepThreads) {
    int j = static_cast<int>(i);
    uint8_t where = kPlacePush;
    for (;;) {
      const int p = parent[j];
      if (p < 0 || ops[p] == kOpNot) break;
      if (first_child[p] != j) {
        where = ops[p] == kOpAnd ? kPlaceAnd : kPlaceOr;
        break;
      }
      if (!flat[p]) break;
      j = p;
    }
    place[i] = where;
  }
  __syncthreads();

  // the program: each thread a run of consecutive ops, its first term's number and its depth
  // at entry from block prefix sums; the folded evaluation's depth is the deepest push
  const int chunk = static_cast<int>((n_ops + kPrepThreads - 1) / kPrepThreads);
  const int64_t c0 = static_cast<int64_t>(tid) * chunk;
  const int64_t c1 = c0 + chunk < n_ops ? c0 + chunk : n_ops;
  int my_terms = 0;
  int my_delta = 0;
  int my_kept = 0;
  for (int64_t i = c0; i < c1; ++i) {
    const uint8_t op = ops[i];
    my_terms += op == kOpTerm ? 1 : 0;
    const bool pops = !flat[i] && op != kOpTerm && op != kOpEmpty;  // AND, OR, NOT
    const bool push = !flat[i] && place[i] == kPlacePush;
    my_delta += (push ? 1 : 0) - (pops ? 1 : 0);
    my_kept += flat[i] ? 0 : 1;
  }
  int total = 0;
  int term = prep_scan_excl(my_terms, red, total);
  int depth = prep_scan_excl(my_delta, red, total);
  int kept_total = 0;
  int at = prep_scan_excl(my_kept, red, kept_total);  // the program leaves flattened nodes out
  int deepest = 0;
  uint32_t* out = prog + b * kProgMaxOps * 2;
  for (int64_t i = c0; i < c1; ++i) {
    const uint8_t op = ops[i];
    uint32_t w0w = 0u;
    uint32_t w1w = 0u;
    uint32_t where = place[i];
    if (flat[i]) {
      // a no-op (its children folded into the parent's level): not in the program, so the
      // sibling TERMs on either side stay one run
      continue;
    } else if (op == kOpTerm) {
      w0w = kKindTerm | term_pos[term][0];
      w1w = term_pos[term][1];
    } else if (op == kOpEmpty) {
      w0w = kKindEmpty;
    } else {
      w0w = op == kOpNot ? kKindNot : kKindPass;
      --depth;
    }
    if (op == kOpTerm) ++term;
    if (where == kPlacePush) {
      ++depth;
      deepest = depth > deepest ? depth : deepest;
    }
    out[2 * at] = w0w | (where << 2);
    out[2 * at + 1] = w1w;
    ++at;
  }
  deepest = prep_max(deepest, red);
  if (tid == 0) {
    write_header(hdr, b, deepest <= kFoldDepth ? kPlanProgram : kPlanStack,
                 static_cast<int32_t>(kept_total), o[6] / 8);
  }
}

// ---- column kernel: programs over LDS-staged bundles -------------------------------------
//
// A workgroup stages two bundles (64 columns, 2 * 64 * 32 words = 32 KiB at 64 bits per doc)
// in LDS once; its four (or eight) waves then run the programs of its plans (wave w: plans w,
// w + waves, ...), lane <-> column, the top of the folded stack in a register and the levels
// below it in LDS.
// Every index word leaves HBM once per workgroup. Lanes of a bundle whose width differs from
// bundle 0's resolve their positions from the stored hashes and read HBM.
// Plans per workgroup from which the column kernel runs eight waves instead of four.
constexpr int64_t kColWidePlans = 64;
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// A term from its stored hashes for a bundle of width w (any width the build allows): the AND of
// the words at the first k distinct hash % w. Duplicates are found in a bitmask of the positions
// taken, so nothing here needs an indexed array (or a private stack).
__device__ inline uint64_t term_from_hashes(const BloomSearchArgs& a, int64_t h0, int64_t term,
                                            const uint64_t* wcol, int64_t w) {
  if (w <= 0) return 0ull;  // a bundle with no bits holds no term
  const uint64_t* h = reinterpret_cast<const uint64_t*>(a.data) + h0 + term * a.hash_k;
  uint64_t seen[kBloomMaxBuildWidth / 64] = {0ull, 0ull, 0ull, 0ull};
  uint64_t r = ~0ull;
  int got = 0;
  for (int s = 0; s < a.hash_k && got < a.k; ++s) {
    const uint32_t p = static_cast<uint32_t>(h[s] % static_cast<uint64_t>(w));
    const uint64_t bit = 1ull << (p & 63u);
    uint64_t taken = 0ull;
#pragma unroll
    for (int q = 0; q < kBloomMaxBuildWidth / 64; ++q) taken |= (p >> 6) == q ? seen[q] & bit : 0;
    if (taken == 0ull) {
#pragma unroll
      for (int q = 0; q < kBloomMaxBuildWidth / 64; ++q) seen[q] |= (p >> 6) == q ? bit : 0ull;
      r &= wcol[static_cast<int64_t>(p) * kBloomWordsPerBundle];
      ++got;
    }
  }
  return r;
}

// A value every lane holds alike, moved to scalar registers.
__device__ inline int64_t uniform64(int64_t x) {
  const uint64_t u = static_cast<uint64_t>(x);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Global-memory views (address space 1, reached by C-style casts): loads and stores through them
// count in vmcnt only, not also in lgkmcnt as flat accesses do, so LDS waits do not wait for
// them.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const i32x4 gi32x4;

// The staged column word at byte offset q (a position's p * 256).
__device__ inline uint64_t column_word(const char* lcol, uint32_t q) {
  return *reinterpret_cast<const uint64_t*>(lcol + q);
}

// AND of a term's KK position words from the staged column (the loads issue back to back).
template <int KK>
__device__ inline uint64_t staged_term(const char* lcol, uint32_t w0, uint32_t w1) {
  uint64_t v = column_word(lcol, (w0 >> 4) & 0x3fffu);
  if constexpr (KK > 1) v &= column_word(lcol, w0 >> 18);
  if constexpr (KK > 2) v &= column_word(lcol, w1 & 0x3fffu);
  if constexpr (KK > 3) v &= column_word(lcol, w1 >> 16);
  return v;
}

// The folded stack machine's state over one plan.
struct FoldState {
  uint64_t top;
  int sp;
  int64_t term;
};

// Ops li = 0 .. cnt-1 of a chunk whose words lane li holds (lo, hi): no memory access but LDS.
// STAGED: every lane's bundle is in LDS (the wave takes no per-lane branch); otherwise lanes
// whose bundle is not staged resolve positions from the stored hashes.
//
// Runs: a TERM followed by TERMs that fold into the top with one operator P (OR or AND) are
// siblings under a P node (a folding TERM's previous sibling is the op just before it), so the
// first one's place is push or P. The run is evaluated as v = T0 P T1 P ... and placed once,
// in a loop with no per-op dispatch; its length comes from a ballot over the chunk's words.
template <int KK, bool STAGED>
__device__ inline void run_ops(FoldState& f, uint32_t lo, uint32_t hi, int cnt,
                               const BloomSearchArgs& a, int64_t h0, const char* lcol,
                               bool mine_staged, const uint64_t* wcol, int64_t my_w,
                               uint64_t (&stk)[kFoldDepth - 1][kWave], int lane) {
  auto term_at = [&](int li) -> uint64_t {
    const uint32_t w0 = __builtin_amdgcn_readlane(lo, li);
    const uint32_t w1 = __builtin_amdgcn_readlane(hi, li);
    uint64_t v;
    if (STAGED || mine_staged) {
      v = staged_term<KK>(lcol, w0, w1);
    } else {
      v = term_from_hashes(a, h0, f.term, wcol, my_w);
    }
    ++f.term;
    return v;
  };
  const bool in_chunk = lane < cnt;
  const bool is_term = (lo & 3u) == kKindTerm;
  const uint64_t or_run = __ballot(in_chunk && is_term && ((lo >> 2) & 3u) == kPlaceOr);
  const uint64_t and_run = __ballot(in_chunk && is_term && ((lo >> 2) & 3u) == kPlaceAnd);
  for (int li = 0; li < cnt;) {
    const uint32_t w0 = __builtin_amdgcn_readlane(lo, li);
    const uint32_t kind = w0 & 3u;
    uint64_t v;
    if (kind == kKindTerm) {
      v = term_at(li);
      // the run's continuation: ops li + 1, li + 2, ... that fold with one operator
      const uint64_t ors = li + 1 < kWave ? or_run >> (li + 1) : 0ull;
      const uint64_t ands = li + 1 < kWave ? and_run >> (li + 1) : 0ull;
      const int n_or = static_cast<int>(__builtin_ctzll(~ors));
      const int n_and = static_cast<int>(__builtin_ctzll(~ands));
      int j = li + 1;
      if (n_or > 0) {
        const int end = j + n_or;
        for (; j + 1 < end; j += 2) {
          const uint64_t x = term_at(j);
          const uint64_t y = term_at(j + 1);
          v |= x | y;
        }
        if (j < end) v |= term_at(j++);
      } else if (n_and > 0) {
        const int end = j + n_and;
        for (; j + 1 < end; j += 2) {
          const uint64_t x = term_at(j);
          const uint64_t y = term_at(j + 1);
          v &= x & y;
        }
        if (j < end) v &= term_at(j++);
      }
      li = j;
    } else {
      if (kind == kKindEmpty) {
        v = ~0ull;
      } else {
        v = kind == kKindNot ? ~f.top : f.top;
        --f.sp;
        if (f.sp >= 1) f.top = stk[f.sp - 1][lane];
      }
      ++li;
    }
    const uint32_t where = (w0 >> 2) & 3u;
    if (where == kPlaceOr) {
      f.top |= v;
    } else if (where == kPlaceAnd) {
      f.top &= v;
    } else {
      if (f.sp >= 1) stk[f.sp - 1][lane] = f.top;
      f.top = v;
      ++f.sp;
    }
  }
}

// One plan: its first 64 ops from the prefetched words (lo0, hi0), any further ones loaded here.
template <int KK, bool STAGED>
__device__ inline uint64_t run_program(const BloomSearchArgs& a, gu32* prog, uint32_t lo0,
                                       uint32_t hi0, int n_ops, int64_t h0, const char* lcol,
                                       bool mine_staged, const uint64_t* wcol, int64_t my_w,
                                       uint64_t (&stk)[kFoldDepth - 1][kWave], int lane) {
  FoldState f{0ull, 0, 0};
  run_ops<KK, STAGED>(f, lo0, hi0, n_ops < kWave ? n_ops : kWave, a, h0, lcol, mine_staged,
                      wcol, my_w, stk, lane);
  for (int c0 = kWave; c0 < n_ops; c0 += kWave) {
    const int cnt = n_ops - c0 < kWave ? n_ops - c0 : kWave;
    const uint32_t lo = prog[2 * (c0 + lane)];
    const uint32_t hi = prog[2 * (c0 + lane) + 1];
    run_ops<KK, STAGED>(f, lo, hi, cnt, a, h0, lcol, mine_staged, wcol, my_w, stk, lane);
  }
  return f.top;
}

// KK = min(k, hash_k): the positions every term's program words carry. THREADS: 256, or 512
// when a workgroup has many plans (its bundles' staging then feeds twice the waves).
typedef __attribute__((address_space(4))) const uint32_t kcu32;
typedef __attribute__((address_space(4))) const int64_t kci64;

// Workgroup barrier over LDS only: this wave's LDS accesses done (lgkmcnt(0)), then
// s_barrier. __syncthreads() would also wait for every global load in flight (its workgroup
// release fence), draining the next bundle pair's prefetch; the column kernel's barriers order
// LDS accesses only. The empty asm statements keep the compiler from moving memory accesses
// across it.
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int KK, int THREADS, bool CLAUSES>
__global__ void __launch_bounds__(THREADS) bloom_column_kernel(BloomSearchArgs a) {
  constexpr int kColThreads = THREADS;
  constexpr int kColWaves = THREADS / kWave;
  __shared__ __attribute__((aligned(16))) uint64_t idx[2 * kColMaxWidth * kBloomWordsPerBundle];
  __shared__ uint64_t fold[kColWaves][kFoldDepth - 1][kWave];
  extern __shared__ uint64_t clause_words[];  // CLAUSES: [a.n_clauses][64 columns]
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  // The wave-uniform tables (bundle offsets, clause and plan descriptors) are read through the
  // constant address space: scalar loads, waited for on lgkmcnt, so they do not wait for the
  // next bundle pair's words in flight as vector loads (in-order vmcnt) would.
  kci64* bundle_off = (kci64*)(a.bundle_off);
  kcu32* clause_ptr = (kcu32*)(a.clause_ptr);
  kcu32* clause_terms = (kcu32*)(a.clause_terms);
  kcu32* plan_desc = (kcu32*)(a.plan_desc);
  kcu32* plan_refs = (kcu32*)(a.plan_refs);
  const int64_t w0 = uniform64(bundle_off[1] - bundle_off[0]);
  // A workgroup takes bundle pairs blockIdx.x, + gridDim.x, ...: the next pair's words are
  // loaded into registers while the current one is searched, so the index read's latency hides
  // behind the work (one or two workgroups fit a CU, the clause words' LDS allowing).
  const int64_t n_pairs = (a.nb + 1) / 2;
  const int n_words = static_cast<int>(w0 >= 1 && w0 <= kColMaxWidth ? w0 : 0) *
                      kBloomWordsPerBundle;  // a staged bundle's words
  constexpr int kIt = kColMaxWidth * kBloomWordsPerBundle / 2 / kColThreads;  // 16-byte slots
  // pair p's bundle offsets, and which of its two bundles are staged (their width is bundle
  // 0's, the programs' positions)
  auto geometry = [&](int64_t pair, int64_t(&off)[3], bool(&st)[2]) {
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      off[h] = 2 * pair + h <= a.nb ? uniform64(bundle_off[2 * pair + h]) : 0;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      st[h] = 2 * pair + h < a.nb && off[h + 1] - off[h] == w0 && n_words > 0;
    }
  };
  // every load of both bundles issued before any is used: 16 bytes a load when the index is
  // 16-byte aligned (a bundle starts at a multiple of 256 bytes from it), else two of 8
  auto fetch = [&](const int64_t(&off)[3], const bool(&st)[2], v4u(&pre)[2][kIt]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t* g = a.words + off[h] * kBloomWordsPerBundle;
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int i = tid + it * kColThreads;
        v4u v{0, 0, 0, 0};
        if (st[h] && 2 * i < n_words) {
          if (a.words_aligned16) {
            v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(g) + i);
          } else {
            const uint64_t x = __builtin_nontemporal_load(g + 2 * i);
            const uint64_t y = __builtin_nontemporal_load(g + 2 * i + 1);
            v = v4u{static_cast<uint32_t>(x), static_cast<uint32_t>(x >> 32),
                    static_cast<uint32_t>(y), static_cast<uint32_t>(y >> 32)};
          }
        }
        pre[h][it] = v;
      }
    }
  };
  int64_t pair = blockIdx.x;
  int64_t noff[3];
  bool nst[2];
  v4u pre[2][kIt];
  geometry(pair, noff, nst);
  fetch(noff, nst, pre);
  for (; pair < n_pairs; pair += gridDim.x) {
  const int64_t beta0 = 2 * pair;
  int64_t off[3] = {noff[0], noff[1], noff[2]};
  bool staged[2] = {nst[0], nst[1]};
  lds_barrier();  // every wave is done with the previous pair's LDS
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    v4u* l = reinterpret_cast<v4u*>(idx + h * kColMaxWidth * kBloomWordsPerBundle);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int i = tid + it * kColThreads;
      if (staged[h] && 2 * i < n_words) l[i] = pre[h][it];
    }
  }
  if (pair + gridDim.x < n_pairs) {
    geometry(pair + gridDim.x, noff, nst);
    fetch(noff, nst, pre);
  }
  lds_barrier();

  const int half = lane >> 5;
  const int j = lane & 31;
  const int64_t col = beta0 * kBloomWordsPerBundle + lane;
  const int64_t ncol = a.nb * kBloomWordsPerBundle;
  const bool valid = beta0 + half < a.nb;
  const bool mine_staged = half == 0 ? staged[0] : staged[1];
  // wave-uniform: both bundles staged (or the second absent)
  const bool all_staged =
      __builtin_amdgcn_readfirstlane(staged[0] && (staged[1] || beta0 + 1 >= a.nb)) != 0;
  const char* lcol =
      reinterpret_cast<const char*>(idx + half * kColMaxWidth * kBloomWordsPerBundle + j);
  const int64_t my_off = half == 0 ? off[0] : off[1];
  const int64_t my_w = valid ? (half == 0 ? off[1] - off[0] : off[2] - off[1]) : 0;
  const uint64_t* wcol = a.words + my_off * kBloomWordsPerBundle + j;
  uint64_t(&stk)[kFoldDepth - 1][kWave] = fold[wave];
  const uint64_t* clause_col = clause_words + lane;
  if constexpr (CLAUSES) {
    // the batch's distinct clauses, each once per column (an OR of its terms: from the staged
    // positions, or for a bundle of another width from the terms' stored hashes)
    // The clauses' terms in clause order are split evenly over the waves (clauses differ in
    // length by 10x): a wave ORs each clause segment of its share in registers, four terms at
    // a time, and merges it into the clause's word with one LDS atomic OR.
    const int n_clauses = __builtin_amdgcn_readfirstlane(a.n_clauses);
    for (int i = tid; i < n_clauses * kWave; i += kColThreads) clause_words[i] = 0ull;
    lds_barrier();
    const int n_terms = __builtin_amdgcn_readfirstlane(clause_ptr[n_clauses]);
    const int share = (n_terms + kColWaves - 1) / kColWaves;
    const int t_lo = wave * share;
    const int t_hi = t_lo + share < n_terms ? t_lo + share : n_terms;
    // STAGED: both bundles staged (wave-uniform), so the loop holds no global load whose wait
    // would also wait for the next pair's words in flight
    auto clause_terms_or = [&](auto staged_c) {
      constexpr bool STAGED = decltype(staged_c)::value;
      auto term = [&](int t) -> uint64_t {
        kcu32* e = clause_terms + 4 * static_cast<int64_t>(t);
        const uint32_t p0 = __builtin_amdgcn_readfirstlane(e[0]);
        const uint32_t p1 = __builtin_amdgcn_readfirstlane(e[1]);
        if constexpr (STAGED) {
          return staged_term<KK>(lcol, p0, p1);
        } else {
          const int64_t hidx = static_cast<int64_t>(
              (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(e[3])) << 32) |
              __builtin_amdgcn_readfirstlane(e[2]));
          return mine_staged ? staged_term<KK>(lcol, p0, p1)
                             : term_from_hashes(a, hidx, 0, wcol, my_w);
        }
      };
      int c = 0;
      while (c < n_clauses && __builtin_amdgcn_readfirstlane(clause_ptr[c + 1]) <= t_lo) ++c;
      for (int t = t_lo; t < t_hi; ++c) {
        const int end_c = __builtin_amdgcn_readfirstlane(clause_ptr[c + 1]);
        const int end = end_c < t_hi ? end_c : t_hi;
        uint64_t v = 0ull;
        for (; t + 3 < end; t += 4) {
          const uint64_t x0 = term(t);
          const uint64_t x1 = term(t + 1);
          const uint64_t x2 = term(t + 2);
          const uint64_t x3 = term(t + 3);
          v |= (x0 | x1) | (x2 | x3);
        }
        for (; t < end; ++t) v |= term(t);
        __hip_atomic_fetch_or(&clause_words[c * kWave + lane], v, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    };
    if (all_staged) {
      clause_terms_or(std::true_type{});
    } else {
      clause_terms_or(std::false_type{});
    }
    lds_barrier();
  }

  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * a.plans_per_wg;
  const int64_t b1 = b0 + a.plans_per_wg < a.plan_count ? b0 + a.plans_per_wg : a.plan_count;
  if constexpr (CLAUSES) {
    if (a.all_clauses && a.out_mask_t != nullptr) {
      // Every plan reads the clause table, so the staged bundles are dead: their LDS holds a
      // chunk of 64 plans' words for the 64 columns, swizzled (word p ^ r of row r) so that
      // both the column-wise stores and the row-wise reads are free of bank conflicts. A
      // column's 64 words then leave as one contiguous 512-byte run of the transposed output,
      // instead of 64 scattered 8-byte stores a plan.
      typedef __attribute__((address_space(1))) int64_t gi64;
      gi64* ot = (gi64*)(a.out_mask_t);
      const int64_t col0 = beta0 * kBloomWordsPerBundle;
      for (int64_t c0 = b0; c0 < b1; c0 += kWave) {
        for (int64_t pb = c0 + wave; pb < b1 && pb < c0 + kWave; pb += kColWaves) {
          const uint32_t desc = __builtin_amdgcn_readfirstlane(plan_desc[pb]);
          kcu32* refs = plan_refs + ((desc >> 12) & 0x7ffffu);
          const int cnt = static_cast<int>(desc & 0xfffu);
          uint64_t top = ~0ull;
          for (int r = 0; r < cnt; ++r) {
            const uint32_t ref = __builtin_amdgcn_readfirstlane(refs[r]);
            const uint64_t w = clause_col[(ref & 0x7fffu) * kWave];
            top &= (ref & 0x8000u) != 0u ? ~w : w;
          }
          const int p = static_cast<int>(pb - c0);
          idx[lane * kWave + (p ^ lane)] = top;
        }
        lds_barrier();
        for (int i = tid; i < kWave * kWave; i += kColThreads) {
          const int r = i / kWave;
          const int p = i % kWave;
          if (c0 + p < b1 && col0 + r < ncol) {
            ot[(col0 + r) * a.out_t_stride + c0 + p] = static_cast<int64_t>(idx[r * kWave + (p ^ r)]);
          }
        }
        lds_barrier();
      }
      continue;
    }
  }
  // each plan's header and first 64 program ops are loaded while the plan before it runs (a
  // plan's slot holds kProgMaxOps >= 64 ops, so the loads stay inside it)
  gu32* progs = (gu32*)(a.prog);
  gi32x4* hdrs = (gi32x4*)(a.hdr);
  int64_t b = b0 + wave;
  i32x4 h_next = {0, 0, 0, 0};
  uint32_t lo_next = 0u;
  uint32_t hi_next = 0u;
  if (b < b1) {
    h_next = hdrs[b];
    lo_next = progs[b * kProgMaxOps * 2 + 2 * lane];
    hi_next = progs[b * kProgMaxOps * 2 + 2 * lane + 1];
  }
  for (; b < b1; b += kColWaves) {
    const i32x4 h = h_next;
    const uint32_t lo = lo_next;
    const uint32_t hi = hi_next;
    // wait for this plan's words here, before the next plan's loads are issued: the waits the
    // compiler would place inside the op loop also cover those newer loads
    asm volatile("" ::"v"(h), "v"(lo), "v"(hi));
    if (b + kColWaves < b1) {
      const int64_t nb = b + kColWaves;
      h_next = hdrs[nb];
      lo_next = progs[nb * kProgMaxOps * 2 + 2 * lane];
      hi_next = progs[nb * kProgMaxOps * 2 + 2 * lane + 1];
    }
    if constexpr (CLAUSES) {
      // a plan of clauses: the AND of its clauses' words (NOT: inverted)
      const uint32_t desc = __builtin_amdgcn_readfirstlane(plan_desc[b]);
      if (desc >> 31) {
        kcu32* refs = plan_refs + ((desc >> 12) & 0x7ffffu);
        const int cnt = static_cast<int>(desc & 0xfffu);
        uint64_t top = ~0ull;
        for (int r = 0; r < cnt; ++r) {
          const uint32_t ref = __builtin_amdgcn_readfirstlane(refs[r]);
          const uint64_t w = clause_col[(ref & 0x7fffu) * kWave];
          top &= (ref & 0x8000u) != 0u ? ~w : w;
        }
        if (valid) write_column(a, b, ncol, col, top);
        continue;
      }
    }
    const int32_t st = __builtin_amdgcn_readfirstlane(h[0]);
    if (st == kPlanStack) continue;  // the stack evaluation writes it
    uint64_t top = 0ull;
    if (st == kPlanProgram) {
      gu32* prog = progs + b * kProgMaxOps * 2;
      const int n_ops = __builtin_amdgcn_readfirstlane(h[1]);  // <= kProgMaxOps
      const int64_t h0 = static_cast<int64_t>(
          (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(h[3])))
           << 32) |
          static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(h[2])));
      if (all_staged) {
        top = run_program<KK, true>(a, prog, lo, hi, n_ops, h0, lcol, true, wcol, my_w, stk,
                                    lane);
      } else {
        top = run_program<KK, false>(a, prog, lo, hi, n_ops, h0, lcol, mine_staged, wcol, my_w,
                                     stk, lane);
      }
    }
    if (valid) write_column(a, b, ncol, col, top);
  }
  }  // bundle pairs
}

// ---- stack evaluation: the plans the program cannot hold --------------------------------
//
// Lane <-> column, the evaluation stack in LDS ([max_stack][256] words), positions resolved
// from the stored hashes per column.

// Plan b over column col (< nb * 32) with this lane's stack column stk[s * kBloomThreads + tid]:
// the post-order evaluation of bloom_index_search_cuda.cu:471-534 / bloom_index_search.cpp:
// 88-166; a malformed plan, or one needing more than max_stack slots, matches nothing.
__device__ inline uint64_t stack_eval(const BloomSearchArgs& a, int64_t b, int64_t col,
                                      uint64_t* stk, int tid) {
  const int64_t beta = col / kBloomWordsPerBundle;
  const int j = static_cast<int>(col % kBloomWordsPerBundle);
  const int64_t off = a.bundle_off[beta];
  const int64_t w = a.bundle_off[beta + 1] - off;
  const uint64_t* wcol = a.words + off * kBloomWordsPerBundle + j;  // position p at wcol[32 p]
  const int64_t* o = a.plan_offsets + 8 * b;
  // a malformed plan evaluates to no match instead of reading out of bounds
  bool bad = !plan_ok(o, a.data_bytes);
  const uint8_t* ops = reinterpret_cast<const uint8_t*>(a.data + o[0]);
  const int64_t n_ops = bad ? 0 : o[1] - o[0];
  const int32_t* offs = reinterpret_cast<const int32_t*>(a.data + o[2]);
  const int64_t n_offs = (o[3] - o[2]) / 4;
  const int64_t h0 = o[6] / 8;
  const int64_t nh = (o[7] - o[6]) / 8;
  int sp = 0;
  int64_t term = 0;
  for (int64_t i = 0; i < n_ops && !bad; ++i) {
    const uint8_t op = ops[i];
    uint64_t r = 0ull;
    if (op == kOpTerm) {
      if ((term + 1) * a.hash_k > nh) {
        bad = true;
        break;
      }
      r = term_from_hashes(a, h0, term, wcol, w);
      ++term;
    } else if (op == kOpAnd || op == kOpOr) {
      if (i + 1 >= n_offs) {
        bad = true;
        break;
      }
      const int n = offs[i + 1] - offs[i];  // children on the stack
      if (n < 1 || n > sp) {
        bad = true;
        break;
      }
      r = op == kOpAnd ? ~0ull : 0ull;
      for (int q = 0; q < n; ++q) {
        const uint64_t x = stk[(--sp) * kBloomThreads + tid];
        r = op == kOpAnd ? (r & x) : (r | x);
      }
    } else if (op == kOpNot) {
      if (sp < 1) {
        bad = true;
        break;
      }
      r = ~stk[(--sp) * kBloomThreads + tid];
    } else if (op == kOpEmpty) {
      r = ~0ull;
    } else {
      bad = true;
      break;
    }
    if (sp >= a.max_stack) {
      bad = true;
      break;
    }
    stk[(sp++) * kBloomThreads + tid] = r;
  }
  return (!bad && sp == 1) ? stk[tid] : 0ull;
}

__global__ void __launch_bounds__(kBloomThreads) bloom_search_kernel(BloomSearchArgs a) {
  extern __shared__ uint64_t stk[];  // [max_stack][kBloomThreads]
  const int tid = threadIdx.x;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * a.plans_per_wg;
  const int64_t b1 = b0 + a.plans_per_wg < a.plan_count ? b0 + a.plans_per_wg : a.plan_count;
  // most launches have no plan for this kernel: leave before touching anything else
  bool mine = false;
  for (int64_t b = b0 + tid; b < b1; b += kBloomThreads) mine |= a.hdr[4 * b] == kPlanStack;
  if (!__syncthreads_or(mine)) return;
  const int64_t ncol = a.nb * kBloomWordsPerBundle;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kBloomThreads + tid;
  const bool valid = col < ncol;
  for (int64_t b = b0; b < b1; ++b) {
    if (a.hdr[4 * b] != kPlanStack) continue;  // the column kernel writes it
    const uint64_t res = stack_eval(a, b, valid ? col : 0, stk, tid);
    if (valid) write_column(a, b, ncol, col, res);
  }
}

// ---- the plans over the probed clusters' columns only ----------------------------------
//
// bloom_index_search_batch_return_partial_response (bloom_index_search_cuda.cu:1739-1940,
// bloom_index_search.cpp:219-345): probed cluster i (row i / per_row of a [rows, per_row]
// probe table) starting at doc position starts[i] spans columns starts[i] / 64 .. + its column
// count; output word j (cumsum[i - 1] <= j < cumsum[i], cumsum inclusive) is row q's plan
// (plan_index[q], or q) evaluated on column starts[i] / 64 + j - cumsum[i - 1]. Words at or past
// the device total cumsum[n - 1] (up to max_columns) are 0. A plan index or column outside the
// plans or the index gives 0. Lane <-> output word, each with its own plan and stack column.
struct BloomColumnsArgs {
  BloomSearchArgs s;
  const int64_t* starts;   // [n_clusters] first doc positions
  const int32_t* cumsum;   // [n_clusters] inclusive column counts
  int64_t n_clusters;
  int64_t per_row;
  const int64_t* plan_index;  // [rows] or null
  int64_t max_columns;
  int64_t* out;  // [max_columns]
};

__global__ void __launch_bounds__(kBloomThreads) bloom_columns_kernel(BloomColumnsArgs a) {
  extern __shared__ uint64_t stk[];  // [max_stack][kBloomThreads]
  const int tid = threadIdx.x;
  const int64_t total = a.n_clusters > 0 ? a.cumsum[a.n_clusters - 1] : 0;
  const int64_t ncol = a.s.nb * kBloomWordsPerBundle;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kBloomThreads + tid; j < a.max_columns;
       j += static_cast<int64_t>(gridDim.x) * kBloomThreads) {
    uint64_t res = 0ull;
    if (j < total) {
      int64_t lo = 0;
      int64_t hi = a.n_clusters - 1;
      while (lo < hi) {  // the first cluster whose inclusive count passes j
        const int64_t mid = (lo + hi) >> 1;
        if (static_cast<int64_t>(a.cumsum[mid]) > j) {
          hi = mid;
        } else {
          lo = mid + 1;
        }
      }
      const int64_t first = lo == 0 ? 0 : static_cast<int64_t>(a.cumsum[lo - 1]);
      const int64_t start = a.starts[lo];
      const int64_t col = (start >= 0 ? start / 64 : -1) + (j - first);
      const int64_t q = lo / a.per_row;
      const int64_t b = a.plan_index != nullptr ? a.plan_index[q] : q;
      if (start >= 0 && col < ncol && b >= 0 && b < a.s.plan_count) {
        res = stack_eval(a.s, b, col, stk, tid);
      }
    }
    a.out[j] = static_cast<int64_t>(res);
  }
}

// ---- per-document bits and the probe -----------------------------------------------------
//
// The row view of the bit-sliced bundles: document d's bits in one word, position p at bit p,
// for the per-candidate Bloom probe of the fused scans (bloom_prog.h, probe_wave). One
// workgroup per bundle stages its w * 32 words in LDS; each thread assembles documents t,
// t + 256, ... of the bundle (a wave's 64 documents share a column: every LDS read is a
// broadcast). A bundle whose width is not `width` gets all ones, so its documents pass every
// probe (the programs' positions are bundle 0's).
__global__ void __launch_bounds__(kBloomThreads) bloom_doc_bits_kernel(const uint64_t* words,
                                                                       const int64_t* off,
                                                                       int64_t n_docs,
                                                                       int64_t width,
                                                                       uint64_t* out) {
  __shared__ uint64_t w[kColMaxWidth * kBloomWordsPerBundle];
  const int64_t beta = blockIdx.x;
  const int64_t o0 = off[beta];
  const int64_t wb = off[beta + 1] - o0;
  const bool ok = wb == width && wb >= 1 && wb <= kColMaxWidth;
  const int n = ok ? static_cast<int>(wb) * kBloomWordsPerBundle : 0;
  for (int i = threadIdx.x; i < n; i += kBloomThreads) w[i] = words[o0 * kBloomWordsPerBundle + i];
  __syncthreads();
  const int64_t d0 = beta * kBloomDocsPerBundle;
  for (int t = threadIdx.x; t < kBloomDocsPerBundle && d0 + t < n_docs; t += kBloomThreads) {
    uint64_t f = ~0ull;
    if (ok) {
      f = 0ull;
      const uint64_t* col = w + (t >> 6);
      const int sh = 63 - (t & 63);
      for (int p = 0; p < static_cast<int>(wb); ++p) {
        f |= ((col[p * kBloomWordsPerBundle] >> sh) & 1ull) << p;
      }
    }
    out[d0 + t] = f;
  }
}

// Every plan over every document through the probe: wave <-> 64 documents of one plan (grid
// y), one word of the scans' mask layout each, the wave evaluating its documents one at a time.
// Documents at or past n_docs are 0.
__global__ void __launch_bounds__(kBloomThreads) bloom_probe_search_kernel(BloomProbe p,
                                                                           int64_t n_docs,
                                                                           int64_t n_words,
                                                                           int64_t* out) {
  const int lane = lane_id();
  const int64_t word = static_cast<int64_t>(blockIdx.x) * (kBloomThreads / kWave) +
                       (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (word >= n_words) return;  // (wave-uniform)
  const int64_t d = word * 64 + lane;
  const uint64_t mine = d < n_docs ? p.doc_bits[d] : 0ull;
  const uint64_t* t = p.tables + p.tables[b];
  bool hit = false;
  for (int l = 0; l < kWave; ++l) {
    const bool pass = probe_wave(t, readlane64(mine, l), lane);
    if (lane == l) hit = pass && d < n_docs;
  }
  const uint64_t bits = __ballot(hit);
  if (lane == 0) out[b * n_words + word] = static_cast<int64_t>(__builtin_bitreverse64(bits));
}

}  // namespace rt

using namespace rt;

extern "C" int rt_bloom_bundle_terms(const int64_t* feature_offsets, int64_t N, int64_t C,
                                     int64_t* max_terms, hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && C >= 1 && C <= (int64_t{1} << 20), "N must be >= 0 and C >= 1");
  const int64_t nb = cdiv(N, kBloomDocsPerBundle);
  if (nb == 0) return kOk;
  bloom_terms_kernel<<<static_cast<unsigned>(nb), kBloomThreads, 0, stream>>>(
      feature_offsets, N, static_cast<int>(C), max_terms);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_bloom_build(const int32_t* feature_ids, int64_t C,
                              const int64_t* feature_offsets, const int64_t* feature_values,
                              int64_t N, const int64_t* bundle_b_offsets, int64_t max_width,
                              int64_t k, uint64_t* words, hipStream_t stream) {
  RT_CHECK_ARG(N >= 0 && C >= 1 && C <= (int64_t{1} << 20), "N must be >= 0 and C >= 1");
  RT_CHECK_ARG(k >= 1 && k <= kBloomMaxK, "k must be in [1, %d], got %lld", kBloomMaxK,
               static_cast<long long>(k));
  RT_CHECK_ARG(max_width >= 0 && max_width <= kBloomMaxBuildWidth,
               "bits per doc must be <= %d, got %lld", kBloomMaxBuildWidth,
               static_cast<long long>(max_width));
  const int64_t nb = cdiv(N, kBloomDocsPerBundle);
  if (nb == 0 || max_width == 0) return kOk;
  BloomBuildArgs a{};
  a.feature_ids = feature_ids;
  a.C = static_cast<int>(C);
  a.fo = feature_offsets;
  a.values = feature_values;
  a.N = N;
  a.bundle_off = bundle_b_offsets;
  a.k = static_cast<int>(k);
  a.words = words;
  const int64_t grid = nb * kBloomDocsPerBundle / kBloomThreads;
  RT_CHECK_ARG(grid < (int64_t{1} << 31), "N too large");
  bloom_build_kernel<<<static_cast<unsigned>(grid), kBloomThreads, 0, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" size_t rt_bloom_search_workspace(int64_t data_bytes, int64_t plan_count) {
  (void)data_bytes;  // the programs are per plan
  const int64_t plans = plan_count > 0 ? plan_count : 0;
  return align_up(static_cast<size_t>(plans) * 16, 256) +
         align_up(static_cast<size_t>(plans) * kProgMaxOps * 2 * sizeof(uint32_t), 256);
}

extern "C" size_t rt_bloom_compiled_bytes(int64_t plan_count) {
  return rt_bloom_search_workspace(0, plan_count);
}

// The checks every search makes of its plans and sizes.
static int bloom_check(int64_t n_bundles, const int8_t* plan_data, int64_t data_bytes,
                       int64_t plan_count, int64_t max_stack, int64_t k, int64_t hash_k) {
  RT_CHECK_ARG(n_bundles >= 0 && plan_count >= 0 && data_bytes >= 0, "sizes must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kBloomMaxK, "k must be in [1, %d], got %lld", kBloomMaxK,
               static_cast<long long>(k));
  RT_CHECK_ARG(hash_k >= 1 && hash_k <= 64, "hash_k must be in [1, 64], got %lld",
               static_cast<long long>(hash_k));
  RT_CHECK_ARG(max_stack >= 1 && max_stack <= kBloomMaxStack,
               "max_stack_size must be in [1, %d], got %lld", kBloomMaxStack,
               static_cast<long long>(max_stack));
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(plan_data) % 8 == 0, "plan data must be 8-aligned");
  RT_CHECK_ARG(plan_count <= (int64_t{1} << 31) - 1, "too many plans");
  return kOk;
}

// The plans' shared fields; hdr / prog point into a compiled buffer (header, then programs).
static BloomSearchArgs bloom_args(const uint64_t* words, const int64_t* bundle_b_offsets,
                                  int64_t n_bundles, const int64_t* plan_offsets,
                                  const int8_t* plan_data, int64_t data_bytes,
                                  int64_t plan_count, int64_t max_stack, int64_t k,
                                  int64_t hash_k, void* compiled) {
  BloomSearchArgs a{};
  a.words = words;
  a.bundle_off = bundle_b_offsets;
  a.nb = n_bundles;
  a.plan_offsets = plan_offsets;
  a.data = plan_data;
  a.data_bytes = data_bytes;
  a.plan_count = plan_count;
  a.max_stack = static_cast<int>(max_stack);
  a.k = static_cast<int>(k);
  a.hash_k = static_cast<int>(hash_k);
  a.words_aligned16 = reinterpret_cast<uintptr_t>(words) % 16 == 0;
  a.hdr = static_cast<int32_t*>(compiled);
  a.prog = reinterpret_cast<uint32_t*>(static_cast<char*>(compiled) +
                                       compiled_prog_offset(plan_count));
  return a;
}

// The column kernel for KK positions a term, 4 or 8 waves, with the shared terms' LDS.
template <int KK, bool CLAUSES>
static int launch_column(const BloomSearchArgs& a, dim3 grid, int waves, size_t lds,
                         hipStream_t stream) {
  const void* fn = waves == 8
                       ? reinterpret_cast<const void*>(&bloom_column_kernel<KK, 512, CLAUSES>)
                       : reinterpret_cast<const void*>(&bloom_column_kernel<KK, 256, CLAUSES>);
  if (lds > 0) {
    RT_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  // as many workgroups over the bundle pairs as stay resident together (each then loops over
  // its pairs, the next one's words in flight)
  int occ = 0;
  int dev = 0;
  int cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, waves * kWave,
                                                   static_cast<int>(lds)) == hipSuccess &&
      hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      occ > 0 && cus > 0) {
    const int64_t resident = static_cast<int64_t>(occ) * cus;
    const int64_t gx = cdiv(resident, static_cast<int64_t>(grid.y));
    if (gx < static_cast<int64_t>(grid.x)) grid.x = static_cast<unsigned>(gx < 1 ? 1 : gx);
  }
  if (waves == 8) {
    bloom_column_kernel<KK, 512, CLAUSES><<<grid, 512, lds, stream>>>(a);
  } else {
    bloom_column_kernel<KK, 256, CLAUSES><<<grid, 256, lds, stream>>>(a);
  }
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// The prep pass: each plan's program (or its stack-path / no-match status) into `a`'s buffers.
static int bloom_compile_into(const BloomSearchArgs& a, hipStream_t stream) {
  bloom_prep_kernel<<<static_cast<unsigned>(a.plan_count), kPrepThreads, 0, stream>>>(
      a, const_cast<int32_t*>(a.hdr), const_cast<uint32_t*>(a.prog));
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// The searches over compiled plans: the column kernel (programs; with a.n_clauses > 0 the
// plans of clauses over the batch's distinct clauses), then the stack evaluation of the rest;
// any of the three outputs.
static int bloom_run(BloomSearchArgs a, hipStream_t stream, bool stack_plans = true) {
  const int64_t n_bundles = a.nb;
  const int64_t plan_count = a.plan_count;
  const int64_t kk = a.k < a.hash_k ? a.k : a.hash_k;  // > kProgMaxPos: the stack path only
  const int64_t n_clauses = a.n_clauses;
  RT_CHECK_ARG(n_clauses >= 0 && n_clauses <= kMaxClauses,
               "clauses must be in [0, %d], got %lld", kMaxClauses,
               static_cast<long long>(n_clauses));
  RT_CHECK_ARG(n_clauses == 0 || (kk <= kProgMaxPos && a.clause_ptr != nullptr &&
                                  a.clause_terms != nullptr && a.plan_desc != nullptr &&
                                  a.plan_refs != nullptr),
               "clauses need at most %d positions a term and their tables", kProgMaxPos);

  // column kernel: two bundles per workgroup, plans split over y when that gives too few
  const int64_t cx = cdiv(n_bundles, 2);
  RT_CHECK_ARG(cx < (int64_t{1} << 31), "too many bundles");
  int64_t cy = cdiv(2048, cx);
  const int col_waves = cdiv(plan_count, cy) >= kColWidePlans ? 8 : 4;
  const int64_t max_cy = cdiv(plan_count, col_waves);
  cy = cy > max_cy ? max_cy : cy;
  cy = cy < 1 ? 1 : cy;
  cy = cy > 65535 ? 65535 : cy;
  a.plans_per_wg = cdiv(plan_count, cy);
  cy = cdiv(plan_count, a.plans_per_wg);
  const dim3 cgrid(static_cast<unsigned>(cx), static_cast<unsigned>(cy));
  const size_t lds = static_cast<size_t>(n_clauses) * kWave * sizeof(uint64_t);
  int st = kOk;
  if (n_clauses > 0) {  // (kk <= kProgMaxPos, checked above)
    if (kk == 1) {
      st = launch_column<1, true>(a, cgrid, col_waves, lds, stream);
    } else if (kk == 2) {
      st = launch_column<2, true>(a, cgrid, col_waves, lds, stream);
    } else if (kk == 3) {
      st = launch_column<3, true>(a, cgrid, col_waves, lds, stream);
    } else {
      st = launch_column<4, true>(a, cgrid, col_waves, lds, stream);
    }
  } else if (kk == 1) {
    st = launch_column<1, false>(a, cgrid, col_waves, 0, stream);
  } else if (kk == 2) {
    st = launch_column<2, false>(a, cgrid, col_waves, 0, stream);
  } else if (kk == 3) {
    st = launch_column<3, false>(a, cgrid, col_waves, 0, stream);
  } else if (kk == 4) {
    st = launch_column<4, false>(a, cgrid, col_waves, 0, stream);
  }
  if (st != kOk) return st;

  if (!stack_plans) return kOk;  // (the compile pass gave every plan a program)
  // stack evaluation of the rest (its workgroups skip the plans the column kernel wrote)
  const int64_t gx = cdiv(n_bundles * kBloomWordsPerBundle, kBloomThreads);
  RT_CHECK_ARG(gx < (int64_t{1} << 31), "too many bundles");
  int64_t gy = cdiv(2048, gx);
  gy = gy < 1 ? 1 : gy;
  gy = gy > plan_count ? plan_count : gy;
  gy = gy > 65535 ? 65535 : gy;
  a.plans_per_wg = cdiv(plan_count, gy);
  gy = cdiv(plan_count, a.plans_per_wg);
  const size_t slds = static_cast<size_t>(a.max_stack) * kBloomThreads * sizeof(uint64_t);
  if (slds > 64 * 1024) {
    RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&bloom_search_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(slds)));
  }
  bloom_search_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                        kBloomThreads, slds, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

// The search behind rt_bloom_search and rt_bloom_search_t: the plans compiled into the
// workspace, then searched; any of the three outputs.
static int bloom_search(const uint64_t* words, const int64_t* bundle_b_offsets, int64_t n_bundles,
                        const int64_t* plan_offsets, const int8_t* plan_data, int64_t data_bytes,
                        int64_t plan_count, int64_t max_stack, int64_t k, int64_t hash_k,
                        int64_t* out_mask, uint8_t* out_bool, uint64_t* out_mask_t,
                        int64_t out_t_stride, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  int st = bloom_check(n_bundles, plan_data, data_bytes, plan_count, max_stack, k, hash_k);
  if (st != kOk) return st;
  RT_CHECK_ARG(out_mask != nullptr || out_bool != nullptr || out_mask_t != nullptr, "no output");
  RT_CHECK_ARG(out_mask_t == nullptr || out_t_stride >= plan_count,
               "the transposed output's stride must be >= plan_count");
  if (n_bundles == 0 || plan_count == 0) return kOk;
  const size_t need = rt_bloom_search_workspace(data_bytes, plan_count);
  if (workspace_bytes < need) {
    set_error("workspace too small: %zu < %zu", workspace_bytes, need);
    return kWorkspaceTooSmall;
  }
  BloomSearchArgs a = bloom_args(words, bundle_b_offsets, n_bundles, plan_offsets, plan_data,
                                 data_bytes, plan_count, max_stack, k, hash_k, workspace);
  a.out_mask = out_mask;
  a.out_bool = out_bool;
  a.out_mask_t = out_mask_t;
  a.out_t_stride = out_t_stride;
  st = bloom_compile_into(a, stream);
  if (st != kOk) return st;
  return bloom_run(a, stream);
}

extern "C" int rt_bloom_search(const uint64_t* words, const int64_t* bundle_b_offsets,
                               int64_t n_bundles, const int64_t* plan_offsets,
                               const int8_t* plan_data, int64_t data_bytes, int64_t plan_count,
                               int64_t max_stack, int64_t k, int64_t hash_k, int64_t* out_mask,
                               uint8_t* out_bool, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  return bloom_search(words, bundle_b_offsets, n_bundles, plan_offsets, plan_data, data_bytes,
                      plan_count, max_stack, k, hash_k, out_mask, out_bool, nullptr, 0, workspace,
                      workspace_bytes, stream);
}

extern "C" int rt_bloom_search_t(const uint64_t* words, const int64_t* bundle_b_offsets,
                                 int64_t n_bundles, const int64_t* plan_offsets,
                                 const int8_t* plan_data, int64_t data_bytes, int64_t plan_count,
                                 int64_t max_stack, int64_t k, int64_t hash_k, uint64_t* out_mask_t,
                                 int64_t out_t_stride, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  RT_CHECK_ARG(out_mask_t != nullptr, "out_mask_t is null");
  return bloom_search(words, bundle_b_offsets, n_bundles, plan_offsets, plan_data, data_bytes,
                      plan_count, max_stack, k, hash_k, nullptr, nullptr, out_mask_t,
                      out_t_stride, workspace, workspace_bytes, stream);
}

extern "C" int rt_bloom_compile(const int64_t* bundle_b_offsets, int64_t n_bundles,
                                const int64_t* plan_offsets, const int8_t* plan_data,
                                int64_t data_bytes, int64_t plan_count, int64_t max_stack,
                                int64_t k, int64_t hash_k, void* compiled, size_t compiled_bytes,
                                hipStream_t stream) {
  int st = bloom_check(n_bundles, plan_data, data_bytes, plan_count, max_stack, k, hash_k);
  if (st != kOk) return st;
  if (plan_count == 0) return kOk;
  RT_CHECK_ARG(n_bundles >= 1, "compiling needs the index's bundle widths (no bundles given)");
  RT_CHECK_ARG(compiled != nullptr && compiled_bytes >= rt_bloom_compiled_bytes(plan_count),
               "the compiled buffer needs %zu bytes", rt_bloom_compiled_bytes(plan_count));
  const BloomSearchArgs a = bloom_args(nullptr, bundle_b_offsets, n_bundles, plan_offsets,
                                       plan_data, data_bytes, plan_count, max_stack, k, hash_k,
                                       compiled);
  return bloom_compile_into(a, stream);
}

extern "C" int rt_bloom_search_compiled(const uint64_t* words, const int64_t* bundle_b_offsets,
                                        int64_t n_bundles, const int64_t* plan_offsets,
                                        const int8_t* plan_data, int64_t data_bytes,
                                        int64_t plan_count, int64_t max_stack, int64_t k,
                                        int64_t hash_k, const void* compiled,
                                        size_t compiled_bytes, const uint32_t* clause_ptr,
                                        const uint32_t* clause_terms, const uint32_t* plan_desc,
                                        const uint32_t* plan_refs, int64_t n_clauses,
                                        int64_t plan_flags, int64_t* out_mask,
                                        uint64_t* out_mask_t, int64_t out_t_stride,
                                        hipStream_t stream) {
  int st = bloom_check(n_bundles, plan_data, data_bytes, plan_count, max_stack, k, hash_k);
  if (st != kOk) return st;
  RT_CHECK_ARG((out_mask != nullptr) != (out_mask_t != nullptr), "one output");
  RT_CHECK_ARG(out_mask_t == nullptr || out_t_stride >= plan_count,
               "the transposed output's stride must be >= plan_count");
  if (n_bundles == 0 || plan_count == 0) return kOk;
  RT_CHECK_ARG(compiled != nullptr && compiled_bytes >= rt_bloom_compiled_bytes(plan_count),
               "the compiled buffer needs %zu bytes", rt_bloom_compiled_bytes(plan_count));
  BloomSearchArgs a = bloom_args(words, bundle_b_offsets, n_bundles, plan_offsets, plan_data,
                                 data_bytes, plan_count, max_stack, k, hash_k,
                                 const_cast<void*>(compiled));
  a.out_mask = out_mask;
  a.out_mask_t = out_mask_t;
  a.out_t_stride = out_t_stride;
  a.clause_ptr = clause_ptr;
  a.clause_terms = clause_terms;
  a.plan_desc = plan_desc;
  a.plan_refs = plan_refs;
  RT_CHECK_ARG(n_clauses >= 0 && n_clauses <= kMaxClauses, "clauses must be in [0, %d]",
               kMaxClauses);
  a.n_clauses = static_cast<int>(n_clauses);
  a.all_clauses = n_clauses > 0 && (plan_flags & kPlansAllClauses) != 0;
  return bloom_run(a, stream, (plan_flags & kPlansNoStack) == 0);
}

extern "C" int rt_bloom_doc_bits(const uint64_t* words, const int64_t* bundle_b_offsets,
                                 int64_t n_bundles, int64_t n_docs, int64_t width,
                                 uint64_t* out_doc_bits, hipStream_t stream) {
  RT_CHECK_ARG(n_bundles >= 0 && n_docs >= 0, "sizes must be >= 0");
  RT_CHECK_ARG(n_docs <= n_bundles * kBloomDocsPerBundle,
               "n_docs %lld is above the index's %lld bundles of %d documents",
               static_cast<long long>(n_docs), static_cast<long long>(n_bundles),
               kBloomDocsPerBundle);
  RT_CHECK_ARG(width >= 1 && width <= kColMaxWidth, "width must be in [1, %d], got %lld",
               kColMaxWidth, static_cast<long long>(width));
  if (n_docs == 0) return kOk;
  RT_CHECK_ARG(words != nullptr && bundle_b_offsets != nullptr && out_doc_bits != nullptr,
               "words, bundle offsets and the output must not be null");
  const int64_t grid = cdiv(n_docs, kBloomDocsPerBundle);
  RT_CHECK_ARG(grid < (int64_t{1} << 31), "too many bundles");
  bloom_doc_bits_kernel<<<static_cast<unsigned>(grid), kBloomThreads, 0, stream>>>(
      words, bundle_b_offsets, n_docs, width, out_doc_bits);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_bloom_probe_search(const uint64_t* doc_bits, int64_t n_docs,
                                     const uint64_t* probe_tables, int64_t plan_count,
                                     int64_t* out_mask, hipStream_t stream) {
  RT_CHECK_ARG(n_docs >= 0 && plan_count >= 0, "sizes must be >= 0");
  RT_CHECK_ARG(plan_count <= 65535, "plan_count must be <= 65535, got %lld",
               static_cast<long long>(plan_count));
  const int64_t n_words = cdiv(n_docs, 64);
  if (n_words == 0 || plan_count == 0) return kOk;
  RT_CHECK_ARG(doc_bits != nullptr && probe_tables != nullptr && out_mask != nullptr,
               "doc_bits, probe_tables and out_mask must not be null");
  BloomProbe p;
  p.doc_bits = doc_bits;
  p.tables = probe_tables;
  const int64_t gx = cdiv(n_words, kBloomThreads / kWave);
  RT_CHECK_ARG(gx < (int64_t{1} << 31), "too many documents");
  bloom_probe_search_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(plan_count)),
                              kBloomThreads, 0, stream>>>(p, n_docs, n_words, out_mask);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}

extern "C" int rt_bloom_search_columns(const uint64_t* words, const int64_t* bundle_b_offsets,
                                       int64_t n_bundles, const int64_t* plan_offsets,
                                       const int8_t* plan_data, int64_t data_bytes,
                                       int64_t plan_count, int64_t max_stack, int64_t k,
                                       int64_t hash_k, const int64_t* cluster_starts,
                                       const int32_t* column_counts_cumsum, int64_t n_clusters,
                                       int64_t clusters_per_row, const int64_t* query_plan_index,
                                       int64_t max_columns, int64_t* out_words,
                                       hipStream_t stream) {
  RT_CHECK_ARG(n_bundles >= 0 && plan_count >= 0 && data_bytes >= 0 && n_clusters >= 0 &&
                   max_columns >= 0,
               "sizes must be >= 0");
  RT_CHECK_ARG(k >= 1 && k <= kBloomMaxK, "k must be in [1, %d], got %lld", kBloomMaxK,
               static_cast<long long>(k));
  RT_CHECK_ARG(hash_k >= 1 && hash_k <= 64, "hash_k must be in [1, 64], got %lld",
               static_cast<long long>(hash_k));
  RT_CHECK_ARG(max_stack >= 1 && max_stack <= kBloomMaxStack,
               "max_stack_size must be in [1, %d], got %lld", kBloomMaxStack,
               static_cast<long long>(max_stack));
  RT_CHECK_ARG(clusters_per_row >= 1, "clusters_per_row must be >= 1");
  RT_CHECK_ARG(reinterpret_cast<uintptr_t>(plan_data) % 8 == 0, "plan data must be 8-aligned");
  if (max_columns == 0) return kOk;
  RT_CHECK_ARG(out_words != nullptr, "out_words must not be null");
  // (no clusters, bundles or plans: the kernel writes the zeros, no memset, so a captured
  // graph holds kernels only)
  RT_CHECK_ARG(n_clusters == 0 || (cluster_starts != nullptr && column_counts_cumsum != nullptr),
               "cluster_starts and column_counts_cumsum must not be null");
  RT_CHECK_ARG(n_bundles == 0 || plan_count == 0 ||
                   (words != nullptr && bundle_b_offsets != nullptr && plan_offsets != nullptr &&
                    plan_data != nullptr),
               "the index and the plans must not be null");
  BloomColumnsArgs a{};
  a.s.words = words;
  a.s.bundle_off = bundle_b_offsets;
  a.s.nb = n_bundles;
  a.s.plan_offsets = plan_offsets;
  a.s.data = plan_data;
  a.s.data_bytes = data_bytes;
  a.s.plan_count = plan_count;
  a.s.max_stack = static_cast<int>(max_stack);
  a.s.k = static_cast<int>(k);
  a.s.hash_k = static_cast<int>(hash_k);
  a.starts = cluster_starts;
  a.cumsum = column_counts_cumsum;
  a.n_clusters = n_clusters;
  a.per_row = clusters_per_row;
  a.plan_index = query_plan_index;
  a.max_columns = max_columns;
  a.out = out_words;
  int64_t grid = cdiv(max_columns, kBloomThreads);
  grid = grid < 4096 ? grid : 4096;
  const size_t lds = static_cast<size_t>(max_stack) * kBloomThreads * sizeof(uint64_t);
  if (lds > 64 * 1024) {
    RT_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&bloom_columns_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds)));
  }
  bloom_columns_kernel<<<static_cast<unsigned>(grid), kBloomThreads, lds, stream>>>(a);
  RT_CHECK_HIP(hipGetLastError());
  return kOk;
}
