// Host front end of libtforge_hip: the tforge program text, the
// --tforge-gpu-pipeline option string, and the plan that maps a verified
// program onto kernel launches.  Plain C++ (no HIP calls), so it runs on a
// machine without a GPU.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace tff {

struct Loc {
  int line = 0, col = 0;
};

// A type as written in the program.  Only ranked static f32 tensors are
// legal tforge values; the rest are kept so the verifier can name them.
struct Type {
  bool is_tensor = false;
  bool ranked = true;
  std::vector<int64_t> shape;  // -1 for a dynamic ('?') dimension
  std::string elem;            // "f32", "f16", "i32", ...
  std::string text;            // canonical spelling, e.g. tensor<64x32xf32>
  bool static_shape() const;
  int64_t numel() const;
};

struct Op {
  std::string name;  // "matmul", "bias_add", "relu", "add"
  std::vector<std::string> operands;
  std::vector<Type> operand_types;
  std::string result;
  Type result_type;
  Loc loc;
};

struct Program {
  std::string source_name;
  std::string func_name;
  std::vector<std::string> arg_names;
  std::vector<Type> arg_types;
  std::vector<Type> result_types;
  std::vector<Op> ops;
  bool has_return = false;
  std::string ret_value;
  Type ret_type;
  Loc func_loc, ret_loc;
};

// GpuPipelineOptions (reference include/TensorForge/Pipelines.h:45-72) plus
// the backend's own knobs.
struct Options {
  bool fuse_elementwise = true;
  std::vector<int64_t> block_tile;   // default 16,16
  std::vector<int64_t> thread_tile;  // default 1,1
  int64_t tile_k = 0;
  bool promote = false;
  bool vectorize = false;
  bool print_after_each = false;
  bool print_script = false;
  bool xcd_swizzle = true;  // backend: XCD-aware tile order for staged kernels
  int64_t split_k = 1;      // backend: workgroups per output tile along K (staged kernels)
  bool mask_edges = false;  // backend: staged kernels take any shape (masked edge tiles, no padding)
  bool wave_split_k = false;  // backend: the waves of a workgroup split K, partial tiles summed in LDS
  // Derived (reference lib/Pipelines/Pipelines.cpp:214-263).
  int64_t bm = 16, bn = 16, tm = 1, tn = 1;
  bool align_vectors = false;
};

enum BufRole : int { BUF_INPUT = 0, BUF_OUTPUT = 1, BUF_INTERMEDIATE = 2 };

struct Buffer {
  std::string name;
  int role = BUF_INPUT;
  std::vector<int64_t> shape;
  int64_t numel() const;
};

struct EpiOp {
  int kind;  // tfk::EpiKind
  int buf;   // operand buffer, -1 if none
};

enum StageKind : int { STAGE_GEMM = 0, STAGE_ELEMENTWISE = 1 };

struct Stage {
  int kind = STAGE_GEMM;
  int a = -1, b = -1;  // GEMM operands (buffer ids)
  int x = -1;          // element-op stage input
  int out = -1;
  int64_t M = 0, N = 0, K = 0;
  std::vector<EpiOp> epi;
  std::string ops;  // e.g. "matmul+bias_add+relu"
  Loc loc;
};

// Buffers 0..nargs-1 are the entry arguments, nargs is the result
// (out-param), the rest are library-owned intermediates.
struct Plan {
  int nargs = 0;
  std::vector<Buffer> buffers;
  std::vector<Stage> stages;
};

bool parse_program(const std::string &text, const std::string &source_name, Program &out,
                   std::string &err);
bool verify_program(const Program &p, std::string &err);
bool parse_options(const std::string &text, Options &out, std::string &err);
bool plan_program(const Program &p, const Options &o, Plan &out, std::string &err);

std::string format_error(const std::string &source_name, Loc loc, const std::string &msg);

}  // namespace tff
