// xt-opt: MLIR-free driver for the `xt` subset.  Mirrors the command line the
// reference's lit tests use (xt-opt/xt-opt.cpp:18-33, test/lit.cfg.py:22):
//
//   xt-opt [--xt-serialize] [--canonicalize] [--xt-to-nova] [--split-input-file] [-o out] [file|-]
//
// Each input chunk is parsed and verified, the requested passes run in the
// order given, and the result is printed.  Diagnostics go to stderr as
// `<file>:<line>:<col>: error: <message>`; the exit status is 1 if any chunk
// failed.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "ir.h"

static void usage() {
  std::fprintf(stderr,
               "usage: xt-opt [--xt-serialize] [--canonicalize] [--xt-to-nova] [--split-input-file] "
               "[-o <file>] [<file>|-]\n");
}

int main(int argc, char** argv) {
  std::vector<std::string> passes;
  bool split = false;
  std::string input = "-", output;
  for (int k = 1; k < argc; ++k) {
    std::string a = argv[k];
    if (a == "--xt-serialize" || a == "-xt-serialize") passes.push_back("xt-serialize");
    else if (a == "--canonicalize" || a == "-canonicalize") passes.push_back("canonicalize");
    else if (a == "--xt-to-nova" || a == "-xt-to-nova") passes.push_back("xt-to-nova");
    else if (a == "--split-input-file" || a == "-split-input-file") split = true;
    else if (a == "-o" && k + 1 < argc) output = argv[++k];
    else if (a == "-h" || a == "--help") {
      usage();
      return 0;
    } else if (!a.empty() && a[0] == '-' && a != "-") {
      std::fprintf(stderr, "xt-opt: unknown option '%s'\n", a.c_str());
      usage();
      return 2;
    } else {
      input = a;
    }
  }

  std::stringstream buf;
  if (input == "-") {
    buf << std::cin.rdbuf();
  } else {
    std::ifstream in(input);
    if (!in) {
      std::fprintf(stderr, "xt-opt: cannot open '%s'\n", input.c_str());
      return 2;
    }
    buf << in.rdbuf();
  }
  std::string text = buf.str();
  std::vector<std::string> chunks = split ? xt::split_input_chunks(text)
                                          : std::vector<std::string>{text};

  // Line numbers of a chunk are reported relative to the whole file, as MLIR does.
  std::string out_text;
  bool any_failed = false;
  int line_offset = 0;
  std::string src = input == "-" ? "<stdin>" : input;
  for (size_t c = 0; c < chunks.size(); ++c) {
    std::string padded = std::string(line_offset, '\n') + chunks[c];
    int chunk_lines = 0;
    for (char ch : chunks[c]) chunk_lines += ch == '\n';
    line_offset += chunk_lines + 1;  // the separator line

    xt::Diag diag;
    auto m = xt::parse_module(padded, diag, src);
    bool ok = m != nullptr;
    for (const std::string& p : passes) {
      if (!ok) break;
      if (p == "xt-serialize") ok = xt::pass_xt_serialize(*m, diag);
      else if (p == "canonicalize") ok = xt::pass_canonicalize(*m, diag);
      else if (p == "xt-to-nova") ok = xt::pass_xt_to_nova(*m, diag);
      if (ok) ok = xt::verify_module(*m, diag);
    }
    if (!ok) {
      any_failed = true;
      std::fprintf(stderr, "%s\n", diag.joined().c_str());
      continue;
    }
    if (c > 0) out_text += "// -----\n";
    out_text += xt::print_module(*m);
  }
  if (output.empty()) {
    std::fwrite(out_text.data(), 1, out_text.size(), stdout);
  } else {
    std::ofstream out(output);
    out << out_text;
  }
  return any_failed ? 1 : 0;
}
