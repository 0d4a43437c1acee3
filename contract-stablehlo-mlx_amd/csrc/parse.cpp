// A dependency-free reader of StableHLO's generic operation form, with the
// grammar of StablehloMlx/Parse.lean: `%r = "stablehlo.add"(%a, %b) {attrs} :
// (T, T) -> T`, regions for while/reduce/composite bodies, `%x:n` / `%x#k`
// multi-results, printed func.return / return terminators, inside
// `module { func.func ... }`.  Attribute values stay raw text.
#include <cctype>
#include <cstring>

#include "stablehlo.h"

namespace shlo {

std::string Ty::str() const {
  std::string s = "tensor<";
  for (int64_t d : dims) s += std::to_string(d) + "x";
  return s + el + ">";
}

const std::string *Op::attr(const std::string &k) const {
  for (auto &kv : attrs)
    if (kv.first == k) return &kv.second;
  return nullptr;
}

const Func *Module::func(const std::string &n) const {
  for (auto &f : funcs)
    if (f.name == n) return &f;
  return nullptr;
}

namespace {

struct Parser {
  const std::string &s;
  size_t i = 0;
  explicit Parser(const std::string &t) : s(t) {}

  [[noreturn]] void error(const std::string &msg) {
    std::string ctx = s.substr(i, 60);
    fail(strf("parse error at %zu: %s; next: \"%s\"", i, msg.c_str(), ctx.c_str()));
  }
  int peek() const { return i < s.size() ? (unsigned char)s[i] : -1; }

  void ws() {  // Parse.lean:28-41
    while (i < s.size()) {
      const char c = s[i];
      if (c == ' ' || c == '\n' || c == '\t' || c == '\r') {
        i++;
      } else if (c == '/' && i + 1 < s.size() && s[i + 1] == '/') {
        while (i < s.size() && s[i] != '\n') i++;
      } else {
        break;
      }
    }
  }
  bool starts_with(const char *lit) const { return s.compare(i, strlen(lit), lit) == 0; }
  bool try_lit(const char *lit) {
    ws();
    if (starts_with(lit)) {
      i += strlen(lit);
      return true;
    }
    return false;
  }
  void lit(const char *l) {
    if (!try_lit(l)) error(strf("expected \"%s\"", l));
  }
  static bool id_char(int c) { return std::isalnum(c) || c == '_' || c == '.' || c == '$' || c == '-'; }
  std::string take_while(bool (*p)(int)) {
    size_t b = i;
    while (i < s.size() && p((unsigned char)s[i])) i++;
    return s.substr(b, i - b);
  }
  static bool is_digit(int c) { return c >= '0' && c <= '9'; }

  // `%name`, `%name#k`, or `%name:n` (a multi-result definition)
  std::pair<std::string, int64_t> ssa() {
    ws();
    if (peek() != '%') error("expected %");
    i++;
    std::string n = take_while(id_char);
    if (peek() == '#') {
      i++;
      std::string k = take_while(is_digit);
      return {"%" + n + "#" + k, -1};
    }
    if (peek() == ':' && i + 1 < s.size() && is_digit((unsigned char)s[i + 1])) {
      i++;
      std::string k = take_while(is_digit);
      return {"%" + n, std::stoll(k)};
    }
    return {"%" + n, -1};
  }
  std::string ssa_use() { return ssa().first; }

  Ty ty() {
    ws();
    Ty t;
    if (try_lit("tensor<")) {
      for (;;) {
        std::string d = take_while(is_digit);
        if (d.empty()) {
          size_t b = i;
          while (i < s.size() && s[i] != '>') i++;
          t.el = s.substr(b, i - b);
          break;
        }
        t.dims.push_back(std::stoll(d));
        if (peek() != 'x') error("expected x in tensor type");
        i++;
      }
      lit(">");
      return t;
    }
    t.el = take_while(id_char);
    if (t.el.empty()) error("expected a type");
    return t;
  }

  template <class T, class P>
  std::vector<T> sep_by(P p, const char *close) {
    std::vector<T> xs;
    if (try_lit(close)) return xs;
    xs.push_back(p());
    while (try_lit(",")) xs.push_back(p());
    lit(close);
    return xs;
  }

  std::vector<Ty> ty_list() {
    if (try_lit("(")) return sep_by<Ty>([&] { return ty(); }, ")");
    return {ty()};
  }

  // Raw text of one attribute value, up to a top-level `,` or `}`
  // (Parse.lean:117-135).
  std::string raw_value() {
    ws();
    std::string acc;
    int depth = 0;
    while (i < s.size()) {
      const char c = s[i];
      if (depth == 0 && (c == ',' || c == '}')) break;
      if (c == '"') {
        i++;
        size_t b = i;
        while (i < s.size() && s[i] != '"') i++;
        acc += "\"" + s.substr(b, i - b) + "\"";
        if (i < s.size()) i++;
        continue;
      }
      if (c == '(' || c == '[' || c == '{' || c == '<') {
        depth++;
      } else if (c == ')' || c == ']' || c == '}' || c == '>') {
        if (!(c == '>' && !acc.empty() && acc.back() == '-')) depth--;  // `->` is an arrow
      }
      acc.push_back(c);
      i++;
    }
    size_t a = acc.find_first_not_of(" \t\n\r"), e = acc.find_last_not_of(" \t\n\r");
    return a == std::string::npos ? std::string() : acc.substr(a, e - a + 1);
  }

  std::vector<std::pair<std::string, std::string>> attr_dict() {
    lit("{");
    return sep_by<std::pair<std::string, std::string>>(
        [&] {
          ws();
          std::string k = take_while(id_char);
          if (k.empty()) error("expected an attribute name");
          if (try_lit("=")) return std::make_pair(k, raw_value());
          return std::make_pair(k, std::string("unit"));
        },
        "}");
  }

  Block block() {  // Parse.lean:147-163
    lit("{");
    Block b;
    if (try_lit("^")) {
      take_while(id_char);
      if (try_lit("("))
        b.args = sep_by<std::pair<std::string, Ty>>(
            [&] {
              std::string n = ssa_use();
              lit(":");
              Ty t = ty();
              return std::make_pair(n, t);
            },
            ")");
      lit(":");
    }
    for (;;) {
      if (try_lit("}")) break;
      Op o = op();
      if (o.name == "stablehlo.return" || o.name == "func.return" || o.name == "return") b.ret = o.operands;
      else b.ops.push_back(std::move(o));
    }
    return b;
  }

  Op op() {  // Parse.lean:165-208
    ws();
    Op o;
    std::vector<std::string> results;
    if (peek() == '%') {
      std::vector<std::pair<std::string, int64_t>> defs{ssa()};
      while (try_lit(",")) defs.push_back(ssa());
      lit("=");
      for (auto &d : defs) {
        if (d.second >= 0)
          for (int64_t k = 0; k < d.second; k++) results.push_back(d.first + "#" + std::to_string(k));
        else
          results.push_back(d.first);
      }
    }
    ws();
    if (peek() == '"') {
      i++;
      size_t b = i;
      while (i < s.size() && s[i] != '"') i++;
      o.name = s.substr(b, i - b);
      if (i < s.size()) i++;
      lit("(");
      o.operands = sep_by<std::string>([&] { return ssa_use(); }, ")");
      if (try_lit("(")) o.regions = sep_by<Block>([&] { return block(); }, ")");
      ws();
      if (peek() == '{') o.attrs = attr_dict();
      lit(":");
      lit("(");
      o.in_tys = sep_by<Ty>([&] { return ty(); }, ")");
      lit("->");
      o.out_tys = ty_list();
      // Multi-result ops name their results %w#0 …; single-result keep the bare name.
      if (results.size() == 1 && o.out_tys.size() > 1) {
        std::string base = results[0];
        results.clear();
        for (size_t k = 0; k < o.out_tys.size(); k++) results.push_back(base + "#" + std::to_string(k));
      }
      o.results = results;
      return o;
    }
    std::string name = take_while(id_char);
    if (name == "func.return" || name == "return" || name == "stablehlo.return") {
      o.name = name;
      ws();
      if (peek() == '%') {
        o.operands.push_back(ssa_use());
        while (try_lit(",")) o.operands.push_back(ssa_use());
        lit(":");
        ty();
        while (try_lit(",")) ty();
      }
      return o;
    }
    error("unsupported op syntax \"" + name + "\" (the generic form is expected)");
  }

  void skip_attrs() {
    ws();
    if (peek() == '{') attr_dict();
  }

  Func func() {  // Parse.lean:216-230
    lit("func.func");
    try_lit("public");
    try_lit("private");
    lit("@");
    Func f;
    f.name = take_while(id_char);
    lit("(");
    auto args = sep_by<std::pair<std::string, Ty>>(
        [&] {
          std::string n = ssa_use();
          lit(":");
          Ty t = ty();
          skip_attrs();
          return std::make_pair(n, t);
        },
        ")");
    if (try_lit("->")) {
      if (try_lit("("))
        f.out_tys = sep_by<Ty>(
            [&] {
              Ty t = ty();
              skip_attrs();
              return t;
            },
            ")");
      else
        f.out_tys = {ty()};
    }
    if (try_lit("attributes")) attr_dict();
    Block b = block();
    f.body.args = std::move(args);
    f.body.ops = std::move(b.ops);
    f.body.ret = std::move(b.ret);
    return f;
  }

  Module module() {  // Parse.lean:232-245
    Module m;
    const bool wrapped = try_lit("module");
    if (wrapped) {
      if (try_lit("@")) take_while(id_char);
      if (try_lit("attributes")) attr_dict();
      lit("{");
    }
    for (;;) {
      ws();
      if (starts_with("func.func")) m.funcs.push_back(func());
      else break;
    }
    if (wrapped) lit("}");
    ws();
    if (i < s.size()) error("trailing text after the module");
    return m;
  }
};

}  // namespace

Module parse_module(const std::string &text) {
  Parser p(text);
  return p.module();
}

Loaded load_module(const std::string &text) {
  Loaded l;
  l.module = parse_module(text);
  if (!l.module.func("main")) fail("the module has no @main");
  return l;
}

}  // namespace shlo
