'use strict';
/*
 * strip-types.js — erases the TypeScript syntax of src/index.ts into CommonJS JavaScript that
 * Node 12 runs (this image has Node but no TypeScript compiler).  It understands the subset the
 * backend's source is written in:
 *   - `interface` blocks and `type X = ...;` aliases (removed);
 *   - annotations `: T` on parameters (also `name?: T`, `...rest: T`), return types, `const`/`let`
 *     declarations and class fields, where T is a union of names with type arguments and array
 *     suffixes, string literals, object types `{ ... }` or parenthesised types;
 *   - `x as T` casts, type arguments `name<...>(`, and the modifiers private / public / protected /
 *     readonly, the type operator `readonly T[]`, the type parameters of `class Name<T>` and its
 *     `implements A, B` clause;
 *   - `export` on classes, functions, `const` and `export { ... }` lists (collected into
 *     module.exports).
 * Strings, template literals and comments are copied untouched.  Anything outside the subset is
 * left as is, and `node --check` on the output (tests/test_node_backend.py) catches it.
 *
 * Usage: node strip-types.js IN.ts OUT.js
 */
const fs = require('fs');

const src = fs.readFileSync(process.argv[2], 'utf8');

// ---- a cursor over the source that skips strings, template literals and comments ---------------
function skipNonCode(s, i) {
  const c = s[i];
  if (c === '/' && s[i + 1] === '/') { const e = s.indexOf('\n', i); return e < 0 ? s.length : e; }
  if (c === '/' && s[i + 1] === '*') { const e = s.indexOf('*/', i + 2); return e < 0 ? s.length : e + 2; }
  if (c === "'" || c === '"') {
    let j = i + 1;
    while (j < s.length && s[j] !== c) j += s[j] === '\\' ? 2 : 1;
    return j + 1;
  }
  if (c === '`') {
    let j = i + 1;
    while (j < s.length && s[j] !== '`') {
      if (s[j] === '\\') j += 2;
      else if (s[j] === '$' && s[j + 1] === '{') j = matchClose(s, j + 1) + 1;
      else j += 1;
    }
    return j + 1;
  }
  return i;
}

// Index of the bracket closing the one at i (any of ( [ { <), skipping non-code.
function matchClose(s, i) {
  const open = s[i];
  const close = { '(': ')', '[': ']', '{': '}', '<': '>' }[open];
  let depth = 0;
  let j = i;
  while (j < s.length) {
    const k = skipNonCode(s, j);
    if (k !== j) { j = k; continue; }
    if (s[j] === open) depth += 1;
    else if (s[j] === close) { depth -= 1; if (depth === 0) return j; }
    j += 1;
  }
  throw new Error(`strip-types: unbalanced ${open} at ${i}`);
}

function skipSpace(s, i) {
  while (i < s.length && /\s/.test(s[i])) i += 1;
  return i;
}

// End of a type expression starting at i: primaries joined by | or & (not || / &&).
function typeEnd(s, i) {
  let j = skipSpace(s, i);
  for (;;) {
    if (s[j] === '{' || s[j] === '(' || s[j] === '[') j = matchClose(s, j) + 1;
    else if (s[j] === "'" || s[j] === '"') j = skipNonCode(s, j);
    else {
      const m = /^[A-Za-z_$][\w$.]*/.exec(s.slice(j));
      if (!m) throw new Error(`strip-types: no type at ${j}: ${s.slice(Math.max(0, j - 60), j + 30)}`);
      j += m[0].length;
      // `readonly T[]`: the operator, then the type it applies to
      if (m[0] === 'readonly' && /\s/.test(s[j])) { j = skipSpace(s, j); continue; }
      if (s[j] === '<') j = matchClose(s, j) + 1;
    }
    while (s[j] === '[' && s[j + 1] === ']') j += 2;
    const k = skipSpace(s, j);
    if ((s[k] === '|' && s[k + 1] !== '|') || (s[k] === '&' && s[k + 1] !== '&')) { j = skipSpace(s, k + 1); continue; }
    // a function type `(a: T) => R`: its return type ends the type
    if (s[k] === '=' && s[k + 1] === '>' && s[skipSpace(s, i)] === '(') return typeEnd(s, k + 2);
    return j;
  }
}

// ---- pass 1: remove interface blocks, type aliases and modifiers, line based -------------------
const exported = [];
let lines = src.split('\n');
const kept = [];
for (let n = 0; n < lines.length; ++n) {
  let line = lines[n];
  if (/^(export\s+)?interface\s/.test(line)) {
    while (!/^\}/.test(lines[n])) n += 1;
    continue;
  }
  if (/^(export\s+)?type\s+\w+(<[^>]*>)?\s*=/.test(line)) {
    while (!/;\s*$/.test(lines[n])) n += 1;
    continue;
  }
  let m = /^export\s+\{([^}]*)\};?\s*$/.exec(line);
  if (m) { m[1].split(',').forEach((x) => { if (x.trim()) exported.push(x.trim()); }); continue; }
  m = /^export\s+(async\s+function|function|class|const|let)\s+([A-Za-z_$][\w$]*)/.exec(line);
  if (m) { exported.push(m[2]); line = line.replace(/^export\s+/, ''); }
  line = line.replace(/^(\s*)((?:private|public|protected|readonly)\s+)+/, '$1');
  kept.push(line);
}
let s = kept.join('\n');

// ---- pass 2: annotations, casts and type arguments, with a cursor over code only ---------------
const CONTROL = new Set(['if', 'for', 'while', 'switch', 'catch', 'return', 'typeof', 'await', 'new']);

function stripParams(p) {
  // p: the text between ( and ); remove `?` and `: T` of each top-level parameter.
  let out = '';
  let i = 0;
  while (i < p.length) {
    const k = skipNonCode(p, i);
    if (k !== i) { out += p.slice(i, k); i = k; continue; }
    const c = p[i];
    if (c === '(' || c === '[' || c === '{') { const e = matchClose(p, i); out += stripExpr(p.slice(i, e + 1)); i = e + 1; continue; }
    if (c === '?' && p[i + 1] === ':') { i += 1; continue; }
    if (c === ':') { i = typeEnd(p, i + 1); continue; }
    out += c;
    i += 1;
  }
  return out;
}

function stripExpr(t) {
  let out = '';
  let i = 0;
  while (i < t.length) {
    const k = skipNonCode(t, i);
    if (k !== i) {
      const piece = t.slice(i, k);
      out += piece[0] === '`' ? stripTemplate(piece) : piece;
      i = k;
      continue;
    }
    // `x as T`
    let m = /^\sas\s+/.exec(t.slice(i));
    if (m && /[\w$)\]]/.test(t[i - 1] || '')) { i = typeEnd(t, i + m[0].length); continue; }
    // declarations `const x: T` / `let x: T`
    m = /^(const|let|var)\s+[A-Za-z_$][\w$]*\s*:/.exec(t.slice(i));
    if (m && !/[\w$]/.test(t[i - 1] || '')) {
      out += m[0].slice(0, -1);
      i = typeEnd(t, i + m[0].length);
      continue;
    }
    // `class Name<T> extends Base<U> implements A, B {`: type parameters, type arguments and the
    // implements clause go
    m = /^(class\s+[A-Za-z_$][\w$]*)(\s*<[^{]*?>)?(\s+extends\s+[A-Za-z_$][\w$.]*)?(\s*<[^{]*?>)?\s+implements\s+[^{]*\{/
      .exec(t.slice(i));
    if (m && !/[\w$]/.test(t[i - 1] || '')) {
      out += m[1] + (m[3] || '') + ' {';
      i += m[0].length;
      continue;
    }
    // type parameters of a class: `class Name<T, U>`
    m = /^class\s+[A-Za-z_$][\w$]*\s*</.exec(t.slice(i));
    if (m && !/[\w$]/.test(t[i - 1] || '')) {
      out += m[0].slice(0, -1);
      i = matchClose(t, i + m[0].length - 1) + 1;
      continue;
    }
    // class fields at line start: `  name?: T` followed by = or ;
    m = /^\n(\s+)([A-Za-z_$][\w$]*)\??:\s/.exec(t.slice(i));
    if (m) {
      // (an object literal continued on a new line, `  key: 1, ...`, is not a field: its value
      // does not parse as a type followed by ; or =)
      let e = -1;
      try { e = typeEnd(t, i + m[0].length - 1); } catch (err) { e = -1; }
      const after = e < 0 ? -1 : skipSpace(t, e);
      if (e >= 0 && (t[after] === ';' || t[after] === '=')) { out += `\n${m[1]}${m[2]}`; i = e; continue; }
    }
    // type arguments `name<...>(`
    if (t[i] === '<' && /[\w$]/.test(t[i - 1] || '') && t[i - 1] !== ' ') {
      try {
        const e = matchClose(t, i);
        if (t[e + 1] === '(' && /^[\w$., \[\]|]*$/.test(t.slice(i + 1, e))) { i = e + 1; continue; }
      } catch (err) { /* a comparison: keep */ }
    }
    if (t[i] === '(') {
      const e = matchClose(t, i);
      const before = /([A-Za-z_$][\w$]*)\s*$/.exec(out);
      const word = before ? before[1] : '';
      let j = skipSpace(t, e + 1);
      let ret = -1;
      if (t[j] === ':') {
        try { const r = skipSpace(t, typeEnd(t, j + 1)); ret = j; j = r; } catch (err) { ret = -1; }
      }
      // a definition: parameters followed by a body (not after if / for / while / ...) or by =>
      const arrow = t[j] === '=' && t[j + 1] === '>';
      const isDef = arrow || (t[j] === '{' && !CONTROL.has(word));
      if (!isDef) j = skipSpace(t, e + 1);
      const inner = t.slice(i + 1, e);
      out += '(' + (isDef ? stripParams(inner) : stripExpr(inner)) + ')';
      i = e + 1;
      if (isDef && ret >= 0) { out += ' '; i = j; }
      continue;
    }
    out += t[i];
    i += 1;
  }
  return out;
}

function stripTemplate(piece) {
  let out = '';
  let i = 0;
  while (i < piece.length) {
    if (piece[i] === '$' && piece[i + 1] === '{') {
      const e = matchClose(piece, i + 1);
      out += '${' + stripExpr(piece.slice(i + 2, e)) + '}';
      i = e + 1;
    } else { out += piece[i]; i += 1; }
  }
  return out;
}

s = stripExpr(s);
s = "'use strict';\n" + s.replace(/^'use strict';\n/, '') + `\nmodule.exports = { ${exported.join(', ')} };\n`;
fs.writeFileSync(process.argv[3], s);
