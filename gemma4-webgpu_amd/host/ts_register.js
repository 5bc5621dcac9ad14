'use strict';
// Runs the host's TypeScript sources on Node without a TypeScript compiler:
// a require() hook for `.ts` files that erases the type-only syntax and maps
// ES import/export to CommonJS. Emitted code keeps every line where it was
// (stack traces point at the .ts source).
//
// Supported (the subset the host sources are written in):
//   import { a, b } from './x';   import * as n from 'x';   import type ...;
//   export function / class / const / let;   export interface / type
//   interface X { ... }   type X = ...;   declare ...;
//   annotations on parameters, return types, variables and class fields;
//   optional parameters (x?: T);   `expr as T`;   `implements I`;
//   access modifiers on class members (private/public/protected/readonly).
// Not supported (and not used): enums, namespaces, decorators, generic
// parameters on functions, non-null `!`, parameter properties, annotated
// arrow-function parameters, regular-expression literals, and type syntax
// inside template-literal interpolations.

const fs = require('fs');
const Module = require('module');

// ---- tokenizer -----------------------------------------------------------

function tokenize(src) {
  const toks = [];
  let i = 0;
  const n = src.length;
  const push = (type, s, e) => toks.push({ type, text: src.slice(s, e) });
  while (i < n) {
    const c = src[i];
    const s = i;
    if (c === ' ' || c === '\t' || c === '\r' || c === '\n') {
      while (i < n && /[ \t\r\n]/.test(src[i])) i++;
      push('ws', s, i);
    } else if (c === '/' && src[i + 1] === '/') {
      while (i < n && src[i] !== '\n') i++;
      push('comment', s, i);
    } else if (c === '/' && src[i + 1] === '*') {
      const e = src.indexOf('*/', i + 2);
      i = e < 0 ? n : e + 2;
      push('comment', s, i);
    } else if (c === '"' || c === "'") {
      i++;
      while (i < n && src[i] !== c) i += src[i] === '\\' ? 2 : 1;
      i++;
      push('str', s, i);
    } else if (c === '`') {
      i++;
      let depth = 0;
      while (i < n) {
        if (src[i] === '\\') { i += 2; continue; }
        if (depth === 0 && src[i] === '`') { i++; break; }
        if (src[i] === '$' && src[i + 1] === '{') { depth++; i += 2; continue; }
        if (depth > 0 && src[i] === '}') { depth--; i++; continue; }
        i++;
      }
      push('str', s, i);
    } else if (/[A-Za-z_$]/.test(c)) {
      while (i < n && /[A-Za-z0-9_$]/.test(src[i])) i++;
      push('id', s, i);
    } else if (/[0-9]/.test(c)) {
      while (i < n && /[0-9A-Za-z_.]/.test(src[i])) i++;
      push('num', s, i);
    } else {
      const three = src.slice(i, i + 3), two = src.slice(i, i + 2);
      if (['===', '!==', '...', '**=', '>>>', '<<=', '>>='].includes(three)) i += 3;
      else if (['=>', '==', '!=', '<=', '>=', '&&', '||', '??', '?.', '++', '--', '+=', '-=', '*=', '/=',
        '|=', '&=', '**', '<<', '>>'].includes(two)) i += 2;
      else i += 1;
      push('punct', s, i);
    }
  }
  return toks;
}

// ---- stripper ----------------------------------------------------------------

const MODIFIERS = new Set(['private', 'public', 'protected', 'readonly', 'abstract', 'override']);
const OPEN = { '(': ')', '[': ']', '{': '}', '<': '>' };

function strip(src) {
  const t = tokenize(src);
  const out = t.map((x) => x.text);
  const exported = [];
  const sig = (i) => { while (i < t.length && (t[i].type === 'ws' || t[i].type === 'comment')) i++; return i; };
  const prevSig = (i) => { i--; while (i >= 0 && (t[i].type === 'ws' || t[i].type === 'comment')) i--; return i; };
  const is = (i, text) => i < t.length && t[i].text === text && t[i].type !== 'str';
  // Blank out tokens [a, b) keeping newlines, so line numbers survive.
  const erase = (a, b) => { for (let k = a; k < b; k++) out[k] = t[k].text.replace(/[^\n]/g, ' '); };

  // End (exclusive) of a type expression starting at i: stops at a stop-set token at depth 0.
  function typeEnd(i, stops) {
    let depth = 0;
    for (; i < t.length; i++) {
      const x = t[i];
      if (x.type === 'ws' || x.type === 'comment' || x.type === 'str') continue;
      if (depth === 0 && stops.includes(x.text)) return i;
      if (x.text === '=>' && depth === 0 && !stops.includes('=>')) continue;
      if ('([{<'.includes(x.text)) depth++;
      else if (')]}>'.includes(x.text)) {
        if (depth === 0) return i;
        depth--;
      }
    }
    return t.length;
  }
  // Index of the bracket matching the opener at i.
  function match(i) {
    const open = t[i].text, close = OPEN[open];
    let depth = 0;
    for (let k = i; k < t.length; k++) {
      if (t[k].type === 'str' || t[k].type === 'comment') continue;
      if (t[k].text === open) depth++;
      else if (t[k].text === close && --depth === 0) return k;
    }
    throw new Error('ts_register: unbalanced ' + open);
  }
  // Strip annotations inside a parameter list (open paren at i); returns the close index.
  function params(i) {
    const close = match(i);
    let k = sig(i + 1);
    while (k < close) {
      // one parameter: [...]name[?][: T][= default]
      if (t[k].text === '...') k = sig(k + 1);
      if (t[k].text === '{' || t[k].text === '[') k = match(k) + 1;
      else k++;
      let j = sig(k);
      if (is(j, '?')) { erase(j, j + 1); j = sig(j + 1); }
      if (is(j, ':')) {
        const e = typeEnd(j + 1, [',', '=', ')']);
        erase(j, e);
        j = e;
      }
      // skip a default value to the next top-level comma
      let depth = 0;
      for (; j < close; j++) {
        const x = t[j].text;
        if (t[j].type === 'str') continue;
        if ('([{'.includes(x)) depth++;
        else if (')]}'.includes(x)) depth--;
        else if (x === ',' && depth === 0) break;
      }
      k = sig(j + 1);
    }
    return close;
  }
  // Return type after a parameter list closing at c: `: T` up to `{` or `=>`.
  function returnType(c) {
    const j = sig(c + 1);
    if (!is(j, ':')) return;
    const e = typeEnd(j + 1, ['{', '=>', ';']);
    erase(j, e);
  }
  function removeDecl(i) {  // interface/type/declare statement starting at token i
    let k = i;
    for (; k < t.length; k++) {
      if (t[k].type === 'str' || t[k].type === 'comment') continue;
      if (t[k].text === '{') { k = match(k); if (t[i].text === 'interface') break; continue; }
      if (t[k].text === '(' || t[k].text === '[') { k = match(k); continue; }
      if (t[k].text === ';') break;
    }
    erase(i, k + 1);
    return k + 1;
  }

  function classBody(open) {
    const close = match(open);
    let k = sig(open + 1);
    while (k < close) {
      const start = k;
      let j = k;
      while (t[j].type === 'id' && MODIFIERS.has(t[j].text) && t[sig(j + 1)].type === 'id') j = sig(j + 1);
      if (t[j].text === 'static') j = sig(j + 1);
      if (t[j].text === 'get' || t[j].text === 'set') { const q = sig(j + 1); if (t[q].type === 'id') j = q; }
      const name = j;
      let q = sig(name + 1);
      if (is(q, '?')) q = sig(q + 1);
      if (is(q, '(')) {  // method
        for (let m = start; m < name; m++) if (t[m].type === 'id' && MODIFIERS.has(t[m].text)) erase(m, m + 1);
        const c = params(q);
        returnType(c);
        let b = sig(c + 1);
        while (b < close && t[b].text !== '{') b++;
        const be = match(b);
        walk(b + 1, be);
        k = sig(be + 1);
        continue;
      }
      // field: [mods] name[?|!][: T][= init];
      let e = q;
      if (is(e, ':')) e = typeEnd(e + 1, ['=', ';']);
      if (is(sig(e), '=')) {
        for (let m = start; m < name; m++) if (t[m].type === 'id' && MODIFIERS.has(t[m].text)) erase(m, m + 1);
        erase(sig(name + 1), sig(e));
        let z = sig(e) + 1, depth = 0;
        for (; z < close; z++) {
          if (t[z].type === 'str') continue;
          const x = t[z].text;
          if ('([{'.includes(x)) depth++;
          else if (')]}'.includes(x)) depth--;
          else if (x === ';' && depth === 0) break;
        }
        walk(sig(e) + 1, z);
        k = sig(z + 1);
      } else {  // declaration only: drop it
        let z = sig(e);
        erase(start, z + 1);
        k = sig(z + 1);
      }
    }
    return close;
  }

  function walk(a, b) {
    for (let i = a; i < b; i++) {
      const x = t[i];
      if (x.type !== 'id' && x.type !== 'punct') continue;
      const p = prevSig(i);
      const atStmt = p < 0 || [';', '{', '}'].includes(t[p].text) || (t[p].text === 'export');
      if (x.text === 'import' && atStmt && p < 0 || x.text === 'import' && atStmt) {
        let e = i;
        while (e < t.length && t[e].text !== ';') e++;
        const body = t.slice(i, e).filter((y) => y.type !== 'ws' && y.type !== 'comment').map((y) => y.text);
        if (body[1] === 'type') { erase(i, e + 1); i = e; continue; }
        const from = body.indexOf('from');
        const mod = body[from + 1];
        let lhs;
        if (body[1] === '*') lhs = body[3];
        else if (body[1] === '{') lhs = '{ ' + body.slice(2, body.indexOf('}')).join(' ').replace(/ ,/g, ',') + ' }';
        else lhs = body[1];
        erase(i, e);
        out[i] = `const ${lhs} = require(${mod})`;
        i = e;
        continue;
      }
      if (x.text === 'export' && atStmt) {
        const j = sig(i + 1);
        erase(i, j);
        const kw = t[j].text;
        if (kw === 'interface' || kw === 'type' || kw === 'declare') { i = removeDecl(j) - 1; continue; }
        if (kw === 'function' || kw === 'class') exported.push(t[sig(j + 1)].text);
        else if (kw === 'const' || kw === 'let') exported.push(t[sig(j + 1)].text);
        continue;
      }
      if ((x.text === 'interface' || x.text === 'declare') && atStmt && t[sig(i + 1)].type === 'id') {
        i = removeDecl(i) - 1;
        continue;
      }
      if (x.text === 'type' && atStmt && t[sig(i + 1)].type === 'id' && is(sig(sig(i + 1) + 1), '=')) {
        i = removeDecl(i) - 1;
        continue;
      }
      if (x.text === 'function') {
        let j = sig(i + 1);
        if (t[j].type === 'id') j = sig(j + 1);
        if (is(j, '(')) { const c = params(j); returnType(c); i = c; }
        continue;
      }
      if (x.text === 'class') {
        let j = sig(i + 1);
        while (j < t.length && t[j].text !== '{') {
          if (t[j].text === 'implements') {
            let e = j;
            while (t[e].text !== '{') e++;
            erase(j, e);
            j = e;
            break;
          }
          j++;
        }
        i = classBody(j);
        continue;
      }
      if ((x.text === 'const' || x.text === 'let' || x.text === 'var')) {
        const nm = sig(i + 1);
        if (t[nm].type === 'id') {
          const c = sig(nm + 1);
          if (is(c, ':')) erase(c, typeEnd(c + 1, ['=', ';', ',']));
        }
        continue;
      }
      if (x.text === 'as' && p >= 0 && (t[p].type === 'id' || t[p].type === 'str' || t[p].type === 'num' ||
          [')', ']', '}'].includes(t[p].text))) {
        const e = typeEnd(i + 1, [')', ',', ';', ']', '}', '=', '?', ':']);
        erase(i, e);
        i = e - 1;
        continue;
      }
      if (x.text === '(') {
        // arrow-function parameter list with a return type: (...): T =>
        const c = match(i);
        const j = sig(c + 1);
        if (is(j, '=>')) { params(i); }
        else if (is(j, ':')) {
          const e = typeEnd(j + 1, ['=>', ';', ',', ')']);
          if (is(e, '=>')) { params(i); erase(j, e); }
        }
      }
    }
  }

  walk(0, t.length);
  let js = out.join('');
  if (exported.length) js += '\n' + exported.map((nm) => `exports.${nm} = ${nm};`).join(' ') + '\n';
  return js;
}

function register() {
  if (Module._extensions['.ts']) return;
  Module._extensions['.ts'] = function compileTs(module, filename) {
    const js = strip(fs.readFileSync(filename, 'utf8'));
    module._compile(js, filename);
  };
}

module.exports = { strip, register, tokenize };
