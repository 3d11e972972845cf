"use strict";
/* The C ABI of the MI355X library (include/dj.h) through the N-API addon (dj_napi.cc), wrapped as the Node
 * host's device layer — what gpu.ts's requestDevice / storage buffers / Weight / recorder() give the
 * reference's engines (gpu.ts:38-54, 90-281):
 *   Context    dj_init / dj_destroy; buffers, weights, graphs, timers
 *   DevBuf     a device allocation (dj_buf_*); `at(bytes)` is a pointer inside it
 *   Weight     a quantized (or direct f16) linear on the device (dj_weight_q)
 *   Recorder   one forward: the named ops, snapshot(buf) and finish() (a Promise: the forward runs off the
 *              event loop)
 * Device pointers and handles are BigInt. The addon is built next to libdj.so; a missing build throws. */
const path = require("path");

let addon = null;
function lib() {
  if (!addon) {
    const file = path.join(__dirname, "..", "lib", "dj_napi.node");
    try {
      addon = require(file);
    } catch (e) {
      throw new Error(`decision.js: the native library is not built (${file}): run decision.js_amd/csrc/build.py (${e.message})`);
    }
    if (addon.abiVersion() !== addon.ABI_VERSION) throw new Error("decision.js: libdj.so and its N-API binding disagree on the ABI version");
  }
  return addon;
}

class DevBuf {
  constructor(ctx, ptr, bytes) {
    this.ctx = ctx;
    this.ptr = ptr;
    this.bytes = bytes;
  }
  at(offset) {
    return this.ptr + BigInt(offset);
  }
  write(typed) {
    lib().bufWrite(this.ctx.h, this.ptr, typed);
  }
  upload(typed) {
    lib().upload(this.ctx.h, this.ptr, typed);
  }
  copyFrom(src, bytes) {
    lib().bufCopy(this.ctx.h, this.ptr, src.ptr, bytes === undefined ? Math.min(this.bytes, src.bytes) : bytes);
  }
  read(Ctor, n) {
    const out = new Ctor(n);
    lib().bufRead(this.ctx.h, out, this.ptr);
    return out;
  }
  free() {
    if (this.ptr) lib().bufFree(this.ctx.h, this.ptr);
    this.ptr = 0n;
  }
}

class Weight {
  constructor(ctx, h, N, K, bits, layout) {
    Object.assign(this, { ctx, h, N, K, bits, layout, shape: [N, K] });
  }
  get nbytes() {
    return lib().weightBytes(this.h);
  }
  free() {
    if (this.h) lib().weightFree(this.ctx.h, this.h);
    this.h = 0n;
  }
}

class Context {
  constructor(ordinal = 0) {
    this.h = lib().init(ordinal);
  }
  info() {
    return lib().deviceInfo(this.h);
  }
  alloc(bytes) {
    return new DevBuf(this, lib().bufAlloc(this.h, Math.max(bytes, 1)), bytes);
  }
  array(typed) {
    const b = this.alloc(typed.byteLength);
    b.write(typed);
    return b;
  }
  weightQ(codes, scales, N, K, bits, layout) {
    return new Weight(this, lib().weightQ(this.h, codes, scales, N, K, bits, layout), N, K, bits, layout);
  }
  recorder(key = 0n) {
    return new Recorder(this, key);
  }
  graphClear() {
    lib().graphClear(this.h);
  }
  graphDrop(key) {
    lib().graphDrop(this.h, BigInt(key));
  }
  graphCount() {
    return lib().graphCount(this.h);
  }
  timerBegin() {
    lib().timerBegin(this.h);
  }
  timerEnd() {
    return lib().timerEnd(this.h);
  }
  close() {
    if (this.h) lib().destroy(this.h);
    this.h = 0n;
  }
}

class Recorder {
  constructor(ctx, key) {
    this.ctx = ctx;
    const [h, replay] = lib().recBegin(ctx.h, BigInt(key));
    this.h = h;
    this.replay = replay;
    this.snaps = [];
  }
  gatherQ(ids, T, embed, X) { lib().gatherQ(this.h, ids, T, embed.h, X); }
  addRmsnorm(T, H, add, eps, X, Y, w, O) { lib().addRmsnorm(this.h, T, H, add ? 1 : 0, eps, X, Y, w, O); }
  sandwich(T, H, eps, scale, X, Y, w1, w2, O) { lib().sandwich(this.h, T, H, eps, scale, X, Y, w1, w2, O); }
  matmul(X, w, Y, M) { lib().matmul(this.h, X, w.h, Y, M); }
  matmulGlu(X, w, H, M, act) { lib().matmulGlu(this.h, X, w.h, H, M, act); }
  qkNormRope(T, heads, kv, D, stride, Z, qn, kn, vnorm, pos, posStride, eps, theta, rot, mode) {
    lib().qkNormRope(this.h, T, heads, kv, D, stride, Z, qn, kn, vnorm ? 1 : 0, pos, posStride, eps, theta, rot, mode);
  }
  ropeTable(T, pos, posStride, theta, rot, tab, mode = lib().ROPE_POW_NEG) { lib().ropeTable(this.h, T, pos, posStride, theta, rot, mode, tab); }
  matmulResidual(X, w, M, R, nw, XW, SS) { lib().matmulResidual(this.h, X, w.h, M, R, nw, XW, SS); }
  /** act: -1 plain, else a gated activation (ACT_*) */
  matmulNormed(XW, w, Y, M, act, SS, H, eps) { lib().matmulNormed(this.h, XW, w.h, Y, M, act, SS, H, eps); }
  matmulQkvRopeNormed(XW, w, Z, M, heads, kv, D, qn, kn, vnorm, pos, posStride, eps, theta, tab, SS, H, normEps, rot = D,
    mode = lib().ROPE_POW_NEG) {
    lib().matmulQkvRopeNormed(this.h, XW, w.h, Z, M, heads, kv, D, qn, kn, vnorm ? 1 : 0, pos, posStride, eps, theta, rot, mode,
      tab, SS, H, normEps);
  }
  matmulQkvRope(X, w, Z, M, heads, kv, D, qn, kn, vnorm, pos, posStride, eps, theta, tab, rot = D, mode = lib().ROPE_POW_NEG) {
    lib().matmulQkvRope(this.h, X, w.h, Z, M, heads, kv, D, qn, kn, vnorm ? 1 : 0, pos, posStride, eps, theta, rot, mode, tab);
  }
  attention(T, heads, kv, D, Q, qStride, A, B, rng, scale, O) {
    lib().attention(this.h, T, heads, kv, D, Q, qStride, A, B, rng, scale, O);
  }
  attentionQkRope(T, heads, kv, D, Q, qStride, A, B, rng, scale, qn, kn, eps, tab, O, rot = D) {
    lib().attentionQkRope(this.h, T, heads, kv, D, Q, qStride, A, B, rng, scale, qn, kn, eps, tab, rot, O);
  }
  attentionGated(T, heads, kv, D, Q, qStride, A, B, rng, scale, G, gStride, O) {
    lib().attentionGated(this.h, T, heads, kv, D, Q, qStride, A, B, rng, scale, G, gStride, O);
  }
  pleMix(T, P, G, E, w, eps, O) { lib().pleMix(this.h, T, P, G, E, w, eps, O); }
  poolProject(T, S, H, N, X, seqs, W, out) { lib().poolProject(this.h, T, S, H, N, X, seqs, W, out); }
  gdn(T, nspans, spans, LH, stride, Z, convW, Alog, dtBias, gnorm, eps, Y) {
    lib().gdn(this.h, T, nspans, spans, LH, stride, Z, convW, Alog, dtBias, gnorm, eps, Y);
  }
  kvStore(T, kv, D, Z, stride, kCol, cache, row0) { lib().kvStore(this.h, T, kv, D, Z, stride, kCol, cache, row0); }
  meanPool(T, S, H, X, seqs, out) { lib().meanPool(this.h, T, S, H, X, seqs, out); }
  readout(T, P, H, X, R, codes, pairs, out) { lib().readout(this.h, T, P, H, X, R, codes, pairs, out); }
  shortConv(T, H, Z, w, taps, Y) { lib().shortConv(this.h, T, H, Z, w, taps, Y); }
  addRows(T, H, Xi, idx, E, rows, Xo) { lib().addRows(this.h, T, H, Xi, idx, E, rows, Xo); }
  biasAct(T, N, Y, b, act = 0) { lib().biasAct(this.h, T, N, Y, b, act); }
  addLayernorm(T, H, add, eps, X, Y, w, b, O) { lib().addLayernorm(this.h, T, H, add ? 1 : 0, eps, X, Y, w, b, O); }
  gatherRows(M, H, T, X, rows, G) { lib().gatherRows(this.h, M, H, T, X, rows, G); }
  score(M, H, Y, w, b, out) { lib().score(this.h, M, H, Y, w, b, out); }
  denseF32(M, inp, w, out) { lib().denseF32(this.h, M, inp, w.h, out); }
  leafLogits(T, L, H, nIds, eps, X, leaves, w, ids, embed, out) {
    lib().leafLogits(this.h, T, L, H, nIds, eps, X, leaves, w, ids, embed.h, out);
  }
  /** The device bytes at `ptr`, as a new typed array (Ctor, n) filled when the forward completes. */
  snapshot(ptr, Ctor, n) {
    const host = new Ctor(n);
    lib().recSnapshot(this.h, ptr, host);
    this.snaps.push(host);
    return this.snaps.length - 1;
  }
  /** Ends a recording that failed (dj_rec_abort): nothing more runs and the context is free for the next
   * forward. Its own status is not thrown: the error being handled is the one to report. */
  abort() {
    if (!this.h) return;
    const h = this.h;
    this.h = 0n;
    try {
      lib().recAbort(h);
    } catch (e) {
      // the original error is reported by the caller
    }
  }
  /** Runs `body(this)` (the op calls); on any error aborts the recording and rethrows. */
  record(body) {
    try {
      return body(this);
    } catch (e) {
      this.abort();
      throw e;
    }
  }
  /** Submits the forward (or replays its captured graph); resolves to the snapshots. */
  async finish() {
    const h = this.h;
    this.h = 0n;
    await lib().recFinishAsync(h);
    return this.snaps;
  }
}

const kvSrc = (base, rows, stride, kCol, vCol) => ({ base, rows, stride, kCol, vCol });

module.exports = { lib, Context, DevBuf, Weight, Recorder, kvSrc, consts: () => lib() };
