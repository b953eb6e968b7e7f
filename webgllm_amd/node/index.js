'use strict'
/**
 * HipGpu: the reference's GPU-backend contract (class Gpu,
 * src/gpu/gl.ts:47; PendingRead and GpuError, src/gpu/types.ts:12-14) over
 * the N-API addon webgllm_hip.node and libwebgllm_hip.so, plus an `ops`
 * object of native kernels, which an engine detects as it detects
 * `nativeProgram` on WebGPU (src/engine.ts:5039). A texture is a flat
 * device buffer with the same bytes, rows of `width` texels.
 *
 * CommonJS, so that Node 12 loads it as it is.
 */
const path = require('path')

const addon = require(path.join(__dirname, 'webgllm_hip.node'))

/** The WebGL 2 formats the engine makes textures in (src/gpu/types.ts:21-41). */
const GL = {
  RGBA32F: 0x8814,
  RGBA4: 0x8056,
  RGBA8: 0x8058,
  RGBA16F: 0x881a,
  R32F: 0x822e,
  R32UI: 0x8236,
  R8UI: 0x8232,
  RGBA32UI: 0x8d70,
  RGBA8UI: 0x8d7c,
  RGBA8I: 0x8d8e
}

/** Bytes a texel of each format holds. */
const TEXEL_BYTES = {
  [GL.RGBA32F]: 16,
  [GL.RGBA4]: 2,
  [GL.RGBA8]: 4,
  [GL.RGBA16F]: 8,
  [GL.R32F]: 4,
  [GL.R32UI]: 4,
  [GL.R8UI]: 1,
  [GL.RGBA32UI]: 16,
  [GL.RGBA8UI]: 4,
  [GL.RGBA8I]: 4
}

class GpuError extends Error {}

/** The addon's errors as GpuError, keeping the status name and number. */
function rethrow (e) {
  if (e && e.name === 'GpuError' && !(e instanceof GpuError)) {
    const g = new GpuError(e.message)
    g.code = e.code
    g.status = e.status
    throw g
  }
  throw e
}

function call (fn, ...args) {
  try {
    return fn(...args)
  } catch (e) {
    rethrow(e)
  }
}

function bytesOf (view) {
  return Buffer.from(view.buffer, view.byteOffset, view.byteLength)
}

/** A rectangle's texels as floats, out of the rows [rect.y, rect.y + height) read whole. */
function cut (ab, t, rect, texel) {
  if (rect.x === 0 && rect.width === t.width) return new Float32Array(ab)
  const out = new Uint8Array(rect.width * rect.height * texel)
  const all = new Uint8Array(ab)
  for (let r = 0; r < rect.height; r++) {
    const s = (r * t.width + rect.x) * texel
    out.set(all.subarray(s, s + rect.width * texel), r * rect.width * texel)
  }
  return new Float32Array(out.buffer)
}

/** A device operand as the addon takes it: a texture, or a view of one (gpu.view). */
function operand (t) {
  if (t === null || t === undefined) return null
  if (t.viewOf) return [t.viewOf.tex, t.offset]
  return t.tex
}

/** An object's texture fields as operands, its other fields as they are. */
function operands (o) {
  if (!o) return null
  const out = {}
  for (const [k, v] of Object.entries(o)) out[k] = v && typeof v === 'object' && ('tex' in v || 'viewOf' in v) ? operand(v) : v
  return out
}

/** A QuantMatrix {N, K, layout, zero, quants, scales?, zeros?} with textures. */
function matrix (w) {
  return {
    N: w.N,
    K: w.K,
    layout: w.layout,
    zero: w.zero,
    quants: operand(w.quants),
    scales: operand(w.scales),
    zeros: operand(w.zeros)
  }
}

class HipGpu {
  constructor (device = 0) {
    this.ctx = call(addon.ctxCreate, device)
    const lim = call(addon.ctxLimits, this.ctx)
    // GpuLimits (src/gpu/types.ts:3-9) from the device: a texture is one
    // allocation, so its side is bounded by the bytes an allocation may
    // take at 16 bytes a texel (and by the 32-bit texel offsets the kernels
    // use); a launch's operands are pointers in HIP's 4 KiB of kernel
    // arguments, 8 bytes each, which bounds both inputs and outputs.
    const KERNARG_BYTES = 4096
    this.limits = {
      maxTextureSize: Math.min(2 ** 31 - 1, Math.floor(lim.maxAllocBytes / 16)),
      maxDrawBuffers: KERNARG_BYTES / 8,
      maxTextureUnits: KERNARG_BYTES / 8,
      renderer: lim.renderer,
      computeUnits: lim.computeUnits,
      globalBytes: lim.globalBytes,
      maxAllocBytes: lim.maxAllocBytes,
      ldsBytesPerBlock: lim.ldsBytesPerBlock,
      waveSize: lim.waveSize
    }
    this.nextId = 1
    this.live = new Set()
    this.lost = false
  }

  /** Device bytes the textures hold (Gpu.bytes). */
  get bytes () { return call(addon.bytesLive, this.ctx) }

  isLost () { return this.lost }

  /** Gpu.texture (gl.ts:263-305). `data.pixels`: the texels' bytes, row-major. */
  texture (internal, width, height, data) {
    if (!(width >= 1 && height >= 1)) throw new GpuError(`A ${width}×${height} texture is empty.`)
    const max = this.limits.maxTextureSize
    if (width > max || height > max) throw new GpuError(`A ${width}×${height} texture is over this GPU's ${max}-texel limit.`)
    const bytes = width * height * (TEXEL_BYTES[internal] || 16)
    if (bytes > this.limits.maxAllocBytes) throw new GpuError(`A ${bytes}-byte texture is over this GPU's allocation limit.`)
    let init = null
    if (data) {
      init = bytesOf(data.pixels)
      if (init.length !== bytes) throw new GpuError(`${init.length} bytes for a ${bytes}-byte texture.`)
    }
    const tex = call(addon.bufCreate, this.ctx, bytes, init)
    const t = { id: this.nextId++, tex, width, height, internal, bytes }
    this.live.add(t)
    return t
  }

  /** A byte-addressed view into a texture, for an op's operand (rows of a batch, a cache row). */
  view (t, byteOffset) {
    if (!(byteOffset >= 0 && byteOffset <= t.bytes)) throw new GpuError(`Offset ${byteOffset} is outside a ${t.bytes}-byte texture.`)
    return { viewOf: t, offset: byteOffset }
  }

  /** Gpu.write (gl.ts:354-374): the rectangle's texels, row by row. */
  write (target, rect, data) {
    const texel = target.bytes / (target.width * target.height)
    const src = bytesOf(data.pixels)
    const rowBytes = rect.width * texel
    if (src.length < rowBytes * rect.height) throw new GpuError('Too few bytes for the rectangle.')
    if (rect.x === 0 && rect.width === target.width) {
      call(addon.bufWrite, this.ctx, target.tex, rect.y * rowBytes, src.subarray(0, rowBytes * rect.height))
      return
    }
    for (let r = 0; r < rect.height; r++) {
      const off = ((rect.y + r) * target.width + rect.x) * texel
      call(addon.bufWrite, this.ctx, target.tex, off, src.subarray(r * rowBytes, (r + 1) * rowBytes))
    }
  }

  /** Bytes into a texture at a byte offset (an upload of ids, a position). */
  writeBytes (target, byteOffset, view) {
    call(addon.bufWrite, this.ctx, target.tex, byteOffset, bytesOf(view))
  }

  /** Gpu.zero (gl.ts:710-726). */
  zero (t) { call(addon.bufZero, this.ctx, t.tex) }

  /** Gpu.delete (gl.ts:448-461). */
  delete (t) {
    if (!this.live.delete(t)) return
    call(addon.bufDelete, this.ctx, t.tex)
  }

  /**
   * Gpu.readStart (gl.ts:740-782): the rectangle's bytes read back behind
   * the work already queued, as a PendingRead: call it for a Promise of the
   * floats (polling the fence between event-loop turns), or cancel it.
   */
  readStart (t, rect = { x: 0, y: 0, width: t.width, height: t.height }) {
    const texel = t.bytes / (t.width * t.height)
    const band = rect.height * t.width * texel
    const fence = call(addon.readStart, this.ctx, t.tex, rect.y * t.width * texel, band)
    let done = false
    const wait = async () => {
      if (done) throw new Error('This read was cancelled or already taken.')
      while (!call(addon.fenceReady, fence)) await new Promise((resolve) => setImmediate(resolve))
      done = true
      return cut(call(addon.readFinish, fence, band), t, rect, texel)
    }
    return Object.assign(wait, {
      cancel: () => {
        if (done) return
        done = true
        call(addon.readCancel, fence)
      }
    })
  }

  /** Gpu.read: readStart, awaited. */
  read (t, rect) { return this.readStart(t, rect)() }

  /** Gpu.readNow (gl.ts:658-700): blocking. */
  readNow (t, rect = { x: 0, y: 0, width: t.width, height: t.height }) {
    const texel = t.bytes / (t.width * t.height)
    const band = rect.height * t.width * texel
    const ab = call(addon.readNow, this.ctx, t.tex, rect.y * t.width * texel, band)
    return cut(ab, t, rect, texel)
  }

  /** A texture's bytes [byteOffset, byteOffset + bytes), blocking (Gpu.readBytes, gl.ts:786-835). */
  readBytes (t, byteOffset = 0, bytes = t.bytes - byteOffset) {
    return call(addon.readNow, this.ctx, t.tex, byteOffset, bytes)
  }

  // PacedGpu's fences (src/gpu/paced.ts:11-22): fence() ends the work issued
  // so far behind a fence, fenceReady looks once, deleteFence drops one, wait
  // resolves once the GPU is past it, readBack blocks until the queue is done.
  fence () { return call(addon.fence, this.ctx) }
  fenceReady (f) { return call(addon.fenceReady, f) }
  deleteFence (f) { call(addon.readCancel, f) }
  async wait (f) {
    if (!f) return
    while (!call(addon.fenceReady, f)) await new Promise((resolve) => setImmediate(resolve))
    call(addon.readFinish, f)
  }

  readBack () {
    this.finish()
    return true
  }

  /** Gpu.flush (gl.ts:729-732); PacedGpu.finish. */
  flush () { call(addon.flush, this.ctx) }
  finish () { call(addon.finish, this.ctx) }

  /** Gpu.dispose (gl.ts:316-331): every texture and the context. */
  dispose () {
    if (this.lost) return
    this.lost = true
    this.live.clear()
    call(addon.ctxDestroy, this.ctx)
  }

  /**
   * Native kernels over textures, one per family of the engine's passes
   * (the way the reference detects `nativeProgram` on WebGPU,
   * src/engine.ts:5039). A matrix is {N, K, layout, zero, quants, scales?,
   * zeros?} with textures holding the QuantMatrix arrays
   * (src/weights.ts:1-31). Operands are textures or views (gpu.view); an
   * operand smaller than its shape needs is refused with a GpuError before
   * anything runs.
   */
  get ops () {
    const ctx = this.ctx
    const o = operand
    const gpu = this
    return {
      /** The loaders' packers on the GPU (packQ4_0, packQ4_K: src/repack.ts:60-168); srcRows an Int32Array. */
      repack: (kind, w, row0, rows, src, srcRows) =>
        call(addon.repack, ctx, kind, matrix(w), row0, rows, o(src), srcRows || null),
      /** matrixRow (src/repack.ts:865-891) into an R32F texture. */
      dequant: (w, row0, rows, out) => call(addon.dequant, ctx, matrix(w), row0, rows, o(out)),
      /** packQ4_K's half scales and zero points of a Q4_K-records matrix (N K / 32 halves each),
       *  kept for the prompt GEMMs: with its quants they form the half-zero-point matrix. */
      q4kRecordHalves: (w, scales, zeros) =>
        call(addon.q4kRecordHalves, ctx, matrix(w), o(scales), o(zeros)),
      /**
       * splitPartials + pf and the passes folded into it (src/engine.ts:5241-5377,
       * src/gpu/kernels.ts:744-895, :1169-1361): y = x W^T for M <= 8 rows of
       * halves, with an epilogue (mode EPI_STORE | EPI_SWIGLU | EPI_ROPE_KV |
       * EPI_SHORT_CONV: the short conv of convFused over the B | C | x rows,
       * src/gpu/kernels.ts:1447-1523, into out16, convState(Out) and
       * convPrefixes; it throws WG_ERR_UNSUPPORTED for a layout or shape its
       * kernels do not take, where gemv with EPI_STORE and shortConv follow).
       */
      gemv: (w, x, M, y, epilogue = null, ldx = null, ldy = null) =>
        call(addon.gemv, ctx, matrix(w), o(x), M, o(y), operands(epilogue), ldx, ldy),
      /** Engine.matmul for a prompt batch (src/engine.ts:4969-5234): {lda, ldc, residual, ldr, rowScale, colOf}. */
      gemm: (w, A, M, C, opts = null) => call(addon.gemm, ctx, matrix(w), o(A), M, o(C), operands(opts)),
      /** The gate|up GEMM with SwiGLU folded in (src/gpu/native.ts:33). */
      gemmSwiglu: (w, A, M, out16, rowScale = null, lda = null, ldo = null) =>
        call(addon.gemmSwiglu, ctx, matrix(w), o(A), M, o(out16), o(rowScale), lda, ldo),
      /** embed / embedFold (src/gpu/kernels.ts:1092-1149, :985-1041). */
      embed: (w, ids, M, h, epilogue = null, ldh = null) =>
        call(addon.embed, ctx, matrix(w), o(ids), M, o(h), operands(epilogue), ldh),
      /** NORM_TO_H2 with PRESCALE (src/gpu/kernels.ts:89, :1195-1242). */
      normToH2: (x, M, D, w, eps, out, rowScale, ldx = null, ldo = null) =>
        call(addon.normToH2, ctx, o(x), M, D, o(w), eps, o(out), o(rowScale), ldx, ldo),
      /** headPrep + values (src/gpu/kernels.ts:2196-2322, :3030-3045). */
      headPrep: (qkv, M, shape, qNorm, kNorm, rope, ropeRows, pos0, qOut, kCache, vCache, ctxRows, ldq = null, ldqo = null) =>
        call(addon.headPrep, ctx, o(qkv), M, shape, o(qNorm), o(kNorm), o(rope), ropeRows, o(pos0), o(qOut), o(kCache), o(vCache), ctxRows, ldq, ldqo),
      attnScratchBytes: (M, heads, headDim, maxKeys) => addon.attnScratchBytes(M, heads, headDim, maxKeys),
      /** scores / attend / attendPanel + combine (src/gpu/kernels.ts:2386-2579, :2803-3027). */
      attnDecode: (q, M, shape, kCache, vCache, pos0, maxKeys, out, scratch, ldq = null, ldo = null) =>
        call(addon.attnDecode, ctx, o(q), M, shape, o(kCache), o(vCache), o(pos0), maxKeys, o(out), o(scratch), ldq, ldo),
      /**
       * headPrep + attnDecode in one launch, the heads prepared inside the
       * attention (the same bits); throws WG_ERR_UNSUPPORTED where the
       * kernel does not take the shape (then the two calls).
       */
      attnDecodePrep: (qkv, M, shape, qNorm, kNorm, rope, ropeRows, pos0, kCache, vCache, ctxRows, out, scratch,
                       qOut = null, ldqkv = null, ldo = null) =>
        call(addon.attnDecodePrep, ctx, o(qkv), M, shape, o(qNorm), o(kNorm), o(rope), ropeRows, o(pos0),
             o(kCache), o(vCache), ctxRows, o(out), o(scratch), o(qOut), ldqkv, ldo),
      /** The prompt's attention plan (src/engine.ts:6359-6630). */
      attnPrefill: (q, M, shape, kCache, vCache, pos0, maxKeys, out, ldq = null, ldo = null) =>
        call(addon.attnPrefill, ctx, o(q), M, shape, o(kCache), o(vCache), o(pos0), maxKeys, o(out), ldq, ldo),
      /** convFused + convPrefixes (src/gpu/kernels.ts:1447-1523; Engine.convolve, src/engine.ts:5806-5899). */
      shortConv: (bcx, M, D, W, taps, state, stateOut, prefixes, out, ldb = null, ldo = null) =>
        call(addon.shortConv, ctx, o(bcx), M, D, W, o(taps), o(state), o(stateOut), o(prefixes), o(out), ldb, ldo),
      /** Engine.accept's rollback (src/engine.ts:8063-8086). */
      convAccept: (prefixes, kept, rows, D, W, state) =>
        call(addon.convAccept, ctx, o(prefixes), kept, rows, D, W, o(state)),
      /** The conv layers' rollback operands as a device table for verifyAccept (a texture the caller deletes). */
      convStates: (layers, rows) => {
        const tex = call(addon.convStates, ctx, layers.map((l) => ({ prefixes: o(l.prefixes), state: o(l.state), dim: l.dim, width: l.width })), rows)
        const bytes = layers.length * addon.constants.CONV_STATE_BYTES
        const t = { id: gpu.nextId++, tex, width: bytes, height: 1, internal: GL.R8UI, bytes }
        gpu.live.add(t)
        return t
      },
      /** Engine.accept after a verify batch with the handler's keep rule (src/handler.ts:1811-1887), on the device. */
      verifyAccept: (picks, rows, convs, nConv, maxState, pos, ids, hist, histLen, keptLog, logLen, cursor) =>
        call(addon.verifyAccept, ctx, o(picks), rows, o(convs), nConv, maxState, o(pos), o(ids), o(hist), histLen, o(keptLog), logLen, o(cursor)),
      /** argmaxParts + verifyAccept in one launch (the picks also to picksOut). */
      verifyAcceptParts: (parts, picksOut, rows, convs, nConv, maxState, pos, ids, hist, histLen, keptLog, logLen, cursor) =>
        call(addon.verifyAcceptParts, ctx, o(parts), o(picksOut), rows, o(convs), nConv, maxState, o(pos), o(ids), o(hist),
             histLen, o(keptLog), logLen, o(cursor)),
      /** verifyDrafts + embed in one launch (rows 1.. from the table's row *cursor, also into ids). */
      embedDrafts: (w, ids, rows, table, nSteps, cursor, h, epilogue = null, ldh = null) =>
        call(addon.embedDrafts, ctx, matrix(w), o(ids), rows, o(table), nSteps, o(cursor), o(h), operands(epilogue), ldh),
      /** A verify step's drafts from a device table (src/draft.ts:15-45 runs on the host). */
      verifyDrafts: (ids, rows, table, nSteps, cursor) =>
        call(addon.verifyDrafts, ctx, o(ids), rows, o(table), nSteps, o(cursor)),
      /** Engine.argmax (src/engine.ts:8271-8336): the first largest logit of each row. */
      argmax: (logits, M, V, ids, scratch, tops = null, ld = null) =>
        call(addon.argmax, ctx, o(logits), M, V, o(ids), o(scratch), o(tops), ld),
      argmaxScratchBytes: (M, V) => addon.argmaxScratchBytes(M, V),
      /** One decode step's pick and advance on the device (src/engine.ts:8095-8110, :8318-8336). */
      argmaxAdvance: (logits, V, ids, pos, hist, histLen, scratch, tops = null) =>
        call(addon.argmaxAdvance, ctx, o(logits), V, o(ids), o(pos), o(hist), histLen, o(scratch), o(tops)),
      /**
       * The picks from a head gemv's epilogue.pickParts (its workgroups'
       * share of CHUNK_MAX_AT, src/gpu/kernels.ts:3169-3246): as argmaxRows
       * over its logits, bit for bit; with pos (M = 1) argmaxAdvance's
       * advance. pickPartsBytes(M) sizes the parts buffer.
       */
      argmaxParts: (parts, M, ids, tops = null, pos = null, hist = null, histLen = 0) =>
        call(addon.argmaxParts, ctx, o(parts), M, o(ids), o(tops), o(pos), o(hist), histLen),
      pickPartsBytes: (M) => addon.pickPartsBytes(M),
      pickScratchBytes: (M, V) => addon.pickScratchBytes(M, V),
      /** Engine.pick's penalized chunk candidates (src/engine.ts:8352-8473). */
      pickCandidates: (logits, M, V, count, chunksOut, candidates, scratch, opts = null) =>
        call(addon.pickCandidates, ctx, o(logits), M, V, count, o(chunksOut), o(candidates), o(scratch), operands(opts))
    }
  }
}

/** The matrix arrays' sizes (src/weights.ts:153-178). */
function quantSizes (N, K, layout = addon.constants.LAYOUT_ROWGROUP, zero = addon.constants.ZERO_8) {
  return call(addon.q4Sizes, N, K, layout, zero)
}

module.exports = {
  HipGpu,
  GpuError,
  GL,
  TEXEL_BYTES,
  quantSizes,
  ggufHeader: (p) => call(addon.ggufHeader, p),
  onnxGraph: (p) => call(addon.onnxGraph, p),
  version: () => addon.version(),
  constants: addon.constants,
  addon
}
