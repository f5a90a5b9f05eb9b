//go:build cqhip

// The cqhip build of package cq: the same API as matrix.go, kernel.go and
// lut.go (which the patch in go/patches moves behind !cqhip), bound by cgo
// to libcqhip.so, the MI355X implementation of the CQ products. A Matrix is
// a handle to the library's device copy of the packed index and FP16 norms;
// views share it. Products on host slices copy their operands within the
// call, as cgo requires of Go memory; the outputs are the lut kernel's bit
// for bit (an Exact view: the nibble4 kernel's).
//
// Not compiled in the repository that ships it (no Go toolchain there): the
// C ABI it calls is the one the repository's tests drive on the CPU and on
// the GPU.
package cq

/*
#cgo CFLAGS: -I${SRCDIR}/../../third_party/cqhip/include
#cgo LDFLAGS: -L${SRCDIR}/../../third_party/cqhip/lib -lcqhip -Wl,-rpath,${SRCDIR}/../../third_party/cqhip/lib
#include <stdlib.h>
#include "cqhip.h"
*/
import "C"

import (
	"errors"
	"fmt"
	"runtime"
	"unsafe"

	"github.com/cwbudde/go-whistle/internal/cact"
)

// Matrix is a 2- or 4-bit CQ matrix [out, in] held on the device (cf.
// matrix.go:22-43). It is safe for concurrent use.
type Matrix struct {
	h       *C.cq_matrix
	out, in int
	bits    int
}

// call runs f on a locked OS thread and returns its status with the
// library's message for it: the message is per thread, and a goroutine may
// move between threads between two cgo calls.
func call(f func() C.int) (C.int, string) {
	runtime.LockOSThread()
	defer runtime.UnlockOSThread()

	rc := f()
	if rc == C.CQ_OK {
		return rc, ""
	}

	return rc, C.GoString(C.cq_last_error())
}

// must panics on any failure, as the CPU build panics on misuse
// (kernel.go:101-103, matrix.go:134-136, 162-164); device failures panic too.
func must(f func() C.int) {
	if rc, msg := call(f); rc != C.CQ_OK {
		panic(msg)
	}
}

func wrap(h *C.cq_matrix) *Matrix {
	m := &Matrix{h: h, out: int(C.cq_out(h)), in: int(C.cq_in(h)), bits: int(C.cq_bits(h))}
	runtime.AddCleanup(m, func(h *C.cq_matrix) { C.cq_free(h) }, h)

	return m
}

func newMatrix(p cact.Packed, gather C.int) (*Matrix, error) {
	var (
		h   *C.cq_matrix
		cb  *C.float
		idx *C.uint8_t
		nrm *C.uint8_t
	)

	if len(p.Codebook) > 0 {
		cb = (*C.float)(unsafe.Pointer(&p.Codebook[0]))
	}

	if len(p.Index) > 0 {
		idx = (*C.uint8_t)(unsafe.Pointer(&p.Index[0]))
	}

	if len(p.Norms) > 0 {
		nrm = (*C.uint8_t)(unsafe.Pointer(&p.Norms[0]))
	}

	rc, msg := call(func() C.int {
		return C.cq_new(C.int(p.Out), C.int(p.In), C.int(p.Group), C.int(p.Bits), C.int(p.Width),
			cb, C.size_t(len(p.Codebook)), idx, C.size_t(len(p.Index)), nrm, C.size_t(len(p.Norms)), gather, &h)
	})
	runtime.KeepAlive(p)

	switch rc {
	case C.CQ_OK:
		return wrap(h), nil
	case C.CQ_ERR_ARG: // the reference's "cq: ..." validation text (matrix.go:61-73)
		return nil, errors.New(msg)
	default:
		panic(fmt.Sprintf("%s (status %d)", msg, int(rc)))
	}
}

// New builds a Matrix from a packed CQ tensor and uploads it (matrix.go:46-55).
func New(p cact.Packed) (*Matrix, error) { return newMatrix(p, 0) }

// NewGather builds a Matrix like New (matrix.go:60-96); the device copy is
// the same, so Prepare has nothing left to do.
func NewGather(p cact.Packed) (*Matrix, error) { return newMatrix(p, 1) }

// Out is the number of rows, the length of y.
func (m *Matrix) Out() int { return m.out }

// In is the number of columns, the length of x.
func (m *Matrix) In() int { return m.in }

// Bits is the index width, 2 or 4.
func (m *Matrix) Bits() int { return m.bits }

// Prepare is kept for the API (matrix.go:111-115).
func (m *Matrix) Prepare() {
	must(func() C.int { return C.cq_prepare(m.h) })
	runtime.KeepAlive(m)
}

// Bytes is the memory the matrix holds, with the reference's accounting
// (matrix.go:121-129).
func (m *Matrix) Bytes() int {
	n := int(C.cq_bytes(m.h))
	runtime.KeepAlive(m)

	return n
}

// Rows returns rows [lo, hi) as a Matrix that shares m's storage
// (matrix.go:133-145).
func (m *Matrix) Rows(lo, hi int) *Matrix {
	var v *C.cq_matrix

	must(func() C.int { return C.cq_rows(m.h, C.int(lo), C.int(hi), &v) })
	runtime.KeepAlive(m)

	return wrap(v)
}

// Exact returns a view whose products run the nibble kernels
// (matrix.go:152-157).
func (m *Matrix) Exact() *Matrix {
	var v *C.cq_matrix

	must(func() C.int { return C.cq_exact(m.h, &v) })
	runtime.KeepAlive(m)

	return wrap(v)
}

// Dense returns a view whose products of 16 or more activations run
// Exact's arithmetic as an fp32 MFMA contraction (within float32 rounding
// of Exact, not bit for bit); fewer run the nibble kernels. It has no
// counterpart in the reference: for batched encoder frames that take
// Exact's semantics.
func (m *Matrix) Dense() *Matrix {
	var v *C.cq_matrix

	must(func() C.int { return C.cq_dense(m.h, &v) })
	runtime.KeepAlive(m)

	return wrap(v)
}

func fptr(s []float32) *C.float {
	if len(s) == 0 {
		return nil
	}

	return (*C.float)(unsafe.Pointer(&s[0]))
}

// Row dequantises row r into dst (len In), bit for bit cact.CQ
// (matrix.go:161-181).
func (m *Matrix) Row(dst []float32, r int) {
	must(func() C.int { return C.cq_row(m.h, fptr(dst), C.size_t(len(dst)), C.int(r)) })
	runtime.KeepAlive(m)
}

// GEMV sets dst = W · x (kernel.go:78-80).
func (m *Matrix) GEMV(dst, x []float32) { m.GEMM(dst, x, 1) }

// GEMM sets dst[r] = W · x[r] for rows activations (kernel.go:85-87).
func (m *Matrix) GEMM(dst, x []float32, rows int) {
	must(func() C.int {
		return C.cq_gemm(m.h, fptr(dst), C.size_t(len(dst)), fptr(x), C.size_t(len(x)), C.int(rows))
	})
	runtime.KeepAlive(m)
}

// GEMMs sets dsts[k] = ms[k].GEMM(x, rows) for matrices that share one input
// (kernel.go:134-158), in one launch per index width.
func GEMMs(ms []*Matrix, dsts [][]float32, x []float32, rows int) {
	if len(ms) != len(dsts) {
		panic(fmt.Sprintf("cq: GEMMs of %d matrices into %d outputs", len(ms), len(dsts)))
	}

	n := len(ms)
	if n == 0 {
		return
	}

	// cgo forbids Go memory that holds Go pointers: the handle, output and
	// length arrays live in C memory, and the output slices stay pinned.
	word := C.size_t(unsafe.Sizeof(uintptr(0)))
	hs := unsafe.Slice((**C.cq_matrix)(C.malloc(C.size_t(n)*word)), n)
	ds := unsafe.Slice((**C.float)(C.malloc(C.size_t(n)*word)), n)
	ls := unsafe.Slice((*C.size_t)(C.malloc(C.size_t(n)*C.size_t(unsafe.Sizeof(C.size_t(0))))), n)

	defer C.free(unsafe.Pointer(&hs[0]))
	defer C.free(unsafe.Pointer(&ds[0]))
	defer C.free(unsafe.Pointer(&ls[0]))

	var pin runtime.Pinner
	defer pin.Unpin()

	for k, m := range ms {
		hs[k] = m.h

		if len(dsts[k]) > 0 {
			pin.Pin(&dsts[k][0])
		}

		ds[k] = fptr(dsts[k])
		ls[k] = C.size_t(len(dsts[k]))
	}

	must(func() C.int {
		return C.cq_gemms(C.int(n), &hs[0], &ds[0], &ls[0], fptr(x), C.size_t(len(x)), C.int(rows))
	})
	runtime.KeepAlive(ms)
}
