;;;; hip-dit.lisp -- ex-nihilo's DiT backend on an AMD MI355X through libexn-hip.so
;;;;
;;;; The backend trio of src/cuda-dit.lisp (upload-dit :52, dit-velocity :137, dit-release :99)
;;;; with the same signatures, so load-engine, generate, edit and decode-latent
;;;; (src/generate.lisp:37,96,102,134) run unchanged.  Listed in ex-nihilo.asd in place of
;;;; cuda-dit on an MI355X host:
;;;;   (:file "hip-dit" :if-feature (:and :sbcl :linux :exn-hip))
;;;; The C side is include/exn_hip.h; every status other than 0 becomes a Lisp error carrying
;;;; exn_last_error().  The library adds txt_in.text_norm's 1 itself, so the vectors go as read.

(in-package #:ex-nihilo)

(sb-alien:load-shared-object
 (or (uiop:getenv "EXN_HIP_LIB")
     (namestring (asdf:system-relative-pathname "ex-nihilo" "lib/libexn-hip.so"))))

(sb-alien:define-alien-routine ("exn_last_error" %exn-last-error) sb-alien:c-string)
(sb-alien:define-alien-routine ("exn_open" %exn-open) sb-alien:int
  (device sb-alien:int) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_dit_create" %exn-dit-create) sb-alien:int
  (ctx sb-sys:system-area-pointer) (layers sb-alien:int) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_dit_set" %exn-dit-set) sb-alien:int
  (d sb-sys:system-area-pointer) (name sb-alien:c-string) (kind sb-alien:int)
  (data sb-sys:system-area-pointer) (d0 (sb-alien:signed 64)) (d1 (sb-alien:signed 64)))
(sb-alien:define-alien-routine ("exn_dit_check" %exn-dit-check) sb-alien:int (d sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_dit_velocity" %exn-dit-velocity) sb-alien:int
  (d sb-sys:system-area-pointer) (context sb-sys:system-area-pointer) (p sb-alien:int)
  (latent sb-sys:system-area-pointer) (h sb-alien:int) (w sb-alien:int) (sigma sb-alien:double)
  (prefix-key (sb-alien:unsigned 64)) (ref-a sb-alien:int) (ref-latent sb-sys:system-area-pointer)
  (rh sb-alien:int) (rw sb-alien:int) (v sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_dit_release" %exn-dit-release) sb-alien:int (d sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_dit_w8a8" %exn-dit-w8a8) sb-alien:int
  (d sb-sys:system-area-pointer) (on sb-alien:int))
(sb-alien:define-alien-routine ("exn_dit_resident" %exn-dit-resident) sb-alien:int
  (d sb-sys:system-area-pointer) (bf16 sb-alien:int))
(sb-alien:define-alien-routine ("exn_dit_profile" %exn-dit-profile) sb-alien:int
  (d sb-sys:system-area-pointer) (on sb-alien:int))
(sb-alien:define-alien-routine ("exn_dit_profile_read" %exn-dit-profile-read) sb-alien:int
  (d sb-sys:system-area-pointer) (cls sb-alien:int) (ms sb-sys:system-area-pointer)
  (launches sb-sys:system-area-pointer) (flops sb-sys:system-area-pointer) (bytes sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_dit_stats" %exn-dit-stats) sb-alien:int
  (d sb-sys:system-area-pointer) (on sb-alien:int))
(sb-alien:define-alien-routine ("exn_dit_stats_read" %exn-dit-stats-read) sb-alien:int
  (d sb-sys:system-area-pointer) (maxabs sb-sys:system-area-pointer) (nonfinite sb-sys:system-area-pointer)
  (records (sb-alien:signed 64)))

(defvar *int8* nil
  "cuda-dit.lisp's switch (src/cuda-dit.lisp:110-113): true takes every Q8_0 product of 16 rows
   or more as int8 activations (quant_q8 by blocks of 32, the int8 MFMA) -- the CUDA backend's
   default numerics; false (here the default: several times faster on the MI355X, and nearer the
   float reference) multiplies bf16 activations by the exact bf16 dequantisation.")

(defvar *hip-resident* t
  "No counterpart in the reference, whose products read the Q8_0 weights: true (the default)
   keeps a resident bf16 expansion of each block matrix beside its Q8_0 codes -- 14 GB more for
   the DiT, the step about 7% faster on the MI355X; the prompt encoder makes its expansions for
   prompts of more than 256 tokens only -- and false multiplies from the Q8_0 codes alone,
   dequantised inside the products.  The results are the same bit for bit either way.")

(defvar *dit-trace* nil
  "metal-dit.lisp's switch (src/metal-dit.lisp:114-117): when true, each velocity's largest
   values -- before the blocks the stream and txt_in's GELU rows, after each layer the stream,
   the attention's output and the MLP's inner rows -- and their counts of values that are not
   finite are printed after it: where a step first overflows.")

(defparameter +exn-profile-classes+ #("qkv" "attend" "out" "gate_up" "down" "ln_mod" "qkv_prep" "edge")
  "The library's kernel classes (EXN_PROF_* in exn_hip.h), in order.")

(defconstant +exn-q8-0+ 8)
(defconstant +exn-f32+ 0)
(defconstant +exn-bf16+ 30)

(defmacro exn-check (form)
  `(let ((status ,form))
     (unless (zerop status) (error "libexn-hip: ~A" (%exn-last-error)))))

(defun exn-out-pointer (fn &rest args)
  "Call FN with ARGS and a pointer cell; the cell's pointer."
  (let ((cell (make-array 1 :element-type '(unsigned-byte 64))))
    (sb-sys:with-pinned-objects (cell)
      (exn-check (apply fn (append args (list (sb-sys:vector-sap cell))))))
    (sb-sys:int-sap (aref cell 0))))

(defstruct (hdit (:constructor %make-hdit)) ctx handle gguf
  (keys (make-hash-table :test 'equal)))   ; prefix keys (EQUAL Lisp objects) -> 64-bit ids

(defun upload-dit (path &key (device 0))
  "The DiT in the GGUF at PATH on HIP device DEVICE."
  (let* ((g (open-dit path)) (file (il::map-file-vector path))
         (ctx (exn-out-pointer #'%exn-open device))
         (d (%make-hdit :ctx ctx :handle (exn-out-pointer #'%exn-dit-create ctx 32) :gguf g)))
    (dolist (name (gguf-tensor-order g))
      (let* ((ti (gguf-tensor g name)) (short (subseq name (length +dit-prefix+)))
             (dims (tensor-info-dims ti))
             (src (sb-sys:sap+ (sb-sys:vector-sap file) (+ (il::gguf-data-offset g) (il::tensor-info-offset ti)))))
        (sb-sys:with-pinned-objects (file)
          (if (null (rest dims))
              (let ((v (il::load-f32 g name)))          ; norm vectors as floats; the library adds text_norm's 1
                (sb-sys:with-pinned-objects (v)
                  (exn-check (%exn-dit-set (hdit-handle d) short +exn-f32+ (sb-sys:vector-sap v) (length v) 1))))
              (exn-check (%exn-dit-set (hdit-handle d) short
                                       (ecase (tensor-info-type ti) (:q8_0 +exn-q8-0+) (:f32 +exn-f32+) (:bf16 +exn-bf16+))
                                       src (first dims) (reduce #'* (rest dims))))))))
    (exn-check (%exn-dit-check (hdit-handle d)))
    d))

(defun print-dit-trace (d)
  "*dit-trace*'s lines for D's last velocity, in metal-dit.lisp's form (its trace-max, :119-124)."
  (let* ((rows (1+ 32)) (mx (f32vec (* 4 rows)))
         (bad (make-array (* 4 rows) :element-type '(signed-byte 64))))
    (sb-sys:with-pinned-objects (mx bad)
      (exn-check (%exn-dit-stats-read (hdit-handle d) (sb-sys:vector-sap mx) (sb-sys:vector-sap bad) (* 4 rows))))
    (flet ((one (name i)
             (format *error-output* " ~A ~,1F~:[~; (~D not finite)~]" name (aref mx i) (plusp (aref bad i)) (aref bad i))))
      (format *error-output* "~&before:")
      (one "x-all" 0)
      (when (or (plusp (aref mx 3)) (plusp (aref bad 3))) (one "h" 3))
      (terpri *error-output*)
      (loop for il from 0 below 32
            for r = (* 4 (1+ il))
            do (format *error-output* "~&layer ~D:" il) (one "x" r) (one "att" (+ r 1)) (one "ff" (+ r 2))
               (terpri *error-output*)))))

(defun add-gpu-profile (d table)
  "D's last velocity's GPU time by kernel class into TABLE (illatio's *gpu-profile*, seconds by
   name, which tenant-run reports for the request under EXN_PROFILE, src/tenant.lisp:53-62)."
  (let ((cell (make-array 4 :element-type 'double-float :initial-element 0d0))
        (n (make-array 1 :element-type '(signed-byte 64) :initial-element 0)))
    (sb-sys:with-pinned-objects (cell n)
      (loop for cls from 0 below (length +exn-profile-classes+)
            do (exn-check (%exn-dit-profile-read (hdit-handle d) cls (sb-sys:vector-sap cell) (sb-sys:vector-sap n)
                                                 (sb-sys:sap+ (sb-sys:vector-sap cell) 8)
                                                 (sb-sys:sap+ (sb-sys:vector-sap cell) 16)))
               (when (plusp (aref n 0))
                 (incf (gethash (format nil "exn:~A" (aref +exn-profile-classes+ cls)) table 0d0)
                       (/ (aref cell 0) 1d3)))))))

(defun dit-velocity (d context p latent h w sigma &key (prefix-key nil) ref)
  "cuda-dit.lisp's dit-velocity on the MI355X: the same arguments, the same result."
  (let ((v (f32vec (* 64 h w)))
        (profile (and (uiop:getenv "EXN_PROFILE") (boundp 'il::*gpu-profile*)
                      (hash-table-p (symbol-value 'il::*gpu-profile*)) (symbol-value 'il::*gpu-profile*)))
        (key (if prefix-key
                 (or (gethash prefix-key (hdit-keys d))
                     (setf (gethash prefix-key (hdit-keys d)) (1+ (hash-table-count (hdit-keys d)))))
                 0))
        (ref-latent (and ref (second ref))))
    (exn-check (%exn-dit-w8a8 (hdit-handle d) (if *int8* 1 0)))
    (exn-check (%exn-dit-resident (hdit-handle d) (if *hip-resident* 1 0)))
    (exn-check (%exn-dit-stats (hdit-handle d) (if *dit-trace* 1 0)))
    (exn-check (%exn-dit-profile (hdit-handle d) (if profile -1 0)))
    (sb-sys:with-pinned-objects (context latent v ref-latent)
      (exn-check (%exn-dit-velocity (hdit-handle d) (sb-sys:vector-sap context) p (sb-sys:vector-sap latent) h w
                                    (coerce sigma 'double-float) key
                                    (if ref (first ref) 0)
                                    (if ref (sb-sys:vector-sap ref-latent) (sb-sys:int-sap 0))
                                    (if ref (third ref) 0) (if ref (fourth ref) 0)
                                    (sb-sys:vector-sap v))))
    (when profile
      (add-gpu-profile d profile)
      (exn-check (%exn-dit-profile (hdit-handle d) 0)))
    (when *dit-trace* (print-dit-trace d))
    v))

(defun dit-release (d)
  "D's scratch and kept prompt keys and values freed (the weights stay)."
  (exn-check (%exn-dit-release (hdit-handle d))))
