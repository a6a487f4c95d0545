;;;; hip-encoder.lisp -- the prompt encoder's text model on an AMD MI355X through libexn-hip.so
;;;;
;;;; Loaded after src/encoder.lisp, it redefines only the text model's compute -- load-encoder
;;;; (:41), encoder-gpu-p (:50), call-with-picture-rows (:69) and encoder-states (:143), with
;;;; the reference's lambda lists -- so that encoder.lisp's own encode-prompt and
;;;; encode-edit-prompt (:55-141: the ids, the edit prompt's positions and mrope-table, the
;;;; system turn and the picture's rows left out) run unchanged over the library's forward
;;;; (exn_enc_*) in place of illatio's il::cuda-forward-n.  The model encode-prompt receives is
;;;; still illatio's (il::load-model: the vocabulary for il::tokenize, the width and rotary
;;;; settings it reads); the library's encoder for it is found in *hip-encoders*.  The picture's
;;;; rows go to the forward as arguments instead of through il::*after-embed* /
;;;; il::*after-layer*.  Loads after hip-dit.lisp and hip-vision.lisp, whose shared object,
;;;; status check and %exn-open it uses; listed in ex-nihilo.asd after them and encoder.lisp.

(in-package #:ex-nihilo)

(sb-alien:define-alien-routine ("exn_enc_create" %exn-enc-create) sb-alien:int
  (ctx sb-sys:system-area-pointer) (layers sb-alien:int) (rope-base sb-alien:double) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_set" %exn-enc-set) sb-alien:int
  (e sb-sys:system-area-pointer) (name sb-alien:c-string) (kind sb-alien:int)
  (data sb-sys:system-area-pointer) (d0 (sb-alien:signed 64)) (d1 (sb-alien:signed 64)))
(sb-alien:define-alien-routine ("exn_enc_check" %exn-enc-check) sb-alien:int (e sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_states" %exn-enc-states) sb-alien:int
  (e sb-sys:system-area-pointer) (ids sb-sys:system-area-pointer) (n sb-alien:int) (pos sb-sys:system-area-pointer)
  (pic0 sb-alien:int) (m sb-alien:int) (merged sb-sys:system-area-pointer) (deep sb-sys:system-area-pointer)
  (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_states_dev" %exn-enc-states-dev) sb-alien:int
  (e sb-sys:system-area-pointer) (ids sb-sys:system-area-pointer) (n sb-alien:int) (cs sb-sys:system-area-pointer)
  (pic0 sb-alien:int) (m sb-alien:int) (merged sb-sys:system-area-pointer) (deep sb-sys:system-area-pointer)
  (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_release" %exn-enc-release) sb-alien:int (e sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_resident" %exn-enc-resident) sb-alien:int
  (e sb-sys:system-area-pointer) (bf16 sb-alien:int))
(sb-alien:define-alien-routine ("exn_alloc" %exn-alloc) sb-alien:int
  (ctx sb-sys:system-area-pointer) (bytes (sb-alien:unsigned 64)) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_free" %exn-free) sb-alien:int
  (ctx sb-sys:system-area-pointer) (p sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_upload" %exn-upload) sb-alien:int
  (ctx sb-sys:system-area-pointer) (dst sb-sys:system-area-pointer) (src sb-sys:system-area-pointer)
  (bytes (sb-alien:unsigned 64)))
(sb-alien:define-alien-routine ("exn_download" %exn-download) sb-alien:int
  (ctx sb-sys:system-area-pointer) (dst sb-sys:system-area-pointer) (src sb-sys:system-area-pointer)
  (bytes (sb-alien:unsigned 64)))

(defvar *hip-encoders* (make-hash-table :test 'eq :weakness :key)
  "illatio's model (what load-encoder returns) -> (context . exn_enc handle) of its text model
   on the GPU.")

(defvar *hip-picture* nil
  "Inside call-with-picture-rows: (merged deep rows-in), the picture's rows for the forward.")

(defun load-encoder (path &key device (threads (il::default-thread-count)))
  "The prompt encoder in the qwen3vl GGUF at PATH: its text model on HIP device DEVICE (0 when
   NIL), every block's matrices as the file's Q8_0 records, its norms as floats.  Returns
   illatio's model of the file (the vocabulary, the widths and rotary settings encoder.lisp
   reads), the library's encoder recorded for it."
  (let* ((g (read-gguf path)) (file (il::map-file-vector path))
         (ctx (exn-out-pointer #'%exn-open (or device 0)))
         (e (exn-out-pointer #'%exn-enc-create ctx 36 (coerce (meta g "qwen3vl.rope.freq_base") 'double-float))))
    (dolist (name (gguf-tensor-order g))
      (let* ((ti (gguf-tensor g name)) (dims (tensor-info-dims ti)))
        (if (or (null (rest dims)) (eq (tensor-info-type ti) :f32))
            (let ((v (il::load-f32 g name)))
              (sb-sys:with-pinned-objects (v)
                (exn-check (%exn-enc-set e name +exn-f32+ (sb-sys:vector-sap v) (first dims) (reduce #'* (rest dims))))))
            (sb-sys:with-pinned-objects (file)
              (exn-check (%exn-enc-set e name (ecase (tensor-info-type ti) (:q8_0 +exn-q8-0+))
                                       (sb-sys:sap+ (sb-sys:vector-sap file)
                                                    (+ (il::gguf-data-offset g) (il::tensor-info-offset ti)))
                                       (first dims) (reduce #'* (rest dims))))))))
    (exn-check (%exn-enc-check e))
    (let ((model (il::load-model path :threads threads)))
      (setf (gethash model *hip-encoders*) (cons ctx e))
      model)))

(defun encoder-gpu-p (model)
  "Whether MODEL, the prompt encoder, runs on a GPU: here, whether load-encoder made it."
  (and (gethash model *hip-encoders*) t))

(defun call-with-picture-rows (model merged deep d rows-in fn)
  "FN called with the encoder's forward taking a picture's rows: MERGED's (the vision tower's)
   in place of the image pads after the embedding, DEEP's (a list of three) added after the first
   layers.  ROWS-IN: of a pass's first position and count, (values its first picture row, the
   picture's row there, how many), or NIL."
  (declare (ignore model d))
  (let ((*hip-picture* (list merged deep rows-in)))
    (funcall fn)))

(defun rope-cs (rope n)
  "illatio's rope rows (a position's 64 cosines, then its 64 sines) as the library's table: the
   cosine and sine of pair j at 2j and 2j + 1."
  (let ((cs (f32vec (* n 128))))
    (dotimes (s n cs)
      (dotimes (j 64)
        (setf (aref cs (+ (* s 128) (* 2 j))) (aref rope (+ (* s 128) j))
              (aref cs (+ (* s 128) (* 2 j) 1)) (aref rope (+ (* s 128) 64 j)))))))

(defun call-on-device (ctx arrays fn)
  "FN called with a device copy of each of ARRAYS (specialised vectors, or NIL for a null
   pointer); the copies freed after."
  (let ((saps '()))
    (unwind-protect
         (progn
           (dolist (a arrays)
             (if (null a)
                 (push (sb-sys:int-sap 0) saps)
                 (let ((bytes (max 4 (* 4 (length a)))))
                   (push (exn-out-pointer #'%exn-alloc ctx bytes) saps)
                   (sb-sys:with-pinned-objects (a)
                     (exn-check (%exn-upload ctx (first saps) (sb-sys:vector-sap a) (* 4 (length a))))))))
           (apply fn (reverse saps)))
      (dolist (p saps)
        (unless (zerop (sb-sys:sap-int p)) (%exn-free ctx p))))))

(defun encoder-states (model ids &key rope)
  "Every token's state after the text model's last block, before its final norm: (length IDS) x
   4096 floats.  ROPE: rope rows for the positions (mrope-table's, an edit prompt's), else text
   positions; inside call-with-picture-rows the picture's rows too."
  (destructuring-bind (ctx . e) (or (gethash model *hip-encoders*) (error "not a GPU encoder: ~A" model))
    (exn-check (%exn-enc-resident e (if *hip-resident* 1 0)))   ; hip-dit.lisp's switch
    (let* ((n (length ids))
           (iv (make-array n :element-type '(signed-byte 32) :initial-contents (coerce ids 'list)))
           (out (f32vec (* n 4096))))
      (multiple-value-bind (pic0 from m) (and *hip-picture* (funcall (third *hip-picture*) 0 n))
        (let* ((merged (and pic0 (subseq (first *hip-picture*) (* from 4096) (* (+ from m) 4096))))
               (deep (and pic0 (apply #'concatenate '(simple-array single-float (*))
                                      (mapcar (lambda (s) (subseq s (* from 4096) (* (+ from m) 4096)))
                                              (second *hip-picture*))))))
          (if (null rope)
              (sb-sys:with-pinned-objects (iv out merged deep)
                (exn-check (%exn-enc-states e (sb-sys:vector-sap iv) n (sb-sys:int-sap 0) (or pic0 0) (if pic0 m 0)
                                            (if merged (sb-sys:vector-sap merged) (sb-sys:int-sap 0))
                                            (if deep (sb-sys:vector-sap deep) (sb-sys:int-sap 0))
                                            (sb-sys:vector-sap out))))
              (call-on-device ctx (list iv (rope-cs rope n) merged deep out)
                              (lambda (di dcs dm dd dout)
                                (exn-check (%exn-enc-states-dev e di n dcs (or pic0 0) (if pic0 m 0) dm dd dout))
                                (sb-sys:with-pinned-objects (out)
                                  (exn-check (%exn-download ctx (sb-sys:vector-sap out) dout (* 4 n 4096)))))))))
      out)))

(defun encoder-release (model)
  "MODEL's scratch freed (the weights stay)."
  (exn-check (%exn-enc-release (cdr (gethash model *hip-encoders*)))))
